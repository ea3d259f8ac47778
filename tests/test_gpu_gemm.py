"""GPU parity of the verify-forward GEMM (vnx_gemm_bf16) against the fp64
product of the same bf16 inputs.

Bar: |y - ref| <= RTOL * sum_k |x_k w_k| per element (fp32 accumulation of
exact bf16 products, so the error is a few ulps of the running sums, far
below 1e-5 of that magnitude), plus one rounding of the output type (2^-8
relative for bf16, 2^-11 for fp16).  The SwiGLU epilogue is held to the same
bar propagated through silu(g) * u: RTOL * (1.1 * mag_g * |u| + |silu(g)| *
mag_u) times the routing weight (silu' <= 1.1), plus the output rounding."""
import ctypes

import numpy as np
import pytest
import torch

from versenext_amd import _lib

pytestmark = pytest.mark.gpu

RTOL = 1e-5
P = ctypes.c_void_p


def _say(*a):
    print(*a, flush=True)


def _rnd(dtype):
    return {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]


def _pack(w):
    """(batch, N, K) bf16 -> packed (batch, elems) bf16 and the batch stride."""
    L = _lib.lib()
    batch, N, K = w.shape
    elems = L.vnx_pack_bf16_size(N, K) // 2
    out = torch.empty((batch, elems), dtype=torch.bfloat16, device=w.device)
    st = P(torch.cuda.current_stream().cuda_stream)
    for z in range(batch):
        _lib.check(L.vnx_pack_bf16(P(w[z].data_ptr()), K, N, K, P(out[z].data_ptr()), st), "pack")
    return out, elems


def _gemm(x, w, M, N, K, batch, sxb, swb, y, ldy, syb, epi=0, comb=None):
    st = P(torch.cuda.current_stream().cuda_stream)
    wp, swb = _pack(w)
    rc = _lib.lib().vnx_gemm_bf16(P(x.data_ptr()), K, sxb, P(wp.data_ptr()), swb, M, N, K, batch, epi,
                                  P(comb.data_ptr()) if comb is not None else None, batch, P(y.data_ptr()),
                                  _lib.DTYPE_CODES[y.dtype], ldy, syb, st)
    torch.cuda.synchronize()
    return rc


def _inputs(hip, batch_x, batch_w, M, N, K, seed):
    g = torch.Generator(device=hip.torch_device)
    g.manual_seed(seed)
    x = torch.randn((batch_x, M, K), generator=g, device=hip.torch_device).to(torch.bfloat16)
    w = (torch.randn((batch_w, N, K), generator=g, device=hip.torch_device) * 0.05).to(torch.bfloat16)
    return x, w


@pytest.mark.parametrize("M,N,K,batch,shared_x,dtype", [
    (224, 2048, 1024, 1, False, torch.float32), (224, 1024, 2752, 1, False, torch.bfloat16),
    (37, 100, 192, 3, True, torch.float16), (224, 5504, 1024, 1, False, torch.bfloat16),
    (1, 64, 64, 2, False, torch.float32), (257, 33, 128, 1, False, torch.float32),
    # weight-streaming shape (256 x 128 workgroup tiles): many 128-column groups
    (224, 16384, 1024, 1, False, torch.float32), (300, 8192, 192, 1, False, torch.bfloat16),
    (224, 1024, 2688, 16, True, torch.bfloat16), (61, 16400, 64, 1, False, torch.float16)])
def test_plain(hip, M, N, K, batch, shared_x, dtype):
    _say(f"gemm M={M} N={N} K={K} batch={batch} shared_x={shared_x} out={dtype}")
    x, w = _inputs(hip, 1 if shared_x else batch, batch, M, N, K, seed=M + N + K)
    y = torch.empty((batch, M, N), dtype=dtype, device=hip.torch_device)
    _lib.check(_gemm(x, w, M, N, K, batch, 0 if shared_x else M * K, N * K, y, N, M * N), "gemm")
    torch.cuda.synchronize()
    xd = x.double().cpu().expand(batch, M, K)
    wd = w.double().cpu()
    ref = torch.bmm(xd, wd.transpose(1, 2))
    mag = torch.bmm(xd.abs(), wd.abs().transpose(1, 2))
    err = (y.double().cpu() - ref).abs()
    tol = RTOL * mag + _rnd(dtype) * ref.abs()
    worst = float((err / (mag + 1e-300)).max())
    assert bool((err <= tol + 1e-30).all()), f"worst err / mag = {worst:.3e}"
    _say(f"  worst err / mag = {worst:.2e}")


@pytest.mark.parametrize("M,H,K,batch,with_comb,dtype", [
    (224, 2752, 1024, 1, False, torch.bfloat16), (224, 2688, 1024, 4, True, torch.bfloat16),
    (30, 48, 128, 2, True, torch.float32), (5, 16, 64, 1, False, torch.float16)])
def test_swiglu_epilogue(hip, M, H, K, batch, with_comb, dtype):
    """W rows interleaved in blocks of 32 (16 gate rows, 16 up rows);
    y[m, j] = comb[m, z] * silu(gate_j) * up_j."""
    _say(f"gemm swiglu M={M} H={H} K={K} batch={batch} comb={with_comb} out={dtype}")
    N = 2 * H
    x, w = _inputs(hip, 1, batch, M, N, K, seed=H + K)
    comb = None
    if with_comb:
        g = torch.Generator(device=hip.torch_device)
        g.manual_seed(7)
        comb = torch.rand((M, batch), generator=g, device=hip.torch_device)
        comb[comb < 0.4] = 0.0
    y = torch.empty((batch, M, H), dtype=dtype, device=hip.torch_device)
    _lib.check(_gemm(x, w, M, N, K, batch, 0, N * K, y, H, M * H, epi=_lib.VNX_EPI_SWIGLU, comb=comb), "gemm")
    torch.cuda.synchronize()
    xd = x.double().cpu().expand(batch, M, K)
    wd = w.double().cpu()
    acc = torch.bmm(xd, wd.transpose(1, 2))                        # (batch, M, N)
    mag = torch.bmm(xd.abs(), wd.abs().transpose(1, 2))
    blk = torch.arange(N).view(-1, 32)
    gi, ui = blk[:, :16].reshape(-1), blk[:, 16:].reshape(-1)      # hidden j -> gate / up rows
    g_, u_ = acc[..., gi], acc[..., ui]
    silu = g_ * torch.sigmoid(g_)
    cw = comb.double().cpu().t().unsqueeze(-1) if comb is not None else torch.ones(batch, M, 1, dtype=torch.float64)
    ref = cw * silu * u_
    bound = cw * RTOL * (1.1 * mag[..., gi] * u_.abs() + silu.abs() * mag[..., ui]) + _rnd(dtype) * ref.abs()
    err = (y.double().cpu() - ref).abs()
    worst = float((err / (bound + 1e-300)).max())
    assert bool((err <= bound + 1e-30).all()), f"worst err / bound = {worst:.3e}"
    if comb is not None:
        assert bool((y.cpu()[cw.expand_as(ref) == 0] == 0).all())


def test_rejects_bad_shapes(hip):
    x, w = _inputs(hip, 1, 1, 4, 64, 64, seed=1)
    wp, _ = _pack(w)
    y = torch.empty((4, 64), dtype=torch.float32, device=hip.torch_device)
    st = P(torch.cuda.current_stream().cuda_stream)
    L = _lib.lib()
    # K not a multiple of 64
    assert L.vnx_gemm_bf16(P(x.data_ptr()), 64, 0, P(wp.data_ptr()), 0, 4, 64, 32, 1, 0, None, 1,
                           P(y.data_ptr()), _lib.VNX_F32, 64, 0, st) == _lib.VNX_ERR_UNSUPPORTED
    # SwiGLU needs N a multiple of 32
    assert L.vnx_gemm_bf16(P(x.data_ptr()), 64, 0, P(wp.data_ptr()), 0, 4, 48, 64, 1, 1, None, 1,
                           P(y.data_ptr()), _lib.VNX_F32, 64, 0, st) == _lib.VNX_ERR_INVALID_ARG
    # ldy shorter than a row
    assert L.vnx_gemm_bf16(P(x.data_ptr()), 64, 0, P(wp.data_ptr()), 0, 4, 64, 64, 1, 0, None, 1,
                           P(y.data_ptr()), _lib.VNX_F32, 32, 0, st) == _lib.VNX_ERR_INVALID_ARG
    # a batch stride shorter than one packed weight
    assert L.vnx_gemm_bf16(P(x.data_ptr()), 64, 0, P(wp.data_ptr()), 64, 4, 64, 64, 2, 0, None, 1,
                           P(y.data_ptr()), _lib.VNX_F32, 64, 0, st) == _lib.VNX_ERR_INVALID_ARG
    # packing needs K a multiple of 64
    assert L.vnx_pack_bf16(P(w.data_ptr()), 64, 64, 32, P(wp.data_ptr()), st) == _lib.VNX_ERR_UNSUPPORTED


@pytest.mark.parametrize("M,N,K,epi", [(224, 2048, 1024, 0), (224, 5504, 1024, 1), (37, 96, 192, 0),
                                       (5, 64, 2048, 1), (257, 40, 64, 0)])
def test_norm_input(hip, M, N, K, epi):
    """vnx_gemm_bf16_norm: the staged operand is bf16(x * w) exactly as torch
    rounds it, so the reference is that bf16 matrix times W in fp64, scaled by
    the fp64 rstd of the fp32 rows; the GEMM bar plus rstd's fp32 error
    (1e-6 relative) plus one bf16 rounding of the output."""
    _say(f"gemm norm M={M} N={N} K={K} epi={epi}")
    dev = hip.torch_device
    g = torch.Generator(device=dev)
    g.manual_seed(M + N + K)
    x = torch.randn((M, K), generator=g, device=dev) * 2.0
    nw = torch.rand((K,), generator=g, device=dev) + 0.5
    w = (torch.randn((1, N, K), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wp, _ = _pack(w)
    eps = 1e-6
    ncols = N // 2 if epi else N
    y = torch.empty((M, ncols), dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.lib().vnx_gemm_bf16_norm(P(x.data_ptr()), K, P(nw.data_ptr()), eps, P(wp.data_ptr()), M, N, K,
                                             epi, P(y.data_ptr()), ncols, P(torch.cuda.current_stream().cuda_stream)),
               "gemm_norm")
    torch.cuda.synchronize()
    xs = (x * nw).to(torch.bfloat16).double().cpu()                   # the staged operand
    xd = x.double().cpu()
    rstd = 1.0 / torch.sqrt((xd * xd).mean(dim=1, keepdim=True) + eps)
    wd = w[0].double().cpu()
    acc = (xs @ wd.t()) * rstd
    mag = (xs.abs() @ wd.abs().t()) * rstd
    if epi:
        blk = torch.arange(N).view(-1, 32)
        gi, ui = blk[:, :16].reshape(-1), blk[:, 16:].reshape(-1)
        g_, u_ = acc[:, gi], acc[:, ui]
        silu = g_ * torch.sigmoid(g_)
        ref = silu * u_
        tol = (RTOL + 1e-6) * (1.1 * mag[:, gi] * u_.abs() + silu.abs() * mag[:, ui]) + 2.0 ** -8 * ref.abs()
    else:
        ref = acc
        tol = (RTOL + 1e-6) * mag + 2.0 ** -8 * ref.abs()
    err = (y.double().cpu() - ref).abs()
    worst = float((err / (tol + 1e-300)).max())
    assert bool((err <= tol + 1e-30).all()), f"worst err / bound = {worst:.3e}"
    _say(f"  worst err / bound = {worst:.2e}")


@pytest.mark.parametrize("M,N,K", [(224, 2048, 1024), (37, 96, 192), (257, 40, 64), (7, 3072, 2048)])
def test_norm_embed_equals_two_calls(hip, M, N, K):
    """vnx_gemm_bf16_norm_embed against vnx_embed_rmsnorm followed by
    vnx_gemm_bf16_norm (checked against fp64 above): the residual rows it
    writes and the product must be bit-identical, since both stage bf16(x * w)
    of the same fp32 x = emb[id] * scale and scale by the same rstd.  Token
    ids outside the table are clamped, as vnx_embed_rmsnorm clamps them."""
    _say(f"gemm norm embed M={M} N={N} K={K}")
    dev = hip.torch_device
    g = torch.Generator(device=dev)
    g.manual_seed(3 * M + N + K)
    V, scale, eps = 500, 32.0, 1e-6
    emb = torch.randn((V, K), generator=g, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, V, (M,), generator=g, device=dev)
    ids[0], ids[M - 1] = -1, V + 3
    nw = torch.rand((K,), generator=g, device=dev) + 0.5
    w = (torch.randn((1, N, K), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wp, _ = _pack(w)
    L = _lib.lib()
    st = P(torch.cuda.current_stream().cuda_stream)
    outs = []
    for fused in (True, False):
        x = torch.full((M, K), 7.0, dtype=torch.float32, device=dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if fused:
            _lib.check(L.vnx_gemm_bf16_norm_embed(P(ids.data_ptr()), P(emb.data_ptr()), _lib.VNX_BF16, K, V, scale,
                                                  P(x.data_ptr()), K, P(nw.data_ptr()), eps, P(wp.data_ptr()), M, N,
                                                  K, P(y.data_ptr()), N, st), "gemm_norm_embed")
        else:
            h = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
            _lib.check(L.vnx_embed_rmsnorm(P(ids.data_ptr()), P(emb.data_ptr()), _lib.VNX_BF16, K, V, scale,
                                           P(nw.data_ptr()), eps, M, K, P(x.data_ptr()), K, P(h.data_ptr()),
                                           _lib.VNX_BF16, K, st), "embed_rmsnorm")
            _lib.check(L.vnx_gemm_bf16_norm(P(x.data_ptr()), K, P(nw.data_ptr()), eps, P(wp.data_ptr()), M, N, K, 0,
                                            P(y.data_ptr()), N, st), "gemm_norm")
        torch.cuda.synchronize()
        outs.append((x.cpu(), y.cpu()))
    assert torch.equal(outs[0][0], emb.cpu().float()[ids.cpu().clamp(0, V - 1)] * scale)
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


def test_norm_embed_rejects(hip):
    dev = hip.torch_device
    x = torch.zeros((4, 64), dtype=torch.float32, device=dev)
    emb = torch.zeros((8, 72), dtype=torch.bfloat16, device=dev)
    ids = torch.zeros(4, dtype=torch.int64, device=dev)
    nw = torch.ones(64, dtype=torch.float32, device=dev)
    wp = torch.zeros(64 * 64, dtype=torch.bfloat16, device=dev)
    y = torch.zeros((4, 64), dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    st = P(torch.cuda.current_stream().cuda_stream)

    def call(ids_p=P(ids.data_ptr()), dt=_lib.VNX_BF16, lde=72, vocab=8):
        return L.vnx_gemm_bf16_norm_embed(ids_p, P(emb.data_ptr()), dt, lde, vocab, 1.0, P(x.data_ptr()), 64,
                                          P(nw.data_ptr()), 1e-6, P(wp.data_ptr()), 4, 64, 64, P(y.data_ptr()), 64, st)
    assert call(ids_p=None) == _lib.VNX_ERR_INVALID_ARG
    assert call(vocab=0) == _lib.VNX_ERR_INVALID_ARG
    assert call(lde=32) == _lib.VNX_ERR_INVALID_ARG       # a row shorter than K
    assert call(dt=_lib.VNX_F32) == _lib.VNX_ERR_UNSUPPORTED
    assert call(lde=68) == _lib.VNX_ERR_UNSUPPORTED       # rows not 16-byte aligned


@pytest.mark.parametrize("M,N,K", [(224, 1024, 1024), (224, 1024, 2752), (9, 100, 64)])
def test_residual_epilogue(hip, M, N, K):
    """vnx_gemm_bf16_residual: res += x . W^T in fp32; the GEMM bar plus one
    fp32 rounding of the sum."""
    _say(f"gemm residual M={M} N={N} K={K}")
    x, w = _inputs(hip, 1, 1, M, N, K, seed=N + K)
    wp, _ = _pack(w)
    g = torch.Generator(device=hip.torch_device)
    g.manual_seed(3)
    res = torch.randn((M, N), generator=g, device=hip.torch_device)
    res0 = res.double().cpu()
    _lib.check(_lib.lib().vnx_gemm_bf16_residual(P(x.data_ptr()), K, P(wp.data_ptr()), M, N, K, P(res.data_ptr()), N,
                                                 P(torch.cuda.current_stream().cuda_stream)), "gemm_residual")
    torch.cuda.synchronize()
    xd, wd = x[0].double().cpu(), w[0].double().cpu()
    ref = res0 + xd @ wd.t()
    mag = xd.abs() @ wd.abs().t()
    err = (res.double().cpu() - ref).abs()
    assert bool((err <= RTOL * mag + 2.0 ** -24 * ref.abs() + 1e-30).all())

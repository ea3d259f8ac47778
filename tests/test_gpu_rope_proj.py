"""GPU parity of the INT4 q|k|v projection with RoPE and the KV-cache write
fused into its epilogue (vnx_gemv_w4_rope_kv, group-128 weights), against the
fp64 projection of
the same rounded inputs followed by NeoX rotate-half RoPE (the reference of
vnx_rope_kv, TriSparseAttention._apply_rope).

Bar per element: the GEMM bar carried through the rotation,
RTOL * (mag_own * |cos| + mag_partner * |sin|), plus fp32 rounding of the
rotation (1e-6 of |own cos| + |partner sin|) and one bf16 rounding of the
result (2^-8 relative).  Rows whose position falls at or past the cache
capacity are skipped: their q rows and cache rows keep a sentinel."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import quant as Q
from versenext_amd import _lib
from versenext_amd import model as VM

pytestmark = pytest.mark.gpu

RTOL = 1e-5
VP = ctypes.c_void_p
SENT = 7.0


def _say(*a):
    print(*a, flush=True)


def _st():
    return VP(torch.cuda.current_stream().cuda_stream)


def _setup(hip, B, n, H, Hkv, d, cap, T, seed):
    dev = hip.torch_device
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    lens = torch.randint(0, cap - n + 2, (B,), generator=g, dtype=torch.int32)
    lens[0] = cap - n + 1                    # its last row falls past the cache
    ang = torch.rand((T, d), generator=g, dtype=torch.float64) * 6.0
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    q = torch.full((B, H, n, d), SENT, dtype=torch.bfloat16, device=dev)
    kc = torch.full((B, Hkv, cap, d), SENT, dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, SENT)
    return lens, cos, sin, q, kc, vc


def _args(lens_d, cos_d, sin_d, q, kc, vc, n, H, Hkv, d, rope, cap):
    return _lib.RopeKvArgs(VP(lens_d.data_ptr()), n, H, Hkv, d, VP(cos_d.data_ptr()), VP(sin_d.data_ptr()),
                           cos_d.shape[0], rope, VP(q.data_ptr()), VP(kc.data_ptr()), VP(vc.data_ptr()),
                           kc.stride(0), kc.stride(1), kc.stride(2), cap)


def _check(x64, W64, lens, cos, sin, q, kc, vc, B, n, H, Hkv, d, rope, cap, rtol=RTOL):
    heads = H + 2 * Hkv
    acc = (x64 @ W64.t()).view(B, n, heads, d)
    mag = (x64.abs() @ W64.abs().t()).view(B, n, heads, d)
    half = d // 2
    pos = lens.long().view(B, 1) + torch.arange(n).view(1, n)
    ok = pos < cap
    pc = pos.clamp(max=cos.shape[0] - 1)
    c = cos.double()[pc].unsqueeze(2)
    s = sin.double()[pc].unsqueeze(2)
    rot = torch.cat([-acc[..., half:], acc[..., :half]], dim=-1)
    mrot = torch.cat([mag[..., half:], mag[..., :half]], dim=-1)
    rotated = torch.zeros(heads, dtype=torch.bool)
    if rope:
        rotated[:H + Hkv] = True
    rs = rotated.view(1, 1, heads, 1)
    ref = torch.where(rs, acc * c + rot * s, acc)
    arot = torch.where(rs, (acc * c).abs() + (rot * s).abs(), acc.abs())
    bound = torch.where(rs, rtol * (mag * c.abs() + mrot * s.abs()), rtol * mag) + 1e-6 * arot \
        + 2.0 ** -8 * ref.abs() + 1e-30
    qg, kg, vg = q.double().cpu(), kc.double().cpu(), vc.double().cpu()
    worst = 0.0
    for b in range(B):
        for i in range(n):
            if not ok[b, i]:
                assert bool((qg[b, :, i] == SENT).all())
                continue
            p = int(pos[b, i])
            for part, got in ((slice(0, H), qg[b, :, i]), (slice(H, H + Hkv), kg[b, :, p]),
                              (slice(H + Hkv, heads), vg[b, :, p])):
                err = (got - ref[b, i, part]).abs()
                bd = bound[b, i, part]
                worst = max(worst, float((err / bd).max()))
                assert bool((err <= bd).all()), f"row ({b}, {i}) worst err / bound {worst:.3e}"
    # cache rows that no token wrote keep the sentinel
    written = torch.zeros((B, cap), dtype=torch.bool)
    for b in range(B):
        for i in range(n):
            if ok[b, i]:
                written[b, int(pos[b, i])] = True
    assert bool((kg.permute(0, 2, 1, 3)[~written] == SENT).all())
    _say(f"  worst err / bound = {worst:.2e}")


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("B,n,H,Hkv,d,K", [(32, 1, 16, 8, 64, 1024), (20, 2, 4, 2, 64, 256), (3, 1, 2, 1, 128, 128),
                                           (40, 1, 3, 1, 16, 128),
                                           # (H + 2Hkv) d = 4608 rows: more 16-row tiles than CUs, so
                                           # the two-tiles-per-workgroup epilogue variant runs
                                           (8, 1, 56, 8, 64, 512), (24, 1, 56, 8, 64, 1024)])
def test_gemv_w4_rope_kv(hip, B, n, H, Hkv, d, K, norm):
    """norm: x is fp32 residual rows and RMSNorm(x) * w is fused (the staged
    operand fp16(x * w) as numpy rounds it, rows scaled by the fp64 rstd; the
    bar grows by rstd's fp32 error, 1e-6 relative)."""
    _say(f"gemv_w4_rope_kv B={B} n={n} H={H} Hkv={Hkv} d={d} K={K} norm={norm}")
    dev = hip.torch_device
    heads = H + 2 * Hkv
    N, M, cap, T = heads * d, B * n, 40, 48
    rng = np.random.default_rng(N + K)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    p, s = Q.quantize_int4_g(W, 128)
    perm = VM.rope_rows(heads, d, 8).numpy()
    pq = torch.from_numpy(np.ascontiguousarray(p[perm])).to(dev)
    sq = torch.from_numpy(np.ascontiguousarray(s[perm])).to(dev)
    lens, cos, sin, q, kc, vc = _setup(hip, B, n, H, Hkv, d, cap, T, seed=M + d)
    lens_d, cos_d, sin_d = lens.to(dev), cos.to(dev), sin.to(dev)
    rk = _args(lens_d, cos_d, sin_d, q, kc, vc, n, H, Hkv, d, 1, cap)
    if norm:
        x = rng.normal(0, 2.0, (M, K)).astype(np.float32)
        nw = (rng.random(K) + 0.5).astype(np.float32)
        xd, nwd = torch.from_numpy(x).to(dev), torch.from_numpy(nw).to(dev)
        _lib.check(_lib.lib().vnx_gemv_w4_rope_kv(VP(xd.data_ptr()), K, VP(nwd.data_ptr()), 1e-6, VP(pq.data_ptr()),
                                                  pq.stride(0), VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), M, N,
                                                  K, 128, ctypes.byref(rk), _st()), "gemv_w4_rope_kv norm")
        rstd = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
        x64 = torch.from_numpy((x * nw).astype(np.float16).astype(np.float64) * rstd)
    else:
        x16 = rng.normal(0, 1, (M, K)).astype(np.float16)
        xd = torch.from_numpy(x16).to(dev)
        _lib.check(_lib.lib().vnx_gemv_w4_rope_kv(VP(xd.data_ptr()), K, None, 0.0, VP(pq.data_ptr()), pq.stride(0),
                                                  VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), M, N, K, 128,
                                                  ctypes.byref(rk), _st()), "gemv_w4_rope_kv")
        x64 = torch.from_numpy(x16.astype(np.float64))
    torch.cuda.synchronize()
    Wd = torch.from_numpy(Q.dequantize_int4_g(p, s, (N, K), 128).astype(np.float64))
    _check(x64, Wd, lens, cos, sin, q, kc, vc, B, n, H, Hkv, d, 1, cap, rtol=RTOL + (1e-6 if norm else 0.0))


def test_rope_proj_rejects(hip):
    dev = hip.torch_device
    x = torch.zeros((4, 128), dtype=torch.float16, device=dev)
    wq = torch.zeros((64, 64), dtype=torch.uint8, device=dev)
    sc = torch.ones((64, 1), dtype=torch.float16, device=dev)
    lens = torch.zeros(4, dtype=torch.int32, device=dev)
    cs = torch.zeros((8, 16), dtype=torch.float32, device=dev)
    q = torch.zeros(4096, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    rk = _lib.RopeKvArgs(VP(lens.data_ptr()), 1, 2, 1, 8, VP(cs.data_ptr()), VP(cs.data_ptr()), 8, 1,
                         VP(q.data_ptr()), VP(q.data_ptr()), VP(q.data_ptr()), 64, 16, 16, 4)
    args = lambda N: (VP(x.data_ptr()), 128, None, 0.0, VP(wq.data_ptr()), 64, VP(sc.data_ptr()), _lib.VNX_F16, 1, 4,
                      N, 128, 128, ctypes.byref(rk), _st())
    # d = 8 is not a whole 16-row tile of rotate-half pairs
    assert L.vnx_gemv_w4_rope_kv(*args(32)) == _lib.VNX_ERR_UNSUPPORTED
    rk.d, rk.c_sr = 32, 32
    # N must be (H + 2 Hkv) d
    assert L.vnx_gemv_w4_rope_kv(*args(96)) == _lib.VNX_ERR_INVALID_ARG
    # rows must be whole sequences of n tokens
    rk.n = 3
    assert L.vnx_gemv_w4_rope_kv(*args(128)) == _lib.VNX_ERR_INVALID_ARG


@pytest.mark.parametrize("B,n,H,Hkv,d,K", [(32, 1, 16, 8, 64, 1024), (3, 1, 2, 1, 128, 128), (40, 1, 3, 1, 16, 256),
                                           (24, 1, 56, 8, 64, 1024)])
def test_gemv_w4_rope_kv_embed_equals_two_calls(hip, B, n, H, Hkv, d, K):
    """vnx_gemv_w4_rope_kv_embed against vnx_embed_rmsnorm followed by the
    norm form of vnx_gemv_w4_rope_kv (itself checked against the fp64
    projection above): the residual rows it writes, the q rows and the cache
    rows must be bit-identical, since both stage fp16(x * w) of the same fp32
    x = emb[id] * scale and scale by the same rstd.  Token ids outside the
    table are clamped, as vnx_embed_rmsnorm clamps them."""
    _say(f"gemv_w4_rope_kv_embed B={B} n={n} H={H} Hkv={Hkv} d={d} K={K}")
    dev = hip.torch_device
    heads = H + 2 * Hkv
    N, M, cap, T, V, scale = heads * d, B * n, 40, 48, 300, 1.7
    rng = np.random.default_rng(3 * N + K)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    p, s = Q.quantize_int4_g(W, 128)
    perm = VM.rope_rows(heads, d, 8).numpy()
    pq = torch.from_numpy(np.ascontiguousarray(p[perm])).to(dev)
    sq = torch.from_numpy(np.ascontiguousarray(s[perm])).to(dev)
    emb = torch.from_numpy(rng.normal(0, 1.0, (V, K)).astype(np.float32)).to(torch.bfloat16).to(dev)
    ids = torch.from_numpy(rng.integers(0, V, M)).to(dev)
    ids[0], ids[M - 1] = -3, V + 5
    nwd = torch.from_numpy((rng.random(K) + 0.5).astype(np.float32)).to(dev)
    L = _lib.lib()
    outs = []
    for fused in (True, False):
        lens, cos, sin, q, kc, vc = _setup(hip, B, n, H, Hkv, d, cap, T, seed=M + d)
        lens_d, cos_d, sin_d = lens.to(dev), cos.to(dev), sin.to(dev)
        rk = _args(lens_d, cos_d, sin_d, q, kc, vc, n, H, Hkv, d, 1, cap)
        x = torch.full((M, K), SENT, dtype=torch.float32, device=dev)
        if fused:
            _lib.check(L.vnx_gemv_w4_rope_kv_embed(
                VP(ids.data_ptr()), VP(emb.data_ptr()), _lib.VNX_BF16, K, V, scale, VP(x.data_ptr()), K,
                VP(nwd.data_ptr()), 1e-6, VP(pq.data_ptr()), pq.stride(0), VP(sq.data_ptr()), _lib.VNX_F16,
                sq.stride(0), M, N, K, 128, ctypes.byref(rk), _st()), "gemv_w4_rope_kv_embed")
        else:
            y = torch.empty((M, K), dtype=torch.float16, device=dev)
            _lib.check(L.vnx_embed_rmsnorm(
                VP(ids.data_ptr()), VP(emb.data_ptr()), _lib.VNX_BF16, K, V, scale, VP(nwd.data_ptr()), 1e-6, M, K,
                VP(x.data_ptr()), K, VP(y.data_ptr()), _lib.VNX_F16, K, _st()), "embed_rmsnorm")
            _lib.check(L.vnx_gemv_w4_rope_kv(VP(x.data_ptr()), K, VP(nwd.data_ptr()), 1e-6, VP(pq.data_ptr()),
                                             pq.stride(0), VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), M, N,
                                             K, 128, ctypes.byref(rk), _st()), "gemv_w4_rope_kv norm")
        torch.cuda.synchronize()
        outs.append((x.cpu(), q.cpu(), kc.cpu(), vc.cpu()))
    xe = emb.cpu().float()[ids.cpu().clamp(0, V - 1)] * scale
    assert torch.equal(outs[0][0], xe)
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


def test_rope_proj_embed_rejects(hip):
    dev = hip.torch_device
    x = torch.zeros((4, 128), dtype=torch.float32, device=dev)
    emb = torch.zeros((8, 128), dtype=torch.bfloat16, device=dev)
    ids = torch.zeros(4, dtype=torch.int64, device=dev)
    nw = torch.ones(128, dtype=torch.float32, device=dev)
    wq = torch.zeros((64, 64), dtype=torch.uint8, device=dev)
    sc = torch.ones((64, 1), dtype=torch.float16, device=dev)
    lens = torch.zeros(4, dtype=torch.int32, device=dev)
    cs = torch.zeros((8, 32), dtype=torch.float32, device=dev)
    q = torch.zeros(4096, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    rk = _lib.RopeKvArgs(VP(lens.data_ptr()), 1, 1, 0, 32, VP(cs.data_ptr()), VP(cs.data_ptr()), 8, 1,
                         VP(q.data_ptr()), VP(q.data_ptr()), VP(q.data_ptr()), 64, 32, 32, 4)

    def call(ids_p=VP(ids.data_ptr()), dt=_lib.VNX_BF16, lde=128, vocab=8, nw_p=VP(nw.data_ptr())):
        return L.vnx_gemv_w4_rope_kv_embed(ids_p, VP(emb.data_ptr()), dt, lde, vocab, 1.0, VP(x.data_ptr()), 128,
                                           nw_p, 1e-6, VP(wq.data_ptr()), 64, VP(sc.data_ptr()), _lib.VNX_F16, 1, 4,
                                           64, 128, 128, ctypes.byref(rk), _st())
    assert call(ids_p=None) == _lib.VNX_ERR_INVALID_ARG
    assert call(nw_p=None) == _lib.VNX_ERR_INVALID_ARG
    assert call(vocab=0) == _lib.VNX_ERR_INVALID_ARG
    assert call(lde=64) == _lib.VNX_ERR_INVALID_ARG       # a row shorter than K
    assert call(dt=_lib.VNX_F16) == _lib.VNX_ERR_UNSUPPORTED
    assert call(lde=132) == _lib.VNX_ERR_UNSUPPORTED      # rows not 16-byte aligned

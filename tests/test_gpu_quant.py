"""GPU parity of the weight-only quantized path against oracle/quant.py.

Bar: the GPU quantizers and the dequantization kernels are bit-exact with the
oracle; the GEMV (fp16 activations, fp32 accumulation on the matrix cores)
agrees with the fp64 product of the same fp16 activations and dequantized
weights within 1e-5 * sum_k |x_k w_k| per output (the fp32 tolerance of the
north star, relative to the sum of magnitudes the rounding acts on)."""
import numpy as np
import pytest
import torch

from oracle import quant as Q
from versenext_amd import quant as VQ

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def _say(*a):
    print(*a, flush=True)


def _weights(N, K, seed, std=0.02):
    w = np.random.default_rng(seed).normal(0, std, (N, K)).astype(np.float32)
    # exact ties for round-half-to-even in a few rows: multiples of scale/2
    w[0, :8] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 3.5, -3.5, 7.0], np.float32) * std
    return w


@pytest.mark.parametrize("kind", ["int8", "int4", "int4_g128"])
def test_gpu_quantizers_match_oracle(hip, kind):
    _say(f"quantizer {kind}")
    w = _weights(300, 512, 1)
    wt = torch.from_numpy(w).to(hip.torch_device)
    if kind == "int8":
        q, s = VQ.quantize_int8(wt)
        qo, so = Q.quantize_int8(w)
        assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)
    elif kind == "int4":
        q, s = VQ.quantize_int4(wt)
        qo, so = Q.quantize_int4(w)
        assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)
    else:
        q, s = VQ.quantize_int4_g(wt, 128)
        qo, so = Q.quantize_int4_g(w, 128)
        assert np.array_equal(q.cpu().numpy(), qo)
        assert np.array_equal(s.cpu().numpy().view(np.uint16), so.view(np.uint16))


@pytest.mark.parametrize("kind", ["int8", "int4", "int4_g128"])
def test_dequant_kernels_bit_exact(hip, kind):
    _say(f"dequant {kind}")
    N, K = 257, 1024
    w = _weights(N, K, 2)
    if kind == "int8":
        q, s = Q.quantize_int8(w)
        got = hip.dequant_w8(torch.from_numpy(q), torch.from_numpy(s.reshape(-1))).cpu().numpy()
        ref = Q.dequantize_int8(q, s)
    elif kind == "int4":
        p, s = Q.quantize_int4(w)
        got = hip.dequant_w4(torch.from_numpy(p), torch.from_numpy(s), K, K).cpu().numpy()
        ref = Q.dequantize_int4(p, s, (N, K))
    else:
        p, s = Q.quantize_int4_g(w, 128)
        got = hip.dequant_w4(torch.from_numpy(p), torch.from_numpy(s), K, 128).cpu().numpy()
        ref = Q.dequantize_int4_g(p, s, (N, K), 128)
    assert got.dtype == np.float32 and np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


_QCACHE = {}


def _quantized(kind, N, K, seed):
    """Oracle-quantized weights, cached (the full-size head is 1 GB in fp32)."""
    key = (kind, N, K, seed)
    if key not in _QCACHE:
        if len(_QCACHE) > 4:
            _QCACHE.clear()
        w = _weights(N, K, seed)
        if kind == "int8":
            _QCACHE[key] = Q.quantize_int8(w)
        elif kind == "int4":
            _QCACHE[key] = Q.quantize_int4(w)
        else:
            _QCACHE[key] = Q.quantize_int4_g(w, 128)
        del w
    return _QCACHE[key]


def _gemv_check(hip, kind, N, K, B, seed, rows=None):
    x16 = np.random.default_rng(seed + B).normal(0, 1, (B, K)).astype(np.float16)
    xt = torch.from_numpy(x16)
    if kind == "int8":
        q, s = _quantized(kind, N, K, seed)
        y = hip.gemv_w8(xt, torch.from_numpy(q), torch.from_numpy(s.reshape(-1)))
        wd = lambda r: Q.dequantize_int8(q[r], s[r])  # noqa: E731
    elif kind == "int4":
        p, s = _quantized(kind, N, K, seed)
        y = hip.gemv_w4(xt, torch.from_numpy(p), torch.from_numpy(s), K)
        wd = lambda r: Q.dequantize_int4(p[r], s[r], (len(r), K))  # noqa: E731
    else:
        p, s = _quantized(kind, N, K, seed)
        y = hip.gemv_w4(xt, torch.from_numpy(p), torch.from_numpy(s), 128)
        wd = lambda r: Q.dequantize_int4_g(p[r], s[r], (len(r), K), 128)  # noqa: E731
    y = y.cpu().numpy()
    assert y.shape == (B, N) and y.dtype == np.float32
    r = np.arange(N) if rows is None else rows
    W = wd(r)
    ref = Q.gemv_ref(x16, W)
    mag = Q.gemv_abs(x16, W)
    err = np.abs(y[:, r].astype(np.float64) - ref)
    worst = float(np.max(err / (mag + 1e-30)))
    _say(f"  {kind} N={N} K={K} B={B}: max err / sum|xw| = {worst:.2e}")
    assert np.all(err <= RTOL * mag + 1e-30), worst


@pytest.mark.parametrize("kind", ["int8", "int4", "int4_g128"])
@pytest.mark.parametrize("N,K,B", [(4096, 1024, 1), (1000, 384, 3), (1024, 4096, 8), (333, 512, 17),
                                   (512, 1024, 32), (256, 256, 40), (8192, 1024, 32), (1024, 4096, 32),
                                   (40000, 256, 20), (33005, 512, 17), (40003, 1024, 32)])
def test_gemv_parity(hip, kind, N, K, B):
    _gemv_check(hip, kind, N, K, B, seed=N + K + B)


@pytest.mark.parametrize("kind", ["int4_g128", "int8"])
@pytest.mark.parametrize("B", [1, 8, 32])
def test_gemv_tied_head_full_size(hip, kind, B):
    """Config 4's tied LM head, 248,320 x 1024, checked on 4096 sampled rows
    (including both ends and a partial last tile)."""
    N, K = 248320, 1024
    rows = np.unique(np.concatenate([np.arange(16), np.arange(N - 40, N),
                                     np.random.default_rng(B).choice(N, 4040, replace=False)]))
    _gemv_check(hip, kind, N, K, B, seed=5, rows=rows)


def test_quantized_linear_forward(hip):
    _say("QuantizedLinear")
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, (640, 256)).astype(np.float32)
    b = rng.normal(0, 1, 640).astype(np.float32)
    x = rng.normal(0, 1, (2, 3, 256)).astype(np.float32)
    for qtype in VQ.QuantizedLinear.QTYPES:
        ql = VQ.QuantizedLinear(w, b, qtype=qtype)
        y = ql(torch.from_numpy(x)).cpu().numpy()
        wd = ql.dequantize().cpu().numpy().astype(np.float64)
        x16 = x.astype(np.float16).astype(np.float64)
        ref = x16 @ wd.T + b
        assert y.shape == (2, 3, 640)
        assert np.all(np.abs(y - ref) <= RTOL * (np.abs(x16) @ np.abs(wd).T) + 1e-6)


def test_gemv_rejects_bad_shapes(hip):
    x = torch.zeros((2, 100), dtype=torch.float16)
    with pytest.raises(ValueError):
        hip.gemv_w8(x, torch.zeros((8, 100), dtype=torch.int8), torch.ones(8))  # K % 128 != 0


@pytest.mark.parametrize("H,K,B", [(4096, 1024, 32), (4096, 1024, 1), (64, 256, 17), (1000, 512, 40),
                                   (2056, 1024, 32), (2056, 2048, 7)])
def test_gemv_swiglu_parity(hip, H, K, B):
    """vnx_gemv_w4_swiglu: the group-128 GEMV of a [gate; up] weight whose rows
    are interleaved in blocks of 8 gate + 8 up rows, with silu(gate) * up in
    the epilogue (fp16 out).  Bar: the GEMV bar carried through silu(g) * u
    (|silu'| <= 1.1) plus one fp16 rounding (and half an fp16 subnormal step)."""
    import ctypes
    from versenext_amd import _lib
    _say(f"gemv swiglu H={H} K={K} B={B}")
    N = 2 * H
    p, s = _quantized("int4_g128", N, K, seed=H + K)
    x16 = np.random.default_rng(B).normal(0, 1, (B, K)).astype(np.float16)
    perm = np.arange(N).reshape(2, H // 8, 8).transpose(1, 0, 2).reshape(-1)   # packed row -> source row
    dev = hip.torch_device
    pq = torch.from_numpy(np.ascontiguousarray(p[perm])).to(dev)
    sq = torch.from_numpy(np.ascontiguousarray(s[perm])).to(dev)
    xt = torch.from_numpy(x16).to(dev)
    y = torch.full((B, H), float("nan"), dtype=torch.float16, device=dev)
    VP = ctypes.c_void_p
    _lib.check(_lib.lib().vnx_gemv_w4_swiglu(VP(xt.data_ptr()), K, None, 0.0, VP(pq.data_ptr()), pq.stride(0),
                                             VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), B, N, K, 128,
                                             VP(y.data_ptr()), H, VP(torch.cuda.current_stream().cuda_stream)),
               "gemv_w4_swiglu")
    torch.cuda.synchronize()
    W = Q.dequantize_int4_g(p, s, (N, K), 128)
    acc, mag = Q.gemv_ref(x16, W), Q.gemv_abs(x16, W)          # (B, N) fp64, source row order
    g, u = acc[:, :H], acc[:, H:]
    silu = g / (1.0 + np.exp(-g))
    ref = silu * u
    bound = RTOL * (1.1 * mag[:, :H] * np.abs(u) + np.abs(silu) * mag[:, H:]) + 2.0 ** -11 * np.abs(ref) + 2.0 ** -25
    got = y.cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    worst = float(np.max(err / bound))
    _say(f"  worst err / bound = {worst:.2e}")
    assert np.all(err <= bound), worst
    # rejects a weight whose rows are not whole 16-row blocks
    assert _lib.lib().vnx_gemv_w4_swiglu(VP(xt.data_ptr()), K, None, 0.0, VP(pq.data_ptr()), pq.stride(0),
                                         VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), B, N - 8, K, 128,
                                         VP(y.data_ptr()), H,
                                         VP(torch.cuda.current_stream().cuda_stream)) == _lib.VNX_ERR_UNSUPPORTED


@pytest.mark.parametrize("H,K,B", [(4096, 1024, 32), (64, 256, 17), (1000, 512, 40), (2056, 1024, 20)])
def test_gemv_swiglu_norm_input(hip, H, K, B):
    """vnx_gemv_w4_swiglu with norm_w: the staged operand is fp16(x * w) as
    numpy rounds the fp32 product, so the reference is that fp16 matrix times
    the dequantized W in fp64, scaled by the fp64 rstd of the fp32 rows; the
    SwiGLU bar of the plain test plus rstd's fp32 error (1e-6 relative)."""
    import ctypes
    from versenext_amd import _lib
    _say(f"gemv swiglu norm H={H} K={K} B={B}")
    N = 2 * H
    p, s = _quantized("int4_g128", N, K, seed=H + K + 1)
    rng = np.random.default_rng(B + 3)
    x = (rng.normal(0, 2.0, (B, K))).astype(np.float32)
    nw = (rng.random(K) + 0.5).astype(np.float32)
    eps = 1e-6
    perm = np.arange(N).reshape(2, H // 8, 8).transpose(1, 0, 2).reshape(-1)
    dev = hip.torch_device
    pq = torch.from_numpy(np.ascontiguousarray(p[perm])).to(dev)
    sq = torch.from_numpy(np.ascontiguousarray(s[perm])).to(dev)
    xt, nwt = torch.from_numpy(x).to(dev), torch.from_numpy(nw).to(dev)
    y = torch.full((B, H), float("nan"), dtype=torch.float16, device=dev)
    VP = ctypes.c_void_p
    _lib.check(_lib.lib().vnx_gemv_w4_swiglu(VP(xt.data_ptr()), K, VP(nwt.data_ptr()), eps, VP(pq.data_ptr()),
                                             pq.stride(0), VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), B, N, K,
                                             128, VP(y.data_ptr()), H, VP(torch.cuda.current_stream().cuda_stream)),
               "gemv_w4_swiglu norm")
    torch.cuda.synchronize()
    xs = (x * nw).astype(np.float16)
    rstd = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + eps)
    W = Q.dequantize_int4_g(p, s, (N, K), 128)
    acc, mag = Q.gemv_ref(xs, W) * rstd, Q.gemv_abs(xs, W) * rstd
    g, u = acc[:, :H], acc[:, H:]
    silu = g / (1.0 + np.exp(-g))
    ref = silu * u
    bound = (RTOL + 1e-6) * (1.1 * mag[:, :H] * np.abs(u) + np.abs(silu) * mag[:, H:]) + 2.0 ** -11 * np.abs(ref) \
        + 2.0 ** -25
    err = np.abs(y.cpu().numpy().astype(np.float64) - ref)
    worst = float(np.max(err / bound))
    _say(f"  worst err / bound = {worst:.2e}")
    assert np.all(err <= bound), worst


@pytest.mark.parametrize("N,K,B", [(1024, 1024, 32), (1024, 4096, 32), (100, 256, 40), (4104, 1024, 32),
                                   (4104, 2048, 9), (1000, 3072, 5), (512, 8192, 17)])
def test_gemv_residual(hip, N, K, B):
    """vnx_gemv_w4_residual: res += x . W^T (fp32); the GEMV bar plus one fp32
    rounding of the sum."""
    import ctypes
    from versenext_amd import _lib
    _say(f"gemv residual N={N} K={K} B={B}")
    p, s = _quantized("int4_g128", N, K, seed=N + K + 2)
    rng = np.random.default_rng(B + 5)
    x16 = rng.normal(0, 1, (B, K)).astype(np.float16)
    res0 = rng.normal(0, 1, (B, N)).astype(np.float32)
    dev = hip.torch_device
    pq, sq = torch.from_numpy(p).to(dev), torch.from_numpy(s).to(dev)
    xt, res = torch.from_numpy(x16).to(dev), torch.from_numpy(res0).to(dev)
    VP = ctypes.c_void_p
    _lib.check(_lib.lib().vnx_gemv_w4_residual(VP(xt.data_ptr()), K, VP(pq.data_ptr()), pq.stride(0),
                                               VP(sq.data_ptr()), _lib.VNX_F16, sq.stride(0), B, N, K, 128,
                                               VP(res.data_ptr()), N, VP(torch.cuda.current_stream().cuda_stream)),
               "gemv_w4_residual")
    torch.cuda.synchronize()
    W = Q.dequantize_int4_g(p, s, (N, K), 128)
    ref = res0.astype(np.float64) + Q.gemv_ref(x16, W)
    mag = Q.gemv_abs(x16, W)
    err = np.abs(res.cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= RTOL * mag + 2.0 ** -24 * np.abs(ref) + 1e-30)


def _tiles_ref(p, N, K):
    """vnx_pack_w4_tiles' layout restated from its definition in include/vnx.h:
    tile t, piece g, lane l = the 16 bytes W[16t + l % 16][64g + 16(l / 16) ..]
    of the row-major packing, each nibble XOR 8 (offset form); rows past N
    hold q = 0 (0x88 bytes)."""
    tiles = (N + 15) // 16
    full = np.full((tiles * 16, K // 2), 0x00, np.uint8)
    full[:N] = p
    a = full.reshape(tiles, 16, K // 128, 4, 16)          # t, m, g, kq, byte
    a = a.transpose(0, 2, 3, 1, 4)                          # t, g, kq, m, byte -> lane = kq*16 + m
    return (a.reshape(-1) ^ 0x88).astype(np.uint8)


@pytest.mark.parametrize("N,K", [(1000, 512), (40003, 1024), (4096, 1024)])
def test_pack_w4_tiles_layout(hip, N, K):
    p, s = _quantized("int4_g128", N, K, 61)
    got = hip.pack_w4_tiles(torch.from_numpy(p), K).cpu().numpy()
    assert got.size == hip._L.vnx_w4_tiles_bytes(N, K) == (N + 15) // 16 * 16 * K // 2
    assert np.array_equal(got, _tiles_ref(p, N, K))


@pytest.mark.parametrize("N,K,B", [(4096, 1024, 1), (1000, 512, 3), (33005, 512, 17), (40003, 1024, 32),
                                   (40003, 1024, 40), (65536, 1024, 16), (248320, 1024, 1), (248320, 1024, 8),
                                   (248320, 1024, 32)])
def test_gemv_w4_tiles_equals_row_layout(hip, N, K, B):
    """vnx_gemv_w4_tiles on the tiled copy equals the fp64 product of the
    oracle's dequantized weights within the GEMV bar on sampled rows (both
    ends and a partial last tile included), and, from 32,768 rows (where
    vnx_gemv_w4 runs its streaming form: the same products summed in the
    same order), vnx_gemv_w4 on the row layout bit for bit."""
    p, s = _quantized("int4_g128", N, K, 7)
    x16 = np.random.default_rng(N + B).normal(0, 1, (B, K)).astype(np.float16)
    xt = torch.from_numpy(x16)
    wt = hip.pack_w4_tiles(torch.from_numpy(p), K)
    y = hip.gemv_w4_tiles(xt, wt, torch.from_numpy(s), N, K).cpu().numpy()
    assert y.shape == (B, N)
    if N >= 32768:
        y_rows = hip.gemv_w4(xt, torch.from_numpy(p), torch.from_numpy(s), 128).cpu().numpy()
        assert np.array_equal(y.view(np.uint32), y_rows.view(np.uint32))
    r = np.unique(np.concatenate([np.arange(min(N, 40)), np.arange(max(0, N - 40), N),
                                  np.random.default_rng(B).choice(N, min(N, 2000), replace=False)]))
    W = Q.dequantize_int4_g(p[r], s[r], (len(r), K), 128)
    ref = Q.gemv_ref(x16, W)
    mag = Q.gemv_abs(x16, W)
    err = np.abs(y[:, r].astype(np.float64) - ref)
    worst = float(np.max(err / (mag + 1e-30)))
    _say(f"  tiles N={N} K={K} B={B}: max err / sum|xw| = {worst:.2e}")
    assert np.all(err <= RTOL * mag + 1e-30), worst


@pytest.mark.parametrize("N,K,B", [(1000, 512, 3), (40003, 1024, 32), (248320, 1024, 32)])
def test_gemv_w4_tiles_bf16_out_is_rounded_fp32(hip, N, K, B):
    """vnx_gemv_w4_tiles_out with bf16 output writes the fp32 output of the
    same product rounded to nearest even, bit for bit (torch's fp32 -> bf16
    cast rounds the same way)."""
    p, s = _quantized("int4_g128", N, K, 11)
    x16 = np.random.default_rng(N + 3 * B).normal(0, 1, (B, K)).astype(np.float16)
    xt = torch.from_numpy(x16)
    wt = hip.pack_w4_tiles(torch.from_numpy(p), K)
    y32 = hip.gemv_w4_tiles(xt, wt, torch.from_numpy(s), N, K)
    y16 = hip.gemv_w4_tiles(xt, wt, torch.from_numpy(s), N, K, out_dtype=torch.bfloat16)
    assert y16.dtype == torch.bfloat16 and tuple(y16.shape) == (B, N)
    assert torch.equal(y16.cpu().view(torch.int16), y32.to(torch.bfloat16).cpu().view(torch.int16))


def test_gemv_w4_tiles_rejects_bad_shapes(hip):
    p, s = _quantized("int4_g128", 64, 256, 3)
    wt = hip.pack_w4_tiles(torch.from_numpy(p), 256)
    with pytest.raises(ValueError):   # K must be 512 or 1024
        hip.gemv_w4_tiles(torch.zeros((1, 256), dtype=torch.float16), wt, torch.from_numpy(s), 64, 256)

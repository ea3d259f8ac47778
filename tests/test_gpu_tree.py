"""GPU parity of the tree-verify attention kernel (vnx_tree_attn) against
oracle/tree.py.

Bar: with fp32 output, |out - ref| <= RTOL * sum_j p_j |v_j| per element,
where ref is the fp64 attention of the same bf16 inputs.  The kernel's error
sources are the fp32 dot products (exact bf16 x bf16 products, fp32 sums),
exp2 on the transcendental unit, and P carried as bf16 hi + lo parts
(relative error <= 2^-17), each well under 1e-5 of the magnitude the
rounding acts on, so RTOL = 2e-5 leaves a factor of ~4 over the worst case
measured.  With bf16 output the result is additionally rounded once:
|out - ref| <= 2^-8 |ref| + RTOL * mag.  (The north star's bf16 bar is 2e-2.)"""
import numpy as np
import pytest
import torch

from oracle import tree as OT
from versenext_amd import _lib
from versenext_amd import tree as T

pytestmark = pytest.mark.gpu

RTOL = 2e-5


def _say(*a):
    print(*a, flush=True)


def _bf16(rng, shape, std=1.0):
    return torch.from_numpy(rng.normal(0, std, shape).astype(np.float32)).to(torch.bfloat16)


def _np(t):
    return t.float().cpu().numpy() if t is not None else None


def _check(out, ref, mag, bf16=False):
    o = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(o - ref)
    rnd = 2.0 ** -8 if bf16 else (2.0 ** -11 if out.dtype == torch.float16 else 0.0)
    tol = RTOL * mag + rnd * np.abs(ref)
    worst = float(np.max(err / (mag + 1e-300)))
    assert np.all(err <= tol + 1e-30), f"worst err / mag = {worst:.3e}"
    return worst


def _run(hip, B, H, Hkv, N, Tp, d, parent=None, seed=0, out_dtype=torch.float32, per_batch=False,
         cache_extra=0, inplace=False, std=1.0, T2=0, gates=(0.3, 0.8), waves=0, splits=0):
    _say(f"tree_attn B={B} H={H} Hkv={Hkv} N={N} Tp={Tp} d={d} out={out_dtype} per_batch={per_batch} "
         f"cache_extra={cache_extra} inplace={inplace} T2={T2} waves={waves} splits={splits}")
    rng = np.random.default_rng(seed)
    par = T.tree_from_branching((4, 3, 2)) if parent is None else np.asarray(parent, np.int32)
    assert par.size == N
    q = _bf16(rng, (B, H, N, d), std)
    Tcap = Tp + N + cache_extra
    kbuf = _bf16(rng, (B, Hkv, Tcap, d), std)
    vbuf = _bf16(rng, (B, Hkv, Tcap, d))
    dev = hip.torch_device
    kbuf, vbuf, q = kbuf.to(dev), vbuf.to(dev), q.to(dev)
    if inplace:  # tree rows written into the cache right after the prefix
        kc, vc = kbuf[:, :, :Tp], vbuf[:, :, :Tp]
        kt, vt = kbuf[:, :, Tp:Tp + N], vbuf[:, :, Tp:Tp + N]
    else:
        kc, vc = kbuf[:, :, :Tp], vbuf[:, :, :Tp]
        kt = _bf16(rng, (B, Hkv, N, d), std).to(dev)
        vt = _bf16(rng, (B, Hkv, N, d)).to(dev)
    if per_batch:
        words = np.stack([T.ancestor_words(par if b % 2 == 0 else T.chain(N)) for b in range(B)])
    else:
        words = T.ancestor_words(par)
    seg2 = None
    if T2:
        seg2 = (_bf16(rng, (1, Hkv, T2, d), std).to(dev), _bf16(rng, (1, Hkv, T2, d)).to(dev))
    out = hip.tree_attention(q, kc if Tp else None, vc if Tp else None, kt, vt, words, out_dtype=out_dtype,
                             seg2=seg2, gates=np.asarray(gates, np.float32) if T2 else None,
                             force_waves=waves, force_splits=splits)
    torch.cuda.synchronize()
    ref, mag = OT.tree_attention(_np(q), _np(kc) if Tp else None, _np(vc) if Tp else None, _np(kt), _np(vt),
                                 words)
    if T2:
        # the second segment: its T2 rows as a prefix, every tree row masked
        k2 = np.broadcast_to(_np(seg2[0]), (B, Hkv, T2, d))
        v2 = np.broadcast_to(_np(seg2[1]), (B, Hkv, T2, d))
        r2, m2 = OT.tree_attention(_np(q), k2, v2, _np(kt), _np(vt), np.zeros(N, np.uint64))
        g1, g2 = float(np.float32(gates[0])), float(np.float32(gates[1]))
        ref, mag = g1 * ref + g2 * r2, g1 * mag + g2 * m2
    worst = _check(out, ref, mag, bf16=out_dtype == torch.bfloat16)
    _say(f"  worst err / sum p|v| = {worst:.2e}")
    return worst


def _plan(B, H, Hkv, N, Tp, d):
    import ctypes
    s, g, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.lib().vnx_tree_attn_plan(B, H, Hkv, N, Tp, d, ctypes.byref(s), ctypes.byref(g),
                                             ctypes.byref(c)), "plan")
    return s.value, g.value, c.value


def test_config3_shape_fp32(hip):
    """B 16, 16 heads x 64, KV prefix 2048, tree (4,3,2)."""
    _run(hip, 16, 16, 16, 40, 2048, 64, seed=10)


def test_config3_shape_bf16_out(hip):
    _run(hip, 4, 16, 16, 40, 2048, 64, seed=11, out_dtype=torch.bfloat16)


@pytest.mark.parametrize("H,Hkv,N,Tp", [(16, 8, 40, 512), (32, 4, 16, 200), (8, 1, 40, 96)])
def test_gqa_query_groups(hip, H, Hkv, N, Tp):
    par = T.tree_from_branching((4, 3, 2)) if N == 40 else T.tree_from_branching((4, 3))
    _run(hip, 2, H, Hkv, N, Tp, 64, parent=par, seed=H + N)


@pytest.mark.parametrize("H,Hkv,N,Tp", [(4, 2, 20, 300), (2, 2, 7, 33), (8, 2, 64, 0)])
def test_head_dim_128(hip, H, Hkv, N, Tp):
    rng = np.random.default_rng(N)
    par = np.array([-1] + [int(rng.integers(-1, i)) for i in range(1, N)], np.int32)
    _run(hip, 2, H, Hkv, N, Tp, 128, parent=par, seed=N + 1)


@pytest.mark.parametrize("N,Tp", [(64, 0), (1, 77), (7, 1000), (33, 31), (64, 4096), (2, 1)])
def test_edge_sizes(hip, N, Tp):
    rng = np.random.default_rng(N * 7 + Tp)
    par = np.array([-1] + [int(rng.integers(-1, i)) for i in range(1, N)], np.int32)
    _run(hip, 3, 4, 2, N, Tp, 64, parent=par, seed=N + Tp)


def test_chain_tree_per_batch_and_strided_cache(hip):
    _run(hip, 4, 4, 4, 40, 700, 64, per_batch=True, cache_extra=100, seed=3)
    _run(hip, 4, 4, 4, 40, 700, 64, inplace=True, cache_extra=64, seed=4)


def test_splits_cover_one_and_many(hip):
    assert _plan(64, 16, 16, 40, 2048, 64)[0] == 1
    s, g, c = _plan(1, 1, 1, 40, 8192, 64)
    assert s > 8 and g == 1
    assert _plan(1, 2, 1, 40, 64, 64)[1] == 2  # 80 query rows: two groups
    _run(hip, 64, 16, 16, 40, 2048, 64, seed=5)
    _run(hip, 1, 1, 1, 40, 8192, 64, seed=6)


@pytest.mark.parametrize("waves", ["4", "5", "8", "9", "16"])
@pytest.mark.parametrize("B,H,Hkv,N,Tp,d", [(8, 16, 8, 1, 640, 64), (8, 16, 8, 7, 301, 64),
                                            (2, 16, 16, 40, 700, 64), (2, 4, 2, 20, 300, 128)])
def test_workgroup_shapes(hip, waves, B, H, Hkv, N, Tp, d):
    """Every workgroup shape (4 waves, 4 with prefetch, 8, 8 with prefetch, 16; a shape that
    does not fit the query tile falls back to the default) on decode-like
    (N 1, 7) and verify-like (N 40) calls."""
    par = T.chain(N) if N < 40 else None
    if N == 20:
        rng = np.random.default_rng(5)
        par = np.array([-1] + [int(rng.integers(-1, i)) for i in range(1, N)], np.int32)
    _run(hip, B, H, Hkv, N, Tp, d, parent=par, seed=N + Tp, waves=int(waves))


@pytest.mark.parametrize("waves,splits,out_dtype,N,T2,d", [
    ("16", None, torch.float32, 1, 128, 64), ("8", None, torch.bfloat16, 7, 128, 64),
    ("5", None, torch.float16, 7, 100, 64), ("4", "3", torch.float32, 7, 128, 64),
    ("16", "2", torch.float16, 1, 40, 64), ("8", None, torch.float32, 7, 128, 128),
    ("4", "2", torch.bfloat16, 40, 64, 64)])
def test_gated_second_segment(hip, waves, splits, out_dtype, N, T2, d):
    """TriSparse's fused sliding-window + global paths: out = g1 * tree
    attention + g2 * attention over the T2 shared rows, with and without key
    splits (the second segment then merges through its own slot)."""
    par = T.chain(N) if N < 40 else None
    _run(hip, 6, 16, 8, N, 500, d, parent=par, seed=N + T2, out_dtype=out_dtype, T2=T2, waves=int(waves),
         splits=int(splits) if splits else 0)


def test_large_scores(hip):
    """Scores of tens of units: the online max rescaling must hold."""
    _run(hip, 2, 4, 4, 40, 1024, 64, seed=8, std=3.0)


def test_attention_entry_point(hip):
    """DeviceBackend.attention with a tree mask / no mask runs the kernel."""
    rng = np.random.default_rng(12)
    B, H, N, Tp, d = 2, 4, 12, 100, 64
    par = T.tree_from_branching((3, 3))
    dev = hip.torch_device
    q = _bf16(rng, (B, H, N, d)).to(dev)
    k = _bf16(rng, (B, H, Tp + N, d)).to(dev)
    v = _bf16(rng, (B, H, Tp + N, d)).to(dev)
    words = T.ancestor_words(par)
    for mask, w in ((T.mask_from_words(words, Tp), words), (None, np.full(N, (1 << N) - 1, np.uint64))):
        out = hip.attention(q, k, v, mask)
        assert out.dtype == torch.bfloat16 and out.shape == (B, H, N, d)
        ref, mag = OT.tree_attention(_np(q), _np(k[:, :, :Tp]), _np(v[:, :, :Tp]), _np(k[:, :, Tp:]),
                                     _np(v[:, :, Tp:]), w)
        _check(out, ref, mag, bf16=True)


def test_rejects_bad_arguments(hip):
    dev = hip.torch_device
    z = lambda *s: torch.zeros(s, dtype=torch.bfloat16, device=dev)  # noqa: E731
    with pytest.raises(ValueError):  # 65 nodes
        hip.tree_attention(z(1, 1, 65, 64), None, None, z(1, 1, 65, 64), z(1, 1, 65, 64),
                           np.ones(65, np.uint64))
    with pytest.raises(ValueError):  # head dim 96
        hip.tree_attention(z(1, 1, 4, 96), None, None, z(1, 1, 4, 96), z(1, 1, 4, 96), np.ones(4, np.uint64))
    with pytest.raises(ValueError):  # 3 query heads over 2 kv heads
        hip.tree_attention(z(1, 3, 4, 64), None, None, z(1, 2, 4, 64), z(1, 2, 4, 64), np.ones(4, np.uint64))


@pytest.mark.parametrize("B,H,Hkv,N,d,rope,splits", [(32, 16, 8, 7, 64, 1, None), (5, 4, 2, 3, 128, 1, None),
                                                     (4, 8, 2, 7, 64, 0, None), (3, 4, 4, 5, 64, 1, "2")])
def test_qkv_rows_mode_matches_rope_kv_path(hip, B, H, Hkv, N, d, rope, splits):
    """vnx_tree_attn reading the q|k|v projection rows (RoPE and the tree
    rows' cache write inside the call) against vnx_rope_kv followed by the
    q-input call: the same fp32 rotation rounded once to bf16, so the cache
    rows and the outputs must agree bit for bit; rows past the cache stay
    unwritten."""
    import ctypes
    from versenext_amd import _lib
    _say(f"tree attn qkv mode B={B} H={H} Hkv={Hkv} N={N} d={d} rope={rope} splits={splits}")
    dev = hip.torch_device
    g = torch.Generator(device="cpu")
    g.manual_seed(B * N + d)
    cap, T = 96, 120
    heads = H + 2 * Hkv
    qkv = (torch.randn((B * N, heads * d), generator=g) * 2).to(torch.bfloat16).to(dev)
    lens = torch.randint(0, cap - N + 1, (B,), generator=g, dtype=torch.int32)
    lens[0] = cap - N + 2                      # its last rows fall past the cache
    Tp = int(lens.max())
    lens = lens.to(dev)
    ang = torch.rand((T, d), generator=g, dtype=torch.float64) * 6.0
    cos, sin = torch.cos(ang).float().to(dev), torch.sin(ang).float().to(dev)
    kc0 = torch.randn((B, Hkv, cap, d), generator=g).to(torch.bfloat16).to(dev)
    vc0 = torch.randn((B, Hkv, cap, d), generator=g).to(torch.bfloat16).to(dev)
    anc = torch.tensor([(1 << (i + 1)) - 1 for i in range(N)], dtype=torch.int64).to(dev)   # chain
    L = _lib.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(kc, vc, q, out, use_qkv):
        a = _lib.TreeAttnArgs()
        if use_qkv:
            a.qkv = qkv.data_ptr(); a.qkv_ld = qkv.stride(0)
            a.cos_table = cos.data_ptr(); a.sin_table = sin.data_ptr(); a.table_rows = T; a.rope = rope
            a.cap = cap
        else:
            a.q = q.data_ptr(); a.q_strides[:] = list(q.stride()[:3])
        a.k_cache = kc.data_ptr(); a.v_cache = vc.data_ptr(); a.cache_strides[:] = list(kc.stride()[:3])
        a.k_tree = kc.data_ptr(); a.v_tree = vc.data_ptr(); a.tree_strides[:] = list(kc.stride()[:3])
        a.anc = anc.data_ptr(); a.anc_batch_stride = 0
        a.out = out.data_ptr(); a.out_dtype = _lib.VNX_BF16; a.out_strides[:] = [N * H * d, d, H * d]
        a.B, a.H, a.Hkv, a.Tp, a.N, a.d = B, H, Hkv, Tp, N, d
        a.scale = 1.0 / d ** 0.5
        a.tp_batch = lens.data_ptr(); a.tree_follows_prefix = 1
        a.force_splits = int(splits) if splits else 0
        ws = torch.empty(max(256, L.vnx_tree_attn_workspace_args(ctypes.byref(a))), dtype=torch.uint8, device=dev)
        _lib.check(L.vnx_tree_attn(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), st), "tree_attn")

    # reference path: vnx_rope_kv, then queries from q
    kc_a, vc_a = kc0.clone(), vc0.clone()
    q = torch.zeros((B, H, N, d), dtype=torch.bfloat16, device=dev)
    _lib.check(L.vnx_rope_kv(ctypes.c_void_p(qkv.data_ptr()), _lib.VNX_BF16, qkv.stride(0), B, N, H, Hkv, d,
                             ctypes.c_void_p(lens.data_ptr()), ctypes.c_void_p(cos.data_ptr()),
                             ctypes.c_void_p(sin.data_ptr()), T, rope, ctypes.c_void_p(q.data_ptr()),
                             ctypes.c_void_p(kc_a.data_ptr()), ctypes.c_void_p(vc_a.data_ptr()), _lib.VNX_BF16,
                             kc_a.stride(0), kc_a.stride(1), kc_a.stride(2), cap, st), "rope_kv")
    out_a = torch.zeros((B * N, H * d), dtype=torch.bfloat16, device=dev)
    call(kc_a, vc_a, q, out_a, False)
    kc_b, vc_b = kc0.clone(), vc0.clone()
    out_b = torch.zeros((B * N, H * d), dtype=torch.bfloat16, device=dev)
    call(kc_b, vc_b, None, out_b, True)
    torch.cuda.synchronize()
    assert torch.equal(kc_a.cpu(), kc_b.cpu()) and torch.equal(vc_a.cpu(), vc_b.cpu())
    # rows whose positions fit the cache are compared (others are undefined in both)
    ok = (lens.cpu().long().view(B, 1) + torch.arange(N).view(1, N)) < cap
    oa, ob = out_a.cpu().view(B, N, H * d), out_b.cpu().view(B, N, H * d)
    assert torch.equal(oa[ok], ob[ok])


def _run_paths(hip, B, H, Hkv, N, Tp, d, tp, window, alibi, parent=None, T2=0, seed=0, out_dtype=torch.float32,
               alibi_max=1024, waves=0, splits=0):
    """vnx_tree_attn with a sliding window and / or ALiBi against
    oracle.tree.tree_attention_paths (the gated TriSparse paths)."""
    _say(f"tree_attn paths B={B} H={H} Hkv={Hkv} N={N} Tp={Tp} d={d} window={window} alibi={alibi} T2={T2} "
         f"alibi_max={alibi_max} waves={waves} splits={splits}")
    rng = np.random.default_rng(seed)
    par = T.chain(N) if parent is None else np.asarray(parent, np.int32)
    dev = hip.torch_device
    q = _bf16(rng, (B, H, N, d), 2.0).to(dev)
    kc = _bf16(rng, (B, Hkv, Tp, d), 2.0).to(dev)
    vc = _bf16(rng, (B, Hkv, Tp, d)).to(dev)
    kt = _bf16(rng, (B, Hkv, N, d), 2.0).to(dev)
    vt = _bf16(rng, (B, Hkv, N, d)).to(dev)
    words = T.ancestor_words(par)
    gates = np.asarray([0.55, 0.3, 0.7], np.float32)
    seg2 = None
    if T2:
        seg2 = (_bf16(rng, (1, Hkv, T2, d)).to(dev), _bf16(rng, (1, Hkv, T2, d)).to(dev))
    slopes = (1.0 / (2.0 ** (np.arange(1, H + 1, dtype=np.float32) / H))).astype(np.float32) if alibi else None
    out = hip.tree_attention(q, kc, vc, kt, vt, words, out_dtype=out_dtype, seg2=seg2,
                             gates=gates if (T2 or alibi) else None, tp=np.asarray(tp, np.int32), window=window,
                             alibi_slopes=slopes, alibi_max_keys=alibi_max, force_waves=waves, force_splits=splits)
    torch.cuda.synchronize()
    ref, mag = OT.tree_attention_paths(_np(q), _np(kc), _np(vc), _np(kt), _np(vt), words, tp=tp, window=window,
                                       slopes=slopes, alibi_max=alibi_max,
                                       seg2=(_np(seg2[0]), _np(seg2[1])) if T2 else None,
                                       gates=gates if (T2 or alibi) else None)
    worst = _check(out, ref, mag, bf16=out_dtype == torch.bfloat16)
    _say(f"  worst err / sum p|v| = {worst:.2e}")


@pytest.mark.parametrize("window,splits", [(64, 0), (100, 0), (37, 0), (64, 3), (200, 2)])
def test_sliding_window_crossed_by_ragged_rows(hip, window, splits):
    """Path A with the window crossed: ragged prefixes (some shorter than the
    window, some far longer), a chain of 7 new rows, the global rows gated;
    key splits over the windowed range."""
    tp = [300, 12, 63, 64, 299, 150]
    _run_paths(hip, 6, 16, 8, 7, 300, 64, tp, window, False, T2=16, seed=window + splits, splits=splits)


@pytest.mark.parametrize("waves,d,out_dtype", [(4, 64, torch.float32), (8, 64, torch.bfloat16),
                                               (4, 128, torch.float32), (8, 128, torch.float16)])
def test_alibi_path_with_window_and_global_rows(hip, waves, d, out_dtype):
    """All three gated paths (config-1's layout: window, global rows, ALiBi)
    at bf16 head sizes; one row's keys exceed alibi_max, so its ALiBi path
    drops out as in the reference."""
    tp = [90, 5, 40, 61]
    _run_paths(hip, 4, 8, 4, 5, 90, d, tp, 32, True, T2=8, seed=d + waves, out_dtype=out_dtype,
               alibi_max=70, waves=waves)


def test_alibi_without_window_on_a_tree(hip):
    """ALiBi over a token tree (key positions from the tree depths), no
    window and no global rows, and a tree with a window."""
    par = T.tree_from_branching((3, 2, 2))
    N = par.size
    _run_paths(hip, 3, 4, 2, N, 50, 64, [50, 0, 17], 0, True, parent=par, seed=1)
    _run_paths(hip, 3, 4, 2, N, 50, 64, [50, 0, 17], N + 3, True, parent=par, seed=2)
    _run_paths(hip, 3, 4, 2, N, 80, 64, [80, 20, 45], N, False, parent=par, seed=3, T2=4)


def test_window_smaller_than_the_tree_is_rejected(hip):
    dev = hip.torch_device
    z = lambda *s: torch.zeros(s, dtype=torch.bfloat16, device=dev)  # noqa: E731
    with pytest.raises(ValueError):
        hip.tree_attention(z(1, 2, 8, 64), z(1, 2, 10, 64), z(1, 2, 10, 64), z(1, 2, 8, 64), z(1, 2, 8, 64),
                           T.ancestor_words(T.chain(8)), window=7)


def _run_rows_f32(hip, B, H, Hkv, N, Tp, d, tp, window, alibi, parent="chain", T2=0, seed=0,
                  out_dtype=torch.float32, alibi_max=1024):
    """vnx_tree_attn's fp32-rows path (f32_rows: fp32 q / cache / tree rows,
    d 8 / 16 / 32) against oracle.tree.tree_attention_paths; parent "chain"
    passes anc=None (a chain of any length N)."""
    _say(f"tree_attn fp32 rows B={B} H={H} Hkv={Hkv} N={N} Tp={Tp} d={d} window={window} alibi={alibi} "
         f"T2={T2} alibi_max={alibi_max} out={out_dtype} tree={parent if isinstance(parent, str) else 'words'}")
    rng = np.random.default_rng(seed)
    dev = hip.torch_device
    f = lambda *s: torch.from_numpy(rng.normal(0, 1.5, s).astype(np.float32)).to(dev)  # noqa: E731
    q, kt, vt = f(B, H, N, d), f(B, Hkv, N, d), f(B, Hkv, N, d)
    kc, vc = (f(B, Hkv, Tp, d), f(B, Hkv, Tp, d)) if Tp else (None, None)
    words = None if isinstance(parent, str) else T.ancestor_words(np.asarray(parent, np.int32))
    gates = np.asarray([0.55, 0.3, 0.7], np.float32)
    seg2 = (f(1, Hkv, T2, d), f(1, Hkv, T2, d)) if T2 else None
    slopes = (1.0 / (2.0 ** (np.arange(1, H + 1, dtype=np.float32) / H))).astype(np.float32) if alibi else None
    out = hip.tree_attention(q, kc, vc, kt, vt, words, out_dtype=out_dtype, seg2=seg2,
                             gates=gates if (T2 or alibi) else None, tp=np.asarray(tp, np.int32), window=window,
                             alibi_slopes=slopes, alibi_max_keys=alibi_max, fp32_rows=True)
    torch.cuda.synchronize()
    ref, mag = OT.tree_attention_paths(_np(q), _np(kc), _np(vc), _np(kt), _np(vt), words, tp=tp, window=window,
                                       slopes=slopes, alibi_max=alibi_max,
                                       seg2=(_np(seg2[0]), _np(seg2[1])) if T2 else None,
                                       gates=gates if (T2 or alibi) else None)
    worst = _check(out, ref, mag, bf16=out_dtype == torch.bfloat16)
    _say(f"  worst err / sum p|v| = {worst:.2e}")


@pytest.mark.parametrize("d,out_dtype", [(16, torch.float32), (8, torch.float32), (32, torch.bfloat16),
                                         (16, torch.float16)])
def test_fp32_rows_config1_layout(hip, d, out_dtype):
    """The config-1 target's layout (4 heads / 2 kv, window 32, 4 global rows,
    ALiBi) on fp32 rows: a verify chain of 5 over ragged prefixes, one of
    them past alibi_max so its ALiBi path drops out."""
    _run_rows_f32(hip, 3, 4, 2, 5, 150, d, [150, 0, 31], 32, True, T2=4, seed=d, out_dtype=out_dtype,
                  alibi_max=100)


@pytest.mark.parametrize("N,Tp,window,alibi,d", [(66, 84, 32, True, 16), (100, 0, 32, False, 32),
                                                 (150, 0, 32, True, 8), (40, 16, 16, True, 16)])
def test_fp32_rows_long_chains(hip, N, Tp, window, alibi, d):
    """Prefill chunks: chains longer than one mask word and longer than the
    window (anc=None), with and without a cache before them."""
    _run_rows_f32(hip, 2, 4, 2, N, Tp, d, [Tp, Tp // 2], window, alibi, T2=4, seed=N + d)


def test_fp32_rows_on_a_tree(hip):
    """Ancestor words on the fp32 path: tree positions from the depths, a
    window wider than the tree, ALiBi, no global rows; and no paths at all."""
    par = T.tree_from_branching((3, 2, 2))
    N = par.size
    _run_rows_f32(hip, 3, 4, 2, N, 50, 16, [50, 0, 17], N + 3, True, parent=par, seed=5)
    _run_rows_f32(hip, 2, 2, 1, N, 20, 8, [20, 3], 0, False, parent=par, seed=6)


def test_fp32_rows_rejects_bad_arguments(hip):
    """The fp32-rows path takes heads of 8 / 16 / 32 only, at most 64 nodes
    with mask words, and no chain (anc None) on the bf16 path."""
    dev = hip.torch_device
    f = lambda *s: torch.zeros(s, dtype=torch.float32, device=dev)  # noqa: E731
    with pytest.raises(ValueError):  # head dim 64 on fp32 rows
        hip.tree_attention(f(1, 2, 4, 64), None, None, f(1, 1, 4, 64), f(1, 1, 4, 64), None, fp32_rows=True)
    with pytest.raises(ValueError):  # 65 nodes with mask words
        hip.tree_attention(f(1, 1, 65, 16), None, None, f(1, 1, 65, 16), f(1, 1, 65, 16), np.ones(65, np.uint64),
                           fp32_rows=True)
    with pytest.raises(ValueError):  # a chain without words needs fp32 rows
        hip.tree_attention(f(1, 1, 4, 64), None, None, f(1, 1, 4, 64), f(1, 1, 4, 64), None)
    # 65 chain nodes without words are fine
    out = hip.tree_attention(f(1, 1, 65, 16), None, None, f(1, 1, 65, 16), f(1, 1, 65, 16), None, fp32_rows=True)
    torch.cuda.synchronize()
    assert out.shape == (1, 1, 65, 16) and torch.isfinite(out).all()

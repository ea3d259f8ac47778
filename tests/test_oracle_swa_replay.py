"""TriSparse attention paths in the oracle, pinned by replaying the reference's
own consistency tests and against the golden-pinned model restatement.

- test_parallel_sparse_attn.py:85-131: the chunked parallel sliding-window
  attention (tri_sparse_attn.py:258-378: query chunks of W, key slices of
  2W-1 from zero-padded K / V, -1e9 masks) and the serial one (:380-448) agree
  within 1e-3 on the reference's eight cases, position offset included; here
  both are also compared with oracle.model.swa_attention, the one masked
  softmax the oracle uses.
- test_parallel_sparse_attn.py:133-160: the full gated forward (three paths)
  with either sliding-window form.
- oracle.tree.tree_attention_paths (the checker of vnx_tree_attn's window
  and ALiBi) on a chain over a cache == the last rows of
  oracle.model.trisparse_heads over the whole sequence, with the window
  crossed; on trees, node by node against the keys its window and root path
  leave visible.
The two chunked forms below restate the reference's algorithm for these tests
only."""
import numpy as np
import pytest

from oracle import model as OM
from oracle import tree as OT

F32 = np.float32


def _softmax(x):
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def _chunked_parallel(q, k, v, W, off):
    """tri_sparse_attn.py:258-378 (one chunk: the serial form)."""
    B, H, Tq, d = q.shape
    Tk = k.shape[2]
    n = (Tq + W - 1) // W
    if n == 1:
        return _chunked_serial(q, k, v, W, off)
    qp = np.concatenate([q, np.zeros((B, H, n * W - Tq, d), F32)], axis=2)
    K = 2 * W - 1
    kp = np.concatenate([k, np.zeros((B, H, K, d), F32)], axis=2)
    vp = np.concatenate([v, np.zeros((B, H, K, d), F32)], axis=2)
    outs = []
    for c in range(n):
        lo = off + c * W
        klo, khi = max(0, lo - W + 1), min(Tk, lo + W)
        if klo >= khi:
            klo = max(0, khi - 1)
        qg = np.arange(W) + lo
        kg = np.arange(K) + klo
        ok = (kg[None] <= qg[:, None]) & ((qg[:, None] - kg[None]) < W)
        mask = np.where(ok, 0.0, -1e9).astype(F32)
        mask[:, khi - klo:] = -1e9
        s = (qp[:, :, c * W:(c + 1) * W] @ np.swapaxes(kp[:, :, klo:klo + K], -1, -2)) * F32(1.0 / d ** 0.5)
        outs.append(_softmax(s + mask) @ vp[:, :, klo:klo + K])
    return np.concatenate(outs, axis=2)[:, :, :Tq]


def _chunked_serial(q, k, v, W, off):
    """tri_sparse_attn.py:380-448."""
    B, H, Tq, d = q.shape
    Tk = k.shape[2]
    n = (Tq + W - 1) // W
    qp = np.concatenate([q, np.zeros((B, H, n * W - Tq, d), F32)], axis=2)
    outs = []
    for c in range(n):
        lo = off + c * W
        klo, khi = max(0, lo - W + 1), min(Tk, lo + W)
        if klo >= khi:
            klo = max(0, khi - 1)
        qg = np.arange(W) + lo
        kg = np.arange(khi - klo) + klo
        ok = (kg[None] <= qg[:, None]) & ((qg[:, None] - kg[None]) < W)
        mask = np.where(ok, 0.0, -1e9).astype(F32)
        s = (qp[:, :, c * W:(c + 1) * W] @ np.swapaxes(k[:, :, klo:khi], -1, -2)) * F32(1.0 / d ** 0.5)
        outs.append(_softmax(s + mask) @ v[:, :, klo:khi])
    return np.concatenate(outs, axis=2)[:, :, :Tq]


def _qkv(rng, B, T, H, Hkv, d, std=1.0):
    q = rng.normal(0, std, (B, H, T, d)).astype(F32)
    k = np.repeat(rng.normal(0, std, (B, Hkv, T, d)).astype(F32), H // Hkv, axis=1)
    v = np.repeat(rng.normal(0, 1.0, (B, Hkv, T, d)).astype(F32), H // Hkv, axis=1)
    return q, k, v


# test_parallel_sparse_attn.py:85-104 (dim 32: d = 32 / n_head)
CASES = [(1, 6, 8, 4, 2, True, 0), (1, 20, 8, 4, 2, True, 0), (2, 25, 8, 4, 2, True, 0),
         (1, 17, 8, 4, 2, True, 0), (1, 20, 8, 4, 2, False, 0), (1, 20, 8, 4, 2, True, 5),
         (1, 64, 8, 4, 2, True, 0), (1, 20, 8, 4, 4, True, 0)]


@pytest.mark.parametrize("B,T,W,n_head,n_kv,use_alibi,off", CASES)
def test_parallel_vs_serial_swa_replay(B, T, W, n_head, n_kv, use_alibi, off):
    rng = np.random.default_rng(123 + T + off)
    q, k, v = _qkv(rng, B, T, n_head, n_kv, 32 // n_head)
    par = _chunked_parallel(q, k, v, W, off)
    ser = _chunked_serial(q, k, v, W, off)
    assert par.shape == ser.shape == q.shape
    assert np.max(np.abs(par - ser)) < 1e-3          # the reference's bar
    ref = OM.swa_attention(q, k, v, W, off)
    assert np.max(np.abs(par - ref)) < 1e-5 and np.max(np.abs(ser - ref)) < 1e-5


def test_full_gated_forward_replay():
    """test_parallel_sparse_attn.py:133-160: dim 32, 4 heads / 2 kv, W 8,
    ALiBi, B 2, T 20: the three gated paths with either chunked form equal
    oracle.model.trisparse_heads."""
    rng = np.random.default_rng(99)
    B, T, H, Hkv, d, W = 2, 20, 4, 2, 8, 8
    q, k, v = _qkv(rng, B, T, H, Hkv, d)
    kg = np.repeat(rng.normal(0, 0.5, (1, Hkv, 4, d)).astype(F32), H // Hkv, axis=1)
    vg = np.repeat(rng.normal(0, 0.5, (1, Hkv, 4, d)).astype(F32), H // Hkv, axis=1)
    gate = OM._sigmoid(rng.normal(0, 1, 3).astype(F32))
    cfg = OM_cfg(W, True)
    ref = OM.trisparse_heads(q, k, v, kg, vg, gate, cfg)
    glob = OM._attend(q, kg, vg, None)
    alibi = OM.alibi_attention(q, k, v, OM.alibi_slopes(H))
    for swa in (_chunked_parallel, _chunked_serial):
        out = gate[0] * swa(q, k, v, W, 0) + gate[1] * glob + gate[2] * alibi
        assert np.max(np.abs(out - ref)) < 1e-3


class OM_cfg:
    def __init__(self, window, alibi):
        self.window_size = window
        self.use_alibi = alibi


@pytest.mark.parametrize("T,n,W,alibi", [(40, 5, 8, True), (70, 9, 16, False), (30, 1, 32, True),
                                         (100, 7, 64, True), (150, 66, 32, True), (100, 100, 32, False)])
def test_tree_paths_on_a_chain_equal_the_model_paths(T, n, W, alibi):
    """A cache of T - n rows, then n new rows in a chain: the gated paths of
    the new rows equal the last n rows of the whole-sequence restatement.
    Chains longer than one mask word (and prefill, n = T) pass anc=None."""
    rng = np.random.default_rng(T + n)
    B, H, Hkv, d, G = 2, 4, 2, 16, 4
    q, k, v = _qkv(rng, B, T, H, Hkv, d)
    k2 = rng.normal(0, 0.5, (1, Hkv, G, d)).astype(F32)
    v2 = rng.normal(0, 0.5, (1, Hkv, G, d)).astype(F32)
    gate = OM._sigmoid(rng.normal(0, 1, 3).astype(F32))
    ref = OM.trisparse_heads(q, k, v, np.repeat(k2, H // Hkv, axis=1), np.repeat(v2, H // Hkv, axis=1), gate,
                             OM_cfg(W, alibi))[:, :, T - n:]
    kc = k[:, ::H // Hkv]
    vc = v[:, ::H // Hkv]
    words = np.array([(1 << (i + 1)) - 1 for i in range(n)], np.uint64) if n <= 64 else None
    out, _ = OT.tree_attention_paths(q[:, :, T - n:], kc[:, :, :T - n], vc[:, :, :T - n], kc[:, :, T - n:],
                                     vc[:, :, T - n:], words, window=W,
                                     slopes=OM.alibi_slopes(H) if alibi else None, seg2=(k2, v2), gates=gate)
    assert np.max(np.abs(out - ref)) < 2e-5
    # past the ALiBi key limit path C drops out (tri_sparse_attn.py:600-607)
    out2, _ = OT.tree_attention_paths(q[:, :, T - n:], kc[:, :, :T - n], vc[:, :, :T - n], kc[:, :, T - n:],
                                      vc[:, :, T - n:], words, window=W, slopes=OM.alibi_slopes(H),
                                      alibi_max=T - 1, seg2=(k2, v2), gates=gate)
    ref2 = OM.trisparse_heads(q, k, v, np.repeat(k2, H // Hkv, axis=1), np.repeat(v2, H // Hkv, axis=1), gate,
                              OM_cfg(W, False))[:, :, T - n:]
    assert np.max(np.abs(out2 - ref2)) < 2e-5


def test_tree_paths_on_trees_node_by_node():
    """Random trees over ragged prefixes: each node's window path is a plain
    softmax over the prefix keys within the window and its root path; the
    ALiBi path over all of them with the distance bias; with no window and
    no gates the paths reduce to tree_attention."""
    rng = np.random.default_rng(4)
    B, H, Hkv, N, Tp, d, W = 3, 4, 2, 9, 50, 16, 12
    par = np.array([-1, 0, 0, 1, 1, 2, 3, -1, 7], np.int32)
    words = np.zeros(N, np.uint64)
    depth = np.zeros(N, np.int64)
    for i in range(N):
        words[i] = (words[par[i]] if par[i] >= 0 else np.uint64(0)) | np.uint64(1 << i)
        depth[i] = depth[par[i]] + 1 if par[i] >= 0 else 0
    q = rng.normal(0, 1, (B, H, N, d))
    kc = rng.normal(0, 1, (B, Hkv, Tp, d))
    vc = rng.normal(0, 1, (B, Hkv, Tp, d))
    kt = rng.normal(0, 1, (B, Hkv, N, d))
    vt = rng.normal(0, 1, (B, Hkv, N, d))
    tp = np.array([50, 7, 31])
    sl = OM.alibi_slopes(H)
    gate = np.array([0.6, 0.0, 0.3], F32)
    out, _ = OT.tree_attention_paths(q, kc, vc, kt, vt, words, tp=tp, window=W, slopes=sl, gates=gate)
    g = gate.astype(np.float64)
    for b in range(B):
        t = tp[b]
        for h in range(H):
            kh = h // (H // Hkv)
            for i in range(N):
                path = [j for j in range(N) if (int(words[i]) >> j) & 1]
                pos = t + depth[i]
                pre = [j for j in range(t)]
                keys = np.concatenate([kc[b, kh, pre], kt[b, kh, path]])
                vals = np.concatenate([vc[b, kh, pre], vt[b, kh, path]])
                kpos = np.concatenate([np.arange(t), t + depth[path]])
                s = keys @ q[b, h, i] / np.sqrt(d)
                inw = (pos - kpos) < W
                ea = np.exp(s[inw] - s[inw].max())
                oa = (ea / ea.sum()) @ vals[inw]
                sc_ = s - sl[h] * (pos - kpos)
                ec = np.exp(sc_ - sc_.max())
                oc = (ec / ec.sum()) @ vals
                assert np.allclose(out[b, h, i], g[0] * oa + g[2] * oc, atol=1e-12), (b, h, i)
    plain, _ = OT.tree_attention_paths(q, kc, vc, kt, vt, words)
    ref, _ = OT.tree_attention(q, kc, vc, kt, vt, words)
    assert np.allclose(plain, ref, atol=1e-12)

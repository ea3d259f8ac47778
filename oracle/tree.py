"""Tree-verify oracles (test infrastructure only).

Attention (the kernel vnx_tree_attn):
- `tree_attention`: DeviceBackend.attention
  (packages/verse_torch/verse_torch/device.py:260-270: scores = q k^T / sqrt(d)
  + additive mask, softmax over keys, @ v) in fp64, over the KV prefix
  concatenated with the tree rows (the cache concat of
  packages/verse_nex/verse_nex/tri_sparse_attn.py:558-575), the mask 0 / -inf
  from the ancestor words, GQA by repeating each kv head H/Hkv times
  (repeat_kv, tri_sparse_attn.py:577-580).
- `tree_attention_gathered`: the same quantity computed node by node over
  the keys it may see, collected by walking its parent chain; a formulation
  that shares no mask code with `tree_attention`, used to pin it.
- `tree_attention_paths`: TriSparseAttention's gated paths over a cache
  plus tree rows (tri_sparse_attn.py:585-608): node i of batch row b sits at
  position tp_b + depth(i) (depth 0 for a root), prefix row j at j, tree row
  j at tp_b + depth(j); path A the sliding window (pos - key pos < window,
  :258-378), path B the global rows (all visible, :469-495), path C ALiBi
  (bias -m_h * (pos - key pos), no window, only where tp_b + N <= 1024,
  :489-530, :600-607); out = g0 A + g1 B + g2 C.

Greedy tree verification (vnx_tree_greedy; no reference function — the
reference's verifier is the chain case, speculative.py:202-223 and :277-287):
- `argmax_rows`: numpy.argmax per row (first maximal index; NaN wins);
- `tree_greedy`: node i is accepted iff its token equals the argmax of its
  parent's target row (row 0 for the root, 1 + p otherwise) and its parent is
  accepted; the result is the deepest accepted node (lowest BFS index among
  equally deep ones), its root path and the bonus argmax of its own row;
- `tree_greedy_bruteforce`: the same by enumerating every root-to-node path.

Tree expansion (vnx_row_topk):
- `topk_rows`: the b best ids of each row in the order value descending,
  ties by lower id, NaN above every number (so b = 1 is numpy.argmax);
- `expand_tree`: node tokens = the r-th best id of its parent's draft row,
  r = its rank among its siblings.

Pinned by tests/test_oracle_tree.py: chain tree == causal attention
(torch scaled_dot_product_attention, fp64 on the CPU); a single node and an
all-visible mask == plain prefix attention; tree_attention ==
tree_attention_gathered on random trees; tree_greedy == brute force on random
trees and == the reference-pinned chain rule (oracle.speculative
.greedy_verify_batched) on chains; topk_rows == a full stable sort.
tree_attention_paths on a chain == the last rows of oracle.model
.trisparse_heads (itself pinned by reference-written golden logits) with the
window crossed, with and without ALiBi (tests/test_oracle_swa_replay.py), and
on trees == tree_attention where the paths reduce to it.
"""
from __future__ import annotations

import numpy as np


def _parents(parent):
    p = np.asarray(parent, dtype=np.int64).reshape(-1)
    if np.any(p < -1) or np.any(p >= np.arange(p.size)):
        raise ValueError("parent[i] must be -1 or an earlier node")
    return p


def _depths(par):
    d = np.zeros(par.size, np.int64)
    for i, p in enumerate(par):
        d[i] = 1 if p < 0 else d[p] + 1
    return d


def _f64(x):
    x = np.asarray(x)
    if x.dtype == np.uint16:  # raw bf16 bits
        return (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return x.astype(np.float64)


def _words(anc, B, N):
    a = np.asarray(anc, dtype=np.uint64)
    return np.broadcast_to(a, (B, N)) if a.ndim == 1 else a


def tree_attention(q, k_cache, v_cache, k_tree, v_tree, anc, scale=None):
    """(out, mag), both (B, H, N, d) fp64: the attention output and
    sum_j p_j |v_j| (the scale its rounding errors are measured against).
    q (B,H,N,d); caches (B,Hkv,Tp,d) or None; tree rows (B,Hkv,N,d); anc (N,)
    or (B,N) uint64 words.  bf16 inputs may be passed as raw uint16 bits."""
    q = _f64(q)
    kt, vt = _f64(k_tree), _f64(v_tree)
    B, H, N, d = q.shape
    Hkv = kt.shape[1]
    if k_cache is None:
        K, V = kt, vt
        Tp = 0
    else:
        kc, vc = _f64(k_cache), _f64(v_cache)
        Tp = kc.shape[2]
        K, V = np.concatenate([kc, kt], axis=2), np.concatenate([vc, vt], axis=2)
    rep = H // Hkv
    K = np.repeat(K, rep, axis=1)
    V = np.repeat(V, rep, axis=1)
    sc = 1.0 / np.sqrt(d) if scale is None else float(scale)
    scores = np.matmul(q, K.transpose(0, 1, 3, 2)) * sc
    w = _words(anc, B, N)
    bits = ((w[:, :, None] >> np.arange(N, dtype=np.uint64)[None, None, :]) & np.uint64(1)).astype(bool)
    mask = np.zeros((B, N, Tp + N))
    mask[:, :, Tp:][~bits] = -np.inf
    scores = scores + mask[:, None]
    mx = scores.max(axis=-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    e = np.exp(scores - mx)
    den = e.sum(axis=-1, keepdims=True)
    p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
    return np.matmul(p, V), np.matmul(p, np.abs(V))


def tree_attention_paths(q, k_cache, v_cache, k_tree, v_tree, anc, tp=None, window=0, slopes=None,
                         alibi_max=1024, seg2=None, gates=None, scale=None):
    """(out, mag) (B, H, N, d) fp64 of the gated TriSparse paths over each
    batch row's first tp[b] cache rows and its N tree rows (see the module
    docstring).  tp: (B,) prefix lengths (default: all Tp rows); seg2 = (k2,
    v2) (B or 1, Hkv, T2, d); gates (3,) fp32; slopes (H,) or None.  anc None:
    a chain of any length (node i sees tree rows j <= i)."""
    q = _f64(q)
    kt, vt = _f64(k_tree), _f64(v_tree)
    B, H, N, d = q.shape
    Hkv = kt.shape[1]
    rep = H // Hkv
    Tp = 0 if k_cache is None else np.asarray(k_cache).shape[2]
    kc = None if k_cache is None else _f64(k_cache)
    vc = None if v_cache is None else _f64(v_cache)
    tp = np.full(B, Tp, np.int64) if tp is None else np.clip(np.asarray(tp, np.int64), 0, Tp)
    sc = 1.0 / np.sqrt(d) if scale is None else float(scale)
    w = None if anc is None else _words(anc, B, N)
    g = None if gates is None else np.asarray(gates, np.float32).astype(np.float64)
    out = np.zeros((B, H, N, d))
    mag = np.zeros((B, H, N, d))

    def soft(scores, ok, V):
        s = np.where(ok, scores, -np.inf)
        mx = s.max(axis=-1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0.0)
        e = np.exp(s - mx)
        den = e.sum(axis=-1, keepdims=True)
        pr = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
        return pr @ V, pr @ np.abs(V)

    for b in range(B):
        t = int(tp[b])
        if w is None:
            bits = np.tril(np.ones((N, N), bool))
        else:
            bits = ((w[b][:, None] >> np.arange(N, dtype=np.uint64)[None, :]) & np.uint64(1)).astype(bool)  # (N, N)
        depth = bits.sum(axis=1) - 1
        qpos = t + depth                                                     # (N,)
        kpos = np.concatenate([np.arange(t), t + depth])                    # (t + N,)
        vis = np.concatenate([np.ones((N, t), bool), bits], axis=1)         # (N, t + N)
        dist = qpos[:, None] - kpos[None, :]
        K = np.concatenate([kc[b, :, :t], kt[b]], axis=1) if t else kt[b]
        V = np.concatenate([vc[b, :, :t], vt[b]], axis=1) if t else vt[b]
        K = np.repeat(K, rep, axis=0)
        V = np.repeat(V, rep, axis=0)
        scores = q[b] @ K.transpose(0, 2, 1) * sc                           # (H, N, t + N)
        okA = vis & (dist < window) if window else vis
        oA, mA = soft(scores, okA[None], V)
        if g is None:
            out[b], mag[b] = oA, mA
            continue
        o, m = g[0] * oA, g[0] * mA
        if seg2 is not None:
            k2 = _f64(seg2[0])
            v2 = _f64(seg2[1])
            k2 = np.repeat(k2[b if k2.shape[0] > 1 else 0], rep, axis=0)
            v2 = np.repeat(v2[b if v2.shape[0] > 1 else 0], rep, axis=0)
            oB, mB = soft(q[b] @ k2.transpose(0, 2, 1) * sc, np.ones((1, 1, k2.shape[1]), bool), v2)
            o, m = o + g[1] * oB, m + g[1] * mB
        if slopes is not None and t + N <= alibi_max:
            sl = np.asarray(slopes, np.float32).astype(np.float64)
            oC, mC = soft(scores - sl[:, None, None] * dist[None], vis[None], V)
            o, m = o + g[2] * oC, m + g[2] * mC
        out[b], mag[b] = o, m
    return out, mag


def tree_attention_gathered(q, k_cache, v_cache, k_tree, v_tree, parent, scale=None):
    """Per node: softmax over [prefix keys, tree keys on its root path] of
    q . k * scale, times v.  Returns (B, H, N, d) fp64."""
    q = _f64(q)
    kt, vt = _f64(k_tree), _f64(v_tree)
    B, H, N, d = q.shape
    Hkv = kt.shape[1]
    kc = None if k_cache is None else _f64(k_cache)
    vc = None if v_cache is None else _f64(v_cache)
    par = np.asarray(parent)
    sc = 1.0 / np.sqrt(d) if scale is None else float(scale)
    out = np.zeros((B, H, N, d))
    for i in range(N):
        path = []
        j = i
        while j >= 0:
            path.append(j)
            j = int(par[j])
        for b in range(B):
            for h in range(H):
                g = h // (H // Hkv)
                keys = kt[b, g, path]
                vals = vt[b, g, path]
                if kc is not None:
                    keys = np.concatenate([kc[b, g], keys])
                    vals = np.concatenate([vc[b, g], vals])
                s = keys @ q[b, h, i] * sc
                e = np.exp(s - s.max())
                out[b, h, i] = (e / e.sum()) @ vals
    return out


def argmax_rows(x):
    """numpy.argmax over the last axis (speculative.py:158, :220)."""
    return np.argmax(np.asarray(x), axis=-1)


def tree_greedy(target, tokens, parent):
    """target (B, N+1, V) logits (row 0: the root's prediction, row 1+i: after
    node i); tokens (B, N) node tokens; parent (N,) BFS parent array.
    Returns (accept_len (B,) int32 = depth of the chosen node (0 if none),
    best (B,) int32 = chosen node or -1, out_ids (B, maxdepth+1) int64 = its
    root path, the bonus argmax, then -1; pred (B, N+1) int64)."""
    par = _parents(parent)
    dep = _depths(par)
    N = par.size
    tokens = np.asarray(tokens, dtype=np.int64)
    B = tokens.shape[0]
    pred = argmax_rows(target).astype(np.int64)
    prow = np.where(par < 0, 0, par + 1)
    alen = np.zeros(B, np.int32)
    best = np.full(B, -1, np.int32)
    out = np.full((B, int(dep.max()) + 1), -1, np.int64)
    for b in range(B):
        acc = np.zeros(N, bool)
        for i in range(N):
            acc[i] = tokens[b, i] == pred[b, prow[i]] and (par[i] < 0 or acc[par[i]])
        bi, bd = -1, 0
        for i in range(N):
            if acc[i] and dep[i] > bd:
                bi, bd = i, int(dep[i])
        best[b], alen[b] = bi, bd
        path = []
        j = bi
        while j >= 0:
            path.append(int(tokens[b, j]))
            j = int(par[j])
        path = path[::-1]
        out[b, :bd] = path
        out[b, bd] = pred[b, 0 if bi < 0 else bi + 1]
    return alen, best, out, pred


def tree_greedy_bruteforce(target, tokens, parent):
    """(accept_len, best) by trying every node's root path."""
    par = _parents(parent)
    N = par.size
    tokens = np.asarray(tokens, dtype=np.int64)
    pred = argmax_rows(target)
    B = tokens.shape[0]
    alen = np.zeros(B, np.int32)
    best = np.full(B, -1, np.int32)
    for b in range(B):
        for i in range(N):
            path = []
            j = i
            while j >= 0:
                path.append(j)
                j = int(par[j])
            ok = all(tokens[b, n] == pred[b, 0 if par[n] < 0 else par[n] + 1] for n in path)
            if ok and len(path) > alen[b]:
                alen[b], best[b] = len(path), i
    return alen, best


def topk_rows(x, k: int):
    """(rows, k) ids and values: value descending, ties by lower id, NaN first."""
    x = np.asarray(x)
    x2 = x.reshape(-1, x.shape[-1])
    ids = np.empty((x2.shape[0], k), np.int64)
    for r, row in enumerate(x2):
        nan = np.flatnonzero(np.isnan(row))
        rest = np.flatnonzero(~np.isnan(row))
        order = rest[np.argsort(-row[rest].astype(np.float64), kind="stable")]
        ids[r] = np.concatenate([nan, order])[:k]
    vals = np.take_along_axis(x2, ids, axis=1)
    return ids.reshape(*x.shape[:-1], k), vals.reshape(*x.shape[:-1], k)


def expand_tree(draft, parent):
    """Node tokens (B, N) of a tree whose node i takes the r-th best id of its
    parent's draft row (row 0 for the root, 1 + p otherwise), r = the number
    of earlier siblings of i."""
    par = _parents(parent)
    rows = np.where(par < 0, 0, par + 1)
    rank = np.zeros(par.size, np.int64)
    seen: dict[int, int] = {}
    for i, p in enumerate(par):
        rank[i] = seen.get(int(p), 0)
        seen[int(p)] = rank[i] + 1
    kmax = int(rank.max()) + 1
    ids, _ = topk_rows(draft, kmax)  # (B, R, kmax)
    return ids[:, rows, rank]

"""Token trees for tree speculative decoding (host-side structure helpers).

A tree of N draft nodes is held in BFS order as a parent array: parent[i] is
the index of node i's parent, or -1 when its parent is the root (the last
committed token).  BFS order gives parent[i] < i.  The verify kernels read:
- anc[i], a 64-bit word with bit j set iff node j is node i itself or one of
  its ancestors: the attention mask of vnx_tree_attn, so N <= 64;
- the parent array itself for the greedy path search (vnx_tree_greedy).

The reference has no token tree: its verifier is the chain case, parent[i] =
i - 1 (packages/verse_nex/verse_nex/speculative.py:202-223), for which the
mask is causal and the greedy path is the accepted prefix.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

MAX_NODES = 64


def tree_from_branching(branching: Sequence[int]) -> np.ndarray:
    """Parent array (int32, BFS order) of the full tree with branching[d]
    children per node at depth d: (4, 3, 2) -> 4 + 12 + 24 = 40 nodes."""
    parents: list[int] = []
    level = [-1]
    for b in branching:
        if b < 1:
            raise ValueError("branching factors must be >= 1")
        nxt = []
        for par in level:
            for _ in range(int(b)):
                nxt.append(len(parents))
                parents.append(par)
        level = nxt
    return np.asarray(parents, dtype=np.int32)


def chain(n: int) -> np.ndarray:
    """Parent array of a chain of n nodes (the reference's k draft tokens)."""
    return np.arange(-1, n - 1, dtype=np.int32)


def check_parents(parent) -> np.ndarray:
    p = np.asarray(parent, dtype=np.int64).reshape(-1)
    n = p.size
    if n < 1 or n > MAX_NODES:
        raise ValueError(f"a tree holds 1..{MAX_NODES} nodes, got {n}")
    if np.any(p < -1) or np.any(p >= np.arange(n)):
        raise ValueError("parent[i] must be -1 or a node index < i (BFS order)")
    return p.astype(np.int32)


def depths(parent) -> np.ndarray:
    """Depth of every node (children of the root have depth 1)."""
    p = check_parents(parent)
    d = np.zeros(p.size, dtype=np.int32)
    for i, par in enumerate(p):
        d[i] = 1 if par < 0 else d[par] + 1
    return d


def ancestor_words(parent) -> np.ndarray:
    """(N,) uint64: bit j of word i is set iff j is i or an ancestor of i."""
    p = check_parents(parent)
    words = np.zeros(p.size, dtype=np.uint64)
    for i, par in enumerate(p):
        words[i] = np.uint64(1 << i) | (words[par] if par >= 0 else np.uint64(0))
    return words


def draft_rows(parent) -> np.ndarray:
    """Draft-logit row of each node's parent: 0 for the root, 1 + parent index
    for an internal node (row 1 + i holds the draft's prediction after node i)."""
    p = check_parents(parent)
    return np.where(p < 0, 0, p + 1).astype(np.int32)


def mask_from_words(words, Tp: int) -> np.ndarray:
    """The additive (N, Tp + N) fp32 mask the words stand for: 0 where visible,
    -inf elsewhere (DeviceBackend.attention's `mask`, device.py:260-270)."""
    w = np.asarray(words, dtype=np.uint64)
    n = w.size
    bits = ((w[:, None] >> np.arange(n, dtype=np.uint64)[None, :]) & np.uint64(1)).astype(bool)
    m = np.zeros((n, Tp + n), dtype=np.float32)
    m[:, Tp:][~bits] = -np.inf
    return m


def words_from_mask(mask, Tp: int):
    """Inverse of mask_from_words for an additive (N, Tp + N) mask whose prefix
    columns are all visible (0) and whose tree block is 0 / very negative
    (<= -1e4, TriSparse uses -1e9); returns None for any other mask."""
    m = np.asarray(mask, dtype=np.float64)
    if m.ndim != 2:
        return None
    n = m.shape[0]
    if n < 1 or n > MAX_NODES or m.shape[1] != Tp + n:
        return None
    if Tp and np.any(m[:, :Tp] != 0.0):
        return None
    blk = m[:, Tp:]
    vis = blk == 0.0
    if not np.all(vis | (blk <= -1e4)):
        return None
    if not np.all(np.diag(vis)):
        return None
    return (vis.astype(np.uint64) << np.arange(n, dtype=np.uint64)[None, :]).sum(axis=1, dtype=np.uint64)


__all__ = ["MAX_NODES", "tree_from_branching", "chain", "check_parents", "depths", "ancestor_words",
           "draft_rows", "mask_from_words", "words_from_mask"]

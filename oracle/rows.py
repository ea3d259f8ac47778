"""Row-wise reference operations (test infrastructure only).

Restates, in numpy:
- temperature scaling `logits / temperature` on float32 (sampler.py:95);
- the top-k keep rule `scaled >= np.partition(scaled, -k)[-k]` (sampler.py:98-102),
  ties keep more than k;
- NumpyBackend.softmax: exp(x - max) / sum (device.py:305-308);
- numpy.argmax (first maximal index; speculative.py:158, :220);
- the row log-sum-exp in fp64, the exact value the kernels approximate.
"""
from __future__ import annotations

import numpy as np


def scale(logits: np.ndarray, temperature: float) -> np.ndarray:
    """RN(l / T) in float32 — numpy's float32 array / float32 scalar division."""
    x = np.asarray(logits, dtype=np.float32)
    T = np.float32(temperature)
    if T == np.float32(1.0):
        return x.copy()
    return x / T


def topk_threshold(scaled_row: np.ndarray, top_k: int) -> np.float32:
    """The Sampler's kth value: np.partition(scaled, -top_k)[-top_k] (sampler.py:100-101)."""
    if top_k <= 0 or top_k >= scaled_row.size:
        return np.float32(-np.inf)
    return np.float32(np.partition(scaled_row, -top_k)[-top_k])


def apply_threshold(a: np.ndarray, thr) -> np.ndarray:
    """Masks scaled values below the per-row threshold to -inf (keeps ties, sampler.py:102)."""
    if thr is None:
        return a
    thr = np.asarray(thr, dtype=np.float32)[..., None]
    return np.where(a >= thr, a, np.float32(-np.inf)).astype(np.float32)


def lse64(a: np.ndarray) -> np.ndarray:
    """log(sum exp(a)) along the last axis in fp64 (rows of -inf give -inf)."""
    a = np.asarray(a)
    m = np.max(a, axis=-1, keepdims=True).astype(np.float64)
    finite = np.isfinite(m)
    m_safe = np.where(finite, m, 0.0)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        s = np.sum(np.exp(a.astype(np.float64) - m_safe), axis=-1)
        out = m_safe[..., 0] + np.log(s)
    return np.where(finite[..., 0], out, m[..., 0])


def softmax_ref(x: np.ndarray, dim: int = -1) -> np.ndarray:
    """NumpyBackend.softmax, verbatim semantics (device.py:305-308)."""
    x_max = np.max(x, axis=dim, keepdims=True)
    e = np.exp(x - x_max)
    return e / np.sum(e, axis=dim, keepdims=True)


def argmax(x: np.ndarray) -> np.ndarray:
    return np.argmax(x, axis=-1)

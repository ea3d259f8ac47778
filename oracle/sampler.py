"""CPU restatement of Sampler.sample (test infrastructure only: the checker of
vnx_sampler_sample and vnx_logit_calibrate).

Follows packages/verse_infra/verse_infra/verse_inference/sampler.py:70-138
step by step, in the build's canonical arithmetic where the reference's
float32 numpy results are not reproducible bit for bit:
1. temperature 0: numpy.argmax of the raw logits (:88-90);
2. a = RN(l / T) in float32 (:93);
3. top-k (0 < k < V): kth = np.partition(a, -k)[-k]; a = where(a >= kth, a,
   -inf), so ties keep more than k and NaN drops out (:96-102).  CometSpark's
   exactly-k rule instead keeps argpartition(-a, k-1)[:k] (packages/verse_nex/
   verse_nex/cometspark.py:896-898): exactly k tokens, NaN ranked below every
   value, ties at the kth value taken by lower id (numpy leaves them open);
4. M = max(a); if M is not finite, numpy.argmax of the raw logits (:105-108);
5. probabilities p = E(a - L32), E = the canonical exp, L32 = RN32 of the
   fp64 row log-sum-exp (the reference's exp / sum, :109-111);
6. top-p < 1 (:113-131): tokens in descending probability, ties by lower id
   (numpy's argsort leaves their order open); cumulative sums in exact
   fixed point, P = floor(p * 2^60) summed as integers, compared with
   floor(top_p * 2^60); cutoff = the first position whose cumulative sum
   reaches top_p (searchsorted, side 'left'), at most V - 1; the first
   cutoff + 1 tokens are kept;
7. the draw: numpy's Generator.choice rule on the kept probabilities with
   the given uniform (first j with C_j > u * C_V over fp64 cumulative sums,
   :135-137; oracle/canon.c vnx_ref_icdf), over token ids in increasing order
   (CometSpark draws over argpartition's output order, which numpy does not
   fix: the distribution is the same, the token for a given uniform is not).

CometSpark's sampling step (_generate_with_logits, cometspark.py:868-910) is
sample(..., exact_k=True, calib_factor=f): the calibration first, then
temperature 0 -> argmax of the calibrated row, else the steps above.

The logit calibration of VMPC-compressed models (packages/verse_nex/
verse_nex/cometspark.py:922-948): logits / sqrt(var(logits) + 1e-8) *
calib_factor, with the variance taken in fp64 and every later step one
float32 operation in the reference's order.
"""
from __future__ import annotations

import numpy as np

from . import _clib
from . import rows

FIX_BITS = 60
FLAG_CDF_EDGE = 4


def kth_largest(a: np.ndarray, k: int) -> np.float32:
    """np.partition(a, -k)[-k]: the kth largest value, NaN counting as the largest."""
    return np.float32(np.partition(np.asarray(a, np.float32), -k)[-k])


def fixed(p) -> np.ndarray:
    """floor(p * 2^60) as uint64 (exact: scaling by a power of two)."""
    return np.floor(np.asarray(p, np.float64) * float(2 ** FIX_BITS)).astype(np.uint64)


def nucleus(p: np.ndarray, top_p: float):
    """(keep mask, p_star, j_star, cutoff) of the nucleus rule on probabilities p
    (float32, >= 0): order by (p descending, id ascending), exact fixed-point
    cumulative sums, cutoff = first position whose sum reaches top_p, at most
    V - 1; the first cutoff + 1 tokens are kept.  (p_star, j_star) describe the
    last kept token: kept iff p > p_star or (p == p_star and id <= j_star)."""
    p = np.asarray(p, np.float32)
    V = p.size
    order = np.lexsort((np.arange(V), -p.astype(np.float64)))
    c = np.cumsum(fixed(p[order]), dtype=np.uint64)
    target = np.uint64(fixed(np.float64(np.float32(top_p))))
    cutoff = int(np.searchsorted(c, target, side="left"))
    cutoff = min(cutoff, V - 1)
    keep = np.zeros(V, bool)
    keep[order[:cutoff + 1]] = True
    j_star = int(order[cutoff])
    return keep, np.float32(p[j_star]), j_star, cutoff


def exact_k_keep(a: np.ndarray, k: int):
    """(keep mask, kth value, k_star) of argpartition(-a, k-1)[:k] with the
    order fixed: value descending (NaN below every value, -0 == +0), then id
    ascending; k_star is the id of the last kept token."""
    a = np.asarray(a, np.float32)
    V = a.size
    nan = np.isnan(a)
    neg = np.where(nan, 0.0, -a.astype(np.float64))
    order = np.lexsort((np.arange(V), neg, nan))
    keep = np.zeros(V, bool)
    keep[order[:k]] = True
    last = int(order[k - 1])
    return keep, np.float32(a[last]), last


def probabilities(logits, temperature: float, top_k: int = 0, exact_k: bool = False):
    """(a masked, L32, p) of steps 2-5, or None when step 4 falls back to argmax."""
    x = np.asarray(logits, np.float32)
    V = x.size
    a = rows.scale(x, temperature)
    if 0 < top_k < V:
        if exact_k:
            a = np.where(exact_k_keep(a, top_k)[0], a, np.float32(-np.inf)).astype(np.float32)
        else:
            a = rows.apply_threshold(a, kth_largest(a, top_k))
    M = np.max(a)
    if not np.isfinite(M):
        return None
    L32 = np.float32(rows.lse64(a[None])[0])
    p = _clib.exp_canon((a - L32).astype(np.float32))
    return a, L32, p


def sample(logits, temperature: float, top_k: int, top_p: float, u: float, exact_k: bool = False,
           calib_factor=None, eps: float = 1e-8):
    """Sampler.sample restated: (token, flags, info).  info holds the kth value
    (and k_star under exact_k), L32 and the nucleus (p_star, j_star) when they
    apply.  calib_factor (not None) calibrates the row first."""
    x = np.asarray(logits, np.float32).reshape(-1)
    if calib_factor is not None:
        x = logit_calibrate(x, calib_factor, eps)[0]
    V = x.size
    info = {}
    if temperature == 0.0:
        return int(np.argmax(x)), 0, info
    if 0 < top_k < V:
        if exact_k:
            _, info["kth"], info["k_star"] = exact_k_keep(rows.scale(x, temperature), top_k)
        else:
            info["kth"] = kth_largest(rows.scale(x, temperature), top_k)
    pr = probabilities(x, temperature, top_k, exact_k)
    if pr is None:
        return int(np.argmax(x)), 0, info
    a, L32, p = pr
    info["L32"] = L32
    if top_p < 1.0:
        keep, p_star, j_star, cutoff = nucleus(p, top_p)
        p = np.where(keep, p, np.float32(0.0)).astype(np.float32)
        info.update(p_star=p_star, j_star=j_star, cutoff=cutoff)
    j, before, after, total = _clib.icdf(p, u)
    flags = 0
    t = float(u) * total
    if t - before < 1e-12 * total or after - t < 1e-12 * total:
        flags |= FLAG_CDF_EDGE
    return j, flags, info


def logit_calibrate(logits, calib_factor: float, eps: float = 1e-8):
    """(calibrated float32 rows, fp64 variance): x / sqrt(var + eps) * f along
    the last axis (cometspark.py:930, :946-948); var in fp64, then float32
    ops: s = sqrt(RN32(var) + eps), RN(RN(x / s) * f)."""
    x = np.asarray(logits, np.float32)
    var64 = np.var(x.astype(np.float64), axis=-1, keepdims=True)
    var32 = var64.astype(np.float32)
    s = np.sqrt(var32 + np.float32(eps)).astype(np.float32)
    out = ((x / s).astype(np.float32) * np.float32(calib_factor)).astype(np.float32)
    return out, var64[..., 0]

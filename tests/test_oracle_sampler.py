"""The Sampler restatement (oracle/sampler.py) pinned against what numpy and the
mathematics fix: numpy's partition for the kth value, the reference's own
nucleus steps (argsort / cumsum / searchsorted / cutoff + 1, sampler.py:113-131)
run on the same probabilities, the defining properties of the smallest
nucleus when probabilities tie, numpy's Generator.choice for the draw, and a
planted off-by-one that those checks catch."""
import numpy as np
import pytest

from oracle import sampler as OS
from oracle import rows as OR


def _reference_nucleus_keep(probs: np.ndarray, top_p: float) -> np.ndarray:
    """sampler.py:113-125 verbatim in float64 (argsort, cumsum, searchsorted,
    min(cutoff, V - 1), keep the first cutoff + 1); a stable argsort, so tied
    probabilities go by lower id, the order the restatement fixes."""
    sorted_idx = np.argsort(-probs, kind="stable")
    cumsum = np.cumsum(probs[sorted_idx])
    cutoff = np.searchsorted(cumsum, top_p)
    cutoff = min(cutoff, probs.size - 1)
    keep = np.zeros_like(probs, dtype=bool)
    keep[sorted_idx[: cutoff + 1]] = True
    return keep


def test_kth_largest_is_numpy_partition():
    rng = np.random.default_rng(0)
    a = rng.normal(size=5000).astype(np.float32)
    for k in (1, 2, 17, 64, 1000, 4999):
        assert OS.kth_largest(a, k) == np.sort(a)[::-1][k - 1]
    b = a.copy()
    b[[3, 10, 20]] = np.nan
    assert np.isnan(OS.kth_largest(b, 2)) and OS.kth_largest(b, 4) == np.sort(a[~np.isnan(b)])[::-1][0]


@pytest.mark.parametrize("top_p", [0.3, 0.75, 0.9, 0.99])
def test_nucleus_matches_the_reference_steps(top_p):
    rng = np.random.default_rng(int(top_p * 100))
    checked = 0
    for _ in range(20):
        a = OR.scale(rng.normal(0, 2, 3000).astype(np.float32), 0.8)
        _, _, p = OS.probabilities(a, 1.0)
        keep, p_star, j_star, cutoff = OS.nucleus(p, top_p)
        p64 = p.astype(np.float64)
        c = np.cumsum(np.sort(p64)[::-1])
        if np.min(np.abs(c - np.float32(top_p))) < 1e-9:
            continue  # a cumulative sum within rounding of top_p: the two arithmetics may differ
        ref = _reference_nucleus_keep(p64, float(np.float32(top_p)))
        assert np.array_equal(keep, ref)
        assert keep.sum() == cutoff + 1 and keep[j_star] and p[j_star] == p_star
        checked += 1
    assert checked >= 15


def test_nucleus_with_ties_is_the_smallest_prefix_by_probability_then_id():
    rng = np.random.default_rng(5)
    for trial in range(40):
        levels = np.float32(rng.random(6) + 0.01)
        p = levels[rng.integers(0, 6, 500)]
        p = (p / p.sum()).astype(np.float32)
        top_p = float(rng.random() * 0.98 + 0.01)
        keep, p_star, j_star, cutoff = OS.nucleus(p, top_p)
        f = OS.fixed(p)
        target = OS.fixed(np.float64(np.float32(top_p)))
        tot = int(f[keep].sum(dtype=np.uint64))
        assert keep.sum() == cutoff + 1
        assert tot >= int(target) or keep.all()
        # dropping the last kept token (p_star, j_star) falls short of top_p
        assert tot - int(f[j_star]) < int(target)
        # kept tokens outrank dropped ones: higher probability, or equal and lower id
        kept = np.flatnonzero(keep)
        dropped = np.flatnonzero(~keep)
        assert np.all((p[kept] > p_star) | ((p[kept] == p_star) & (kept <= j_star)))
        assert np.all((p[dropped] < p_star) | ((p[dropped] == p_star) & (dropped > j_star)))


def test_planted_off_by_one_fails_the_nucleus_properties():
    """Keeping `cutoff` tokens instead of cutoff + 1 leaves the kept mass below top_p."""
    rng = np.random.default_rng(9)
    p = rng.random(400).astype(np.float32)
    p = (p / p.sum()).astype(np.float32)
    keep, p_star, j_star, cutoff = OS.nucleus(p, 0.6)
    bad = keep.copy()
    bad[j_star] = False
    assert int(OS.fixed(p)[bad].sum(dtype=np.uint64)) < int(OS.fixed(np.float64(np.float32(0.6))))


def test_limits_temperature_zero_tiny_top_p_and_top_k_one():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, 2000).astype(np.float32)
    am = int(np.argmax(x))
    assert OS.sample(x, 0.0, 0, 1.0, 0.7)[0] == am
    for u in (0.01, 0.5, 0.99):
        assert OS.sample(x, 0.8, 0, 1e-9, u)[0] == am
        assert OS.sample(x, 0.8, 1, 1.0, u)[0] == am
    # every logit -inf after masking, or a NaN without top-k: numpy.argmax of the raw row
    y = x.copy()
    y[7] = np.nan
    assert OS.sample(y, 0.8, 0, 1.0, 0.3)[0] == 7
    z = np.full(10, -np.inf, np.float32)
    assert OS.sample(z, 0.8, 0, 0.9, 0.3)[0] == 0


def test_draw_is_numpy_generator_choice_on_the_kept_probabilities():
    rng = np.random.default_rng(11)
    agree = 0
    for seed in range(30):
        x = rng.normal(0, 2, 1000).astype(np.float32)
        top_k, top_p, T = (0, 1.0, 0.8) if seed % 3 == 0 else ((50, 0.9, 0.7) if seed % 3 == 1 else (0, 0.95, 1.3))
        u = np.random.default_rng(seed).random()
        tok, flags, info = OS.sample(x, T, top_k, top_p, np.float32(u))
        a, L32, p = OS.probabilities(x, T, top_k)
        if top_p < 1.0:
            p = np.where(OS.nucleus(p, top_p)[0], p, 0)
        q = p.astype(np.float64) / p.astype(np.float64).sum()
        ref = np.random.default_rng(seed).choice(q.size, p=q)
        if flags == 0 and abs(float(np.float32(u)) - u) < 1e-7:
            agree += tok == ref
            assert tok == ref, (seed, tok, ref)
    assert agree >= 25


def test_logit_calibration_matches_the_reference_formula():
    rng = np.random.default_rng(2)
    x = rng.normal(0.5, 3.0, (4, 5000)).astype(np.float32)
    out, var64 = OS.logit_calibrate(x, 1.7)
    assert np.allclose(var64, np.var(x.astype(np.float64), axis=-1), rtol=0, atol=0)
    ref = x / np.sqrt(np.var(x, axis=-1, keepdims=True) + 1e-8) * 1.7  # cometspark.py:946-948, float32 numpy
    assert np.max(np.abs(out - ref) / np.abs(ref)) < 2e-6
    assert np.allclose(np.std(out.astype(np.float64), axis=-1), 1.7, rtol=1e-5)


def test_exact_k_is_numpy_argpartition_set():
    """Distinct values (with NaN present): the kept set equals
    argpartition(-a, k-1)[:k] (cometspark.py:896-898), NaN never kept while k
    non-NaN values exist."""
    rng = np.random.default_rng(12)
    for k in (1, 5, 64, 300, 999):
        a = rng.normal(0, 2, 3000).astype(np.float32)
        a[rng.integers(0, 3000, 7)] = np.nan
        keep, kth, kstar = OS.exact_k_keep(a, k)
        ref = np.zeros(a.size, bool)
        ref[np.argpartition(-a, kth=k - 1)[:k]] = True
        assert np.array_equal(keep, ref), k
        assert keep.sum() == k and not np.isnan(a[keep]).any()
        assert kth == np.min(a[keep]) and a[kstar] == kth


def test_exact_k_ties_go_by_lower_id():
    rng = np.random.default_rng(13)
    for trial in range(30):
        a = (rng.integers(-6, 6, 800) / 2).astype(np.float32)
        a[a == 0] = np.float32(-0.0) if trial % 2 else np.float32(0.0)  # -0 and +0 tie
        k = int(rng.integers(1, 800))
        keep, kth, kstar = OS.exact_k_keep(a, k)
        assert keep.sum() == k
        # every kept token outranks every dropped one by (value desc, id asc)
        kept, dropped = np.flatnonzero(keep), np.flatnonzero(~keep)
        assert np.all((a[kept] > kth) | ((a[kept] == kth) & (kept <= kstar)))
        assert np.all((a[dropped] < kth) | ((a[dropped] == kth) & (dropped > kstar)))
        # a planted tie rule that takes the highest ids breaks the property whenever ties are split
        ties = np.flatnonzero(a == kth)
        need = k - int(np.sum(a > kth))
        if 0 < need < ties.size:
            bad = (a > kth)
            bad[ties[-need:]] = True
            assert not np.array_equal(bad, keep)


def test_cometspark_step_calibrates_then_draws_exactly_k():
    """sample(exact_k=True, calib_factor=f): greedy is the argmax of the
    calibrated row; the draw is Generator.choice over the softmax of the k kept
    values (cometspark.py:896-904), the kept ids in increasing order."""
    rng = np.random.default_rng(14)
    agree = 0
    for seed in range(20):
        x = rng.normal(0, 3, 2000).astype(np.float32)
        f = 1.3
        xc = OS.logit_calibrate(x, f)[0]
        assert OS.sample(x, 0.0, 40, 1.0, 0.5, exact_k=True, calib_factor=f)[0] == int(np.argmax(xc))
        u = np.random.default_rng(seed).random()
        tok, flags, info = OS.sample(x, 0.8, 40, 1.0, np.float32(u), exact_k=True, calib_factor=f)
        a = (xc / np.float32(0.8)).astype(np.float64)
        idx = np.sort(np.argpartition(-a, 39)[:40])
        q = np.exp(a[idx] - a[idx].max())
        q /= q.sum()
        ref = idx[np.random.default_rng(seed).choice(40, p=q)]
        if flags == 0 and abs(float(np.float32(u)) - u) < 1e-7:
            agree += tok == ref
            assert tok == ref, (seed, tok, ref)
        assert info["k_star"] in idx
    assert agree >= 15

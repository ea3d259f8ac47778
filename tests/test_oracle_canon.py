"""Pins the oracle's canonical arithmetic (oracle/canon.c) against mathematics
and numpy: the canonical exp against math.exp, the Markstein division
against IEEE division, and the inverse-CDF rule against numpy's own
Generator.choice (the sampler's draw, sampler.py:135-137)."""
import math

import numpy as np
import pytest

from oracle import _clib, rows


def test_exp_canon_accuracy_and_specials():
    rng = np.random.default_rng(0)
    t = np.concatenate([rng.uniform(-86.4, 0.0, 200000), rng.uniform(-1e-3, 1e-3, 20000),
                        np.array([0.0, -0.0, -1.0, -2.5, -86.4, 1e-6])]).astype(np.float32)
    e = _clib.exp_canon(t).astype(np.float64)
    ref = np.exp(t.astype(np.float64))
    rel = np.abs(e - ref) / ref
    assert rel.max() < 3e-7, rel.max()  # within ~2.5 ulp of the true exponential
    assert _clib.exp_canon(np.float32(0.0)) == 1.0
    sp = _clib.exp_canon(np.array([-np.inf, np.nan, -86.6, -200.0, 100.0], np.float32))
    assert sp[0] == 0 and sp[1] == 0 and sp[2] == 0 and sp[3] == 0
    assert np.isfinite(sp[4]) and sp[4] > 1e38  # clamped at t = 88
    assert _clib.exp_canon(np.float32(88.0)) == sp[4]


def test_exp_canon_monotone_on_a_fine_grid():
    t = np.linspace(-20, 0, 400001, dtype=np.float32)
    e = _clib.exp_canon(t)
    assert np.all(np.diff(e.astype(np.float64)) >= 0)


@pytest.mark.parametrize("T", [0.8, 0.5, 0.7, 1.3, 0.3, 2.0, 0.123456, 3.14159, 1e-3, 0.9999999])
def test_markstein_division_is_exact(T):
    # Every significand in [1,2); scaling by 2^e covers all normal logits.
    assert _clib.markstein_mismatches(T) == 0


def test_markstein_random_temperatures_and_values():
    rng = np.random.default_rng(1)
    for T in rng.uniform(0.05, 4.0, 20).astype(np.float32):
        for l in rng.normal(0, 20, 200).astype(np.float32):
            assert _clib.div_markstein(l, T) == np.float32(l) / np.float32(T)
    for l in [np.inf, -np.inf, 0.0, -0.0]:
        q = _clib.div_markstein(l, 0.8)
        assert q == np.float32(l) / np.float32(0.8)


def test_icdf_is_numpy_choice_rule():
    """numpy's Generator.choice(V, p=p) is searchsorted(cdf/cdf[-1], random(), 'right');
    the oracle's icdf is the same rule with the normalisation folded into the target."""
    rng = np.random.default_rng(7)
    for trial in range(300):
        V = int(rng.integers(2, 50))
        w = rng.random(V).astype(np.float32)
        w[rng.random(V) < 0.3] = 0
        if w.sum() == 0:
            w[0] = 1
        p = w.astype(np.float64) / w.astype(np.float64).sum()
        seed = int(rng.integers(0, 2**31))
        g1, g2 = np.random.default_rng(seed), np.random.default_rng(seed)
        picked = g1.choice(V, p=p)
        u = g2.random()
        cdf = np.cumsum(p)
        cdf /= cdf[-1]
        assert picked == int(np.searchsorted(cdf, u, side="right"))  # numpy's own rule
        u32 = np.float32(u)
        j, before, after, total = _clib.icdf(w, u32)
        cw = np.cumsum(w.astype(np.float64))
        assert j == int(np.searchsorted(cw, np.float64(u32) * cw[-1], side="right"))
        assert w[j] > 0
        # a float64 uniform is used as drawn, not rounded to float32
        j64 = _clib.icdf(w, u)[0]
        assert j64 == int(np.searchsorted(cw, u * cw[-1], side="right"))


def test_icdf_keeps_the_float64_uniform():
    """Where float32 rounding of the uniform crosses a bucket edge, the
    float64 draw follows the unrounded value."""
    w = np.ones(8, np.float32)
    u = 0.5 - 2.0 ** -40            # float32(u) == 0.5 exactly: the next bucket
    assert np.float32(u) == np.float32(0.5)
    assert _clib.icdf(w, u)[0] == 3
    assert _clib.icdf(w, np.float32(u))[0] == 4


def test_icdf_edges():
    w = np.array([0, 0, 1, 0, 1, 0], np.float32)
    assert _clib.icdf(w, 0.0)[0] == 2
    assert _clib.icdf(w, 0.4999)[0] == 2
    assert _clib.icdf(w, 0.5)[0] == 4  # C_2 = 1 > 0.5*2 is false at exactly the edge: next bucket
    assert _clib.icdf(w, np.float32(1 - 2**-24))[0] == 4
    assert _clib.icdf(np.zeros(5, np.float32), 0.3)[0] == -1


def test_lse64_and_softmax_closed_forms():
    x = np.array([[1000.0, 1001.0, 1002.0]], np.float32)  # device test vector (test_device_backend.py:93-101)
    sm = rows.softmax_ref(x)
    assert np.all(np.isfinite(sm)) and abs(sm.sum() - 1) < 1e-6
    L = rows.lse64(x)[0]
    assert abs(L - (1002 + math.log(1 + math.exp(-1) + math.exp(-2)))) < 1e-12
    assert rows.lse64(np.array([[-np.inf, -np.inf]], np.float32))[0] == -np.inf
    a = np.random.default_rng(2).normal(0, 3, (4, 1000)).astype(np.float32)
    ref = np.log(np.sum(np.exp(a.astype(np.float64)), -1))
    assert np.allclose(rows.lse64(a), ref, rtol=0, atol=1e-12)


def test_topk_threshold_keeps_ties():
    s = np.array([1, 3, 3, 2, 3, 0], np.float32)
    thr = rows.topk_threshold(s, 2)
    kept = rows.apply_threshold(s[None], [thr])[0]
    assert np.sum(np.isfinite(kept)) == 3  # sampler.py:102 keeps all ties of the kth value
    assert rows.topk_threshold(s, 0) == -np.inf and rows.topk_threshold(s, 6) == -np.inf


def test_scale_is_numpy_division():
    x = np.random.default_rng(3).normal(0, 5, 10000).astype(np.float32)
    assert np.array_equal(rows.scale(x, 0.8), x / np.float32(0.8))
    assert np.array_equal(rows.scale(x, 1.0), x)

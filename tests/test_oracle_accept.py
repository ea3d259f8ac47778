"""Pins the stochastic acceptance oracle (no reference implementation exists:
the reference verifier is greedy).  Checks chosen so that plausible mistakes
fail: the T -> 0 limit equals the reference's greedy rule (+ bonus), p == q
accepts everything, p(x) = 0 rejects, and the exact output law on u-grids
equals p (the unbiasedness theorem of arXiv:2211.17192, Thm. 1)."""
import numpy as np
import pytest

from oracle import _clib, rows
from oracle.speculative import (FLAG_BAD_ID, greedy_verify_batched, output_law_on_grid,
                                spec_accept)


def _softmax64(x, T):
    a = rows.scale(x, T).astype(np.float64)
    e = np.exp(a - a.max())
    return e / e.sum()


def test_low_temperature_reduces_to_greedy_with_bonus():
    rng = np.random.default_rng(0)
    B, k, V = 32, 4, 50
    # integer-spaced logits: at T = 0.01 every row is one-hot to machine precision
    tgt = rng.permuted(np.tile(np.arange(V, dtype=np.float32), (B, k + 1, 1)), axis=2)
    dft = rng.permuted(np.tile(np.arange(V, dtype=np.float32), (B, k, 1)), axis=2)
    pred = tgt.argmax(-1)
    ids = np.where(rng.random((B, k)) < 0.6, pred[:, :k], dft.argmax(-1))
    for i in range(k):  # draft rows put their mass on the drafted id
        dft[np.arange(B), i, ids[:, i]] = V + 1
    u = (rng.random((B, k + 1)) * 0.98).astype(np.float32)
    res = spec_accept(tgt, dft, ids, u, 0.01)
    _, _, alen, out = greedy_verify_batched(tgt, ids)
    assert np.array_equal(res["accept_len"], alen)
    assert np.array_equal(res["out_ids"], out)


def test_identical_draft_accepts_everything():
    rng = np.random.default_rng(1)
    B, k, V = 16, 6, 300
    tgt = rng.normal(0, 2, (B, k + 1, V)).astype(np.float32)
    dft = tgt[:, :k].copy()
    ids = rng.integers(0, V, (B, k))
    u = rng.random((B, k + 1)).astype(np.float32)
    res = spec_accept(tgt, dft, ids, u, 0.8)
    assert np.all(res["accept_len"] == k)
    assert np.array_equal(res["out_ids"][:, :k], ids)
    # bonus = inverse-CDF draw from p_k
    for b in range(B):
        w, _ = _clib.resid_weights(tgt[b, k], None, 0.8, -np.inf, -np.inf, res["lse_t"][b, k], 0.0)
        assert res["out_ids"][b, k] == _clib.icdf(w, u[b, k])[0]


def test_zero_target_probability_rejects_and_residual_avoids_it():
    V, k = 20, 3
    tgt = np.zeros((1, k + 1, V), np.float32)
    tgt[0, 0, 5] = -1e4  # p_0(5) underflows to 0
    dft = np.zeros((1, k, V), np.float32)
    dft[0, 0, 5] = 10.0  # q_0 concentrated on 5
    ids = np.array([[5, 1, 2]])
    u = np.array([[0.0, 0.5, 0.5, 0.3]], np.float32)
    res = spec_accept(tgt, dft, ids, u, 1.0)
    assert res["accept_len"][0] == 0
    assert res["out_ids"][0, 0] != 5 and res["out_ids"][0, 1] == -1


def test_bad_ids_are_rejected_and_flagged():
    rng = np.random.default_rng(2)
    tgt = rng.normal(size=(2, 3, 10)).astype(np.float32)
    dft = tgt[:, :2].copy()
    ids = np.array([[1, -3], [11, 0]])
    res = spec_accept(tgt, dft, ids, np.full((2, 3), 0.5, np.float32), 1.0)
    assert res["accept_len"].tolist() == [1, 0]
    assert res["flags"][0, 1] & FLAG_BAD_ID and res["flags"][1, 0] & FLAG_BAD_ID


@pytest.mark.parametrize("seed,T", [(3, 1.0), (4, 0.8), (5, 1.7)])
def test_output_law_equals_target_distribution(seed, T):
    rng = np.random.default_rng(seed)
    V = 6
    p_logits = rng.normal(0, 1.5, (2, V)).astype(np.float32)
    q_logits = (p_logits[:1] + rng.normal(0, 1.0, (1, V))).astype(np.float32)
    q = _softmax64(q_logits[0], T)
    law = output_law_on_grid(p_logits, q_logits, q, T, grid=2048)
    p = _softmax64(p_logits[0], T)
    assert np.abs(law - p).max() < 2.5e-3, (law, p)


def test_law_check_detects_a_planted_mistake():
    """Drafting from the wrong distribution breaks unbiasedness; the same law
    check must see it (shows the check has power)."""
    rng = np.random.default_rng(3)
    V = 6
    p_logits = rng.normal(0, 1.5, (2, V)).astype(np.float32)
    q_logits = (p_logits[:1] + rng.normal(0, 1.0, (1, V))).astype(np.float32)
    wrong = np.full(V, 1.0 / V)  # drafts x uniformly instead of from q
    law = output_law_on_grid(p_logits, q_logits, wrong, 1.0, grid=1024)
    p = _softmax64(p_logits[0], 1.0)
    assert np.abs(law - p).max() > 2e-2


def test_probabilities_agree_with_true_softmax():
    rng = np.random.default_rng(6)
    B, k, V = 4, 3, 5000
    tgt = rng.normal(0, 2, (B, k + 1, V)).astype(np.float32)
    dft = (tgt[:, :k] + rng.normal(0, 0.5, (B, k, V))).astype(np.float32)
    res = spec_accept(tgt, dft, rng.integers(0, V, (B, k)), rng.random((B, k + 1)).astype(np.float32), 0.8)
    for b in range(B):
        for i in range(k + 1):
            w, _ = _clib.resid_weights(tgt[b, i], None, 0.8, -np.inf, -np.inf, res["lse_t"][b, i], 0.0)
            p = _softmax64(tgt[b, i], 0.8)
            assert np.max(np.abs(w - p) / p) < 1e-5  # north-star tolerance for fp32 probabilities

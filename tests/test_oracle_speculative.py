"""The reference's own test vectors (tests/test_speculative_decode.py) replayed
against the numpy restatement of its greedy verifier (oracle.speculative).

Each test names the reference test it mirrors; inputs and expected outputs
are the reference's."""
import numpy as np
import pytest

from oracle.speculative import RefSpeculativeDecoder, greedy_verify_batched


class FakeMainModel:
    """tests/test_speculative_decode.py:36-73: embedding + projection, with
    forced per-position logits."""

    def __init__(self, vocab_size=16, dim=8, next_token_logits=None):
        rng = np.random.RandomState(0)
        self.vocab_size, self.dim = vocab_size, dim
        self.E = rng.randn(vocab_size, dim).astype(np.float32)
        self.W = rng.randn(dim, vocab_size).astype(np.float32)
        self.next_token_logits = next_token_logits

    def __call__(self, idx):
        idx = np.asarray(idx).astype(np.int64)
        hidden = self.E[idx]
        if self.next_token_logits is not None:
            T = idx.shape[1]
            logits = np.broadcast_to(self.next_token_logits[None, :T, :],
                                     (idx.shape[0], T, self.vocab_size)).astype(np.float32).copy()
        else:
            logits = hidden @ self.W
        return logits, hidden


def _forced(targets, T_ctx=3, V=16):
    nl = np.full((32, V), -10.0, dtype=np.float32)
    for i, t in enumerate(targets):
        nl[T_ctx - 1 + i, t] = 10.0
    return nl


def _set_heads(dec, tokens):
    for i, t in enumerate(tokens):
        w = np.zeros((dec.vocab_size, dec.dim), np.float32)
        w[t, :] = 10.0
        dec.head_weights[i] = w


def test_draft_k4_candidate_shape():  # reference :81-93
    dec = RefSpeculativeDecoder(8, 16, 4, seed=0)
    toks, lgs = dec.draft(np.random.randn(1, 1, 8).astype(np.float32))
    assert toks.shape == (1, 4) and len(lgs) == 4
    assert all(lg.shape == (1, 16) for lg in lgs)
    assert np.all((toks >= 0) & (toks < 16))


def test_draft_various_hidden_shapes():  # reference :96-114
    dec = RefSpeculativeDecoder(8, 16, 4, seed=0)
    for h in [np.random.randn(2, 8), np.random.randn(2, 5, 8), np.random.randn(2, 1, 8)]:
        assert dec.draft(h.astype(np.float32))[0].shape == (2, 4)
    assert dec.draft(np.random.randn(1, 8).astype(np.float32))[0].shape == (1, 4)


def test_draft_k_other_than_4():  # reference :117-124
    for k in [2, 8]:
        t, lg = RefSpeculativeDecoder(8, 16, k).draft(np.random.randn(1, 1, 8).astype(np.float32))
        assert t.shape == (1, k) and len(lg) == k


def test_draft_head_invalid_k():  # reference :127-132
    for k in [0, -1]:
        with pytest.raises(ValueError):
            RefSpeculativeDecoder(8, 16, k)


def test_verify_accept_all():  # reference :140-184
    mm = FakeMainModel(next_token_logits=_forced([10, 11, 12, 13]))
    dec = RefSpeculativeDecoder(8, 16, 4)
    _set_heads(dec, [10, 11, 12, 13])
    ctx = np.array([[1, 2, 3]], np.int64)
    toks, _ = dec.draft(mm(ctx)[1])
    assert toks[0].tolist() == [10, 11, 12, 13]
    acc, ok, _ = dec.verify_then_commit(toks, mm, ctx)
    assert ok is True and acc == [10, 11, 12, 13]


def test_verify_accept_partial_prefix():  # reference :187-229
    mm = FakeMainModel(next_token_logits=_forced([10, 11, 12, 13]))
    dec = RefSpeculativeDecoder(8, 16, 4)
    _set_heads(dec, [10, 5, 12, 13])
    ctx = np.array([[1, 2, 3]], np.int64)
    toks, _ = dec.draft(mm(ctx)[1])
    assert toks[0].tolist() == [10, 5, 12, 13]
    acc, ok, _ = dec.verify_then_commit(toks, mm, ctx, max_redraft_rounds=0)
    assert ok is False and acc == [10, 11]


def test_verify_reject_first_position():  # reference :232-266
    mm = FakeMainModel(next_token_logits=_forced([5, 6, 7, 8]))
    dec = RefSpeculativeDecoder(8, 16, 4)
    _set_heads(dec, [0, 1, 2, 3])
    ctx = np.array([[1, 2, 3]], np.int64)
    toks, _ = dec.draft(mm(ctx)[1])
    assert toks[0].tolist() == [0, 1, 2, 3]
    acc, ok, _ = dec.verify_then_commit(toks, mm, ctx, max_redraft_rounds=0)
    assert ok is False and acc == [5]


def test_verify_reject_triggers_redraft():  # reference :274-309
    mm = FakeMainModel(next_token_logits=_forced([10, 11, 12, 13]))
    dec = RefSpeculativeDecoder(8, 16, 4)
    _set_heads(dec, [0, 1, 2, 3])
    ctx = np.array([[1, 2, 3]], np.int64)
    toks, _ = dec.draft(mm(ctx)[1])
    acc, ok, new_ctx = dec.verify_then_commit(toks, mm, ctx, max_redraft_rounds=1)
    assert ok is False and acc[0] == 10
    assert new_ctx.shape[1] == ctx.shape[1] + len(acc)


def test_full_draft_verify_pipeline():  # reference :317-345
    mm = FakeMainModel(vocab_size=32, dim=16)
    dec = RefSpeculativeDecoder(16, 32, 4, seed=10)
    ctx = np.array([[5, 6, 7, 8, 9]], np.int64)
    toks, lgs = dec.draft(mm(ctx)[1])
    mask, pred = dec.verify(toks, mm, ctx)
    assert mask.shape == (1, 4) and pred.shape == (1, 4) and mask.dtype == np.bool_
    acc, ok, new_ctx = dec.verify_then_commit(toks, mm, ctx)
    assert 1 <= len(acc) <= 4 and isinstance(ok, bool)
    assert new_ctx.shape == (1, ctx.shape[1] + len(acc))


def test_verify_batch_mismatch_raises():  # reference :374-380
    dec = RefSpeculativeDecoder(8, 16, 4)
    with pytest.raises(ValueError):
        dec.verify(np.array([[1, 2, 3, 4]]), lambda x: np.zeros((1, 4, 16)), np.array([[1, 2], [3, 4]]))


def test_verify_main_model_returns_tuple_or_tensor():  # reference :383-409
    dec = RefSpeculativeDecoder(8, 16, 4)
    ctx, draft = np.array([[1, 2, 3]]), np.array([[5, 6, 7, 8]])
    m1 = lambda x: np.random.randn(x.shape[0], x.shape[1], 16).astype(np.float32)  # noqa: E731
    m2 = lambda x: (m1(x), np.random.randn(x.shape[0], x.shape[1], 8).astype(np.float32))  # noqa: E731
    for m in (m1, m2):
        acc, pred = dec.verify(draft, m, ctx)
        assert acc.shape == (1, 4) and pred.shape == (1, 4)


# ---- batched greedy verify: row 0 equals the reference rule; brute force ----

def _commit_ref(draft_row, pred_row, k, bonus_pred=None):
    out = []
    for i in range(k):
        if draft_row[i] == pred_row[i]:
            out.append(int(draft_row[i]))
        else:
            out.append(int(pred_row[i]))
            return out, False
    if bonus_pred is not None:
        out.append(int(bonus_pred))
    return out, True


@pytest.mark.parametrize("bonus", [False, True])
def test_greedy_batched_matches_reference_rule(bonus):
    rng = np.random.default_rng(5)
    B, k, V = 64, 5, 7
    rows_t = k + 1 if bonus else k
    logits = rng.integers(0, 4, (B, rows_t, V)).astype(np.float32)  # many ties
    pred = np.argmax(logits, -1)
    ids = np.where(rng.random((B, k)) < 0.7, pred[:, :k], rng.integers(0, V, (B, k)))
    acc, p2, alen, out = greedy_verify_batched(logits, ids)
    assert np.array_equal(p2, pred)
    for b in range(B):
        exp, ok = _commit_ref(ids[b], pred[b], k, pred[b, k] if bonus else None)
        got = [int(v) for v in out[b] if v >= 0]
        assert got == exp
        assert (alen[b] == k) == ok


def test_greedy_row0_equals_reference_verify_then_commit():
    rng = np.random.default_rng(6)
    V, k = 16, 4
    for trial in range(50):
        nl = rng.normal(size=(32, V)).astype(np.float32)
        mm = FakeMainModel(next_token_logits=nl)
        dec = RefSpeculativeDecoder(8, V, k)
        ctx = rng.integers(0, V, (1, 3))
        draft = np.where(rng.random((1, k)) < 0.6, np.argmax(nl[2:2 + k], -1)[None], rng.integers(0, V, (1, k)))
        acc_tokens, ok, _ = dec.verify_then_commit(draft, mm, ctx, max_redraft_rounds=0)
        logits = mm(np.concatenate([ctx, draft], 1))[0][:, 2:2 + k]
        _, _, alen, out = greedy_verify_batched(logits, draft)
        assert [int(v) for v in out[0] if v >= 0] == acc_tokens
        assert (alen[0] == k) == ok

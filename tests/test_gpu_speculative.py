"""The reference's test_speculative_decode.py vectors through the GPU
SpeculativeDecoder (draft-head argmax and verify on the gfx950 kernels), and
the batched greedy verify kernel vs the oracle."""
import numpy as np
import pytest
import torch

from oracle.speculative import greedy_verify_batched

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


class FakeMainModel:
    """tests/test_speculative_decode.py:36-73, returning device tensors."""

    def __init__(self, vocab_size=16, dim=8, next_token_logits=None):
        rng = np.random.RandomState(0)
        self.vocab_size = vocab_size
        self.E = torch.from_numpy(rng.randn(vocab_size, dim).astype(np.float32)).cuda()
        self.W = torch.from_numpy(rng.randn(dim, vocab_size).astype(np.float32)).cuda()
        self.nl = None if next_token_logits is None else torch.from_numpy(next_token_logits).cuda()

    def __call__(self, idx):
        idx = idx.long().cuda()
        hidden = self.E[idx]
        if self.nl is not None:
            T = idx.shape[1]
            logits = self.nl[None, :T, :].expand(idx.shape[0], T, self.vocab_size).contiguous()
        else:
            logits = hidden @ self.W
        return logits, hidden


def _forced(targets, T_ctx=3, V=16):
    nl = np.full((32, V), -10.0, dtype=np.float32)
    for i, t in enumerate(targets):
        nl[T_ctx - 1 + i, t] = 10.0
    return nl


def _decoder(dim=8, V=16, k=4, heads=None):
    from versenext_amd import SpeculativeDecoder
    dec = SpeculativeDecoder(dim=dim, vocab_size=V, num_draft_heads=k, seed=0)
    if heads is not None:
        for i, t in enumerate(heads):
            w = np.zeros((V, dim), np.float32)
            w[t, :] = 10.0
            dec.draft_heads[i].weight = w
    return dec


def test_draft_shapes(hip):
    _say("draft shapes")
    dec = _decoder()
    t, lg = dec.draft(np.random.randn(1, 1, 8).astype(np.float32))
    assert t.shape == (1, 4) and len(lg) == 4 and all(tuple(x.shape) == (1, 16) for x in lg)
    assert np.all((t >= 0) & (t < 16))
    for h in [np.random.randn(2, 8), np.random.randn(2, 5, 8), np.random.randn(2, 1, 8)]:
        assert dec.draft(h.astype(np.float32))[0].shape == (2, 4)
    for k in [2, 8]:
        t, lg = _decoder(k=k).draft(np.random.randn(1, 1, 8).astype(np.float32))
        assert t.shape == (1, k) and len(lg) == k
    from versenext_amd import SpeculativeDecoder
    for k in [0, -1]:
        with pytest.raises(ValueError):
            SpeculativeDecoder(dim=8, vocab_size=16, num_draft_heads=k)


def test_draft_argmax_equals_torch(hip):
    _say("draft argmax vs torch")
    dec = _decoder(dim=64, V=50000, k=4)
    h = torch.randn(3, 64)
    toks, lgs = dec.draft(h)
    ref = torch.stack([lg.detach() for lg in lgs], 1).argmax(-1).cpu().numpy()
    assert np.array_equal(toks, ref)


@pytest.mark.parametrize("targets,heads,expect,ok", [
    ([10, 11, 12, 13], [10, 11, 12, 13], [10, 11, 12, 13], True),  # reference :140-184
    ([10, 11, 12, 13], [10, 5, 12, 13], [10, 11], False),          # reference :187-229
    ([5, 6, 7, 8], [0, 1, 2, 3], [5], False),                      # reference :232-266
])
def test_verify_then_commit_reference_vectors(hip, targets, heads, expect, ok):
    _say(f"verify_then_commit {heads}")
    mm = FakeMainModel(next_token_logits=_forced(targets))
    dec = _decoder(heads=heads)
    ctx = np.array([[1, 2, 3]], np.int64)
    toks, _ = dec.draft(mm(torch.from_numpy(ctx))[1])
    assert toks[0].tolist() == heads
    acc, all_ok, new_ctx = dec.verify_then_commit(toks, mm, ctx, max_redraft_rounds=0)
    assert all_ok is ok and acc == expect
    assert new_ctx.shape == (1, 3 + len(expect))


def test_redraft_and_pipeline(hip):
    _say("redraft + pipeline")
    mm = FakeMainModel(next_token_logits=_forced([10, 11, 12, 13]))
    dec = _decoder(heads=[0, 1, 2, 3])
    ctx = np.array([[1, 2, 3]], np.int64)
    toks, _ = dec.draft(mm(torch.from_numpy(ctx))[1])
    acc, ok, new_ctx = dec.verify_then_commit(toks, mm, ctx, max_redraft_rounds=1)
    assert ok is False and acc[0] == 10 and new_ctx.shape[1] == 3 + len(acc)
    mm2 = FakeMainModel(vocab_size=32, dim=16)
    dec2 = _decoder(dim=16, V=32)
    ctx2 = np.array([[5, 6, 7, 8, 9]], np.int64)
    toks2, _ = dec2.draft(mm2(torch.from_numpy(ctx2))[1])
    mask, pred = dec2.verify(toks2, mm2, ctx2)
    assert mask.shape == (1, 4) and pred.shape == (1, 4) and mask.dtype == np.bool_
    acc2, ok2, nc2 = dec2.verify_then_commit(toks2, mm2, ctx2)
    assert 1 <= len(acc2) <= 4 and isinstance(ok2, bool) and nc2.shape == (1, 5 + len(acc2))


def test_verify_errors_and_model_returns(hip):
    _say("verify errors")
    dec = _decoder()
    with pytest.raises(ValueError):
        dec.verify(np.array([[1, 2, 3, 4]]), lambda x: torch.zeros(1, 4, 16), np.array([[1, 2], [3, 4]]))
    ctx, draft = np.array([[1, 2, 3]]), np.array([[5, 6, 7, 8]])
    m1 = lambda x: torch.randn(x.shape[0], x.shape[1], 16)  # noqa: E731  (host tensor)
    m2 = lambda x: (torch.randn(x.shape[0], x.shape[1], 16).cuda(), torch.randn(1))  # noqa: E731
    m3 = lambda x: np.random.randn(x.shape[0], x.shape[1], 16).astype(np.float32)  # noqa: E731
    for m in (m1, m2, m3):
        acc, pred = dec.verify(draft, m, ctx)
        assert acc.shape == (1, 4) and pred.shape == (1, 4)


def test_draft_loss_positive_and_differentiable(hip):
    _say("draft_loss")
    dec = _decoder()
    toks, lgs = dec.draft(np.random.randn(2, 1, 8).astype(np.float32))
    loss = dec.draft_loss(lgs, np.random.randint(0, 16, (2, 4)))
    assert loss.dim() == 0 and float(loss) > 0
    loss.backward()
    assert all(h.weight.grad is not None for h in dec.draft_heads)


@pytest.mark.parametrize("B,k,V,bonus", [(64, 5, 7, True), (32, 8, 248320, True), (9, 3, 1001, False),
                                         (4, 64, 300, True)])
def test_greedy_verify_parity(hip, B, k, V, bonus):
    _say(f"greedy_verify B={B} k={k} V={V} bonus={bonus}")
    rng = np.random.default_rng(B * k + V)
    rows_t = k + 1 if bonus else k
    if V < 100:
        logits = rng.integers(0, 4, (B, rows_t, V)).astype(np.float32)  # many ties
    else:
        logits = rng.normal(0, 2, (B, rows_t, V)).astype(np.float32)
    pred = logits.argmax(-1)
    ids = np.where(rng.random((B, k)) < 0.8, pred[:, :k], rng.integers(0, V, (B, k)))
    acc, p, alen, out = hip.greedy_verify(torch.from_numpy(logits), torch.from_numpy(ids), rows_t=rows_t)
    ra, rp, ral, rout = greedy_verify_batched(logits, ids)
    assert np.array_equal(acc.cpu().numpy(), ra) and np.array_equal(p.cpu().numpy(), rp)
    assert np.array_equal(alen.cpu().numpy(), ral) and np.array_equal(out.cpu().numpy(), rout)


def test_verify_batch_all_rows(hip):
    _say("verify_batch")
    rng = np.random.default_rng(3)
    B, T, k, V = 6, 5, 4, 64
    nl = rng.normal(size=(B, T + k, V)).astype(np.float32)

    def model(idx):
        return torch.from_numpy(nl[:, :idx.shape[1]]).cuda()

    dec = _decoder(V=V)
    ctx = rng.integers(0, V, (B, T))
    pred = nl.argmax(-1)
    draft = np.where(rng.random((B, k)) < 0.7, pred[:, T - 1:T - 1 + k], rng.integers(0, V, (B, k)))
    alen, out = dec.verify_batch(draft, model, ctx, bonus=True)
    _, _, ral, rout = greedy_verify_batched(nl[:, T - 1:T + k], draft)
    assert np.array_equal(alen.cpu().numpy(), ral) and np.array_equal(out.cpu().numpy(), rout)

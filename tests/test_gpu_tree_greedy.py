"""GPU parity of greedy tree verification (vnx_tree_greedy) and row top-b
(vnx_row_topk, tree expansion) against oracle/tree.py.  Integer outputs:
bit-exact."""
import numpy as np
import pytest
import torch

from oracle import speculative as OS
from oracle import tree as OT
from versenext_amd import tree as T

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _plant(rng, target, tokens, parent, frac):
    """Makes a fraction `frac` of the nodes match their parent's target row
    (the node's token becomes that row's maximum), so paths get accepted."""
    par = np.asarray(parent)
    rows = np.where(par < 0, 0, par + 1)
    B, N = tokens.shape
    for b in range(B):
        for n in range(N):
            if rng.random() < frac:
                r = rows[n]
                target[b, r, tokens[b, n]] = target[b, r].max() + 1.0


def _check_greedy(hip, target_np, tokens, parent, dtype=torch.float32):
    dev = hip.torch_device
    tg = torch.from_numpy(target_np).to(dev).to(dtype)
    alen, best, out, pred = hip.tree_greedy(tg, torch.from_numpy(tokens).to(dev), parent)
    torch.cuda.synchronize()
    ref_in = tg.float().cpu().numpy() if dtype != torch.float32 else target_np
    r_alen, r_best, r_out, r_pred = OT.tree_greedy(ref_in, tokens, parent)
    assert np.array_equal(pred.cpu().numpy(), r_pred)
    assert np.array_equal(alen.cpu().numpy(), r_alen)
    assert np.array_equal(best.cpu().numpy(), r_best)
    o = out.cpu().numpy()
    w = r_out.shape[1]
    assert np.array_equal(o[:, :w], r_out)
    assert np.all(o[:, w:] == -1)
    b_alen, b_best = OT.tree_greedy_bruteforce(ref_in, tokens, parent)
    assert np.array_equal(r_alen, b_alen) and np.array_equal(r_best, b_best)
    return r_alen


def test_config3_tree_greedy(hip):
    """B 16, tree (4,3,2) = 40 nodes, V 248,320, logits
    N(0, 2); node tokens are the top-b of the parent's draft row, and some
    nodes are planted to match so that paths of every depth occur."""
    _say("tree_greedy config 3 B=16 N=40 V=248320 fp32")
    B, V = 16, 248320
    par = T.tree_from_branching((4, 3, 2))
    rng = np.random.default_rng(11)
    target = rng.normal(0, 2, (B, 41, V)).astype(np.float32)
    draft = np.random.default_rng(12).normal(0, 2, (B, 17, V)).astype(np.float32)
    tokens = OT.expand_tree(draft, par)
    _plant(rng, target, tokens, par, 0.6)
    alen = _check_greedy(hip, target, tokens, par)
    _say(f"  accept lengths {alen.tolist()}")
    assert alen.max() >= 2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_random_trees(hip, dtype):
    rng = np.random.default_rng(5)
    for N in (1, 2, 17, 40, 64):
        par = np.array([-1] + [int(rng.integers(-1, i)) for i in range(1, N)], np.int32)
        B, V = 6, 3000 + N
        _say(f"tree_greedy random tree N={N} B={B} V={V} {dtype}")
        target = rng.normal(0, 1, (B, N + 1, V)).astype(np.float32)
        tokens = rng.integers(0, V, (B, N)).astype(np.int64)
        _plant(rng, target, tokens, par, 0.7)
        _check_greedy(hip, target, tokens, par, dtype)


def test_ties_and_nan_follow_numpy_argmax(hip):
    """Tied maxima go to the lowest id, NaN counts as the maximum."""
    rng = np.random.default_rng(9)
    par = T.tree_from_branching((2, 2))
    B, N, V = 4, 6, 4099
    target = rng.normal(0, 1, (B, N + 1, V)).astype(np.float32)
    target[:, :, 100] = 50.0
    target[:, :, 4000] = 50.0           # tie: 100 wins
    target[1, 2, 3000] = np.nan         # NaN wins row (1, 2)
    target[2, 0, 7] = np.nan
    target[2, 0, 5] = np.nan            # first NaN wins
    tokens = np.full((B, N), 100, np.int64)
    tokens[1, 2] = 3000
    _check_greedy(hip, target, tokens, par)


def test_chain_is_reference_prefix_rule_with_bonus(hip):
    """A chain tree gives the reference's accepted prefix (speculative.py:
    277-287) and, when all k match, the bonus argmax of row k."""
    rng = np.random.default_rng(3)
    B, k, V = 8, 6, 5000
    target = rng.normal(0, 1, (B, k + 1, V)).astype(np.float32)
    pred = target.argmax(-1)
    draft = pred[:, :k].copy()
    for b in range(B):
        if b % 3:
            draft[b, rng.integers(0, k)] = (draft[b, 0] + 1) % V
    dev = hip.torch_device
    alen, best, out, _ = hip.tree_greedy(torch.from_numpy(target).to(dev), torch.from_numpy(draft).to(dev),
                                         T.chain(k))
    _, _, r_alen, r_out = OS.greedy_verify_batched(target, draft)
    assert np.array_equal(alen.cpu().numpy(), r_alen)
    assert np.array_equal(out.cpu().numpy(), r_out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V,b", [(5, 1), (17, 4), (1000, 3), (4099, 16), (8193, 8), (248320, 4), (248320, 16),
                                 (600000, 2)])
def test_topk_matches_sorted_order(hip, dtype, V, b):
    _say(f"topk V={V} b={b} {dtype}")
    rng = np.random.default_rng(V + b)
    R = 33
    x = rng.normal(0, 2, (R, V)).astype(np.float32)
    x[0, :] = 1.0                                   # all tied
    x[1, V // 2] = np.nan
    x[2, :] = -np.inf
    if V > 10:
        x[3, 3] = x[3, 9] = 40.0                    # tie at the top
        x[4, :V // 2] = -np.inf
    t = torch.from_numpy(x).to(hip.torch_device).to(dtype)
    ids, vals = hip.topk(t, b)
    ref_in = t.float().cpu().numpy()
    r_ids, r_vals = OT.topk_rows(ref_in, b)
    assert np.array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(vals.cpu().numpy(), r_vals)


def test_expand_tree_matches_oracle(hip):
    rng = np.random.default_rng(21)
    par = T.tree_from_branching((4, 3, 2))
    draft = rng.normal(0, 2, (3, 17, 20000)).astype(np.float32)
    tok = hip.expand_tree(torch.from_numpy(draft).to(hip.torch_device), par)
    assert np.array_equal(tok.cpu().numpy(), OT.expand_tree(draft, par))


def test_rejects_bad_trees(hip):
    dev = hip.torch_device
    tg = torch.zeros((1, 4, 64), device=dev)
    tok = torch.zeros((1, 3), dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        hip.tree_greedy(tg, tok, [-1, 2, 0])          # parent after child
    with pytest.raises(ValueError):
        hip.tree_greedy(tg[:, :3], tok, [-1, 0, 1])   # N+1 rows needed
    with pytest.raises(ValueError):
        hip.topk(tg[0], 17)

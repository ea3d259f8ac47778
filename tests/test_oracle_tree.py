"""Pins oracle/tree.py and the host tree helpers (versenext_amd/tree.py).

Attention: the chain tree must equal causal attention computed by a library
routine (torch's scaled_dot_product_attention in fp64 on the CPU), a single
node / an all-visible mask must equal plain prefix attention, and the masked
formulation must equal the per-node gathered one on random trees.  A
transposed mask (descendants instead of ancestors), a dropped self bit or a
dropped prefix each fail one of these.

Greedy path: tree_greedy must equal brute-force enumeration of every root
path, and on chains the reference's prefix rule (oracle.speculative
.greedy_verify_batched, itself pinned to tests/test_speculative_decode.py's
vectors).  Top-b: equal to a full stable sort."""
import numpy as np
import pytest
import torch

from oracle import speculative as OS
from oracle import tree as OT
from versenext_amd import tree as T


def _qkv(rng, B, H, Hkv, N, Tp, d):
    q = rng.normal(0, 1, (B, H, N, d))
    kc = rng.normal(0, 1, (B, Hkv, Tp, d)) if Tp else None
    vc = rng.normal(0, 1, (B, Hkv, Tp, d)) if Tp else None
    kt = rng.normal(0, 1, (B, Hkv, N, d))
    vt = rng.normal(0, 1, (B, Hkv, N, d))
    return q, kc, vc, kt, vt


def _random_parents(rng, n):
    return np.array([-1] + [int(rng.integers(-1, i)) for i in range(1, n)], np.int32)


def test_branching_tree_shape():
    par = T.tree_from_branching((4, 3, 2))
    assert par.size == 40
    assert np.all(par[:4] == -1) and np.all(par[4:16] == np.repeat(np.arange(4), 3))
    assert np.all(par[16:] == np.repeat(np.arange(4, 16), 2))
    d = T.depths(par)
    assert d.tolist() == [1] * 4 + [2] * 12 + [3] * 24
    w = T.ancestor_words(par)
    pop = np.array([bin(int(x)).count("1") for x in w])
    assert np.array_equal(pop, d)  # ancestors-or-self = depth many nodes
    for i, p in enumerate(par):
        assert int(w[i]) >> i & 1
        if p >= 0:
            assert int(w[p]) & ~int(w[i]) == 0  # a parent's set is inside its child's
    assert T.draft_rows(par).max() == 16  # 17 draft rows: root + 16 internal nodes


def test_words_mask_round_trip_and_rejections():
    rng = np.random.default_rng(0)
    par = _random_parents(rng, 23)
    w = T.ancestor_words(par)
    m = T.mask_from_words(w, 7)
    assert np.array_equal(T.words_from_mask(m, 7), w)
    bad = m.copy()
    bad[3, 2] = -np.inf  # a hidden prefix column is not a tree mask
    assert T.words_from_mask(bad, 7) is None
    bad = m.copy()
    bad[4, 7 + 4] = -np.inf  # no self bit
    assert T.words_from_mask(bad, 7) is None
    assert T.words_from_mask(np.where(np.isinf(m), -1e9, 0.0), 7) is not None  # TriSparse's -1e9
    with pytest.raises(ValueError):
        T.check_parents([0, -1])  # parent must precede the child
    with pytest.raises(ValueError):
        T.ancestor_words(np.full(65, -1))


@pytest.mark.parametrize("Tp", [0, 5, 33])
def test_chain_tree_is_causal_attention(Tp):
    rng = np.random.default_rng(Tp)
    B, H, N, d = 2, 3, 9, 16
    q, kc, vc, kt, vt = _qkv(rng, B, H, H, N, Tp, d)
    words = T.ancestor_words(T.chain(N))
    got, _ = OT.tree_attention(q, kc, vc, kt, vt, words)
    K = kt if kc is None else np.concatenate([kc, kt], 2)
    V = vt if vc is None else np.concatenate([vc, vt], 2)
    allow = np.ones((N, Tp + N), bool)
    allow[:, Tp:] = np.tril(np.ones((N, N), bool))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(K), torch.from_numpy(V), attn_mask=torch.from_numpy(allow)).numpy()
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    if Tp == 0:
        ref2 = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q), torch.from_numpy(K), torch.from_numpy(V), is_causal=True).numpy()
        assert np.allclose(got, ref2, rtol=1e-12, atol=1e-12)


def test_single_node_and_all_visible_are_prefix_attention():
    rng = np.random.default_rng(1)
    B, H, Tp, d = 2, 2, 17, 8
    q, kc, vc, kt, vt = _qkv(rng, B, H, H, 1, Tp, d)
    got, _ = OT.tree_attention(q, kc, vc, kt, vt, np.array([1], np.uint64))
    K, V = np.concatenate([kc, kt], 2), np.concatenate([vc, vt], 2)
    s = np.einsum("bhnd,bhtd->bhnt", q, K) / np.sqrt(d)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.allclose(got, p @ V, rtol=1e-13, atol=1e-13)
    # all bits set: every node sees every key (the mask-free DeviceBackend.attention)
    N = 6
    q, kc, vc, kt, vt = _qkv(rng, B, H, H, N, Tp, d)
    got, _ = OT.tree_attention(q, kc, vc, kt, vt, np.full(N, (1 << N) - 1, np.uint64))
    K, V = np.concatenate([kc, kt], 2), np.concatenate([vc, vt], 2)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(K), torch.from_numpy(V)).numpy()
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed", range(4))
def test_masked_equals_gathered_on_random_trees(seed):
    rng = np.random.default_rng(10 + seed)
    N = int(rng.integers(1, 20))
    Tp = int(rng.integers(0, 12))
    H, Hkv = (4, 2) if seed % 2 else (2, 2)
    q, kc, vc, kt, vt = _qkv(rng, 2, H, Hkv, N, Tp, 8)
    par = _random_parents(rng, N)
    got, mag = OT.tree_attention(q, kc, vc, kt, vt, T.ancestor_words(par))
    ref = OT.tree_attention_gathered(q, kc, vc, kt, vt, par)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert np.all(mag >= np.abs(got) - 1e-12)


def test_per_batch_words_differ_from_shared():
    rng = np.random.default_rng(3)
    q, kc, vc, kt, vt = _qkv(rng, 2, 2, 2, 5, 4, 8)
    w0 = T.ancestor_words(T.chain(5))
    w1 = T.ancestor_words(np.full(5, -1, np.int32))
    got, _ = OT.tree_attention(q, kc, vc, kt, vt, np.stack([w0, w1]))
    a, _ = OT.tree_attention(q[:1], kc[:1], vc[:1], kt[:1], vt[:1], w0)
    b, _ = OT.tree_attention(q[1:], kc[1:], vc[1:], kt[1:], vt[1:], w1)
    assert np.allclose(got, np.concatenate([a, b]))


def _greedy_case(rng, B, par, V, hit=0.7):
    N = par.size
    target = rng.normal(0, 1, (B, N + 1, V)).astype(np.float32)
    pred = target.argmax(-1)
    prow = np.where(par < 0, 0, par + 1)
    tokens = rng.integers(0, V, (B, N))
    agree = rng.random((B, N)) < hit
    tokens = np.where(agree, pred[:, prow], tokens)
    return target, tokens


@pytest.mark.parametrize("seed", range(6))
def test_tree_greedy_matches_bruteforce(seed):
    rng = np.random.default_rng(seed)
    par = T.tree_from_branching((4, 3, 2)) if seed < 2 else _random_parents(rng, int(rng.integers(1, 40)))
    target, tokens = _greedy_case(rng, 16, par, 11)
    alen, best, out, pred = OT.tree_greedy(target, tokens, par)
    alen2, best2 = OT.tree_greedy_bruteforce(target, tokens, par)
    assert np.array_equal(alen, alen2) and np.array_equal(best, best2)
    for b in range(16):
        n = alen[b]
        assert out[b, n] == pred[b, 0 if best[b] < 0 else best[b] + 1]
        assert np.all(out[b, n + 1:] == -1)


def test_tree_greedy_on_chain_is_the_reference_prefix_rule():
    rng = np.random.default_rng(5)
    k = 6
    par = T.chain(k)
    target, tokens = _greedy_case(rng, 32, par, 7, hit=0.8)
    alen, best, out, _ = OT.tree_greedy(target, tokens, par)
    # chain: node i's parent row is row i, so tree rows 0..k are the chain's k+1 rows
    acc, pred, alen2, out2 = OS.greedy_verify_batched(target, tokens)
    assert np.array_equal(alen, alen2)
    full = alen == k
    assert np.array_equal(out[:, :k][~full], out2[:, :k][~full])  # blessed token at the mismatch
    assert np.array_equal(out[full, :k], tokens[full])


def test_topk_rows_is_a_stable_sort_and_expand_tree():
    rng = np.random.default_rng(2)
    x = rng.integers(-3, 3, (5, 40)).astype(np.float32)  # many ties
    x[1, 7] = np.nan
    ids, vals = OT.topk_rows(x, 6)
    for r in range(5):
        row = x[r]
        if np.isnan(row).any():
            assert ids[r, 0] == 7
            continue
        ref = sorted(range(40), key=lambda j: (-row[j], j))[:6]
        assert ids[r].tolist() == ref
    assert np.array_equal(OT.topk_rows(x, 1)[0][:, 0], np.argmax(x, -1))
    par = T.tree_from_branching((3, 2))
    draft = rng.normal(0, 1, (2, 4, 50)).astype(np.float32)
    tok = OT.expand_tree(draft, par)
    top3 = np.argsort(-draft, axis=-1, kind="stable")
    assert np.array_equal(tok[:, :3], top3[:, 0, :3])
    assert np.array_equal(tok[:, 3:5], top3[:, 1, :2]) and np.array_equal(tok[:, 7:9], top3[:, 3, :2])

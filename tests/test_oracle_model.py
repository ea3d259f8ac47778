"""The CPU model oracle (oracle/model.py) against golden vectors the reference
wrote (tests/golden/make_cometspark_small.py): the reference's own forward
logits, greedy stream and greedy speculative decode of the config-1 models,
and a toy model with the mate target's RoPE + MoD top-2 choices."""
import os

import numpy as np
import pytest

from oracle import model as OM
from versenext_amd import model as VM

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cometspark_small.npz")


@pytest.fixture(scope="module")
def gold():
    z = np.load(GOLD)
    return {k: z[k] for k in z.files}


def _w(gold, prefix):
    return {k[len(prefix):]: v for k, v in gold.items() if k.startswith(prefix)}


def rope_cfg():
    return VM.ModelConfig(vocab_size=256, dim=64, n_layer=2, n_head=4, n_kv_head=2,
                          layer_pattern=VM.v02_pattern(2, 2), window_size=32, num_global_tokens=4,
                          use_alibi=False, use_rope=True, num_dense_parts=2, num_experts_per_part=4, top_k=2)


def test_weight_names_and_shapes_match_the_reference_state_dict(gold):
    for prefix, cfg in (("t/", VM.small_target()), ("d/", VM.small_draft()), ("r/", rope_cfg())):
        W = _w(gold, prefix)
        shapes = VM.weight_shapes(cfg)
        assert set(shapes) == set(W) - {"head.weight"}
        for k, s in shapes.items():
            assert W[k].shape == s, k
        assert np.array_equal(W["head.weight"], W["tok_emb.weight"])  # tied head


@pytest.mark.parametrize("prefix,key,cfg", [("t/", "long_target_logits", VM.small_target()),
                                            ("d/", "long_draft_logits", VM.small_draft()),
                                            ("r/", "long_rope_logits", rope_cfg())])
def test_forward_matches_reference_logits(gold, prefix, key, cfg):
    """150 tokens: past the 32-token window (SWA masking), ALiBi on / off,
    RoPE, MoD top-1 of 2 and top-2 of 4."""
    got = OM.forward(_w(gold, prefix), cfg, gold["long_seq"])[:, gold["long_rows"]]
    ref = gold[key]
    assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, float(np.max(np.abs(ref))))


def test_prompt_logits(gold):
    got = OM.forward(_w(gold, "t/"), VM.small_target(), gold["prompt"])
    assert np.max(np.abs(got - gold["logits"])) <= 1e-5


def test_greedy_stream_and_speculative_decode(gold):
    Wt, Wd = _w(gold, "t/"), _w(gold, "d/")
    ct, cd = VM.small_target(), VM.small_draft()
    assert np.array_equal(OM.greedy_stream(Wt, ct, gold["prompt"], 128), gold["greedy128"])
    toks, steps = OM.spec_decode_greedy(Wt, ct, Wd, cd, gold["prompt"], 128, 4)
    assert np.array_equal(toks, gold["spec128"]) and steps == int(gold["spec_steps"])


def test_planted_mistakes_fail(gold):
    """A dropped ALiBi path, a wrong window or a missing RoPE each move the
    logits well past the golden test's tolerance (1e-5 of max|logit|), so
    that check can see them.  (At random init the attention scores are
    small, which is why a missing RoPE moves the logits by only ~2e-4.)"""
    seq = gold["long_seq"]
    rows = gold["long_rows"]
    tol = 1e-5 * 1.6
    W = _w(gold, "t/")
    base = OM.forward(W, VM.small_target(), seq)[:, rows]
    c = VM.small_target()
    c.use_alibi = False
    assert np.max(np.abs(OM.forward(W, c, seq)[:, rows] - base)) > 5 * tol
    c = VM.small_target()
    c.window_size = 16
    assert np.max(np.abs(OM.forward(W, c, seq)[:, rows] - base)) > 5 * tol
    Wr = _w(gold, "r/")
    c = rope_cfg()
    c.use_rope = False
    assert np.max(np.abs(OM.forward(Wr, c, seq)[:, rows] - gold["long_rope_logits"])) > 5 * tol


def test_mate_config_sizes():
    """CometSparkV05(): 20 layers (5 mod + 15 trisparse), ~1.12e9 parameters
    with the tied head (spark/src/base_model.py docstring: 861M + 254M)."""
    cfg = VM.mate_target()
    assert cfg.layer_pattern.count("mod") == 5 and cfg.layer_pattern.count("trisparse") == 15
    n = sum(int(np.prod(s)) for s in VM.weight_shapes(cfg).values())
    assert 1.05e9 < n < 1.2e9, n
    assert cfg.ffn_hidden == 2752 and cfg.expert_hidden_eff == 2688
    d = VM.mate_draft()
    assert d.ffn_hidden == 4096 and d.head_dim == 64

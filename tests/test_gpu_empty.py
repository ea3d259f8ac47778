"""Empty batches through the entry points: B = 0 rows (a serving loop whose
batch drained, numpy's behaviour on empty arrays) returns empty outputs of
the right shapes without a launch, for the acceptance, the draws, the
Sampler, the row reductions, the tree path, the LM head and attention."""
import numpy as np
import pytest
import torch

from versenext_amd import tree as T

pytestmark = pytest.mark.gpu

V, k = 1000, 4


def _z(*s, dtype=torch.float32, dev=None):
    return torch.zeros(s, dtype=dtype, device=dev)


def test_acceptance_and_draws(hip):
    dev = hip.torch_device
    res = hip.spec_accept(_z(0, k + 1, V, dev=dev), _z(0, k, V, dev=dev), _z(0, k, dtype=torch.int64, dev=dev),
                          _z(0, k + 1, dev=dev), temperature=0.8)
    assert tuple(res["accept_len"].shape) == (0,) and tuple(res["out_ids"].shape) == (0, k + 1)
    ids = hip.sample(_z(0, V, dev=dev), _z(0, dev=dev), temperature=0.8)
    assert ids.numel() == 0


def test_sampler_and_row_reductions(hip):
    dev = hip.torch_device
    out = hip.sampler_sample(_z(0, V, dev=dev), _z(0, dev=dev), temperature=0.8, top_k=50, top_p=0.9)
    ids = out["ids"] if isinstance(out, dict) else out
    assert ids.numel() == 0
    assert hip.argmax(_z(0, V, dev=dev)).numel() == 0
    assert hip.softmax(_z(0, V, dev=dev)).shape == (0, V)
    lse = hip.row_lse(_z(0, V, dev=dev))
    assert (lse[0] if isinstance(lse, tuple) else lse).numel() == 0


def test_tree_path_and_head(hip):
    dev = hip.torch_device
    ids, vals = hip.topk(_z(0, V, dev=dev), 4)
    assert ids.shape[0] == 0
    par = T.chain(k)
    alen, best, out, _ = hip.tree_greedy(_z(0, k + 1, V, dev=dev), _z(0, k, dtype=torch.int64, dev=dev), par)
    assert alen.numel() == 0
    r = hip.greedy_verify(_z(0, k + 1, V, dev=dev), _z(0, k, dtype=torch.int64, dev=dev), rows_t=k + 1)
    assert all(t.shape[0] == 0 for t in r if isinstance(t, torch.Tensor))
    logits = hip.lm_head(_z(0, 64, dtype=torch.bfloat16, dev=dev), _z(V, 64, dtype=torch.bfloat16, dev=dev))
    assert tuple(logits.shape) == (0, V)


@pytest.mark.parametrize("fp32_rows", [False, True])
def test_attention(hip, fp32_rows):
    dev = hip.torch_device
    d = 16 if fp32_rows else 64
    dt = torch.float32 if fp32_rows else torch.bfloat16
    out = hip.tree_attention(_z(0, 2, 4, d, dtype=dt, dev=dev), _z(0, 1, 8, d, dtype=dt, dev=dev),
                             _z(0, 1, 8, d, dtype=dt, dev=dev), _z(0, 1, 4, d, dtype=dt, dev=dev),
                             _z(0, 1, 4, d, dtype=dt, dev=dev), T.ancestor_words(T.chain(4)), fp32_rows=fp32_rows)
    assert tuple(out.shape) == (0, 2, 4, d)

"""GPU check of the one-launch round commit (vnx_spec_commit) against a
numpy restatement of the commit rule (SpeculativeDecoder.verify_then_commit,
packages/verse_nex/verse_nex/speculative.py:277-310, per sequence): append
ids[b, :n_b + 1] at count[b], advance count and both cache lengths by
n_b + 1, carry ids[b, n_b] as the next round's first token, and summarise
(min count, max lens_t, max lens_d, sum n_b).  Integer work: bit-exact."""
import ctypes

import numpy as np
import pytest
import torch

from versenext_amd import _lib

pytestmark = pytest.mark.gpu
P = ctypes.c_void_p


def _ref(alen, ids, out, count, c, lt, ld, k, n_cap):
    out, count, c, lt, ld = out.copy(), count.copy(), c.copy(), lt.copy(), ld.copy()
    n = np.clip(alen, 0, k)
    for b in range(len(alen)):
        for j in range(n[b] + 1):
            pos = count[b] + j
            if pos < n_cap:
                out[b, pos] = ids[b, j]
        count[b] += n[b] + 1
        c[b] = ids[b, n[b]]
        lt[b] += n[b] + 1
        ld[b] += n[b] + 1
    info = np.array([count.min(), lt.max(), ld.max(), n.sum()], np.int64)
    return out, count, c, lt, ld, info


@pytest.mark.parametrize("B,k,n_cap", [(32, 6, 40), (1, 1, 3), (70, 8, 12), (1024, 3, 9)])
def test_commit_matches_rule(hip, B, k, n_cap):
    print(f"spec_commit B={B} k={k} n_cap={n_cap}", flush=True)
    rng = np.random.default_rng(B + k)
    dev = hip.torch_device
    alen = rng.integers(-1, k + 2, B).astype(np.int32)          # includes out-of-range values (clamped)
    ids = rng.integers(0, 1000, (B, k + 1)).astype(np.int64)
    out = np.full((B, n_cap + 1), -1, np.int64)
    count = rng.integers(0, n_cap, B).astype(np.int64)           # some rows near / past the end
    c = np.zeros(B, np.int64)
    lt = rng.integers(0, 500, B).astype(np.int32)
    ld = rng.integers(0, 500, B).astype(np.int32)
    t = {name: torch.from_numpy(a.copy()).to(dev) for name, a in
         dict(alen=alen, ids=ids, out=out, count=count, c=c, lt=lt, ld=ld).items()}
    info = torch.zeros(4, dtype=torch.int64, device=dev)
    _lib.check(_lib.lib().vnx_spec_commit(
        P(t["alen"].data_ptr()), P(t["ids"].data_ptr()), k + 1, B, k, P(t["out"].data_ptr()), n_cap + 1, n_cap,
        P(t["count"].data_ptr()), P(t["c"].data_ptr()), P(t["lt"].data_ptr()), P(t["ld"].data_ptr()),
        P(info.data_ptr()), P(torch.cuda.current_stream().cuda_stream)), "spec_commit")
    torch.cuda.synchronize()
    r_out, r_count, r_c, r_lt, r_ld, r_info = _ref(alen, ids, out, count, c, lt, ld, k, n_cap)
    assert np.array_equal(t["out"].cpu().numpy(), r_out)
    assert np.array_equal(t["count"].cpu().numpy(), r_count)
    assert np.array_equal(t["c"].cpu().numpy(), r_c)
    assert np.array_equal(t["lt"].cpu().numpy(), r_lt)
    assert np.array_equal(t["ld"].cpu().numpy(), r_ld)
    assert np.array_equal(info.cpu().numpy(), r_info)


def test_commit_rejects_bad_arguments(hip):
    z = torch.zeros(8, dtype=torch.int64, device=hip.torch_device)
    st = P(torch.cuda.current_stream().cuda_stream)
    L = _lib.lib()
    assert L.vnx_spec_commit(None, P(z.data_ptr()), 2, 1, 1, P(z.data_ptr()), 4, 4, P(z.data_ptr()), P(z.data_ptr()),
                             P(z.data_ptr()), P(z.data_ptr()), P(z.data_ptr()), st) == _lib.VNX_ERR_INVALID_ARG
    assert L.vnx_spec_commit(P(z.data_ptr()), P(z.data_ptr()), 2, 1025, 1, P(z.data_ptr()), 4, 4, P(z.data_ptr()),
                             P(z.data_ptr()), P(z.data_ptr()), P(z.data_ptr()), P(z.data_ptr()), st) \
        == _lib.VNX_ERR_UNSUPPORTED

"""GPU parity: vnx_spec_accept_draft_lse (the acceptance that takes the
draft rows' LSEs from the draws that produced the draft ids) against
vnx_spec_accept, which streams the draft rows itself, and against the
oracle (oracle.speculative.spec_accept).

The draft ids are drawn on the GPU with vnx_sample from q_i / T with the
uniforms spec_inputs.make_inputs uses (so they equal its ids except where a
CDF-edge flag marks a draw); vnx_sample's row LSEs and flags go, as a
(k, B) array, to the new entry.  Bar: accept_len and out_ids bit-exact with
vnx_spec_accept and with the oracle, a row differing only where a flag
marks it (near tie, LSE edge, CDF edge); the draws' LSEs equal
vnx_spec_accept's draft-row LSEs except on LSE-edge rows; the target-row
LSEs are the same values or, at a rounding midpoint, one ulp apart."""
import numpy as np
import pytest
import torch

from oracle.speculative import spec_accept
from spec_inputs import make_inputs

pytestmark = pytest.mark.gpu

EXCUSE = 1 | 2 | 4  # near tie, LSE edge, CDF edge


def _say(*a):
    print(*a, flush=True)


def _draws(hip, df, ux, T, ld=None):
    """k draws of B rows: ids (B, k), lse (k, ld) and flags (k, ld)."""
    B, k, _ = df.shape
    ld = ld or B
    dev = hip.torch_device
    lse = torch.full((k, ld), float("nan"), dtype=torch.float32, device=dev)
    fl = torch.full((k, ld), 255, dtype=torch.uint8, device=dev)
    ids = torch.empty((k, B), dtype=torch.int64, device=dev)
    u = torch.from_numpy(np.ascontiguousarray(ux.T)).to(dev)
    for i in range(k):
        hip.sample(df[:, i], u[i], temperature=T, out=ids[i], lse_out=lse[i, :B], flags_out=fl[i, :B])
    return ids.t().contiguous(), lse[:, :B], fl[:, :B]


def _differs(a, b, flags_a, flags_b):
    rows = []
    for r in range(a["accept_len"].shape[0]):
        if a["accept_len"][r] == b["accept_len"][r] and np.array_equal(a["out_ids"][r], b["out_ids"][r]):
            continue
        upto = max(int(a["accept_len"][r]), int(b["accept_len"][r])) + 1
        rows.append((r, bool(((flags_a[r, :upto] | flags_b[r, :upto]) & EXCUSE).any())))
    return rows


def _case(hip, B, k, V, T, dtype=torch.float32, ld=None, with_flags=True, max_explained=2):
    _say(f"spec_accept_draft_lse B={B} k={k} V={V} T={T} dtype={dtype} ld={ld}")
    tgt, dft, ids_ref, u = make_inputs(B, k, V, T)
    ux = np.random.default_rng(3).random((B, k)).astype(np.float32)  # make_inputs' draw uniforms
    dev = hip.torch_device
    tg = torch.from_numpy(tgt).to(dev).to(dtype)
    df = torch.from_numpy(dft).to(dev).to(dtype)
    ids, lse_dr, fl_dr = _draws(hip, df, ux, T, ld)
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy()
    fl_h = fl_dr.cpu().numpy()
    if dtype == torch.float32:
        # the GPU draws are make_inputs' inverse-CDF draws
        same = ids_h == ids_ref
        assert np.all(same | ((fl_h.T & 4) != 0)), np.argwhere(~same)[:5]
    un = torch.from_numpy(u)
    new = hip.spec_accept(tg, df, ids, un, temperature=T, lse_d_in=lse_dr,
                          flags_d_in=fl_dr if with_flags else None)
    old = hip.spec_accept(tg, df, ids, un, temperature=T)
    torch.cuda.synchronize()
    new = {k_: v.cpu().numpy() for k_, v in new.items()}
    old = {k_: v.cpu().numpy() for k_, v in old.items()}
    # the draws' LSEs are the draft-row LSEs vnx_spec_accept computes
    edge_d = ((old["flags"][:, :k] & 2) != 0) | ((fl_h.T & 2) != 0)
    assert np.all((new["lse_d"] == old["lse_d"]) | edge_d)
    # the target rows are cut into other chunks here (k + 1 rows instead of
    # 2k + 1), so the fp64 LSE may round to the neighbouring fp32 value,
    # which only happens within 1e-7 of a rounding midpoint: one ulp at most
    nt = old["lse_t"].view(np.int32).astype(np.int64)
    dt = np.abs(new["lse_t"].view(np.int32).astype(np.int64) - nt)
    assert dt.max() <= 1 and np.count_nonzero(dt) <= max(1, dt.size // 100), int(np.count_nonzero(dt))
    d_old = _differs(new, old, new["flags"], old["flags"])
    assert all(ok for _, ok in d_old), d_old
    assert len(d_old) <= max_explained, d_old
    # and the oracle on the logits as the kernels read them
    tf, dfl = tg.float().cpu().numpy(), df.float().cpu().numpy()
    o = spec_accept(tf, dfl, ids_h, u, T)
    d_or = _differs(new, o, new["flags"], o["flags"])
    assert all(ok for _, ok in d_or), d_or
    assert len(d_or) <= max_explained, d_or
    _say(f"  mean accept {new['accept_len'].mean():.3f}, vs vnx_spec_accept {len(d_old)} flagged rows differ, "
         f"vs oracle {len(d_or)}")
    return new


@pytest.mark.parametrize("B,k,V,T", [(8, 4, 1000, 1.0), (16, 8, 32000, 0.8), (5, 3, 4099, 1.7), (3, 1, 7, 0.8)])
def test_draft_lse_small(hip, B, k, V, T):
    _case(hip, B, k, V, T)


def test_draft_lse_config2_full_size(hip):
    """B=64, k=8, V=248,320, T=0.8."""
    r = _case(hip, 64, 8, 248320, 0.8)
    assert r["accept_len"].min() >= 0 and r["accept_len"].max() <= 8


def test_draft_lse_config5_shape_bf16(hip):
    """The e2e round's shape: B=32, k=6, V=248,320, T=0.8, bf16 logits,
    the LSE rows in a (k, 40) array (leading dimension above B)."""
    _case(hip, 32, 6, 248320, 0.8, dtype=torch.bfloat16, ld=40)


def test_draft_lse_without_flags(hip):
    _case(hip, 16, 5, 50000, 0.9, with_flags=False)


def test_draft_lse_rejects(hip):
    tgt, dft, ids, u = make_inputs(4, 3, 500, 0.8)
    dev = hip.torch_device
    tg, df = torch.from_numpy(tgt).to(dev), torch.from_numpy(dft).to(dev)
    lse = torch.zeros((3, 4), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError):
        hip.spec_accept(tg, df, ids, u, 0.8, thr_t=np.zeros((4, 4), np.float32), lse_d_in=lse)
    with pytest.raises(ValueError):
        hip.spec_accept(tg, df, ids, u, 0.8, lse_d_in=lse.t())

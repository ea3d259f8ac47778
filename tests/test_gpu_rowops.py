"""GPU parity: vocab-row LSE / max / argmax / softmax kernels vs the fp64 oracle."""
import numpy as np
import pytest
import torch

from oracle import rows

pytestmark = pytest.mark.gpu

SHAPES = [(3, 1), (5, 7), (4, 1000), (7, 4099), (2, 32000), (3, 248320)]


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("R,V", SHAPES)
@pytest.mark.parametrize("T", [1.0, 0.8, 0.37])
def test_row_lse_fp32(hip, R, V, T):
    _say(f"row_lse fp32 R={R} V={V} T={T}")
    x = np.random.default_rng(R * 1000 + V).normal(0, 3, (R, V)).astype(np.float32)
    lse, mx, am = hip.row_lse(torch.from_numpy(x), temperature=T, want_max=True, want_argmax=True)
    torch.cuda.synchronize()
    a = rows.scale(x, T)
    ref = rows.lse64(a)
    err = np.abs(lse.cpu().numpy() - ref).max()
    _say(f"  max |lse - lse64| = {err:.3e}")
    assert err < 2e-7
    assert np.array_equal(mx.cpu().numpy(), a.max(-1))
    assert np.array_equal(am.cpu().numpy(), x.argmax(-1))


@pytest.mark.parametrize("R,V", [(4, 1000), (3, 248320), (6, 4095)])
def test_row_lse_bf16(hip, R, V):
    _say(f"row_lse bf16 R={R} V={V}")
    xt = torch.from_numpy(np.random.default_rng(V).normal(0, 3, (R, V)).astype(np.float32)).to(torch.bfloat16)
    lse, _, am = hip.row_lse(xt, temperature=0.8, want_argmax=True)
    x = xt.float().numpy()
    ref = rows.lse64(rows.scale(x, 0.8))
    assert np.abs(lse.cpu().numpy() - ref).max() < 2e-7
    assert np.array_equal(am.cpu().numpy(), x.argmax(-1))


def test_argmax_ties_nan_inf(hip):
    _say("argmax ties / nan / inf")
    V = 5003
    x = np.zeros((8, V), np.float32)
    x[0, [17, 900, 4000]] = 5.0          # ties -> first index
    x[1, :] = -np.inf                      # all -inf -> 0
    x[2, [3000, 12]] = np.nan              # NaN wins, first NaN
    x[3, 4999] = np.inf
    x[4, V - 1] = 1.0                      # tail element (V % 4 != 0)
    x[5, :] = 7.0                          # all equal -> 0
    x[6, 2500] = -0.0
    x[6, :] = -1.0
    x[6, 2500] = 0.0
    x[7] = np.random.default_rng(0).normal(size=V)
    got = hip.argmax(torch.from_numpy(x)).cpu().numpy()
    assert got.tolist() == np.argmax(x, -1).tolist()


@pytest.mark.parametrize("V", [10, 1000, 248320])
def test_softmax_matches_numpy(hip, V):
    _say(f"softmax V={V}")
    x = np.random.default_rng(V).normal(0, 2, (5, V)).astype(np.float32)
    out = hip.softmax(torch.from_numpy(x)).cpu().numpy()
    ref = rows.softmax_ref(x.astype(np.float64))
    big = ref > 1e-30
    assert np.max(np.abs(out[big] - ref[big]) / ref[big]) < 1e-5
    np.testing.assert_allclose(out.sum(-1), 1.0, atol=1e-5)
    big_vals = np.array([[1000.0, 1001.0, 1002.0]], np.float32)
    assert np.all(np.isfinite(hip.softmax(torch.from_numpy(big_vals)).cpu().numpy()))


def test_softmax_other_dim_and_temperature(hip):
    _say("softmax dim=1, T=0.7")
    x = np.random.default_rng(9).normal(0, 2, (3, 40, 6)).astype(np.float32)
    out = hip.softmax(torch.from_numpy(x), dim=1, temperature=0.7).cpu().numpy()
    ref = rows.softmax_ref(rows.scale(x, 0.7).astype(np.float64), dim=1)
    assert np.max(np.abs(out - ref) / ref) < 1e-5


def test_row_lse_with_topk_thresholds(hip):
    _say("row_lse top-k thresholds")
    R, V, K = 6, 50000, 40
    x = np.random.default_rng(4).normal(0, 2, (R, V)).astype(np.float32)
    a = rows.scale(x, 0.8)
    thr = np.array([rows.topk_threshold(a[r], K) for r in range(R)], np.float32)
    lse, _, _ = hip.row_lse(torch.from_numpy(x), temperature=0.8, thresholds=torch.from_numpy(thr))
    ref = rows.lse64(rows.apply_threshold(a, thr))
    assert np.abs(lse.cpu().numpy() - ref).max() < 2e-7


def test_row_lse_masked_rows(hip):
    _say("row_lse -inf rows")
    x = np.random.default_rng(5).normal(size=(3, 777)).astype(np.float32)
    x[0, :] = -np.inf
    x[1, ::2] = -np.inf
    lse, _, _ = hip.row_lse(torch.from_numpy(x))
    ref = rows.lse64(x)
    got = lse.cpu().numpy()
    assert got[0] == -np.inf
    assert np.abs(got[1:] - ref[1:]).max() < 2e-7

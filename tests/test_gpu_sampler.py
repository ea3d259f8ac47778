"""vnx_sampler_sample and vnx_logit_calibrate against the CPU restatement
(oracle/sampler.py) through the C ABI: the kth value and the nucleus (p*, j*)
bit for bit, the drawn token bit for bit except rows the kernel flags
(CDF_EDGE: the target within 1e-12 of a bucket edge; LSE_EDGE: the fp64 LSE
within 1e-7 of an fp32 rounding midpoint), on 248,320-wide rows, with ties,
NaN and -inf rows, fp32 and bf16 logits."""
import numpy as np
import pytest
import torch

from oracle import sampler as OS
from oracle.model import bf16_round
from versenext_amd import _lib
from versenext_amd.sampler import Sampler

pytestmark = pytest.mark.gpu

V = 248320


def _say(*a):
    print(*a, flush=True)


def _check(hip, x, T, top_k, top_p, u, dtype=torch.float32, exact_k=False, calib_factor=None):
    """x (B, V) float32 host rows (already representable in dtype)."""
    B = x.shape[0]
    res = hip.sampler_sample(torch.from_numpy(x).to(dtype), torch.from_numpy(u), T, top_k, top_p, return_all=True,
                             exact_k=exact_k, calib_factor=calib_factor)
    torch.cuda.synchronize()
    ids = res["ids"].cpu().numpy()
    flags = res["flags"].cpu().numpy()
    kth = res["kth"].cpu().numpy()
    ps = res["p_star"].cpu().numpy()
    js = res["j_star"].cpu().numpy()
    ks = res["k_star"].cpu().numpy()
    bad = 0
    for b in range(B):
        ref, rflags, info = OS.sample(x[b], T, top_k, top_p, u[b], exact_k=exact_k, calib_factor=calib_factor)
        if "kth" in info:
            assert (np.isnan(kth[b]) and np.isnan(info["kth"])) or kth[b] == info["kth"], (b, kth[b], info["kth"])
        if "k_star" in info:
            assert ks[b] == info["k_star"], (b, ks[b], info["k_star"])
        lse_edge = flags[b] & _lib.FLAG_LSE_EDGE
        if "p_star" in info and not (ps[b] == info["p_star"] and js[b] == info["j_star"]):
            # a flagged LSE may round to the neighbouring float32 and shift every p by an ulp
            assert lse_edge, (b, ps[b], js[b], info)
        if ids[b] != ref:
            assert flags[b] != 0 or rflags != 0, (b, ids[b], ref, T, top_k, top_p)
            bad += 1
    return ids, flags, bad


@pytest.mark.parametrize("T,top_k,top_p", [(0.8, 0, 1.0), (0.7, 50, 1.0), (1.0, 0, 0.9), (0.8, 20, 0.95),
                                           (1.3, 1000, 0.5), (0.6, 64, 0.99), (0.8, 1, 1.0), (0.0, 0, 1.0)])
def test_sampler_matches_oracle_full_vocab(hip, T, top_k, top_p):
    rng = np.random.default_rng(int(T * 10 + top_k + top_p * 100))
    B = 12
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    ids, flags, bad = _check(hip, x, T, top_k, top_p, u)
    _say(f"T={T} top_k={top_k} top_p={top_p}: ids {ids[:6].tolist()} flagged {int((flags != 0).sum())}, "
         f"differing {bad}")
    assert bad <= 1


def test_sampler_ties_and_bf16(hip):
    """Logits on a coarse grid: many equal values at the kth value and in the
    nucleus; bf16 rows."""
    rng = np.random.default_rng(5)
    B = 8
    x = (np.round(rng.normal(0, 2.0, (B, V)) * 4) / 4).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    for (T, k, p) in ((1.0, 200, 1.0), (1.0, 0, 0.8), (1.0, 30, 0.7), (0.5, 0, 0.3)):
        ids, flags, bad = _check(hip, x, T, k, p, u)
        assert bad <= 1, (T, k, p)
    xb = bf16_round(rng.normal(0, 2.0, (B, V)).astype(np.float32))
    ids, flags, bad = _check(hip, xb, 0.8, 40, 0.9, u, dtype=torch.bfloat16)
    assert bad <= 1


def test_sampler_special_rows(hip):
    """NaN without top-k, all -inf, more NaN than k, top_k >= V, tiny top_p,
    a short odd-width vocabulary."""
    rng = np.random.default_rng(8)
    B = 6
    x = rng.normal(0, 2.0, (B, 1003)).astype(np.float32)
    x[0, 17] = np.nan
    x[1, :] = -np.inf
    x[2, [3, 9, 11]] = np.nan
    u = rng.random(B).astype(np.float32)
    for (T, k, p) in ((0.8, 0, 1.0), (0.8, 2, 1.0), (0.8, 5000, 1.0), (0.8, 0, 1e-6), (0.9, 7, 0.6)):
        ids, flags, bad = _check(hip, x, T, k, p, u)
        assert bad == 0, (T, k, p)
    assert hip.sampler_sample(torch.from_numpy(x), torch.from_numpy(u), 0.8)[0].item() == 17


def test_sampler_errors_match_the_reference(hip):
    x = torch.zeros((1, 16))
    u = torch.zeros(1)
    for kw in (dict(temperature=-0.1), dict(top_k=-1), dict(top_p=0.0), dict(top_p=1.01)):
        with pytest.raises(ValueError):
            hip.sampler_sample(x, u, **kw)
    with pytest.raises(ValueError):
        Sampler(top_p=0.0)


def test_sampler_class_reproduces_numpy_choice_stream(hip):
    """The Sampler class with a seed draws its uniform from default_rng(seed):
    with top_k 0 / top_p 1 the tokens equal numpy's Generator.choice on the
    canonical probabilities (the reference's sampler.py:135-137 rule)."""
    rng = np.random.default_rng(2)
    s = Sampler(temperature=0.9, seed=123)
    gen = np.random.default_rng(123)
    for _ in range(5):
        x = rng.normal(0, 2.0, 5000).astype(np.float32)
        tok = s.sample(x)
        _, _, p = OS.probabilities(x, 0.9)
        q = p.astype(np.float64) / p.astype(np.float64).sum()
        assert tok == gen.choice(q.size, p=q)


def test_sampler_class_stream_3000_draws_full_vocab(hip):
    """3,000 seeded draws of the Sampler class at V = 248,320 on near-flat
    rows, where every bucket is about 1/V wide, so rounding the uniform to
    float32 would move about one draw in 400: the tokens equal numpy's
    Generator.choice on the canonical probabilities with the same seed, draw
    for draw (the kernel gets numpy's float64 uniform unrounded)."""
    Vf = 248320
    rng = np.random.default_rng(8)
    rows = rng.normal(0, 0.05, (6, Vf)).astype(np.float32)
    probs = []
    for r in rows:
        _, _, p = OS.probabilities(r, 1.0)
        probs.append(p.astype(np.float64) / p.astype(np.float64).sum())
    s = Sampler(temperature=1.0, seed=321)
    gen = np.random.default_rng(321)
    dev_rows = [torch.from_numpy(r).to(hip.torch_device) for r in rows]
    diff = []
    for i in range(3000):
        tok = s.sample(dev_rows[i % 6])
        ref = int(gen.choice(Vf, p=probs[i % 6]))
        if tok != ref:
            diff.append((i, tok, ref))
    _say(f"3000 draws at V={Vf}: {len(diff)} differ from numpy's choice stream")
    assert not diff, diff[:5]


def test_logit_calibration_matches_oracle(hip):
    rng = np.random.default_rng(3)
    x = rng.normal(0.3, 2.5, (6, V)).astype(np.float32)
    out, var = hip.logit_calibrate(torch.from_numpy(x), 1.5, return_var=True)
    torch.cuda.synchronize()
    ref, var64 = OS.logit_calibrate(x, 1.5)
    var = var.cpu().numpy()
    assert np.max(np.abs(var - var64) / var64) < 1e-12
    got = out.cpu().numpy()
    for b in range(6):
        # the fp32 rounding of var decides every output bit; skip a row whose
        # fp64 variance sits within reassociation error of a rounding midpoint
        v32 = np.float32(var64[b])
        mid = (float(v32) + float(np.nextafter(v32, np.float32(np.inf)))) / 2
        if abs(var64[b] - mid) < 1e-13 * var64[b]:
            continue
        assert np.array_equal(got[b], ref[b]), b
    xb = bf16_round(x)
    outb = hip.logit_calibrate(torch.from_numpy(xb).to(torch.bfloat16), 0.7).cpu().numpy()
    assert np.max(np.abs(outb - OS.logit_calibrate(xb, 0.7)[0])) <= 1e-6


@pytest.mark.parametrize("k", [1, 64, 1000, 50000])
def test_exact_k_matches_oracle(hip, k):
    """CometSpark's exactly-k top-k: kth value, the last kept tie k*, the token."""
    rng = np.random.default_rng(20 + k)
    B = 6
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    x[1] = (np.round(x[1] * 2) / 2).astype(np.float32)  # heavy ties, -0 and +0 among them
    x[2, rng.integers(0, V, 9)] = np.nan
    u = rng.random(B).astype(np.float32)
    ids, flags, bad = _check(hip, x, 0.9, k, 1.0, u, exact_k=True)
    _say(f"exact k={k}: ids {ids.tolist()} flagged {int((flags != 0).sum())}, differing {bad}")
    assert bad <= 1


def test_exact_k_with_ties_split_at_the_kth_value(hip):
    """Values on a grid of 1/4: k falls inside a run of ties, so k* decides
    which of them are kept; bf16 rows too."""
    rng = np.random.default_rng(31)
    B = 4
    x = (np.round(rng.normal(0, 1.5, (B, V)) * 4) / 4).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    for k in (7, 333, 4096):
        _check(hip, x, 1.0, k, 1.0, u, exact_k=True)
    xb = bf16_round(rng.normal(0, 2.0, (B, V)).astype(np.float32))
    _check(hip, xb, 0.7, 100, 1.0, u, dtype=torch.bfloat16, exact_k=True)


def test_top_k_outside_the_candidate_search(hip):
    """The single-workgroup form behind the candidate search: rows longer than
    64 chunks of 8192 logits, and rows whose ties at the chunk thresholds
    overflow the candidate segments (a flat row with a few larger values)."""
    rng = np.random.default_rng(51)
    xw = rng.normal(0, 2.0, (2, 600_000)).astype(np.float32)
    uw = rng.random(2).astype(np.float32)
    for (T, k, p, ex) in ((0.8, 50, 1.0, False), (0.8, 50, 0.9, False), (1.0, 40, 1.0, True)):
        ids, flags, bad = _check(hip, xw, T, k, p, uw, exact_k=ex)
        assert bad == 0 or (flags != 0).any(), (T, k, p, ex)
    xf = np.ones((3, V), np.float32)
    xf[:, rng.choice(V, 10, replace=False)] = 2.0
    xf[2, :1000] = 0.5
    uf = rng.random(3).astype(np.float32)
    for (T, k, p, ex) in ((1.0, 50, 1.0, False), (1.0, 50, 1.0, True), (0.9, 20, 0.5, False)):
        ids, flags, bad = _check(hip, xf, T, k, p, uf, exact_k=ex)
        assert bad == 0 or (flags != 0).any(), (T, k, p, ex)


def test_fused_calibration_matches_oracle(hip):
    """VNX_SAMPLE_CALIBRATE: the CometSpark step (calibrate, then greedy or
    exactly-k sampling) and the Sampler rules on calibrated rows."""
    rng = np.random.default_rng(41)
    B = 8
    x = rng.normal(0.4, 3.0, (B, V)).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    ids, _, _ = _check(hip, x, 0.0, 0, 1.0, u, calib_factor=1.7)
    assert ids.tolist() == [int(np.argmax(OS.logit_calibrate(x[b], 1.7)[0])) for b in range(B)]
    for (T, k, p, ex) in ((0.8, 50, 1.0, True), (1.0, 0, 0.9, False), (0.7, 64, 0.95, False)):
        ids, flags, bad = _check(hip, x, T, k, p, u, exact_k=ex, calib_factor=1.7)
        assert bad <= 1, (T, k, p, ex)
    xb = bf16_round(x)
    ids, flags, bad = _check(hip, xb, 0.9, 200, 1.0, u, dtype=torch.bfloat16, exact_k=True, calib_factor=0.6)
    assert bad <= 1


def test_cometspark_sample_step(hip):
    """cometspark_sample: greedy with calibration, and exactly-k draws with
    host uniforms, against the oracle's CometSpark step."""
    from versenext_amd.sampler import cometspark_sample
    rng = np.random.default_rng(51)
    x = rng.normal(0, 2.5, (4, V)).astype(np.float32)
    xt = torch.from_numpy(x)
    g = cometspark_sample(hip, xt, 0.0, 40, calib_factor=1.2).cpu().numpy()
    assert g.tolist() == [OS.sample(x[b], 0.0, 0, 1.0, 0.0, calib_factor=1.2)[0] for b in range(4)]
    u = rng.random(4).astype(np.float32)
    t = cometspark_sample(hip, xt, 0.85, 30, calib_factor=1.2, uniforms=u).cpu().numpy()
    for b in range(4):
        ref, fl, _ = OS.sample(x[b], 0.85, 30, 1.0, u[b], exact_k=True, calib_factor=1.2)
        assert t[b] == ref or fl, b
    # the reference's top_k=None means no top-k
    t2 = cometspark_sample(hip, xt, 0.85, None, uniforms=u).cpu().numpy()
    for b in range(4):
        ref, fl, _ = OS.sample(x[b], 0.85, 0, 1.0, u[b])
        assert t2[b] == ref or fl, b

"""The end-to-end speculative round on the GPU (versenext_amd/e2e.py
SpecDecodeEngine) against the CPU oracle, with caller-supplied uniforms.

- Config 1 (fp32 golden weights the reference wrote, k = 4, T = 0.8): every
  round's committed tokens equal oracle.model.spec_round_cpu's on the same
  context and uniforms (the reference's verify path: full re-forward, no KV
  cache, speculative.py:202-223, with the canonical acceptance).  The GPU
  and CPU logits differ by fp32 summation order (~1e-7), so a decision whose
  margin is below 1e-4 may go either way: at most one such round is allowed,
  and only when its margin on the CPU is below that band.
- Config 5 shapes (the 20-layer CometSparkV05 mate target in bf16, the
  2-layer INT4 group-128 draft, V = 248,320, k = 6, 2 sequences): the verify
  logits and the draft logits agree with the oracle forward on the weights
  the GPU models store (bf16 / dequantized INT4), and every decision of the
  round (the k draft draws, the acceptance tests, the residual / bonus draw,
  the commit) equals the oracle's rule applied to the GPU's own logits, bit
  for bit except positions the kernels' flags mark.  Run with the tied-scale
  draft (every draft accepted) and with the VerseNex draft without the
  embedding scale (cometspark.py:670-690; drafts rejected, residual draws)."""
import os

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import rows as OR
from oracle import _clib
from oracle.speculative import spec_accept
from versenext_amd import model as VM
from versenext_amd.e2e import SpecDecodeEngine

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cometspark_small.npz")
MARGIN = 1e-4


def _say(*a):
    print(*a, flush=True)


def _w(gold, prefix):
    return {k[len(prefix):]: v for k, v in gold.items() if k.startswith(prefix) and not k.endswith("head.weight")}


def _draw_margin(logits, u, T):
    """Relative distance of u * total to the nearest CDF bucket edge of
    softmax(RN(logits / T)) (canonical weights), and the drawn id."""
    a = OR.scale(np.asarray(logits, np.float32)[None], np.float32(T))[0]
    L = np.float32(OR.lse64(a[None])[0])
    w = _clib.exp_canon((a - L).astype(np.float32)).astype(np.float64)
    c = np.cumsum(w)
    t = float(u) * c[-1]
    return float(np.min(np.abs(c - t)) / c[-1])


def _round_margin(Wt, ct, Wd, cd, seq, k, T, ud, ua):
    """Smallest decision margin of the CPU round on this context: the draft
    draws, the acceptance tests |u - p/q| and the final draw."""
    ctx = list(seq)
    V = ct.vocab_size
    q = np.empty((1, k, V), np.float32)
    xs = []
    m = 1.0
    for i in range(k):
        q[0, i] = OM.forward(Wd, cd, np.asarray(ctx)[None], last_n=1)[0, -1]
        m = min(m, _draw_margin(q[0, i], ud[i], T))
        r = spec_accept(q[:, i:i + 1], np.zeros((1, 0, V), np.float32), np.zeros((1, 0), np.int64),
                        np.asarray([[ud[i]]], np.float32), T)
        xs.append(int(r["out_ids"][0, 0]))
        ctx.append(xs[-1])
    p = OM.forward(Wt, ct, np.asarray(ctx)[None], last_n=k + 1)
    res = spec_accept(p, q, np.asarray([xs]), np.asarray(ua, np.float32).reshape(1, k + 1), T)
    for i in range(int(res["accept_len"][0]) + 1):
        if i < k:
            pp = float(np.exp(np.float64(OR.scale(p[0, i, xs[i]:xs[i] + 1], np.float32(T))[0]) - res["lse_t64"][0, i]))
            qq = float(np.exp(np.float64(OR.scale(q[0, i, xs[i]:xs[i] + 1], np.float32(T))[0]) - res["lse_d64"][0, i]))
            if qq > 0:
                m = min(m, abs(float(ua[i]) - min(1.0, pp / qq)))
    n = int(res["accept_len"][0])
    m = min(m, _draw_margin(p[0, n], ua[k], T)) if n == k else m
    return m


def test_config1_rounds_equal_spec_round_cpu(hip):
    torch.backends.cuda.matmul.allow_tf32 = False
    z = np.load(GOLD)
    gold = {k: z[k] for k in z.files}
    Wt, Wd = _w(gold, "t/"), _w(gold, "d/")
    ct, cd = VM.small_target(), VM.small_draft()
    dev = hip.torch_device
    k, T = 4, 0.8
    t = VM.CometSparkGPU(ct, Wt, hip, batch=1, capacity=256, dtype=torch.float32)
    d = VM.CometSparkGPU(cd, Wd, hip, batch=1, capacity=256, dtype=torch.float32)
    eng = SpecDecodeEngine(t, d, hip, k=k, temperature=T)
    prompt = gold["prompt"].astype(np.int64)
    eng.prefill(torch.from_numpy(prompt[None]).to(dev), 200)
    seq = [int(x) for x in prompt]
    rng = np.random.default_rng(12)
    explained, lens = 0, []
    for r in range(24):
        ud = rng.random((k, 1)).astype(np.float32)
        ua = rng.random((1, k + 1)).astype(np.float32)
        c0 = int(eng.count[0])
        eng.step((ud, ua))
        c1 = int(eng.count[0])
        got = [int(x) for x in eng.out[0, c0:c1].cpu()]
        ref = OM.spec_round_cpu(Wt, ct, Wd, cd, seq, k, T, ud[:, 0], ua[0])
        if got != ref:
            m = _round_margin(Wt, ct, Wd, cd, seq, k, T, ud[:, 0], ua[0])
            _say(f"round {r}: gpu {got} cpu {ref}, CPU decision margin {m:.2e}")
            assert m < MARGIN, (r, got, ref, m)
            explained += 1
        lens.append(len(got))
        seq += got
    _say(f"config-1 T=0.8: 24 rounds, committed per round {lens}, {explained} near-edge rounds")
    assert explained <= 1
    assert min(lens) < k + 1 < max(lens) + 1  # both rejections and full acceptance occurred


# ---------------------------------------------------------------------------
# Config 5 shapes
# ---------------------------------------------------------------------------
B5, T0, K5, TEMP, NEW5 = 2, 64, 6, 0.8, 24
CAP5 = T0 + NEW5 + 2 * (K5 + 1) + 16


@pytest.fixture(scope="module")
def mate(hip):
    dev = hip.torch_device
    tcfg = VM.mate_target()
    Wt = VM.init_weights(tcfg, seed=0, device=dev)
    Wt_host = {k: v.cpu().numpy() for k, v in Wt.items()}
    target = VM.CometSparkGPU(tcfg, Wt, hip, batch=B5, capacity=CAP5, dtype=torch.bfloat16)
    del Wt
    torch.cuda.empty_cache()
    Wt_o, _ = OM.stored_weights(Wt_host)
    del Wt_host
    return target, Wt_o


def _mate_draft(hip, scale: bool):
    dev = hip.torch_device
    dcfg = VM.mate_draft(2)
    dcfg.embedding_scale = scale
    Wd = VM.init_weights(dcfg, seed=1, device=dev)
    Wd_host = {k: v.cpu().numpy() for k, v in Wd.items()}
    draft = VM.CometSparkGPU(dcfg, Wd, hip, batch=B5, capacity=CAP5, dtype=torch.bfloat16,
                             int4=True)
    del Wd
    Wd_o, head = OM.stored_weights(Wd_host, int4=True)
    return draft, dcfg, Wd_o, head


def _close(got, ref, name):
    """logits within 3e-2 of the reference's scale and probabilities at T
    within 2e-2 (the bf16 bar); returns the two measures."""
    rel = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    pg = torch.softmax(torch.from_numpy(got).double() / TEMP, -1)
    pr = torch.softmax(torch.from_numpy(ref).double() / TEMP, -1)
    dp = float((pg - pr).abs().max())
    _say(f"  {name}: logits rel {rel:.2e}, probabilities max abs {dp:.2e}")
    assert rel <= 3e-2 and dp <= 2e-2, (name, rel, dp)
    return rel, dp


@pytest.mark.parametrize("scale", [True, False], ids=["tied_scale_draft", "versenex_draft"])
def test_mate_round_matches_oracle(hip, mate, scale):
    target, Wt_o = mate
    draft, dcfg, Wd_o, head = _mate_draft(hip, scale)
    tcfg = target.cfg
    dev = hip.torch_device
    V = tcfg.vocab_size
    rng = np.random.default_rng(40)
    prompts = rng.integers(0, V, (B5, T0))
    eng = SpecDecodeEngine(target, draft, hip, k=K5, temperature=TEMP)
    eng.prefill(torch.from_numpy(prompts).to(dev), NEW5)
    seqs = [list(map(int, p)) for p in prompts]
    accepted = []
    for r in range(3):
        ud = rng.random((K5, B5)).astype(np.float32)
        ua = rng.random((B5, K5 + 1)).astype(np.float32)
        c0 = eng.count.cpu().numpy().copy()
        eng.step((ud, ua))
        torch.cuda.synchronize()
        c1 = eng.count.cpu().numpy()
        p = eng.pbuf.float().cpu().numpy()   # (bf16 logits upcast exactly)
        q = eng.qbuf.float().cpu().numpy()
        xs = eng.toks[:, 1:].cpu().numpy()
        alen = eng.last["accept_len"].cpu().numpy()
        oids = eng.last["out_ids"].cpu().numpy()
        flags = eng.last["flags"].cpu().numpy()
        out = eng.out.cpu().numpy()
        _say(f"round {r} ({'tied-scale' if scale else 'VerseNex'} draft): accept_len {alen.tolist()}")
        # draft draws: the oracle's inverse-CDF rule on the GPU's draft logits
        for i in range(K5):
            ref = spec_accept(q[:, i:i + 1], np.zeros((B5, 0, V), np.float32), np.zeros((B5, 0), np.int64),
                              ud[i].reshape(B5, 1), TEMP)
            ok = ref["out_ids"][:, 0] == xs[:, i]
            assert np.all(ok | (ref["flags"][:, 0] != 0)), (r, i, ref["out_ids"][:, 0], xs[:, i])
        # acceptance, residual / bonus draw: the oracle on the GPU's logits
        ref = spec_accept(p, q, xs, ua, TEMP)
        flagged = (flags != 0).any(axis=1) | (ref["flags"] != 0).any(axis=1)
        same = (ref["accept_len"] == alen) & (ref["out_ids"] == oids).all(axis=1)
        assert np.all(same | flagged), (r, ref["accept_len"], alen, ref["out_ids"], oids)
        for b in range(B5):
            n = int(alen[b])
            assert c1[b] - c0[b] == n + 1
            assert np.array_equal(out[b, c0[b]:c1[b]], oids[b, :n + 1])
        if r == 0:
            # logits of this round against the oracle forward on the stored weights
            for b in range(B5):
                ctx = seqs[b] + list(map(int, xs[b]))
                ref_p = OM.forward(Wt_o, tcfg, np.asarray(ctx)[None], last_n=K5 + 1)[0]
                _close(p[b], ref_p, f"verify logits b={b}")
                ref_q = OM.forward(Wd_o, dcfg, np.asarray(ctx[:-1])[None], last_n=K5, head=head)[0]
                _close(q[b], ref_q, f"draft logits b={b}")
        for b in range(B5):
            seqs[b] += list(map(int, out[b, c0[b]:c1[b]]))
        accepted += alen.tolist()
    _say(f"accepted drafts per round and row: {accepted}")
    if scale:
        assert max(accepted) == K5
    else:
        assert min(accepted) < K5

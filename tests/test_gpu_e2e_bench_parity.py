"""Config 5 at the bench's own workload: the models bench.build_e2e builds
(the 20-layer CometSparkV05 mate target in bf16; the 2-layer INT4
group-128 draft in its three forms: with the tied x sqrt(D) embedding scale,
without it as CometSparkNexLM.forward has it, cometspark.py:670-690, and with
its final-norm weight scaled by bench.PARTIAL_ALPHA), B = 32 sequences, the
bench's 512-token prompts (torch's generator on the device, seed 30),
k = 6, T = 0.8, the round replayed as the captured HIP graph.

For each draft, 3 rounds with caller-supplied uniforms (default_rng(31)):
- every draft draw (6 per round and sequence) equals the oracle's
  inverse-CDF rule on the GPU's own draft logits
  (oracle.speculative.spec_accept with k = 0);
- every acceptance test, residual draw and bonus draw equals
  oracle.speculative.spec_accept on the GPU's own verify and draft logits
  (the reference's verify semantics, speculative.py:202-223 and :277-287,
  generalised to the stochastic rule);
- the commit appends exactly out_ids[b, :n_b + 1] to sequence b;
- in the first and the last round, the verify logits (k + 1 rows) and the
  draft logits (k rows) of two sequences equal oracle.model.forward over the
  whole context (prompt + committed tokens + drafts) on the weights the GPU
  models store, within the bf16 bar (probabilities at T within 2e-2,
  logits within 3e-2 of the row's logit scale).
A decision may differ only where a flag of the kernel or the oracle marks
it (LSE_EDGE, NEAR_TIE, CDF_EDGE).  The partial-acceptance draft must show
mid-round rejections (0 < accept_len < k)."""
import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle.speculative import spec_accept
from versenext_amd import model as VM
from versenext_amd.e2e import SpecDecodeEngine

pytestmark = pytest.mark.gpu

ROUNDS = 3
CHECK_ROWS = (0, 31)
EXCUSE = 1 | 2 | 4  # near tie, LSE edge, CDF edge


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def bench_models(hip):
    import bench
    dev = hip.torch_device
    target, d_tied, d_vnx, d_part = bench.build_e2e(hip, n_new=bench.E2E_NEW, versenex=True)
    # the same weights on the host: init_weights draws from torch's generator
    # on the device with the seeds build_e2e uses.  The target's stored bf16
    # values (OM.stored_weights) are rounded on the device, which is the
    # conversion OM.bf16_round restates (round to nearest even, pinned
    # against torch's conversion on the CPU), so the host holds one fp32
    # copy of the 1.1 G weights instead of two
    Wt_o = {k: (v.to(torch.bfloat16).float() if k.endswith(OM._MATRICES) or k == "tok_emb.weight" else v)
            .cpu().numpy() for k, v in VM.init_weights(target.cfg, seed=0, device=dev).items()}
    Wd = VM.init_weights(VM.mate_draft(2), seed=1, device=dev)
    Wd_host = {k: v.cpu().numpy() for k, v in Wd.items()}
    Wd_o, head = OM.stored_weights(Wd_host, int4=True)
    Wd_part = dict(Wd_o)
    Wd_part["norm.weight"] = (Wd["norm.weight"] * bench.PARTIAL_ALPHA).cpu().numpy()
    del Wd, Wd_host
    g = torch.Generator(device=dev)
    g.manual_seed(30)
    prompts = torch.randint(0, target.cfg.vocab_size, (bench.E2E_B, bench.E2E_T0), generator=g, device=dev)
    torch.cuda.synchronize()
    drafts = {"tied_scale": (d_tied, Wd_o), "versenex": (d_vnx, Wd_o), "partial": (d_part, Wd_part)}
    return dict(target=target, Wt_o=Wt_o, head=head, drafts=drafts, prompts=prompts, bench=bench)


def _close(got, ref, T, name):
    """The bf16 bar: logits within 3e-2 of the row's logit scale and
    probabilities at temperature T within 2e-2."""
    rel = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    pg = torch.softmax(torch.from_numpy(got).double() / T, -1)
    pr = torch.softmax(torch.from_numpy(ref).double() / T, -1)
    dp = float((pg - pr).abs().max())
    top = float(pr.max(-1).values.min())
    _say(f"  {name}: logits rel {rel:.2e}, probabilities max abs {dp:.2e} (smallest row max p {top:.3f})")
    assert rel <= 3e-2 and dp <= 2e-2, (name, rel, dp)


@pytest.mark.parametrize("which", ["tied_scale", "versenex", "partial"])
def test_bench_workload_rounds_match_oracle(hip, bench_models, which):
    M = bench_models
    bench = M["bench"]
    target, Wt_o, head = M["target"], M["Wt_o"], M["head"]
    draft, Wd_o = M["drafts"][which]
    B, K, T = bench.E2E_B, bench.E2E_K, bench.E2E_TEMP
    V = target.cfg.vocab_size
    prompts = M["prompts"]
    eng = SpecDecodeEngine(target, draft, hip, k=K, temperature=T, seed=31, use_graph=True)
    eng.prefill(prompts, bench.E2E_NEW)
    eng._capture()
    seqs = [list(map(int, p)) for p in prompts.cpu().numpy()]
    rng = np.random.default_rng(31)
    accepted, n_flagged = [], 0
    for r in range(ROUNDS):
        ud = rng.random((K, B)).astype(np.float32)
        ua = rng.random((B, K + 1)).astype(np.float32)
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
        _say(f"{which} draft, round {r}: accept_len {alen.tolist()}")
        # the draft draws: the oracle's inverse-CDF rule on the GPU's draft logits
        for i in range(K):
            ref = spec_accept(q[:, i:i + 1], np.zeros((B, 0, V), np.float32), np.zeros((B, 0), np.int64),
                              ud[i].reshape(B, 1), T)
            ok = ref["out_ids"][:, 0] == xs[:, i]
            assert np.all(ok | ((ref["flags"][:, 0] & EXCUSE) != 0)), (r, i, np.nonzero(~ok)[0])
            n_flagged += int(np.count_nonzero(~ok))
        # acceptance tests, residual / bonus draws: the oracle on the GPU's logits
        ref = spec_accept(p, q, xs, ua, T)
        explained = 0
        for b in range(B):
            if ref["accept_len"][b] == alen[b] and np.array_equal(ref["out_ids"][b], oids[b]):
                continue
            upto = max(int(alen[b]), int(ref["accept_len"][b])) + 1
            fl = (flags[b, :upto] | ref["flags"][b, :upto]) & EXCUSE
            assert fl.any(), (r, b, int(ref["accept_len"][b]), int(alen[b]), ref["out_ids"][b], oids[b])
            explained += 1
        assert explained <= 2, (r, explained)
        n_flagged += explained
        # the commit
        for b in range(B):
            n = int(alen[b])
            assert c1[b] - c0[b] == n + 1
            assert np.array_equal(out[b, c0[b]:c1[b]], oids[b, :n + 1])
        if r in (0, ROUNDS - 1):
            # logits of two sequences over their whole context
            for b in CHECK_ROWS:
                ctx = seqs[b] + list(map(int, xs[b]))
                ref_p = OM.forward(Wt_o, target.cfg, np.asarray(ctx)[None], last_n=K + 1)[0]
                _close(p[b], ref_p, T, f"round {r} verify logits b={b} (context {len(ctx)})")
                ref_q = OM.forward(Wd_o, draft.cfg, np.asarray(ctx[:-1])[None], last_n=K, head=head)[0]
                _close(q[b], ref_q, T, f"round {r} draft logits b={b}")
        for b in range(B):
            seqs[b] += list(map(int, out[b, c0[b]:c1[b]]))
        accepted += alen.tolist()
    hist = np.bincount(np.asarray(accepted), minlength=K + 1)
    _say(f"{which} draft: accept_len histogram over {ROUNDS} x {B} (n = 0..{K}): {hist.tolist()}, "
         f"{n_flagged} flagged decisions differed")
    if which == "tied_scale":
        assert hist[K] > 0
    elif which == "versenex":
        assert hist[K] < len(accepted)
    else:
        assert hist[1:K].sum() > 0, "no mid-round rejection at the bench workload"

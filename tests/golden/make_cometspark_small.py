"""Writes tests/golden/cometspark_small.npz: golden vectors of the reference's
config-1 models, produced by the reference implementation itself (run in the
build container only; the GPU box never reads /root/reference).

What only the reference can pin (its exact forward pass for given weights):
- target = CometSparkV05Small() (spark/src/base_model.py:842-918) built after
  np.random.seed(0); draft = the same family at n_embd=32, one 'trisparse'
  layer, built right after it;
- their state_dicts (the weights the oracle and the GPU model load);
- target.forward(prompt) logits for a 16-token prompt
  (default_rng(0).integers(0, 256, 16)), and target / draft logits for a
  150-token random sequence (default_rng(1)), which runs past the 32-token
  sliding window (the random-init tied model's greedy stream repeats one
  token, so the long sequence is what exercises the window);
- the target's greedy continuation of 128 tokens by full re-forward;
- a third model with the mate target's attention and routing choices at toy
  width (RoPE on, ALiBi off, MoD top-2 of 4 experts; n_embd 64, 2 layers,
  window 32), and its logits for the 150-token sequence;
- the reference's greedy speculative decode (SpeculativeDecoder.verify_then_commit,
  packages/verse_nex/verse_nex/speculative.py:230-310) with k = 4 draft tokens
  from the draft model's argmax, until 128 tokens are committed.

The prebuilt Rust extension verse_torch.verse_rs shipped in the reference is
blocked before import (its designed ImportError fallback is pure numpy).
"""
import os
import sys

import numpy as np

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cometspark_small.npz")
# Positions of the 150-token sequence whose logits are kept (every 5th).
LONG_ROWS = np.arange(0, 150, 5)


def main():
    sys.modules["verse_torch.verse_rs"] = None  # never load the shipped binary
    for p in (REF, os.path.join(REF, "packages", "verse_torch"), os.path.join(REF, "packages", "verse_nex"),
              os.path.join(REF, "packages", "verse_infra")):
        if p not in sys.path:
            sys.path.insert(0, p)
    from spark.src.base_model import CometSparkV05Small, CometSparkV05LM
    from spark.src.base_config import CometSparkV05Config
    from verse_nex.speculative import SpeculativeDecoder
    from verse_torch import Tensor, no_grad

    np.random.seed(0)
    target = CometSparkV05Small()
    dcfg = CometSparkV05Config(arch="versenex", vocab_size=256, n_layer=1, n_embd=32, n_head=4, n_kv_head=2,
                               seq_len=64, layer_pattern=["trisparse"], window_size=32, num_global_tokens=4,
                               use_alibi=True, use_rope=False, max_position_embeddings=256)
    draft = CometSparkV05LM(dcfg)
    rcfg = CometSparkV05Config(arch="versenex", vocab_size=256, n_layer=2, n_embd=64, n_head=4, n_kv_head=2,
                               seq_len=64, mod_every=2, num_dense_parts=2, num_experts_per_part=4, top_k=2,
                               window_size=32, num_global_tokens=4, use_alibi=False, use_rope=True,
                               max_position_embeddings=256)
    rope_model = CometSparkV05LM(rcfg)

    prompt = np.random.default_rng(0).integers(0, 256, 16).astype(np.int64)
    with no_grad():
        logits = target.forward(prompt[None]).data.astype(np.float32)
        long_seq = np.random.default_rng(1).integers(0, 256, 150).astype(np.int64)
        long_t = target.forward(long_seq[None]).data.astype(np.float32)
        long_d = draft.forward(long_seq[None]).data.astype(np.float32)
        long_r = rope_model.forward(long_seq[None]).data.astype(np.float32)
        seq = list(prompt)
        greedy = []
        for _ in range(128):
            t = int(np.argmax(target.forward(np.asarray(seq)[None]).data[0, -1]))
            greedy.append(t)
            seq.append(t)

        dec = SpeculativeDecoder(dim=64, vocab_size=256, num_draft_heads=4)
        ctx = prompt[None].copy()
        spec, steps = [], 0
        while len(spec) < 128:
            c = list(ctx[0])
            dt = []
            for _ in range(4):
                t = int(np.argmax(draft.forward(np.asarray(c)[None]).data[0, -1]))
                dt.append(t)
                c.append(t)
            acc, _, ctx = dec.verify_then_commit(np.asarray([dt], dtype=np.int64), target.forward, ctx,
                                                 max_redraft_rounds=0)
            steps += 1
            spec.extend(int(t) for t in acc)
    arrays = {"prompt": prompt, "logits": logits, "greedy128": np.asarray(greedy, np.int64),
              "long_seq": long_seq, "long_rows": LONG_ROWS, "long_target_logits": long_t[:, LONG_ROWS],
              "long_draft_logits": long_d[:, LONG_ROWS], "long_rope_logits": long_r[:, LONG_ROWS],
              "spec128": np.asarray(spec[:128], np.int64), "spec_steps": np.asarray(steps, np.int64)}
    for name, v in target.net.state_dict().items():
        arrays["t/" + name] = np.asarray(v, np.float32)
    for name, v in draft.net.state_dict().items():
        arrays["d/" + name] = np.asarray(v, np.float32)
    for name, v in rope_model.net.state_dict().items():
        arrays["r/" + name] = np.asarray(v, np.float32)
    np.savez(OUT, **arrays)
    print(f"wrote {OUT}: {len(arrays)} arrays, spec steps {steps}")


if __name__ == "__main__":
    main()

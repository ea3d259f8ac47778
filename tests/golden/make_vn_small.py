"""Writes .vn model files with the reference's own writer (run in the build
container only; the GPU box never reads /root/reference):

- tests/golden/cometspark_small_st.vn: the config-1 target
  (CometSparkV05Small(), spark/src/base_model.py:842-918, built after
  np.random.seed(0): the weights of tests/golden/cometspark_small.npz)
  saved through CometSparkV05LM.save_vn (spark/src/base_model.py:616-660),
  i.e. VNFileWriter (packages/verse_torch/verse_torch/vn_format.py:266-382)
  with safetensors available: a model.safetensors payload;
- tests/golden/cometspark_small_npz.vn: the same model saved with the
  writer's safetensors path switched off (its _HAS_SAFETENSORS flag), so the
  writer takes its npz fallback (vn_format.py:353-375);
- tests/golden/untied_small.vn: a one-layer V05 model with tie_weights=False
  (its own head.weight, cometspark.py:396-398) and temperature_scaling=0.7
  (spark/src/base_config.py:266), built after np.random.seed(7);
- tests/golden/vn_small.npz: the untied model's logits for the config-1
  prompt from its own forward (the only output of that model a test needs).

The prebuilt Rust extension verse_torch.verse_rs shipped in the reference is
blocked before import (its designed ImportError fallback is pure numpy).
"""
import os
import sys

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    sys.modules["verse_torch.verse_rs"] = None  # never load the shipped binary
    for p in (REF, os.path.join(REF, "packages", "verse_torch"), os.path.join(REF, "packages", "verse_nex"),
              os.path.join(REF, "packages", "verse_infra")):
        if p not in sys.path:
            sys.path.insert(0, p)
    from spark.src.base_model import CometSparkV05Small, CometSparkV05LM
    from spark.src.base_config import CometSparkV05Config
    from verse_torch import no_grad
    import verse_torch.vn_format as vf

    np.random.seed(0)
    target = CometSparkV05Small()
    gold = np.load(os.path.join(HERE, "cometspark_small.npz"))
    for name, v in target.net.state_dict().items():
        assert np.array_equal(np.asarray(v, np.float32), gold["t/" + name]), name

    st_path = os.path.join(HERE, "cometspark_small_st.vn")
    target.save_vn(st_path)
    flag = vf._HAS_SAFETENSORS
    vf._HAS_SAFETENSORS = False
    try:
        target.save_vn(os.path.join(HERE, "cometspark_small_npz.vn"))
    finally:
        vf._HAS_SAFETENSORS = flag

    np.random.seed(7)
    ucfg = CometSparkV05Config(arch="versenex", vocab_size=256, n_layer=1, n_embd=64, n_head=4, n_kv_head=2,
                               seq_len=64, layer_pattern=["trisparse"], window_size=32, num_global_tokens=4,
                               use_alibi=False, use_rope=True, max_position_embeddings=256, tie_weights=False,
                               temperature_scaling=0.7)
    untied = CometSparkV05LM(ucfg)
    sd = untied.net.state_dict()
    assert not np.array_equal(np.asarray(sd["head.weight"]), np.asarray(sd["tok_emb.weight"]))
    untied.save_vn(os.path.join(HERE, "untied_small.vn"))
    prompt = gold["prompt"].astype(np.int64)
    with no_grad():
        logits = untied.forward(prompt[None]).data.astype(np.float32)
    np.savez(os.path.join(HERE, "vn_small.npz"), prompt=prompt, untied_logits=logits)
    for f in ("cometspark_small_st.vn", "cometspark_small_npz.vn", "untied_small.vn", "vn_small.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()

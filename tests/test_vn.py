"""The streamed .vn reader (versenext_amd/vn.py) against the libraries that
define the two weight payloads: every tensor, read in row chunks, equals
safetensors' own loader (fp32, fp16, bf16, int64) and numpy's .npy reader
(the npz fallback); VNFileReader's checks (vn_format.py:557-620) hold; the
config maps to the model's."""
import json
import zipfile

import numpy as np
import pytest
import torch

from versenext_amd import vn as VN
from versenext_amd.model import ModelConfig
from tests.vn_fixture import write_vn


def _state(rng):
    return {
        "tok_emb.weight": rng.normal(0, 1, (300, 256)).astype(np.float32),
        "blocks.0.attn.wq.weight": rng.normal(0, 1, (256, 256)).astype(np.float32),
        "blocks.0.norm1.weight": rng.random(256).astype(np.float32),
        "blocks.0.attn.gate_logits": np.zeros(3, np.float32),
        "half": rng.normal(0, 1, (7, 33)).astype(np.float16),
        "ids": np.arange(10, dtype=np.int64),
        "scalar": np.array(2.5, np.float32),
    }


def _read_all(path, rows_per_chunk=5):
    out = {}
    with VN.VNReader(path) as r:
        for t in r.tensors():
            parts = []
            left = t.rows
            buf = bytearray(max(1, rows_per_chunk) * t.row_bytes)
            while left:
                n = min(rows_per_chunk, left)
                parts.append(bytes(t.read_into(memoryview(buf), n)))
                left -= n
            out[t.name] = (t.dtype, t.shape, b"".join(parts))
    return out


@pytest.mark.parametrize("fmt", ["safetensors", "npz"])
def test_streamed_tensors_equal_the_library_loaders(tmp_path, fmt):
    rng = np.random.default_rng(0)
    st = _state(rng)
    p = tmp_path / f"m_{fmt}.vn"
    write_vn(p, st, {"dim": 256}, fmt=fmt)
    got = _read_all(p)
    with zipfile.ZipFile(p) as zf:
        payload = zf.read("model.safetensors" if fmt == "safetensors" else "model.npz")
    if fmt == "safetensors":
        from safetensors.numpy import load
        ref = load(payload)
    else:
        import io
        ref = dict(np.load(io.BytesIO(payload), allow_pickle=False))
    assert set(got) == set(ref) == set(st)
    for k, (dt, shape, raw) in got.items():
        r = ref[k]
        assert shape == r.shape, k
        assert raw == np.ascontiguousarray(r).tobytes(), k


def test_bf16_payload_equals_safetensors_torch(tmp_path):
    rng = np.random.default_rng(1)
    st = {"a": rng.normal(0, 1, (64, 128)).astype(np.float32), "b": rng.normal(0, 1, (5, 128)).astype(np.float32)}
    p = tmp_path / "bf.vn"
    write_vn(p, st, {"dim": 128}, bf16_names=("a",))
    got = _read_all(p, rows_per_chunk=7)
    with zipfile.ZipFile(p) as zf:
        from safetensors.torch import load
        ref = load(zf.read("model.safetensors"))
    assert got["a"][0] == "BF16" and got["b"][0] == "F32"
    for k in st:
        assert got[k][2] == ref[k].contiguous().view(torch.uint8).numpy().tobytes(), k


def test_reader_checks_match_the_reference(tmp_path):
    st = {"w": np.ones((2, 128), np.float32)}
    ok1 = tmp_path / "v1.vn"
    write_vn(ok1, st, {"dim": 128}, version=None)        # v1: no version field
    with VN.VNReader(ok1) as r:
        assert r.read_meta()["weight_format"] == "safetensors" and r.vn_format_version == 1
    bad = tmp_path / "v3.vn"
    write_vn(bad, st, {"dim": 128}, version=3)
    with pytest.raises(ValueError):
        VN.VNReader(bad).read_meta()
    for drop in ("meta", "config", "weights"):
        q = tmp_path / f"no_{drop}.vn"
        write_vn(q, st, {"dim": 128}, drop=(drop,))
        with VN.VNReader(q) as r, pytest.raises(ValueError):
            if drop == "config":
                r.read_config()
            else:
                list(r.tensors())


def test_config_mapping_both_flavours():
    W = {"blocks.1.ffn.w_gate.weight": VN.Int4Weight(torch.zeros((4096, 512), dtype=torch.uint8),
                                                      torch.zeros((4096, 8), dtype=torch.float16))}
    nex = {"vocab_size": 248320, "dim": 1024, "n_layer": 2, "n_head": 16, "n_kv_head": 8,
           "layer_pattern": ["mod", "trisparse"], "max_seq_len": 2048, "tie_weights": True, "window_size": 1024,
           "num_global_tokens": 128, "use_alibi": False, "use_rope": True, "rope_theta": 10000.0,
           "num_dense_parts": 4, "num_experts_per_part": 4, "top_k": 2, "expert_hidden": None}
    c = VN.config_from_vn(nex, W)
    assert isinstance(c, ModelConfig) and c.dim == 1024 and not c.embedding_scale and c.ffn_hidden == 4096
    assert c.layer_pattern == ("mod", "trisparse")
    v05 = {"arch": "versenex", "vocab_size": 256, "n_layer": 8, "n_embd": 64, "n_head": 4, "n_kv_head": None,
           "layer_pattern": None, "mod_every": 4, "window_size": 32, "num_global_tokens": 4, "use_alibi": True,
           "use_rope": False, "embedding_scale": True}
    c5 = VN.config_from_vn(v05, {})
    assert c5.dim == 64 and c5.n_kv_head == 4 and c5.embedding_scale
    assert c5.layer_pattern == ("mod", "trisparse", "trisparse", "trisparse") * 2


def test_config_carries_tie_weights_and_temperature_scaling():
    """tie_weights (cometspark.py:1233, base_config.py:239) and the V05
    temperature_scaling (base_config.py:266) reach ModelConfig; the NexLM
    config has no temperature_scaling (1.0)."""
    from versenext_amd.model import generate_temperature
    v05 = {"vocab_size": 256, "n_layer": 2, "n_embd": 64, "n_head": 4, "n_kv_head": 2, "layer_pattern": None,
           "mod_every": 2, "tie_weights": False, "temperature_scaling": 0.7}
    c = VN.config_from_vn(v05, {})
    assert not c.tie_weights and c.temperature_scaling == pytest.approx(0.7)
    assert "head.weight" in __import__("versenext_amd.model", fromlist=["x"]).weight_shapes(c)
    nex = {"vocab_size": 256, "dim": 64, "n_layer": 1, "n_head": 4, "layer_pattern": ["trisparse"],
           "temperature_scaling": 0.5}
    cn = VN.config_from_vn(nex, {})
    assert cn.tie_weights and cn.temperature_scaling == 1.0
    # CometSparkV05LM.generate: the default T 1.0 becomes temperature_scaling
    # (no top_k); CometSparkNexLM.generate: T == 1.0 without top_k is greedy
    assert generate_temperature(c) == pytest.approx(0.7)
    assert generate_temperature(c, 0.9) == pytest.approx(0.9)
    assert generate_temperature(c, 1.0, top_k=50) == 1.0
    assert generate_temperature(cn) == 0.0 and generate_temperature(cn, 0.8) == pytest.approx(0.8)
    assert generate_temperature(cn, 0.0) == 1e-8
    c1 = VN.config_from_vn(dict(v05, temperature_scaling=1.0), {})
    assert generate_temperature(c1) == 0.0
    c0 = VN.config_from_vn(dict(v05, temperature_scaling=0.0), {})
    assert generate_temperature(c0) == 0.0


GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__import__("os").path.abspath(__file__)), "golden")


def _arrays(path, rows_per_chunk=5):
    """{name: ndarray} of the streamed fp32 tensors."""
    out = {}
    for name, (dt, shape, raw) in _read_all(path, rows_per_chunk).items():
        assert dt == "F32", (name, dt)
        out[name] = np.frombuffer(raw, np.float32).reshape(shape).copy()
    return out


@pytest.mark.parametrize("fname,fmt", [("cometspark_small_st.vn", "safetensors"),
                                       ("cometspark_small_npz.vn", "npz")])
def test_reads_the_reference_written_vn(fname, fmt):
    """.vn files written by the reference's CometSparkV05LM.save_vn
    (tests/golden/make_vn_small.py): meta, config and every tensor of the
    config-1 target equal the state_dict the reference wrote into
    cometspark_small.npz, and the config maps to small_target()."""
    import os
    from versenext_amd import model as VM
    path = os.path.join(GOLDEN, fname)
    gold = np.load(os.path.join(GOLDEN, "cometspark_small.npz"))
    with VN.VNReader(path) as r:
        meta = r.read_meta()
        conf = r.read_config()
        assert r.weight_format == fmt and meta["vn_format_version"] == 2
    W = _arrays(path, rows_per_chunk=7)
    want = {k[2:]: gold[k] for k in gold.files if k.startswith("t/")}
    assert set(W) == set(want)
    for k, v in want.items():
        assert W[k].dtype == np.float32 and np.array_equal(W[k], v), k
    c = VN.config_from_vn(conf, W)
    ref = VM.small_target()
    for f in ("vocab_size", "dim", "n_layer", "n_head", "n_kv_head", "layer_pattern", "window_size",
              "num_global_tokens", "use_alibi", "use_rope", "num_dense_parts", "num_experts_per_part", "top_k",
              "embedding_scale", "tie_weights", "temperature_scaling", "ffn_hidden", "expert_hidden_eff"):
        assert getattr(c, f) == getattr(ref, f), f


def test_reference_written_untied_vn_matches_its_logits():
    """The reference's untied one-layer V05 model (tie_weights False,
    temperature_scaling 0.7): the config maps, and the oracle forward on the
    stored weights, with the stored head.weight as the head, reproduces the
    logits the reference computed for the config-1 prompt."""
    import os
    from oracle import model as OM
    from versenext_amd.model import generate_temperature
    path = os.path.join(GOLDEN, "untied_small.vn")
    z = np.load(os.path.join(GOLDEN, "vn_small.npz"))
    with VN.VNReader(path) as r:
        conf = r.read_config()
    W = _arrays(path)
    c = VN.config_from_vn(conf, W)
    assert not c.tie_weights and c.temperature_scaling == pytest.approx(0.7) and c.embedding_scale
    assert generate_temperature(c) == pytest.approx(0.7)
    got = OM.forward(W, c, z["prompt"][None])
    err = float(np.max(np.abs(got - z["untied_logits"])))
    assert err <= 1e-5, err
    tied = OM.forward(W, VN.config_from_vn(dict(conf, tie_weights=True), W), z["prompt"][None])
    assert float(np.max(np.abs(tied - z["untied_logits"]))) > 1e-2

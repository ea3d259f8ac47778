"""vnx_quantize_w4_g and the streamed .vn draft load on the GPU.

- The device quantizer equals oracle/quant.py's quantize_int4_g byte for byte
  (packed nibbles and fp16 scales) on fp32, fp16 and bf16 rows, all-zero
  groups included, and counts groups it cannot quantize.
- CometSparkGPU.from_vn (INT4 draft) holds the same INT4 buffers as the model
  built from the same weights in memory, and its forward returns the same
  hidden states bit for bit, with small chunks (many per matrix), from the
  safetensors and the npz payloads; the device memory it takes while loading
  stays below a full-precision copy of the embedding."""
import ctypes
import gc

import numpy as np
import pytest
import torch

from oracle import quant as OQ
from oracle.model import bf16_round
from tests.vn_fixture import write_vn
from versenext_amd import _lib
from versenext_amd import model as VM
from versenext_amd.vn import Int4Weight

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _quantize(hip, w: torch.Tensor, bad=None):
    N, K = w.shape
    dev = hip.torch_device
    wq = torch.empty((N, K // 2), dtype=torch.uint8, device=dev)
    sc = torch.empty((N, K // 128), dtype=torch.float16, device=dev)
    wd = w.to(dev).contiguous()
    _lib.check(hip._L.vnx_quantize_w4_g(ctypes.c_void_p(wd.data_ptr()), _lib.DTYPE_CODES[wd.dtype], N, K, K, 128,
                                        ctypes.c_void_p(wq.data_ptr()), wq.stride(0), ctypes.c_void_p(sc.data_ptr()),
                                        sc.stride(0), ctypes.c_void_p(bad.data_ptr()) if bad is not None else None,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "quantize_w4_g")
    torch.cuda.synchronize()
    return wq.cpu().numpy(), sc.cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_device_quantizer_equals_the_oracle(hip, dtype):
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.05, (333, 1024)).astype(np.float32)
    w[5, 128:256] = 0.0                       # an all-zero group: scale 1/7
    w[7, :128] *= 400.0                       # a wide group
    w[9, 512:640] = np.float32(3.5) * (np.arange(128) % 3 - 1)   # exact halves at the scale
    wt = torch.from_numpy(w).to(dtype)
    ref_in = wt.float().numpy()               # the values the kernel reads
    wq, sc = _quantize(hip, wt)
    rq, rs = OQ.quantize_int4_g(ref_in, 128)
    assert np.array_equal(wq, rq) and np.array_equal(sc.view(np.uint16), rs.view(np.uint16))
    _say(f"quantize_w4_g {dtype}: bit-exact on {w.shape}")


def test_device_quantizer_counts_bad_groups(hip):
    dev = hip.torch_device
    w = np.random.default_rng(4).normal(0, 1, (4, 256)).astype(np.float32)
    w[1, :128] *= 1e-12                        # scale underflows fp16
    w[3, 200] = np.nan
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    _quantize(hip, torch.from_numpy(w), bad)
    assert int(bad.item()) == 2


def _draft_cfg():
    return VM.ModelConfig(vocab_size=40000, dim=256, n_layer=2, n_head=4, n_kv_head=2,
                          layer_pattern=("trisparse", "trisparse"), window_size=1024, num_global_tokens=8,
                          use_alibi=False, use_rope=True, mlp_hidden=512, embedding_scale=False)


def _nex_config(cfg):
    return {"vocab_size": cfg.vocab_size, "dim": cfg.dim, "n_layer": cfg.n_layer, "n_head": cfg.n_head,
            "n_kv_head": cfg.n_kv_head, "layer_pattern": list(cfg.layer_pattern), "max_seq_len": 2048,
            "tie_weights": True, "aux_loss_weight": 0.01, "window_size": cfg.window_size,
            "num_global_tokens": cfg.num_global_tokens, "use_alibi": cfg.use_alibi, "use_rope": cfg.use_rope,
            "rope_theta": cfg.rope_theta}


@pytest.mark.parametrize("fmt,chunk", [("safetensors", 1 << 20), ("npz", 300 << 10), ("safetensors", 64 << 20)])
def test_from_vn_equals_the_in_memory_int4_draft(hip, tmp_path, fmt, chunk):
    cfg = _draft_cfg()
    W = VM.init_weights(cfg, seed=11)
    state = {k: v.numpy().astype(np.float32) for k, v in W.items()}
    state["head.weight"] = state["tok_emb.weight"]          # the reference's tied state_dict holds both
    path = tmp_path / f"draft_{fmt}.vn"
    write_vn(path, state, _nex_config(cfg), fmt=fmt)
    dev = hip.torch_device
    B = 3
    gc.collect()                                            # earlier tests' models freed before the baseline
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    m = VM.CometSparkGPU.from_vn(str(path), hip, batch=B, capacity=64, dtype=torch.bfloat16, int4=True,
                                 chunk_bytes=chunk)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev) - base
    final = torch.cuda.memory_allocated(dev) - base          # the loaded model's own buffers
    ref = VM.CometSparkGPU(cfg, W, hip, batch=B, capacity=64, dtype=torch.bfloat16, int4=True)
    assert m.cfg.dim == cfg.dim and m.cfg.ffn_hidden == cfg.ffn_hidden and not m.cfg.embedding_scale
    assert torch.equal(m.head.wq, ref.head.wq) and torch.equal(m.head.sc, ref.head.sc)
    assert torch.equal(m.emb, ref.emb)
    for a, b in zip(m.layers, ref.layers):
        assert torch.equal(a.wqkv.wq, b.wqkv.wq) and torch.equal(a.wqkv.sc, b.wqkv.sc)
        assert torch.equal(a.wqkv.wq_rope, b.wqkv.wq_rope)
        assert torch.equal(a.ffn["gu"].wq_sw, b.ffn["gu"].wq_sw) and torch.equal(a.ffn["down"].wq, b.ffn["down"].wq)
        assert torch.equal(a.gk, b.gk) and torch.equal(a.gv, b.gv)
    rng = np.random.default_rng(2)
    toks = torch.from_numpy(rng.integers(0, cfg.vocab_size, (B, 12))).to(dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    ha = m.forward(toks, lens, 0)
    hb = ref.forward(toks, lens, 0)
    lens += 12
    step = torch.from_numpy(rng.integers(0, cfg.vocab_size, (B, 1))).to(dev)
    da = m.forward(step, lens, 12)
    db = ref.forward(step, lens, 12)
    assert torch.equal(ha, hb) and torch.equal(da, db)
    emb_fp32 = cfg.vocab_size * cfg.dim * 4
    _say(f"from_vn {fmt} chunk {chunk}: peak {peak / 2**20:.1f} MiB (fp32 embedding alone {emb_fp32 / 2**20:.1f} MiB)")
    if chunk < emb_fp32:
        # above the loaded model's own buffers: two staging chunks and one 8 MiB
        # fp32 block of the prefill copy's dequantization, never an fp32 copy
        # of a whole matrix (the embedding alone is 39 MiB here)
        _say(f"  peak above the loaded model: {(peak - final) / 2**20:.1f} MiB")
        assert peak - final <= 2 * chunk + (8 << 20) + (2 << 20) < emb_fp32


def test_from_vn_reads_bf16_weights(hip, tmp_path):
    """Weights stored as BF16 quantize from the bf16 values."""
    cfg = _draft_cfg()
    W = VM.init_weights(cfg, seed=12)
    state = {k: bf16_round(v.numpy().astype(np.float32)) for k, v in W.items()}
    path = tmp_path / "bf.vn"
    mats = [k for k in state if k.endswith("weight") and state[k].ndim == 2]
    write_vn(path, state, _nex_config(cfg), bf16_names=tuple(mats))
    m = VM.CometSparkGPU.from_vn(str(path), hip, batch=2, capacity=32, chunk_bytes=1 << 20)
    ref = VM.CometSparkGPU(cfg, {k: torch.from_numpy(v) for k, v in state.items()}, hip, batch=2, capacity=32,
                           int4=True)
    assert torch.equal(m.head.wq, ref.head.wq) and torch.equal(m.layers[1].proj.wq, ref.layers[1].proj.wq)
    assert isinstance(Int4Weight(m.head.wq, m.head.sc), Int4Weight)


@pytest.mark.parametrize("int4", [True, False], ids=["int4", "bf16"])
def test_from_vn_untied_head(hip, tmp_path, int4):
    """tie_weights false (cometspark.py:396-398): the stored head.weight,
    not the embedding, is the LM head.  The .vn model equals the in-memory
    model of the same weights bit for bit, and its logits follow the oracle
    forward with that head (its INT4 group-128 dequantization for int4)."""
    from oracle import model as OM
    cfg = _draft_cfg()
    cfg.tie_weights = False
    W = VM.init_weights(cfg, seed=13)
    assert "head.weight" in W
    state = {k: v.numpy().astype(np.float32) for k, v in W.items()}
    conf = dict(_nex_config(cfg), tie_weights=False)
    path = tmp_path / "untied.vn"
    write_vn(path, state, conf)
    dev = hip.torch_device
    B = 2
    m = VM.CometSparkGPU.from_vn(str(path), hip, batch=B, capacity=32, dtype=torch.bfloat16, int4=int4,
                                 chunk_bytes=1 << 20)
    assert not m.cfg.tie_weights
    ref = VM.CometSparkGPU(cfg, W, hip, batch=B, capacity=32, dtype=torch.bfloat16, int4=int4)
    if int4:
        assert torch.equal(m.head.wq, ref.head.wq) and torch.equal(m.head.sc, ref.head.sc)
    else:
        assert torch.equal(m.head_w, ref.head_w) and not torch.equal(m.head_w, m.emb)
    rng = np.random.default_rng(6)
    toks = rng.integers(0, cfg.vocab_size, (B, 9))
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    tt = torch.from_numpy(toks).to(dev)
    la = m.logits(m.forward(tt, lens, 0, out_dtype=m.act_dtype)[:, -2:])
    lb = ref.logits(ref.forward(tt, lens, 0, out_dtype=ref.act_dtype)[:, -2:])
    torch.cuda.synchronize()
    assert torch.equal(la, lb)
    Wo, _ = OM.stored_weights(state, int4=int4)
    head = OM.int4_g_stored(state["head.weight"], 128) if int4 else OM.bf16_round(state["head.weight"])
    want = OM.forward(Wo, cfg, toks, last_n=2, head=head)
    tied = OM.forward(Wo, cfg, toks, last_n=2, head=Wo["tok_emb.weight"])
    got = la.cpu().numpy()
    rel = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    rel_tied = float(np.max(np.abs(got - tied)) / np.max(np.abs(tied)))
    _say(f"untied head ({'int4' if int4 else 'bf16'}): logits rel {rel:.2e} vs the stored head, "
         f"{rel_tied:.2e} vs the embedding")
    # the tied result is far off (its scale is set by the self-token peak)
    assert rel <= 3e-2 and rel_tied > 20 * rel


GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__import__("os").path.abspath(__file__)), "golden")


@pytest.mark.parametrize("fname", ["cometspark_small_st.vn", "cometspark_small_npz.vn"])
def test_from_vn_reference_file_reproduces_golden_logits(hip, fname):
    """A .vn file the reference wrote (CometSparkV05LM.save_vn with and
    without safetensors, tests/golden/make_vn_small.py), loaded by
    CometSparkGPU.from_vn in fp32: the config-1 target's logits for the
    150-token sequence equal the reference's own within 1e-4."""
    import os
    torch.backends.cuda.matmul.allow_tf32 = False
    gold = np.load(os.path.join(GOLDEN, "cometspark_small.npz"))
    m = VM.CometSparkGPU.from_vn(os.path.join(GOLDEN, fname), hip, batch=1, capacity=256, dtype=torch.float32,
                                 int4=False)
    assert m.cfg.layer_pattern == ("mod", "trisparse") and m.cfg.use_alibi and m.cfg.tie_weights
    dev = hip.torch_device
    seq = gold["long_seq"][None]
    lens = torch.zeros(1, dtype=torch.int32, device=dev)
    out, t = [], 0
    for n in (16, 5, 1, 40, 7, 81):
        h = m.forward(torch.from_numpy(seq[:, t:t + n]).to(dev), lens, int(lens.max()))
        out.append(m.logits(h).cpu().numpy())
        lens += n
        t += n
    got = np.concatenate(out, axis=1)[:, gold["long_rows"]]
    err = float(np.max(np.abs(got - gold["long_target_logits"])))
    _say(f"from_vn {fname} (fp32): max abs err {err:.2e} vs the reference's logits")
    assert err <= 1e-4


def test_from_vn_reference_untied_file_reproduces_its_logits(hip):
    """The reference's untied model file (tie_weights False, its own
    head.weight): from_vn in fp32 reproduces the reference's logits for the
    config-1 prompt within 1e-4."""
    import os
    torch.backends.cuda.matmul.allow_tf32 = False
    z = np.load(os.path.join(GOLDEN, "vn_small.npz"))
    m = VM.CometSparkGPU.from_vn(os.path.join(GOLDEN, "untied_small.vn"), hip, batch=1, capacity=64,
                                 dtype=torch.float32, int4=False)
    assert not m.cfg.tie_weights and not torch.equal(m.head_w, m.emb)
    dev = hip.torch_device
    lens = torch.zeros(1, dtype=torch.int32, device=dev)
    h = m.forward(torch.from_numpy(z["prompt"][None]).to(dev), lens, 0)
    got = m.logits(h).cpu().numpy()
    err = float(np.max(np.abs(got - z["untied_logits"])))
    _say(f"untied .vn (fp32): max abs err {err:.2e}")
    assert err <= 1e-4

"""CometSpark (VerseNex) target and draft models on one MI355X, for end-to-end
speculative decoding with an incremental (KV-cached) verify pass.

Architecture (the reference's, restated for PyTorch-ROCm tensors):
- CometSparkNexLM (packages/verse_nex/verse_nex/cometspark.py:294-449) with
  the CometSparkV05LM embedding scale x sqrt(D) (spark/src/base_model.py:161,
  :201-207): tok_emb -> blocks -> RMSNorm -> tied head;
- VerseNexBlock (cometspark.py:209-247): x += attn(norm1(x)); x += ffn(norm2(x));
  RMSNorm x / sqrt(mean(x^2) + 1e-6) * w (vnnn.py:593-615, :468-508);
- TriSparseAttention (tri_sparse_attn.py:536-613): GQA projections, NeoX
  rotate-half RoPE on q and k (:167-221), sigmoid(gate_logits) weighted sum of
  a causal sliding-window path (window W), a path over the learnable global
  sink tokens projected by wk / wv (:225-258, :469-495), and, when use_alibi
  and the key count is at most 1024, a causal ALiBi path (:501-534);
- FFN: SwiGLU w_down(silu(w_gate x) * w_up x) (vnnn.py:779-807) on
  "trisparse" layers, MoD (mod.py:600-803) on "mod" layers: a soft part
  router over all parts, inside each part a top-k expert router whose
  softmax over the k selected logits weights SwiGLU experts.

The incremental verify differs from the reference's only in what is
recomputed: the reference re-runs the whole sequence without a KV cache
(speculative.py:202-213) and reads logits at the k+1 verified positions; here
every sequence keeps its own committed length in `lens` (the per-sequence
lengths of ParallelKVCache, kv_cache_parallel.py:42-286), the k+1 new rows
are written into the cache at lens[b] .. lens[b]+k, and a rejected suffix is
rolled back by not advancing lens[b].  The rows the verifier reads see the
same keys either way.

Kernels of libvnx_hip.so (gfx950) on the decode and verify forwards:
- attention of the new rows over the cache, all three TriSparse paths
  (vnx_tree_attn with per-row prefix lengths; RoPE and the cache write of
  the new rows inside the call for bf16 verify-size forwards);
- the target's verify-size projections and SwiGLU FFNs on vnx_gemm_bf16
  (RMSNorm staged into the q|k|v and gate-up products, the residual add in
  the output and down products' epilogues, the first layer's token
  embedding gathered by its q|k|v product), the MoD routing
  (vnx_mod_route_x) and the routed expert products (vnx_expert_gemm_bf16);
- the INT4 group-128 draft GEMVs (vnx_gemv_w4 and its fused RMSNorm / RoPE /
  SwiGLU / residual forms) and the verify-pass LM head (vnx_lm_head).
Prefill-size forwards (more rows than one verify round) run their dense
products on PyTorch-ROCm (hipBLASLt / rocBLAS); the attention of every
forward runs on vnx_tree_attn where the head size allows it.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import Dict, Optional, Sequence

import numpy as np
import torch

from . import _lib
from . import quant as VQ
from .vn import Int4Weight


# ---------------------------------------------------------------------------
# Configurations
# ---------------------------------------------------------------------------
@dataclass
class ModelConfig:
    vocab_size: int
    dim: int
    n_layer: int
    n_head: int
    n_kv_head: int
    layer_pattern: Sequence[str]
    window_size: int
    num_global_tokens: int
    use_alibi: bool
    use_rope: bool
    rope_theta: float = 10000.0
    num_dense_parts: int = 4
    num_experts_per_part: int = 4
    top_k: int = 2
    expert_hidden: Optional[int] = None
    mlp_hidden: Optional[int] = None
    embedding_scale: bool = True
    init_std: float = 0.02
    eps: float = 1e-6
    name: str = ""
    # the LM head shares the embedding table (cometspark.py:396-398); False:
    # a separate (V, D) 'head.weight'
    tie_weights: bool = True
    # CometSparkV05Config.temperature_scaling (spark/src/base_config.py:266),
    # the default temperature of generate (see generate_temperature)
    temperature_scaling: float = 1.0

    def __post_init__(self):
        self.layer_pattern = tuple(self.layer_pattern)
        if len(self.layer_pattern) != self.n_layer:
            raise ValueError("layer_pattern must have n_layer entries")
        if any(k not in ("trisparse", "mod") for k in self.layer_pattern):
            raise ValueError("layer kinds are 'trisparse' or 'mod'")
        if self.dim % self.n_head or self.n_head % self.n_kv_head:
            raise ValueError("dim % n_head and n_head % n_kv_head must be 0")

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_head

    @property
    def ffn_hidden(self) -> int:
        """SwiGLUMLP hidden: 2/3 of 4*D rounded up to 64 (vnnn.py:794)."""
        if self.mlp_hidden:
            return int(self.mlp_hidden)
        return int((4 * self.dim * 2 / 3 + 63) // 64) * 64

    @property
    def expert_hidden_eff(self) -> int:
        """MoD expert hidden: floor(D*8/3/64)*64, at least 64 (mod.py:688)."""
        if self.expert_hidden:
            return int(self.expert_hidden)
        return max(int(self.dim * 8 / 3 / 64) * 64, 64)


def generate_temperature(cfg: ModelConfig, temperature: float = 1.0, top_k: Optional[int] = None) -> float:
    """The SpecDecodeEngine temperature (0 = greedy) of the reference's
    generate(temperature, top_k) on this model: CometSparkV05LM.generate
    replaces the default temperature 1.0 by config.temperature_scaling when
    that is positive and not 1.0 and no top_k is given
    (spark/src/base_model.py:312-319); CometSparkNexLM.generate then decodes
    greedily when temperature == 1.0 and top_k is None, and otherwise
    samples from softmax(logits / max(temperature, 1e-8))
    (cometspark.py:817-818, :895)."""
    t = float(temperature)
    if t == 1.0 and top_k is None and cfg.temperature_scaling > 0 and cfg.temperature_scaling != 1.0:
        t = float(cfg.temperature_scaling)
    if t == 1.0 and top_k is None:
        return 0.0
    return max(t, 1e-8)


def v02_pattern(n_layer: int, mod_every: int) -> list:
    """_build_v02_pattern (cometspark.py:1347-1370): 'mod' at i % mod_every == 0."""
    if mod_every < 1:
        raise ValueError("mod_every must be >= 1")
    return ["mod" if i % mod_every == 0 else "trisparse" for i in range(n_layer)]


def mate_target() -> ModelConfig:
    """CometSparkV05() (spark/src/base_model.py:760-838): the config-5 target."""
    return ModelConfig(vocab_size=248320, dim=1024, n_layer=20, n_head=16, n_kv_head=8,
                       layer_pattern=v02_pattern(20, 4), window_size=1024, num_global_tokens=128,
                       use_alibi=False, use_rope=True, num_dense_parts=4, num_experts_per_part=4, top_k=2,
                       name="CometSparkV05 (mate target)")


def small_target() -> ModelConfig:
    """CometSparkV05Small() (spark/src/base_model.py:842-918): the config-1 target."""
    return ModelConfig(vocab_size=256, dim=64, n_layer=2, n_head=4, n_kv_head=2,
                       layer_pattern=v02_pattern(2, 2), window_size=32, num_global_tokens=4,
                       use_alibi=True, use_rope=False, num_dense_parts=2, num_experts_per_part=2, top_k=1,
                       name="CometSparkV05Small (config-1 target)")


def small_draft() -> ModelConfig:
    """Config-1 draft: one 'trisparse' layer of the same family at D = 32."""
    return ModelConfig(vocab_size=256, dim=32, n_layer=1, n_head=4, n_kv_head=2, layer_pattern=("trisparse",),
                       window_size=32, num_global_tokens=4, use_alibi=True, use_rope=False,
                       name="config-1 draft (1 x trisparse, D=32)")


def mate_draft(n_layer: int = 2) -> ModelConfig:
    """Config-5 draft: mate-width 'trisparse' layers (D = 1024, SwiGLU ffn 4096,
    the config-4 GEMV shapes) with the tied 248,320-row head."""
    return ModelConfig(vocab_size=248320, dim=1024, n_layer=n_layer, n_head=16, n_kv_head=8,
                       layer_pattern=("trisparse",) * n_layer, window_size=1024, num_global_tokens=128,
                       use_alibi=False, use_rope=True, mlp_hidden=4096,
                       name=f"VerseNex draft ({n_layer} x trisparse, D=1024, ffn 4096)")


# ---------------------------------------------------------------------------
# Weights
# ---------------------------------------------------------------------------
def weight_shapes(cfg: ModelConfig) -> Dict[str, tuple]:
    """Parameter names (the reference's module paths) and shapes."""
    D, H, Hkv, d = cfg.dim, cfg.n_head, cfg.n_kv_head, cfg.head_dim
    s = {"tok_emb.weight": (cfg.vocab_size, D), "norm.weight": (D,)}
    for i, kind in enumerate(cfg.layer_pattern):
        p = f"blocks.{i}."
        s[p + "norm1.weight"] = (D,)
        s[p + "norm2.weight"] = (D,)
        s[p + "attn.wq.weight"] = (H * d, D)
        s[p + "attn.wk.weight"] = (Hkv * d, D)
        s[p + "attn.wv.weight"] = (Hkv * d, D)
        s[p + "attn.proj.weight"] = (D, H * d)
        s[p + "attn.global_tokens.weight"] = (cfg.num_global_tokens, D)
        s[p + "attn.gate_logits"] = (3,)
        if kind == "trisparse":
            Hf = cfg.ffn_hidden
            s[p + "ffn.w_gate.weight"] = (Hf, D)
            s[p + "ffn.w_up.weight"] = (Hf, D)
            s[p + "ffn.w_down.weight"] = (D, Hf)
        else:
            He, P, E = cfg.expert_hidden_eff, cfg.num_dense_parts, cfg.num_experts_per_part
            s[p + "ffn.part_router.gate.weight"] = (P, D)
            for q in range(P):
                s[p + f"ffn.parts.{q}.router.gate.weight"] = (E, D)
                for e in range(E):
                    ep = p + f"ffn.parts.{q}.experts.{e}."
                    s[ep + "w_gate.weight"] = (He, D)
                    s[ep + "w_up.weight"] = (He, D)
                    s[ep + "w_down.weight"] = (D, He)
    if not cfg.tie_weights:
        s["head.weight"] = (cfg.vocab_size, D)
    return s


def init_weights(cfg: ModelConfig, seed: int = 0, device="cpu") -> Dict[str, torch.Tensor]:
    """Random-init fp32 weights with the reference's scheme
    (CometSparkNexLM._init_weights, cometspark.py:455-481): every Linear /
    Embedding ~ N(0, init_std), attn.proj and the trisparse w_down scaled by
    1/sqrt(2*n_layer), RMSNorm weights 1, gate logits 0, global tokens
    N(0, 0.02).  The values come from torch's generator (the reference draws
    from numpy's legacy stream), so only the distribution is the reference's."""
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    res = 1.0 / math.sqrt(2 * cfg.n_layer)
    out = {}
    for name, shape in weight_shapes(cfg).items():
        if name.endswith("norm1.weight") or name.endswith("norm2.weight") or name == "norm.weight":
            t = torch.ones(shape, dtype=torch.float32, device=device)
        elif name.endswith("gate_logits"):
            t = torch.zeros(shape, dtype=torch.float32, device=device)
        else:
            t = torch.randn(shape, generator=g, dtype=torch.float32, device=device) * cfg.init_std
            if name.endswith("attn.proj.weight") or (name.endswith("ffn.w_down.weight") and ".parts." not in name):
                t = t * res
        out[name] = t
    return out


def rope_tables(head_dim: int, max_len: int, theta: float):
    """cos / sin tables of TriSparseAttention._build_rope_table
    (tri_sparse_attn.py:167-180), computed in float32 as numpy does."""
    half = head_dim // 2
    i = np.arange(half, dtype=np.float32)
    inv_freq = np.float32(1.0) / (np.float32(theta) ** (np.float32(2.0) * i / np.float32(head_dim)))
    pos = np.arange(max_len, dtype=np.float32)
    ang = np.outer(pos, inv_freq).astype(np.float32)
    cos = np.concatenate([np.cos(ang), np.cos(ang)], axis=-1).astype(np.float32)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], axis=-1).astype(np.float32)
    return cos, sin


def alibi_slopes(n_head: int) -> np.ndarray:
    """m_h = 1 / 2^(h / n_head), h = 1..n_head (tri_sparse_attn.py:150-153)."""
    return (1.0 / (2.0 ** (np.arange(1, n_head + 1, dtype=np.float32) / n_head))).astype(np.float32)


# ---------------------------------------------------------------------------
# The model
# ---------------------------------------------------------------------------
@dataclass
class _Layer:
    kind: str
    norm1: torch.Tensor
    norm2: torch.Tensor
    wqkv: object
    proj: object
    gk: torch.Tensor          # (1, Hkv, G, d) global keys (compute dtype)
    gv: torch.Tensor
    gates: torch.Tensor       # sigmoid(gate_logits), fp32 (3,)
    ffn: Dict[str, object] = field(default_factory=dict)


def rope_rows(heads: int, d: int, blk: int) -> torch.Tensor:
    """Row order of a q|k|v weight for the RoPE epilogues: per head, blocks
    of blk dims t*blk .. +blk followed by their rotate-half partners d/2 +
    t*blk .. +blk (entry i = the source row of packed row i)."""
    half = d // 2
    t = torch.arange(half // blk).view(-1, 1, 1)
    r = torch.arange(blk).view(1, 1, -1)
    blocks = torch.cat([t * blk + r, half + t * blk + r], dim=1).reshape(-1)      # one head
    return (torch.arange(heads).view(-1, 1) * d + blocks.view(1, -1)).reshape(-1)


def _deq_int4(w, hip) -> torch.Tensor:
    """fp32 q * s of w quantized to INT4 group 128 with fp16 scales (exact);
    w a dense tensor or an Int4Weight already in that format."""
    if isinstance(w, Int4Weight):
        return hip.dequant_w4(w.wq, w.sc, w.shape[1], 128)
    wq, sc = VQ.quantize_int4_g(w.float(), 128)
    return hip.dequant_w4(wq, sc, w.shape[1], 128)


def _cat(ws):
    """Row concatenation of dense tensors or of Int4Weights (per-row groups,
    so the packed rows and scales concatenate as they are)."""
    if isinstance(ws[0], Int4Weight):
        return Int4Weight.cat(ws)
    return torch.cat(ws, 0)


def _pack(w: torch.Tensor, hip) -> torch.Tensor:
    """vnx_pack_bf16 of a contiguous (N, K) bf16 weight: the matrix-core
    operand order read by vnx_gemm_bf16 / vnx_expert_gemm_bf16."""
    N, K = w.shape
    L = hip._L
    out = torch.empty(L.vnx_pack_bf16_size(N, K) // 2, dtype=torch.bfloat16, device=hip.torch_device)
    _lib.check(L.vnx_pack_bf16(ctypes.c_void_p(w.data_ptr()), K, N, K, ctypes.c_void_p(out.data_ptr()),
                               ctypes.c_void_p(torch.cuda.current_stream(hip.torch_device).cuda_stream)), "pack_bf16")
    return out


class _Linear:
    """y (M, N) fp32 = x (M, K) . W^T.  Dense weights run F.linear in the
    compute dtype; INT4 group-128 weights (fp16 scales) run vnx_gemv_w4 for
    M <= 64 rows and a dequantized copy (bit-exact q * s) for larger M
    (prefill)."""

    def __init__(self, w, dtype, hip, int4: bool, swiglu: bool = False, rope_head_dim: int = 0):
        self.N, self.K = w.shape
        self.wq_rope = None
        self.wt = None
        self.dtype = dtype
        self.hip = hip
        pre = isinstance(w, Int4Weight)  # already quantized (streamed from a .vn file)
        self.int4 = pre or (bool(int4) and self.K % 128 == 0)
        self.wp = None
        self.swiglu = bool(swiglu) and self.N % 32 == 0
        if self.int4:
            wq, sc = (w.wq, w.sc) if pre else VQ.quantize_int4_g(w.float(), 128)
            self.wq, self.sc = wq.contiguous(), sc.contiguous()
            if self.swiglu:
                # rows reordered for vnx_gemv_w4_swiglu: blocks of 8 gate +
                # 8 up rows (per-row quantization, so a pure permutation)
                H = self.N // 2
                self.wq_sw = wq.view(2, H // 8, 8, -1).transpose(0, 1).reshape(self.N, -1).contiguous()
                self.sc_sw = sc.view(2, H // 8, 8, -1).transpose(0, 1).reshape(self.N, -1).contiguous()
            if rope_head_dim and rope_head_dim % 16 == 0 and self.N % rope_head_dim == 0:
                # rows in the order of vnx_gemv_w4_rope_kv's epilogue
                perm = rope_rows(self.N // rope_head_dim, rope_head_dim, 8).to(wq.device)
                self.wq_rope, self.sc_rope = wq[perm].contiguous(), sc[perm].contiguous()
            # the dense copy for prefill-size products, dequantized in row
            # blocks so no fp32 copy of a large matrix (the tied head) exists
            self.wd = torch.empty((self.N, self.K), dtype=dtype, device=hip.torch_device)
            rb = max(1, (8 << 20) // (4 * self.K))
            for r0 in range(0, self.N, rb):
                r1 = min(self.N, r0 + rb)
                self.wd[r0:r1] = hip.dequant_w4(self.wq[r0:r1], self.sc[r0:r1], self.K, 128)
            L = hip._L
            self._ws = torch.zeros(max(256, L.vnx_gemv_workspace(64, self.N, self.K)), dtype=torch.uint8,
                                   device=hip.torch_device)
            # large N (a tied LM head): a tiled copy for vnx_gemv_w4_tiles
            # (1 KB per wave load, nibbles in offset form)
            self.wt = None
            if self.N >= self.TILES_MIN_N and self.K in (512, 1024) and self.sc.dtype == torch.float16:
                self.wt = torch.empty(L.vnx_w4_tiles_bytes(self.N, self.K), dtype=torch.uint8,
                                      device=hip.torch_device)
                _lib.check(L.vnx_pack_w4_tiles(ctypes.c_void_p(self.wq.data_ptr()), self.wq.stride(0), self.N,
                                               self.K, ctypes.c_void_p(self.wt.data_ptr()),
                                               ctypes.c_void_p(torch.cuda.current_stream(hip.torch_device)
                                                               .cuda_stream)), "pack_w4_tiles")
        else:
            self.wd = w.to(dtype).contiguous()
            # verify-size products (M <= GEMM_MAX_M) run vnx_gemm_bf16 on a
            # packed copy; for a fused [gate; up] weight its rows are
            # interleaved in blocks of 16 gate + 16 up rows first (the
            # SwiGLU epilogue's order)
            if dtype == torch.bfloat16 and self.K % 64 == 0:
                src = self.wd
                if self.swiglu:
                    H = self.N // 2
                    src = self.wd.view(2, H // 16, 16, self.K).transpose(0, 1).reshape(self.N, self.K).contiguous()
                L = hip._L
                self.wp = torch.empty(L.vnx_pack_bf16_size(self.N, self.K) // 2, dtype=torch.bfloat16,
                                      device=hip.torch_device)
                _lib.check(L.vnx_pack_bf16(ctypes.c_void_p(src.data_ptr()), self.K, self.N, self.K,
                                           ctypes.c_void_p(self.wp.data_ptr()),
                                           ctypes.c_void_p(torch.cuda.current_stream(hip.torch_device).cuda_stream)),
                           "pack_bf16")


    GEMM_MAX_M = 256
    # rows from which an INT4 weight also keeps the tiled copy (the LM head)
    TILES_MIN_N = 32768

    def gemm(self, x: torch.Tensor, epilogue: int = 0, out_dtype=None) -> Optional[torch.Tensor]:
        """vnx_gemm_bf16 of the packed weight for x (M <= GEMM_MAX_M, bf16
        rows): (M, N), or (M, N/2) with the SwiGLU epilogue; None when this
        weight or x does not qualify."""
        M = x.shape[0]
        if self.wp is None or M > self.GEMM_MAX_M or x.dtype != torch.bfloat16 or x.stride(1) != 1:
            return None
        if epilogue and not self.swiglu:
            return None
        ncols = self.N // 2 if epilogue else self.N
        y = torch.empty((M, ncols), dtype=out_dtype or self.dtype, device=x.device)
        _lib.check(self.hip._L.vnx_gemm_bf16(
            ctypes.c_void_p(x.data_ptr()), x.stride(0), 0, ctypes.c_void_p(self.wp.data_ptr()), 0, M, self.N, self.K,
            1, int(epilogue), None, 1, ctypes.c_void_p(y.data_ptr()), _lib.DTYPE_CODES[y.dtype], ncols, 0,
            ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemm_bf16")
        return y

    def gemm_norm(self, x: torch.Tensor, norm_w: torch.Tensor, eps: float, epilogue: int = 0) -> Optional[torch.Tensor]:
        """vnx_gemm_bf16_norm: RMSNorm(x) * norm_w (x (M, K) fp32 residual rows)
        times the packed weight, (M, N) or with SwiGLU (M, N/2), bf16; None
        when this weight or x does not qualify."""
        M = x.shape[0]
        if (self.wp is None or M > self.GEMM_MAX_M or x.dtype != torch.float32 or x.stride(1) != 1
                or self.K > 2048 or (epilogue and not self.swiglu)):
            return None
        ncols = self.N // 2 if epilogue else self.N
        y = torch.empty((M, ncols), dtype=torch.bfloat16, device=x.device)
        _lib.check(self.hip._L.vnx_gemm_bf16_norm(
            ctypes.c_void_p(x.data_ptr()), x.stride(0), ctypes.c_void_p(norm_w.data_ptr()), float(eps),
            ctypes.c_void_p(self.wp.data_ptr()), M, self.N, self.K, int(epilogue), ctypes.c_void_p(y.data_ptr()),
            ncols, ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemm_bf16_norm")
        return y

    def gemm_norm_embed(self, tokens: torch.Tensor, emb: torch.Tensor, scale: float, x: torch.Tensor,
                        norm_w: torch.Tensor, eps: float) -> Optional[torch.Tensor]:
        """gemm_norm of x = emb[tokens] * scale, which the same call writes
        into x (vnx_gemm_bf16_norm_embed: the first layer's input straight
        from the bf16 token embedding); None (nothing done) when it does not
        apply."""
        M = x.shape[0]
        if (self.wp is None or M > self.GEMM_MAX_M or x.dtype != torch.float32 or x.stride(1) != 1
                or self.K > 2048 or emb.dtype != torch.bfloat16 or emb.stride(1) != 1 or emb.stride(0) % 8
                or emb.data_ptr() % 16):
            return None
        y = torch.empty((M, self.N), dtype=torch.bfloat16, device=x.device)
        P = ctypes.c_void_p
        _lib.check(self.hip._L.vnx_gemm_bf16_norm_embed(
            P(tokens.data_ptr()), P(emb.data_ptr()), _lib.VNX_BF16, emb.stride(0), emb.shape[0], float(scale),
            P(x.data_ptr()), x.stride(0), P(norm_w.data_ptr()), float(eps), P(self.wp.data_ptr()), M, self.N,
            self.K, P(y.data_ptr()), self.N, P(torch.cuda.current_stream(x.device).cuda_stream)),
            "gemm_bf16_norm_embed")
        return y

    def gemm_residual(self, x: torch.Tensor, res: torch.Tensor) -> bool:
        """res (M, N) fp32 += x . W^T (vnx_gemm_bf16_residual); False (nothing
        done) when this weight or x does not qualify."""
        M = x.shape[0]
        if self.wp is None or M > self.GEMM_MAX_M or x.dtype != torch.bfloat16 or x.stride(1) != 1:
            return False
        _lib.check(self.hip._L.vnx_gemm_bf16_residual(
            ctypes.c_void_p(x.data_ptr()), x.stride(0), ctypes.c_void_p(self.wp.data_ptr()), M, self.N, self.K,
            ctypes.c_void_p(res.data_ptr()), res.stride(0),
            ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemm_bf16_residual")
        return True

    def _gemv_x(self, x: torch.Tensor, norm_w):
        """(x pointer, row pitch, norm pointer): fp32 residual rows when a norm
        weight is given (the GEMV applies RMSNorm), else fp16 rows."""
        if norm_w is not None:
            return ctypes.c_void_p(x.data_ptr()), x.stride(0), ctypes.c_void_p(norm_w.data_ptr()), x
        x16 = x.to(torch.float16).contiguous()
        return ctypes.c_void_p(x16.data_ptr()), self.K, None, x16

    def rope_kv(self, x: torch.Tensor, rk, norm_w: Optional[torch.Tensor] = None, eps: float = 0.0) -> bool:
        """The q|k|v projection of x with RoPE and the KV-cache write fused
        (vnx_gemv_w4_rope_kv, INT4 weights, M <= 64; with norm_w, x is the
        fp32 residual stream and RMSNorm(x) * norm_w is fused too); False
        (nothing done) when it does not apply.  (The bf16 verify projection
        keeps a separate vnx_rope_kv: in its GEMM's epilogue the store pattern
        cost more than the launch it saves.)"""
        M = x.shape[0]
        if self.wq_rope is None or M > 64 or (norm_w is not None and x.dtype != torch.float32):
            return False
        xp, ldx, nwp, keep = self._gemv_x(x, norm_w)
        _lib.check(self.hip._L.vnx_gemv_w4_rope_kv(
            xp, ldx, nwp, float(eps), ctypes.c_void_p(self.wq_rope.data_ptr()), self.wq_rope.stride(0),
            ctypes.c_void_p(self.sc_rope.data_ptr()), _lib.VNX_F16, self.sc_rope.stride(0), M, self.N, self.K, 128,
            ctypes.byref(rk), ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemv_w4_rope_kv")
        return True

    def rope_kv_embed(self, tokens: torch.Tensor, emb: torch.Tensor, scale: float, x: torch.Tensor, rk,
                      norm_w: torch.Tensor, eps: float) -> bool:
        """rope_kv of RMSNorm(x) * norm_w where x = emb[tokens] * scale is
        written by the same call (vnx_gemv_w4_rope_kv_embed: the first
        layer's input straight from the bf16 token embedding); False (nothing
        done) when it does not apply."""
        M = x.shape[0]
        if (self.wq_rope is None or M > 64 or x.dtype != torch.float32 or emb.dtype != torch.bfloat16
                or emb.stride(1) != 1 or emb.stride(0) % 8 or emb.data_ptr() % 16 or x.stride(1) != 1):
            return False
        P = ctypes.c_void_p
        _lib.check(self.hip._L.vnx_gemv_w4_rope_kv_embed(
            P(tokens.data_ptr()), P(emb.data_ptr()), _lib.VNX_BF16, emb.stride(0), emb.shape[0], float(scale),
            P(x.data_ptr()), x.stride(0), P(norm_w.data_ptr()), float(eps), P(self.wq_rope.data_ptr()),
            self.wq_rope.stride(0), P(self.sc_rope.data_ptr()), _lib.VNX_F16, self.sc_rope.stride(0), M, self.N,
            self.K, 128, ctypes.byref(rk), P(torch.cuda.current_stream(x.device).cuda_stream)),
            "gemv_w4_rope_kv_embed")
        return True

    def gemv_swiglu(self, x: torch.Tensor, norm_w: Optional[torch.Tensor] = None,
                    eps: float = 0.0) -> Optional[torch.Tensor]:
        """silu(gate) * up (M, N/2) fp16 of a fused [gate; up] INT4 weight for
        M <= 64 rows (vnx_gemv_w4_swiglu; with norm_w, of RMSNorm(x) * norm_w
        of the fp32 rows x); None when it does not apply."""
        M = x.shape[0]
        if not (self.int4 and self.swiglu and M <= 64) or (norm_w is not None and x.dtype != torch.float32):
            return None
        xp, ldx, nwp, keep = self._gemv_x(x, norm_w)
        H = self.N // 2
        y = torch.empty((M, H), dtype=torch.float16, device=x.device)
        _lib.check(self.hip._L.vnx_gemv_w4_swiglu(
            xp, ldx, nwp, float(eps), ctypes.c_void_p(self.wq_sw.data_ptr()), self.wq_sw.stride(0),
            ctypes.c_void_p(self.sc_sw.data_ptr()), _lib.VNX_F16, self.sc_sw.stride(0), M, self.N, self.K, 128,
            ctypes.c_void_p(y.data_ptr()), H, ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)),
            "gemv_w4_swiglu")
        return y

    def gemv_residual(self, x: torch.Tensor, res: torch.Tensor) -> bool:
        """res (M, N) fp32 += x . W^T for INT4 weights and M <= 64
        (vnx_gemv_w4_residual); False (nothing done) when it does not apply."""
        M = x.shape[0]
        if not self.int4 or M > 64 or self.N >= 32768:
            return False
        x16 = x.to(torch.float16).contiguous()
        _lib.check(self.hip._L.vnx_gemv_w4_residual(
            ctypes.c_void_p(x16.data_ptr()), self.K, ctypes.c_void_p(self.wq.data_ptr()), self.wq.stride(0),
            ctypes.c_void_p(self.sc.data_ptr()), _lib.VNX_F16, self.sc.stride(0), M, self.N, self.K, 128,
            ctypes.c_void_p(res.data_ptr()), res.stride(0),
            ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemv_w4_residual")
        return True

    def __call__(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x (M, K); returns (M, N) in the compute dtype (dense) or fp32
        (INT4 GEMV, written into `out` when given: an (M, N) view with unit
        column stride, fp32, or bf16 for the tiled large-N product)."""
        M = x.shape[0]
        if self.int4 and M <= 64:
            x16 = x.to(torch.float16).contiguous()
            y = out if out is not None else torch.empty((M, self.N), dtype=torch.float32, device=x.device)
            L = self.hip._L
            if self.wt is not None:
                if y.dtype not in (torch.float32, torch.bfloat16):
                    raise ValueError("the INT4 head writes fp32 or bf16 logits")
                _lib.check(L.vnx_gemv_w4_tiles_out(
                    ctypes.c_void_p(x16.data_ptr()), self.K, ctypes.c_void_p(self.wt.data_ptr()),
                    ctypes.c_void_p(self.sc.data_ptr()), self.sc.stride(0), M, self.N, self.K,
                    ctypes.c_void_p(y.data_ptr()), _lib.VNX_BF16 if y.dtype == torch.bfloat16 else _lib.VNX_F32,
                    y.stride(0), ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemv_w4_tiles")
                return y
            if y.dtype != torch.float32:
                raise ValueError("the INT4 GEMV writes fp32")
            _lib.check(L.vnx_gemv_w4(
                ctypes.c_void_p(x16.data_ptr()), self.K, ctypes.c_void_p(self.wq.data_ptr()), self.wq.stride(0),
                ctypes.c_void_p(self.sc.data_ptr()), _lib.VNX_F16, self.sc.stride(0), M, self.N, self.K, 128,
                ctypes.c_void_p(y.data_ptr()), y.stride(0), ctypes.c_void_p(self._ws.data_ptr()),
                self._ws.numel(), ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)), "gemv_w4")
            return y
        y = self.gemm(x) if out is None else None
        if y is not None:
            return y
        y = torch.nn.functional.linear(x.to(self.dtype), self.wd)
        if out is not None:
            out.copy_(y)
            return out
        return y


class CometSparkGPU:
    """A CometSpark target or draft on one GPU with a per-sequence KV cache.

    forward(tokens (B, n), lens (B,) int32) runs the n new tokens of every
    sequence at positions lens[b] .. lens[b]+n-1, writes their keys / values
    into the cache there and returns the final-norm hidden states (B, n, D)
    fp32.  Committing a verify result is `lens += accepted + 1` (the rest of
    the written rows is overwritten by the next call)."""

    def __init__(self, cfg: ModelConfig, weights: Dict[str, torch.Tensor], hip, batch: int, capacity: int,
                 dtype=torch.bfloat16, int4: bool = False):
        self.cfg = cfg
        self.hip = hip
        self.dev = hip.torch_device
        self.dtype = dtype
        self.B = int(batch)
        self.cap = int(capacity)
        dev, D, d = self.dev, cfg.dim, cfg.head_dim
        # Int4Weight entries (a .vn file streamed by load_vn_weights) stay as
        # they are; everything else becomes fp32 on the device
        W = {k: v if isinstance(v, Int4Weight) else
             (v if isinstance(v, torch.Tensor) else torch.from_numpy(np.asarray(v))).to(dev, torch.float32)
             for k, v in weights.items()}
        E = W["tok_emb.weight"]
        if isinstance(E, Int4Weight):
            if not int4:
                raise ValueError("an INT4 embedding needs int4=True")
            self.emb = (E.dense if E.dense is not None else _deq_int4(E, hip)).to(dtype).contiguous()
        else:
            self.emb = E.to(dtype).contiguous()
        self.emb_scale = math.sqrt(D) if cfg.embedding_scale else 1.0
        self.norm = W["norm.weight"]
        # the LM head: the embedding table when tied (cometspark.py:396-398),
        # else the model's own (V, D) head.weight
        if cfg.tie_weights:
            Hw = E
        else:
            if "head.weight" not in W:
                raise ValueError("an untied model (tie_weights False) needs 'head.weight'")
            Hw = W["head.weight"]
            if tuple(Hw.shape) != (cfg.vocab_size, D):
                raise ValueError(f"head.weight has shape {tuple(Hw.shape)}, expected {(cfg.vocab_size, D)}")
            if isinstance(Hw, Int4Weight) and not int4:
                raise ValueError("an INT4 head needs int4=True")
        self.head = _Linear(Hw, dtype, hip, int4) if int4 else None
        # the dense head matrix of the bf16 / fp32 logits path
        self.head_w = None if int4 else (self.emb if cfg.tie_weights else Hw.to(dtype).contiguous())
        self.layers = []
        for i, kind in enumerate(cfg.layer_pattern):
            p = f"blocks.{i}."
            wq, wk, wv = W[p + "attn.wq.weight"], W[p + "attn.wk.weight"], W[p + "attn.wv.weight"]
            g = W[p + "attn.global_tokens.weight"]
            G = g.shape[0]
            # the global sinks go through the same k / v weights as the tokens:
            # with INT4 weights, their exact dequantization q * s
            wk_g, wv_g = (wk, wv) if not (int4 and D % 128 == 0) else (_deq_int4(wk, hip), _deq_int4(wv, hip))
            gk = (g @ wk_g.t()).reshape(G, cfg.n_kv_head, d).permute(1, 0, 2).unsqueeze(0)
            gv = (g @ wv_g.t()).reshape(G, cfg.n_kv_head, d).permute(1, 0, 2).unsqueeze(0)
            L = _Layer(kind=kind, norm1=W[p + "norm1.weight"], norm2=W[p + "norm2.weight"],
                       wqkv=_Linear(_cat([wq, wk, wv]), dtype, hip, int4,
                                    rope_head_dim=d if dtype == torch.bfloat16 and int4 else 0),
                       proj=_Linear(W[p + "attn.proj.weight"], dtype, hip, int4),
                       gk=gk.to(dtype).contiguous(), gv=gv.to(dtype).contiguous(),
                       gates=torch.sigmoid(W[p + "attn.gate_logits"].float()).contiguous())
            if kind == "trisparse":
                L.ffn["gu"] = _Linear(_cat([W[p + "ffn.w_gate.weight"], W[p + "ffn.w_up.weight"]]),
                                      dtype, hip, int4, swiglu=True)
                L.ffn["down"] = _Linear(W[p + "ffn.w_down.weight"], dtype, hip, int4)
            else:
                P, E = cfg.num_dense_parts, cfg.num_experts_per_part
                # routing logits [part router | expert routers, part-major] in
                # one fp32 product
                L.ffn["route"] = torch.cat([W[p + "ffn.part_router.gate.weight"]]
                                           + [W[p + f"ffn.parts.{q}.router.gate.weight"] for q in range(P)],
                                           0).contiguous()
                w1, w2 = [], []
                for q in range(P):
                    for e in range(E):
                        ep = p + f"ffn.parts.{q}.experts.{e}."
                        w1.append(torch.cat([W[ep + "w_gate.weight"], W[ep + "w_up.weight"]], 0))
                        w2.append(W[ep + "w_down.weight"])
                # batched-product operands, untransposed and contiguous:
                # (P*E, D, 2He) gate|up and (P*E, He, D) down
                L.ffn["w1"] = torch.stack([w.t() for w in w1]).to(dtype).contiguous()
                L.ffn["w2"] = torch.stack([w.t() for w in w2]).to(dtype).contiguous()
                if dtype == torch.bfloat16 and D % 64 == 0 and cfg.expert_hidden_eff % 64 == 0:
                    # packed per-expert copies for the routed products of
                    # verify-size forwards (vnx_expert_gemm_bf16); gate|up
                    # rows interleaved in blocks of 16 for the SwiGLU epilogue
                    He = cfg.expert_hidden_eff
                    L.ffn["w1p"] = torch.stack([_pack(w.to(dtype).view(2, He // 16, 16, D).transpose(0, 1)
                                                      .reshape(2 * He, D).contiguous(), hip) for w in w1])
                    L.ffn["w2p"] = torch.stack([_pack(w.to(dtype).contiguous(), hip) for w in w2])
            self.layers.append(L)
        cos, sin = rope_tables(d, self.cap + 64, cfg.rope_theta)
        self.cos = torch.from_numpy(cos).to(dev)
        self.sin = torch.from_numpy(sin).to(dev)
        self.slopes = torch.from_numpy(alibi_slopes(cfg.n_head)).to(dev)
        Hkv = cfg.n_kv_head
        self.kc = [torch.zeros((self.B, Hkv, self.cap, d), dtype=dtype, device=dev) for _ in self.layers]
        self.vc = [torch.zeros((self.B, Hkv, self.cap, d), dtype=dtype, device=dev) for _ in self.layers]
        self._words = {}
        self._neg = torch.full((), -1e9, dtype=torch.float32, device=dev)  # the reference's mask value
        # vnx_tree_attn covers all three paths (window, global rows, ALiBi) for
        # bf16 heads of 64 / 128 (verify-size chunks) and fp32 heads of 8 / 16 /
        # 32 (chunks of any length)
        self.f32_rows = dtype == torch.float32 and d in (8, 16, 32)
        self.kernel_attention = (dtype == torch.bfloat16 and d in (64, 128)) or self.f32_rows
        # dtype of the activations fed to the projections: fp16 for the INT4
        # GEMVs, else the compute dtype
        self.act_dtype = torch.float16 if int4 else dtype
        # the first layer's q|k|v product gathers the token embedding itself
        # (INT4 decode and bf16 verify-size forwards; False: vnx_embed_rmsnorm
        # first, the form it is tested against)
        self.embed_fold = True

    @classmethod
    def from_vn(cls, path: str, hip, batch: int, capacity: int, dtype=torch.bfloat16, int4: bool = True,
                chunk_bytes: int = 64 << 20, cfg: Optional[ModelConfig] = None) -> "CometSparkGPU":
        """The model saved in a .vn file (CometSparkNexLM.save_vn /
        CometSparkV05LM.save_vn, cometspark.py:1014-1060; loaded by the
        reference through VNFileReader, spark/mate/model/model.py:271-285),
        its weights streamed onto the device: with int4 the projections, the
        trisparse FFNs and the LM head are quantized chunk by chunk into
        their INT4 group-128 buffers on the GPU (vnx_quantize_w4_g), never
        held in full precision.  A tied model's state_dict holds the
        embedding twice (as 'head.weight' too): that copy is skipped.  With
        tie_weights false in the config (cometspark.py:396-398) the stored
        'head.weight' is the LM head."""
        from .vn import VNReader, config_from_vn, int4_matrix, load_vn_weights
        with VNReader(path) as r:
            r.read_meta()
            conf = r.read_config()
            tied = cfg.tie_weights if cfg is not None else bool(conf.get("tie_weights", True))
            W = load_vn_weights(r, hip, quantize=int4_matrix if int4 else (lambda n, s: False), dense_dtype=dtype,
                                chunk_bytes=chunk_bytes, skip=lambda n: tied and n == "head.weight")
        if cfg is None:
            cfg = config_from_vn(conf, W, name=f"{path} (.vn)")
        return cls(cfg, W, hip, batch, capacity, dtype, int4)

    # ---- pieces ---------------------------------------------------------
    def _st(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)

    def _rms(self, x: torch.Tensor, res: Optional[torch.Tensor], w: torch.Tensor, y: torch.Tensor) -> None:
        """x += res (in place, res may be None); y = RMSNorm(x) * w (vnx_rmsnorm)."""
        M, D = x.shape
        P = ctypes.c_void_p
        _lib.check(self.hip._L.vnx_rmsnorm(
            P(x.data_ptr()), x.stride(0), P(res.data_ptr()) if res is not None else None,
            _lib.DTYPE_CODES[res.dtype] if res is not None else _lib.VNX_F32, res.stride(0) if res is not None else D,
            P(w.data_ptr()), float(self.cfg.eps), M, D, P(x.data_ptr()), x.stride(0), P(y.data_ptr()),
            _lib.DTYPE_CODES[y.dtype], y.stride(0), self._st()), "rmsnorm")

    def _chain_words(self, n: int) -> torch.Tensor:
        w = self._words.get(n)
        if w is None:
            a = np.array([(1 << (i + 1)) - 1 for i in range(n)], dtype=np.uint64)
            w = torch.from_numpy(a.view(np.int64)).to(self.dev)
            self._words[n] = w
        return w

    def _tree_call(self, q, kc, vc, cstr, tree_k, tree_v, tstr, anc, B, H, Hkv, Tp, n, d, tp, follows, out,
                   seg2=None, gates=None, qkv=None, out_sb=None, alibi_max=1024):
        a = _lib.TreeAttnArgs()
        if qkv is not None:
            # queries from the q|k|v rows, RoPE and the cache write in the kernel
            a.q = None; a.q_strides[:] = [0, 0, 0]
            a.qkv = qkv.data_ptr(); a.qkv_ld = qkv.stride(0)
            a.cos_table = self.cos.data_ptr(); a.sin_table = self.sin.data_ptr()
            a.table_rows = self.cos.shape[0]; a.rope = int(self.cfg.use_rope); a.cap = self.cap
        else:
            a.q = q.data_ptr(); a.q_strides[:] = list(q.stride()[:3])
        a.k_cache = kc.data_ptr(); a.v_cache = vc.data_ptr(); a.cache_strides[:] = cstr
        a.k_tree = tree_k.data_ptr(); a.v_tree = tree_v.data_ptr(); a.tree_strides[:] = tstr
        a.anc = anc.data_ptr() if anc is not None else None; a.anc_batch_stride = 0   # None: a chain (fp32 rows)
        a.f32_rows = int(self.f32_rows)
        # output rows in (B, n, H, d) order: the proj input layout
        a.out = out.data_ptr(); a.out_dtype = _lib.DTYPE_CODES[out.dtype]
        a.out_strides[:] = [n * H * d if out_sb is None else out_sb, d, H * d]
        a.B, a.H, a.Hkv, a.Tp, a.N, a.d = B, H, Hkv, Tp, n, d
        a.scale = 1.0 / math.sqrt(d)
        a.window = self.cfg.window_size
        if self.cfg.use_alibi:
            a.alibi_slopes = self.slopes.data_ptr(); a.alibi_max_keys = max(0, int(alibi_max))
            a.gates = gates.data_ptr()
        a.tp_batch = tp.data_ptr() if tp is not None else None
        a.tree_follows_prefix = 1 if follows else 0
        if seg2 is not None:
            k2, v2 = seg2
            a.k_seg2 = k2.data_ptr(); a.v_seg2 = v2.data_ptr()
            a.seg2_strides[:] = [0, k2.stride(1), k2.stride(2)]
            a.T2 = k2.shape[2]
            a.gates = gates.data_ptr()
        L = self.hip._L
        ws = self.hip._workspace(L.vnx_tree_attn_workspace(B, H, Hkv, n, Tp, d))
        _lib.check(L.vnx_tree_attn(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), self._st()),
                   "tree_attn")

    def _attn_kernel(self, q, li, lens, n, Tmax, qkv=None):
        """Sliding-window and global paths in one vnx_tree_attn call: each
        row's prefix of lens[b] cache rows, then its n new rows (written in
        place right after it) under the chain mask, and the G global rows as
        the gated second segment; writes the proj input (B*n, H*d) in the
        activation dtype.  fp32 models with heads of 8 / 16 / 32 take the
        kernel's fp32-rows path (a chain of any n, no mask words).  q (B, H,
        n, d) in the model dtype, or qkv (B*n, (H+2Hkv) d) bf16
        projection rows (RoPE and the new rows' cache write done by the
        kernel; q unused)."""
        cfg = self.cfg
        B, H, d = self.B, cfg.n_head, cfg.head_dim
        kc, vc = self.kc[li], self.vc[li]
        Ly = self.layers[li]
        o = torch.empty((B * n, H * d), dtype=self.act_dtype, device=self.dev)
        cstr = list(kc.stride()[:3])
        anc = None if self.f32_rows else self._chain_words(n)
        self._tree_call(q, kc, vc, cstr, kc, vc, cstr, anc, B, H, cfg.n_kv_head, Tmax, n, d, lens,
                        True, o, seg2=(Ly.gk, Ly.gv), gates=Ly.gates, qkv=qkv)
        return o

    def _attn_kernel_chunked(self, q, li, lens, n, Tmax):
        """bf16 forwards of more rows than one vnx_tree_attn call takes
        (prefill): the n new rows (already in the cache) in chunks of at
        most min(64, window) queries, chunk [c0, c1) seeing each row's
        lens[b] + c0 prefix rows and its own rows under the chain mask.  The
        ALiBi path keeps the whole call's rule (lens[b] + n <= 1024,
        tri_sparse_attn.py:600-607): a chunk passes 1024 - (n - c1) as its
        key limit.  q (B, H, n, d) bf16."""
        cfg = self.cfg
        B, H, d = self.B, cfg.n_head, cfg.head_dim
        kc, vc = self.kc[li], self.vc[li]
        Ly = self.layers[li]
        o = torch.empty((B * n, H * d), dtype=self.act_dtype, device=self.dev)
        cstr = list(kc.stride()[:3])
        step = min(64, cfg.window_size) if cfg.window_size > 0 else 64
        for c0 in range(0, n, step):
            c1 = min(n, c0 + step)
            m = c1 - c0
            lens_c = lens + c0 if c0 else lens
            self._tree_call(q[:, :, c0:c1], kc, vc, cstr, kc, vc, cstr, self._chain_words(m), B, H, cfg.n_kv_head,
                            Tmax + c0, m, d, lens_c, True, o[c0:], seg2=(Ly.gk, Ly.gv), gates=Ly.gates,
                            out_sb=n * H * d, alibi_max=1024 - (n - c1))
        return o

    def _attn_torch(self, q, li, lens, n, Tmax):
        """The same three paths with explicit fp32 masks: bf16 prefill chunks
        longer than 64 rows or than the window, and head sizes the kernel does
        not take.  q (B, H, n, d)."""
        cfg = self.cfg
        B, H, _, d = q.shape
        rep = H // cfg.n_kv_head
        Tk = Tmax + n
        k = self.kc[li][:, :, :Tk].float().repeat_interleave(rep, dim=1)
        v = self.vc[li][:, :, :Tk].float().repeat_interleave(rep, dim=1)
        qf = q.float()
        scale = 1.0 / math.sqrt(d)
        scores = torch.matmul(qf, k.transpose(-1, -2).contiguous()) * scale        # (B, H, n, Tk)
        qpos = lens.long().view(B, 1) + torch.arange(n, device=self.dev).view(1, n)  # (B, n)
        kpos = torch.arange(Tk, device=self.dev).view(1, 1, Tk)
        dist = qpos.unsqueeze(-1) - kpos                                            # (B, n, Tk)
        causal = dist >= 0
        swa_ok = causal & (dist < cfg.window_size)
        neg = self._neg
        s_swa = torch.where(swa_ok.unsqueeze(1), scores, neg)
        out = torch.matmul(torch.softmax(s_swa, dim=-1), v)
        Ly = self.layers[li]
        gk = Ly.gk.float().repeat_interleave(rep, dim=1)
        gv = Ly.gv.float().repeat_interleave(rep, dim=1)
        sg = torch.matmul(qf, gk.transpose(-1, -2).contiguous()) * scale
        out_g = torch.matmul(torch.softmax(sg, dim=-1), gv)
        res = Ly.gates[0] * out + Ly.gates[1] * out_g
        if cfg.use_alibi:
            # path C while the sequence holds at most 1024 keys (:600-607)
            bias = -self.slopes.view(1, H, 1, 1) * dist.unsqueeze(1).float()
            s_c = torch.where(causal.unsqueeze(1), scores + bias, neg)
            out_c = torch.matmul(torch.softmax(s_c, dim=-1), v)
            use_c = ((lens.long() + n) <= 1024).view(B, 1, 1, 1)
            res = res + torch.where(use_c, Ly.gates[2] * out_c, torch.zeros_like(out_c))
        return res

    def _mod_fused(self, L: _Layer, x: torch.Tensor) -> None:
        """The MoD FFN of a verify-size forward with norm2 and the residual
        add fused: x (M, D) fp32 residual stream += MoD(RMSNorm(x) * norm2).
        vnx_mod_route_x normalizes, routes and writes the experts' bf16 input
        rows; vnx_expert_gemm_bf16 runs each expert on its routed rows only
        (gate|up with SwiGLU and routing weight fused, then down on the compact
        rows); vnx_sum_expert_rows adds each row's experts into x."""
        cfg = self.cfg
        P, E, k = cfg.num_dense_parts, cfg.num_experts_per_part, cfg.top_k
        PE, He, D = P * E, cfg.expert_hidden_eff, cfg.dim
        M = x.shape[0]
        P_ = ctypes.c_void_p
        L_ = self.hip._L
        comb = torch.empty((M, PE), dtype=torch.float32, device=self.dev)
        wr = L.ffn["route"]                                                        # (P + PE, D) fp32
        xh = torch.empty((M, D), dtype=torch.bfloat16, device=self.dev)
        _lib.check(L_.vnx_mod_route_x(P_(x.data_ptr()), x.stride(0), P_(L.norm2.data_ptr()), float(cfg.eps),
                                      P_(wr.data_ptr()), wr.stride(0), M, D, P, E, k, P_(comb.data_ptr()), PE,
                                      P_(xh.data_ptr()), D, 0, 1, self._st()), "mod_route_x")
        rows = torch.empty((PE, M), dtype=torch.int32, device=self.dev)
        counts = torch.empty((PE,), dtype=torch.int32, device=self.dev)
        slots = torch.empty((M, PE), dtype=torch.int32, device=self.dev)
        w1p, w2p = L.ffn["w1p"], L.ffn["w2p"]
        act = torch.empty((PE, M, He), dtype=torch.bfloat16, device=self.dev)
        _lib.check(L_.vnx_expert_gemm_bf16(
            P_(xh.data_ptr()), D, 0, P_(w1p.data_ptr()), w1p.stride(0), M, 2 * He, D, PE, _lib.VNX_EPI_SWIGLU,
            P_(comb.data_ptr()), PE, 1, P_(rows.data_ptr()), P_(counts.data_ptr()), P_(slots.data_ptr()),
            P_(act.data_ptr()), _lib.VNX_BF16, He, M * He, self._st()), "expert_gemm w1")
        y = torch.empty((PE, M, D), dtype=torch.bfloat16, device=self.dev)
        _lib.check(L_.vnx_expert_gemm_bf16(
            P_(act.data_ptr()), He, M * He, P_(w2p.data_ptr()), w2p.stride(0), M, D, He, PE, _lib.VNX_EPI_NONE,
            None, 0, 0, None, P_(counts.data_ptr()), None, P_(y.data_ptr()), _lib.VNX_BF16, D, M * D,
            self._st()), "expert_gemm w2")
        _lib.check(L_.vnx_sum_expert_rows(P_(y.data_ptr()), _lib.VNX_BF16, D, M * D, P_(slots.data_ptr()), M, PE,
                                          D, P_(x.data_ptr()), x.stride(0), 1, self._st()), "sum_expert_rows")

    def _mod(self, L: _Layer, h: torch.Tensor) -> torch.Tensor:
        """MoD FFN on (M, D) fp32 normalized rows.  Verify-size forwards (bf16,
        M <= 256): the routing weights (vnx_mod_route_x), each expert's
        products on its routed rows only (vnx_expert_gemm_bf16) and the sum
        over each row's experts (vnx_sum_expert_rows).  Otherwise fp32 routing
        logits in one product and the routing weights (vnx_mod_route); every
        expert's gate|up and down as batched products over the P*E experts,
        with the weighted activations in between (vnx_mod_swiglu; zero for
        unselected experts) and the sum over experts after (vnx_sum_experts)."""
        cfg = self.cfg
        P, E, k = cfg.num_dense_parts, cfg.num_experts_per_part, cfg.top_k
        PE, He, D = P * E, cfg.expert_hidden_eff, cfg.dim
        M = h.shape[0]
        P_ = ctypes.c_void_p
        L_ = self.hip._L
        comb = torch.empty((M, PE), dtype=torch.float32, device=self.dev)
        wr = L.ffn["route"]                                                        # (P + PE, D) fp32
        if P + PE <= 32 and "w1p" in L.ffn and M <= 256:
            # routed products: router + routing rule (one bf16 copy of h),
            # then each expert's gate|up with the SwiGLU and routing weight
            # fused and its down product on its own rows only, then the sum
            # over each row's experts
            xh = torch.empty((M, D), dtype=torch.bfloat16, device=self.dev)
            _lib.check(L_.vnx_mod_route_x(P_(h.data_ptr()), h.stride(0), None, 0.0, P_(wr.data_ptr()), wr.stride(0), M,
                                          D, P, E, k, P_(comb.data_ptr()), PE, P_(xh.data_ptr()), D, 0, 1,
                                          self._st()), "mod_route_x")
            rows = torch.empty((PE, M), dtype=torch.int32, device=self.dev)
            counts = torch.empty((PE,), dtype=torch.int32, device=self.dev)
            slots = torch.empty((M, PE), dtype=torch.int32, device=self.dev)
            w1p, w2p = L.ffn["w1p"], L.ffn["w2p"]
            act = torch.empty((PE, M, He), dtype=torch.bfloat16, device=self.dev)
            _lib.check(L_.vnx_expert_gemm_bf16(
                P_(xh.data_ptr()), D, 0, P_(w1p.data_ptr()), w1p.stride(0), M, 2 * He, D, PE, _lib.VNX_EPI_SWIGLU,
                P_(comb.data_ptr()), PE, 1, P_(rows.data_ptr()), P_(counts.data_ptr()), P_(slots.data_ptr()),
                P_(act.data_ptr()), _lib.VNX_BF16, He, M * He, self._st()), "expert_gemm w1")
            y = torch.empty((PE, M, D), dtype=torch.bfloat16, device=self.dev)
            _lib.check(L_.vnx_expert_gemm_bf16(
                P_(act.data_ptr()), He, M * He, P_(w2p.data_ptr()), w2p.stride(0), M, D, He, PE, _lib.VNX_EPI_NONE,
                None, 0, 0, None, P_(counts.data_ptr()), None, P_(y.data_ptr()), _lib.VNX_BF16, D, M * D,
                self._st()), "expert_gemm w2")
            out = torch.empty((M, D), dtype=torch.float32, device=self.dev)
            _lib.check(L_.vnx_sum_expert_rows(P_(y.data_ptr()), _lib.VNX_BF16, D, M * D, P_(slots.data_ptr()), M, PE,
                                              D, P_(out.data_ptr()), D, 0, self._st()), "sum_expert_rows")
            return out
        if P + PE <= 32 and self.dtype == torch.bfloat16:
            # router products and routing rule in one launch, which also
            # writes the experts' bf16 input rows (one copy per expert)
            xb = torch.empty((PE, M, D), dtype=self.dtype, device=self.dev)
            _lib.check(L_.vnx_mod_route_x(P_(h.data_ptr()), h.stride(0), None, 0.0, P_(wr.data_ptr()), wr.stride(0), M,
                                          D, P, E, k, P_(comb.data_ptr()), PE, P_(xb.data_ptr()), D, M * D, PE,
                                          self._st()), "mod_route_x")
        else:
            logits = torch.nn.functional.linear(h, wr)                             # (M, P + PE) fp32
            _lib.check(L_.vnx_mod_route(P_(logits.data_ptr()), logits.stride(0), M, P, E, k, P_(comb.data_ptr()),
                                        PE, self._st()), "mod_route")
            xb = h.to(self.dtype).unsqueeze(0).expand(PE, M, D).contiguous()
        gu = torch.matmul(xb, L.ffn["w1"])                                        # (PE, M, 2He)
        act = torch.empty((PE, M, He), dtype=self.dtype, device=self.dev)
        _lib.check(L_.vnx_mod_swiglu(P_(gu.data_ptr()), _lib.DTYPE_CODES[gu.dtype], 2 * He, M * 2 * He,
                                     P_(comb.data_ptr()), PE, M, PE, He, P_(act.data_ptr()),
                                     _lib.DTYPE_CODES[act.dtype], He, M * He, self._st()), "mod_swiglu")
        y = torch.matmul(act, L.ffn["w2"])                                        # (PE, M, D)
        out = torch.empty((M, D), dtype=torch.float32, device=self.dev)
        _lib.check(L_.vnx_sum_experts(P_(y.data_ptr()), _lib.DTYPE_CODES[y.dtype], M, PE, D, P_(out.data_ptr()),
                                      self._st()), "sum_experts")
        return out

    def _ffn(self, L: _Layer, h: torch.Tensor) -> torch.Tensor:
        if L.kind == "mod":
            return self._mod(L, h)
        Hf = self.cfg.ffn_hidden
        act = L.ffn["gu"].gemm(h, epilogue=_lib.VNX_EPI_SWIGLU, out_dtype=self.act_dtype)
        if act is None and self.act_dtype == torch.float16:
            act = L.ffn["gu"].gemv_swiglu(h)     # INT4 draft decode
        if act is not None:                      # gate|up product with the SwiGLU epilogue
            return L.ffn["down"](act)
        gu = L.ffn["gu"](h)
        act = torch.empty((h.shape[0], Hf), dtype=self.act_dtype, device=self.dev)
        _lib.check(self.hip._L.vnx_swiglu(ctypes.c_void_p(gu.data_ptr()), _lib.DTYPE_CODES[gu.dtype], gu.stride(0),
                                          h.shape[0], Hf, ctypes.c_void_p(act.data_ptr()),
                                          _lib.DTYPE_CODES[act.dtype], Hf, self._st()), "swiglu")
        return L.ffn["down"](act)

    # ---- forward --------------------------------------------------------
    def _embed_rms(self, tokens: torch.Tensor, w: torch.Tensor, x: torch.Tensor, y: torch.Tensor) -> None:
        """x = emb[tokens] * emb_scale (fp32); y = RMSNorm(x) * w (vnx_embed_rmsnorm)."""
        M, D = x.shape
        P = ctypes.c_void_p
        _lib.check(self.hip._L.vnx_embed_rmsnorm(
            P(tokens.data_ptr()), P(self.emb.data_ptr()), _lib.DTYPE_CODES[self.emb.dtype], self.emb.stride(0),
            self.emb.shape[0], float(self.emb_scale), P(w.data_ptr()), float(self.cfg.eps), M, D, P(x.data_ptr()),
            x.stride(0), P(y.data_ptr()), _lib.DTYPE_CODES[y.dtype], y.stride(0), self._st()), "embed_rmsnorm")

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, lens: torch.Tensor, Tmax: Optional[int] = None,
                out_dtype=torch.float32, cache_only: bool = False) -> Optional[torch.Tensor]:
        """tokens (B, n) int64, lens (B,) int32 on this device; Tmax >= max(lens)
        (read back from the device when not given).  Returns (B, n, D) final-norm
        hidden states in out_dtype (fp32 by default).  cache_only: the caller
        needs only the new rows' keys and values in every layer's cache (a
        draft's last step of a round), so the forward stops once the last
        layer has written them and returns None (where that layer's cache write
        happens inside its attention call, the forward runs to the end)."""
        cfg = self.cfg
        B, n = tokens.shape
        if B != self.B:
            raise ValueError(f"batch {B} != the cache's {self.B}")
        if lens.dtype != torch.int32 or lens.numel() != B:
            raise ValueError("lens must be (B,) int32")
        if Tmax is None:
            Tmax = int(lens.max())
        if Tmax + n > self.cap:
            raise ValueError(f"cache capacity {self.cap} exceeded ({Tmax} + {n})")
        H, Hkv, d, D = cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.dim
        M = B * n
        P = ctypes.c_void_p
        L_ = self.hip._L
        tok = tokens.reshape(-1).contiguous()
        if not self.layers:
            x = (self.emb[tok].float() * self.emb_scale).contiguous()
        else:
            x = torch.empty((M, D), dtype=torch.float32, device=self.dev)                # fp32 residual stream
        use_kernel = self.kernel_attention and (self.f32_rows or (n <= 64 and n <= cfg.window_size))
        # longer bf16 forwards (prefill): the same kernel over query chunks
        chunked = self.kernel_attention and not use_kernel
        pending = None
        for li, L in enumerate(self.layers):
            # verify-size bf16 forwards: the norms and the residual adds live in
            # the projections (vnx_gemm_bf16_norm / _residual) and in the MoD
            # routing / expert sum, so x is the up-to-date residual stream
            fused = (L.wqkv.wp is not None and L.proj.wp is not None and M <= _Linear.GEMM_MAX_M
                     and self.dtype == torch.bfloat16 and D <= 2048
                     and pending is None
                     and ("w1p" in L.ffn if L.kind == "mod" else
                          (L.ffn["gu"].wp is not None and L.ffn["gu"].swiglu and L.ffn["down"].wp is not None)))
            # the INT4 draft's decode: the same fusions on its GEMVs
            qfused = (not fused and L.kind == "trisparse" and L.wqkv.wq_rope is not None and L.proj.int4
                      and L.ffn["gu"].int4 and L.ffn["gu"].swiglu and L.ffn["down"].int4 and M <= 64
                      and pending is None)
            h = None
            qkv = None
            q = torch.empty((B, H, n, d), dtype=self.dtype, device=self.dev)
            kc, vc = self.kc[li], self.vc[li]
            rk = _lib.RopeKvArgs(P(lens.data_ptr()), n, H, Hkv, d, P(self.cos.data_ptr()), P(self.sin.data_ptr()),
                                 self.cos.shape[0], int(cfg.use_rope), P(q.data_ptr()), P(kc.data_ptr()),
                                 P(vc.data_ptr()), kc.stride(0), kc.stride(1), kc.stride(2), self.cap)
            done = False                                   # q and the cache rows written
            if li == 0 and qfused and self.embed_fold and L.wqkv.rope_kv_embed(
                    tok, self.emb, self.emb_scale, x, rk, L.norm1, cfg.eps):
                done = True                                # embedding, norm, q|k|v, RoPE, cache rows: one call
            elif li == 0 and fused and self.embed_fold and (qkv := L.wqkv.gemm_norm_embed(
                    tok, self.emb, self.emb_scale, x, L.norm1, cfg.eps)) is not None:
                pass                                       # embedding, norm and q|k|v: one call
            elif li == 0:
                h = torch.empty((M, D), dtype=self.act_dtype, device=self.dev)
                self._embed_rms(tok, L.norm1, x, h)        # token embedding folded into the first norm
            elif fused:
                qkv = L.wqkv.gemm_norm(x, L.norm1, cfg.eps)
            elif qfused:
                done = L.wqkv.rope_kv(x, rk, L.norm1, cfg.eps)
            else:
                h = torch.empty((M, D), dtype=self.act_dtype, device=self.dev)
                self._rms(x, pending, L.norm1, h)
                pending = None
            if not done and qkv is None:
                done = L.wqkv.rope_kv(h, rk)               # INT4: projection with RoPE + cache write fused
            attn_qkv = None
            if not done:
                if qkv is None:
                    qkv = L.wqkv(h)                                                  # (M, (H+2Hkv) d)
                if use_kernel and qkv.dtype == torch.bfloat16 and qkv.stride(1) == 1:
                    attn_qkv = qkv                         # RoPE + cache write inside the attention call
                    done = True
            if not done:
                _lib.check(L_.vnx_rope_kv(
                    P(qkv.data_ptr()), _lib.DTYPE_CODES[qkv.dtype], qkv.stride(0), B, n, H, Hkv, d,
                    P(lens.data_ptr()), P(self.cos.data_ptr()), P(self.sin.data_ptr()), self.cos.shape[0],
                    int(cfg.use_rope), P(q.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()),
                    _lib.DTYPE_CODES[self.dtype], kc.stride(0), kc.stride(1), kc.stride(2), self.cap, self._st()),
                    "rope_kv")
            if cache_only and attn_qkv is None and li == len(self.layers) - 1:
                return None                                # every layer's new cache rows are written
            if use_kernel:
                o = self._attn_kernel(q, li, lens, n, Tmax, qkv=attn_qkv)
            elif chunked:
                o = self._attn_kernel_chunked(q, li, lens, n, Tmax)
            else:
                o = self._attn_torch(q, li, lens, n, Tmax).permute(0, 2, 1, 3).reshape(M, H * d)
                o = o.to(self.act_dtype).contiguous()
            if fused and L.proj.gemm_residual(o, x):
                # x += proj(o); then the FFN of RMSNorm(x) * norm2, added into x
                if L.kind == "mod":
                    self._mod_fused(L, x)
                else:
                    act = L.ffn["gu"].gemm_norm(x, L.norm2, cfg.eps, epilogue=_lib.VNX_EPI_SWIGLU)
                    if act is None or not L.ffn["down"].gemm_residual(act, x):
                        raise RuntimeError("fused FFN path unavailable for this layer")
                continue
            if qfused and L.proj.gemv_residual(o, x):
                act = L.ffn["gu"].gemv_swiglu(x, L.norm2, cfg.eps)
                if act is None or not L.ffn["down"].gemv_residual(act, x):
                    raise RuntimeError("fused INT4 FFN path unavailable for this layer")
                continue
            a = L.proj(o)
            # MoD layers route on fp32 rows, as the reference does
            h2 = torch.empty((M, D), dtype=torch.float32 if L.kind == "mod" else self.act_dtype, device=self.dev)
            self._rms(x, a, L.norm2, h2)
            pending = self._ffn(L, h2)
        out = torch.empty((M, D), dtype=out_dtype, device=self.dev)
        self._rms(x, pending, self.norm, out)
        return out.view(B, n, D)

    def head_writes_bf16(self) -> bool:
        """Whether logits(out=<bf16 tensor>) is written by the head itself:
        the bf16 LM head (vnx_lm_head), or an INT4 head on its tiled copy
        (vnx_gemv_w4_tiles_out)."""
        if self.head is not None:
            return self.head.wt is not None if self.head.int4 else self.dtype == torch.bfloat16
        return self.dtype == torch.bfloat16

    def logits(self, hidden: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """(B, n, V) logits of the LM head (the tied embedding, or
        head.weight when untied), fp32 or in out's dtype (bf16 where
        head_writes_bf16()): vnx_lm_head (bf16, matrix cores) for the verify
        pass, vnx_gemv_w4 for an INT4 draft, F.linear for an fp32 model."""
        B, n, D = hidden.shape
        V = self.cfg.vocab_size
        h2 = hidden.reshape(B * n, D)
        if self.head is not None:
            if out is not None:
                self.head(h2, out=out.view(B * n, V))
                return out
            return self.head(h2).view(B, n, V)
        if self.dtype == torch.bfloat16 and D % 64 == 0 and B * n <= 256:
            if out is None:
                out = torch.empty((B, n, V), dtype=torch.float32, device=self.dev)
            self.hip.lm_head(h2.to(torch.bfloat16), self.head_w, out=out.view(B * n, V))
            return out
        y = torch.nn.functional.linear(h2.to(self.dtype), self.head_w).float()
        if out is not None:
            out.view(B * n, V).copy_(y)
            return out
        return y.view(B, n, V)

"""Weight-only INT8 / INT4 quantization for the draft model and the tied LM head.

Quantizers (weight preparation, run once at load time, in PyTorch on any
device) follow packages/verse_torch/verse_torch/quantize.py:
- `quantize_int8` (:187-214): per-output-channel for 2-D weights (per-tensor for
  1-D), scale = max|w| / 127 in fp32 (a zero max gives 1/127),
  q = round_half_even(w / scale).clip(-127, 127);
- `quantize_int4` (:231-258): the same with 7 and clip(-8, 7), then `pack_int4`
  (:36-68): byte j = (q[2j+1] & 0xF) << 4 | (q[2j] & 0xF);
- `quantize_int4_g`: the group-128 form with fp16 scales (a build extension for
  BASELINE config 4), s = fp16(max|w_g| / 7), q = clip(rint(w / fp32(s)), -8, 7).

`QuantizedLinear` mirrors the reference class (quantize.py:382-582): it holds
the packed weight and scales on the GPU and runs `forward` on the gfx950
dequant-GEMV kernels (vnx_gemv_w4 / vnx_gemv_w8), y = x @ W^T (+ bias).
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from .device import get_backend


def _div(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Elementwise a / b with b a tensor of a's shape, so PyTorch runs a true
    division (the correctly rounded fp32 quotient numpy computes); dividing by a
    Python number lets it multiply by the reciprocal on the GPU instead."""
    return torch.div(a, b.contiguous())


def _f32(w) -> torch.Tensor:
    if isinstance(w, np.ndarray):
        w = torch.from_numpy(np.ascontiguousarray(w))
    return w.to(torch.float32)


def quantize_int8(w):
    """(q int8, scale fp32): (out, 1) scales for 2-D w, a scalar for 1-D w."""
    w = _f32(w)
    if w.dim() == 1:
        max_abs = float(w.abs().max()) if w.numel() else 0.0
        if max_abs == 0.0:
            return torch.zeros_like(w, dtype=torch.int8), torch.tensor(1.0, dtype=torch.float32)
        scale = torch.tensor(np.float32(max_abs / 127.0), device=w.device)  # fp64 division, then fp32
        return torch.round(_div(w, scale.expand_as(w))).clamp(-127, 127).to(torch.int8), scale
    max_abs = w.abs().amax(dim=-1, keepdim=True)
    safe = torch.where(max_abs > 0, max_abs, torch.ones_like(max_abs))
    scale = _div(safe, torch.full_like(safe, 127.0))
    return torch.round(_div(w, scale.expand_as(w))).clamp(-127, 127).to(torch.int8), scale


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """int8 values in [-8, 7] -> uint8, two per byte, low nibble = even index."""
    q = q.to(torch.int8)
    one = q.dim() == 1
    if one:
        q = q[None]
    if q.shape[1] % 2:
        q = torch.cat([q, torch.zeros((q.shape[0], 1), dtype=torch.int8, device=q.device)], dim=1)
    lo = q[:, 0::2].to(torch.uint8) & 0x0F
    hi = q[:, 1::2].to(torch.uint8) & 0x0F
    out = (hi << 4) | lo
    return out[0] if one else out


def unpack_int4(packed: torch.Tensor, shape) -> torch.Tensor:
    p = packed.to(torch.uint8)
    if len(shape) == 1:
        p = p[None]
    lo = (p & 0x0F).to(torch.int16)
    hi = ((p >> 4) & 0x0F).to(torch.int16)
    lo = torch.where(lo >= 8, lo - 16, lo).to(torch.int8)
    hi = torch.where(hi >= 8, hi - 16, hi).to(torch.int8)
    out = torch.stack([lo, hi], dim=-1).reshape(p.shape[0], -1)[:, :shape[-1]]
    return out[0] if len(shape) == 1 else out


def quantize_int4(w):
    """(packed uint8 (out, ceil(in/2)), scale fp32 (out, 1)) per output channel."""
    w = _f32(w)
    if w.dim() == 1:
        max_abs = float(w.abs().max()) if w.numel() else 0.0
        if max_abs == 0.0:
            return pack_int4(torch.zeros_like(w, dtype=torch.int8)), torch.tensor(1.0, dtype=torch.float32)
        scale = torch.tensor(np.float32(max_abs / 7.0), device=w.device)
        return pack_int4(torch.round(_div(w, scale.expand_as(w))).clamp(-8, 7).to(torch.int8)), scale
    max_abs = w.abs().amax(dim=-1, keepdim=True)
    safe = torch.where(max_abs > 0, max_abs, torch.ones_like(max_abs))
    scale = _div(safe, torch.full_like(safe, 7.0))
    return pack_int4(torch.round(_div(w, scale.expand_as(w))).clamp(-8, 7).to(torch.int8)), scale


def quantize_int4_g(w, group: int = 128):
    """(packed uint8 (N, K/2), scales fp16 (N, K/group)) for a 2-D (N, K) weight."""
    w = _f32(w)
    N, K = w.shape
    if K % group:
        raise ValueError(f"K={K} is not a multiple of the group size {group}")
    wg = w.reshape(N, K // group, group)
    max_abs = wg.abs().amax(dim=-1)
    safe = torch.where(max_abs > 0, max_abs, torch.ones_like(max_abs))
    s16 = _div(safe, torch.full_like(safe, 7.0)).to(torch.float16)
    if bool((s16 == 0).any()):
        raise ValueError("a group scale underflows fp16")
    s32 = s16.to(torch.float32)[..., None].expand_as(wg)
    q = torch.round(_div(wg, s32)).clamp(-8, 7).to(torch.int8).reshape(N, K)
    return pack_int4(q), s16


class QuantizedLinear:
    """Weight-only quantized Linear on the GPU (quantize.py:382-582).

    qtype "int8": per-channel int8; "int4": per-channel int4 with fp32 scales
    (the reference's format); "int4_g128": group-128 int4 with fp16 scales.
    forward(x) takes (..., in) activations (cast to fp16, as the kernels read)
    and returns (..., out) fp32."""

    QTYPES = ("int8", "int4", "int4_g128")

    def __init__(self, weight, bias=None, qtype: str = "int4_g128", device: str = "rocm"):
        if qtype not in self.QTYPES:
            raise ValueError(f"qtype must be one of {self.QTYPES}, got {qtype!r}")
        self.backend = get_backend(device)
        dev = self.backend.torch_device
        w = _f32(weight).to(dev)
        if w.dim() != 2:
            raise ValueError("weight must be (out_features, in_features)")
        self.out_features, self.in_features = w.shape
        self.qtype = qtype
        if qtype == "int8":
            q, s = quantize_int8(w)
            self.wq, self.scale = q.contiguous(), s.reshape(-1).contiguous()
        elif qtype == "int4":
            q, s = quantize_int4(w)
            self.wq, self.scale = q.contiguous(), s.reshape(-1, 1).contiguous()
        else:
            q, s = quantize_int4_g(w, 128)
            self.wq, self.scale = q.contiguous(), s.contiguous()
        self.bias = None if bias is None else _f32(bias).to(dev)

    def dequantize(self) -> torch.Tensor:
        """The fp32 weight the kernels multiply by (bit-exact q * s)."""
        if self.qtype == "int8":
            return self.backend.dequant_w8(self.wq, self.scale)
        group = self.in_features if self.qtype == "int4" else 128
        return self.backend.dequant_w4(self.wq, self.scale, self.in_features, group)

    def forward(self, x) -> torch.Tensor:
        if self.qtype == "int8":
            y = self.backend.gemv_w8(x, self.wq, self.scale)
        else:
            group = self.in_features if self.qtype == "int4" else 128
            y = self.backend.gemv_w4(x, self.wq, self.scale, group)
        return y if self.bias is None else y + self.bias

    __call__ = forward


def weight_bytes(qtype: str, N: int, K: int) -> int:
    """Bytes a GEMV reads for the weight and its scales."""
    if qtype == "int8":
        return N * K + 4 * N
    if qtype == "int4":
        return N * K // 2 + 4 * N
    return N * K // 2 + 2 * N * (K // 128)


__all__ = ["quantize_int8", "quantize_int4", "quantize_int4_g", "pack_int4", "unpack_int4",
           "QuantizedLinear", "weight_bytes"]

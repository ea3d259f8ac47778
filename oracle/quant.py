"""Weight quantization oracles (test infrastructure only).

Restated in numpy from packages/verse_torch/verse_torch/quantize.py:
- `quantize_int8` (:187-214): per-output-channel (2-D) or per-tensor (1-D)
  scale = RN32(max|w| / 127) (a zero max gives scale 1/127),
  q = round_half_even(RN32(w / scale)).clip(-127, 127);
- `quantize_int4` (:231-258) the same with 7 and clip(-8, 7), packed by
  `pack_int4` (:36-68): byte j = (q[2j+1] & 0xF) << 4 | (q[2j] & 0xF), low
  nibble = even index, an odd length padded with 0;
- `unpack_int4` (:71-99), `dequantize_int8` (:216-224) q * scale,
  `dequantize_int4` (:261-274), `matmul_int4` (:277-309) (x @ q.T) * scale.
Build extension (no reference counterpart):
- `quantize_int4_g` symmetric per group of G input columns with fp16 scales,
  s = fp16(RN32(max|w_g| / 7)), q = clip(round_half_even(RN32(w / fp32(s))), -8, 7),
  packed as above; `dequantize_int4_g` = q * fp32(s), exact in fp32 (a 4-bit
  integer times an 11-bit significand).

Pinned (tests/test_oracle_quant.py) by hand-computed vectors of the docstring
rules (nibble order, two's-complement nibbles, round-half-to-even), the
reference's own consistency check (fused == dequantize-then-matmul,
tests/test_compress_v13.py:291-304) and its error-ratio threshold
(tests/benchmark_quantize.py:133-135, INT4 <= 0.05).
"""
from __future__ import annotations

import numpy as np


def quantize_int8(w):
    w = np.asarray(w, dtype=np.float32)
    if w.ndim == 1:
        max_abs = float(np.max(np.abs(w))) if w.size else 0.0
        if max_abs == 0.0:
            return np.zeros_like(w, dtype=np.int8), np.float32(1.0)
        scale = np.float32(max_abs / 127.0)  # Python (fp64) division, then fp32 (quantize.py:205)
        return np.round(w / scale).clip(-127, 127).astype(np.int8), scale
    max_abs = np.max(np.abs(w), axis=-1, keepdims=True)
    safe = np.where(max_abs > 0, max_abs, np.float32(1.0)).astype(np.float32)
    scale = (safe / 127.0).astype(np.float32)  # fp32 array / weak Python float: fp32 division
    return np.round(w / scale).clip(-127, 127).astype(np.int8), scale


def pack_int4(q):
    q = np.asarray(q, dtype=np.int8)
    if q.ndim == 1:
        q = q[None, :]
        one = True
    else:
        one = False
    rows, cols = q.shape
    if cols % 2:
        q = np.concatenate([q, np.zeros((rows, 1), np.int8)], axis=1)
    low = q[:, 0::2].astype(np.uint8) & 0x0F
    high = q[:, 1::2].astype(np.uint8) & 0x0F
    out = (high << 4) | low
    return out[0] if one else out


def unpack_int4(packed, shape):
    packed = np.asarray(packed, dtype=np.uint8)
    if len(shape) == 1:
        packed = packed[None, :]
        n = int(shape[0])
        rows = 1
    else:
        rows, n = int(shape[0]), int(shape[1])
    low = (packed & 0x0F).astype(np.int16)
    high = ((packed >> 4) & 0x0F).astype(np.int16)
    low = np.where(low >= 8, low - 16, low).astype(np.int8)
    high = np.where(high >= 8, high - 16, high).astype(np.int8)
    out = np.empty((rows, packed.shape[1] * 2), np.int8)
    out[:, 0::2] = low
    out[:, 1::2] = high
    out = out[:, :n]
    return out[0] if len(shape) == 1 else out


def quantize_int4(w):
    w = np.asarray(w, dtype=np.float32)
    if w.ndim == 1:
        max_abs = float(np.max(np.abs(w))) if w.size else 0.0
        if max_abs == 0.0:
            return pack_int4(np.zeros_like(w, dtype=np.int8)), np.float32(1.0)
        scale = np.float32(max_abs / 7.0)  # Python (fp64) division, then fp32 (quantize.py:251)
        return pack_int4(np.round(w / scale).clip(-8, 7).astype(np.int8)), scale
    max_abs = np.max(np.abs(w), axis=-1, keepdims=True)
    safe = np.where(max_abs > 0, max_abs, np.float32(1.0)).astype(np.float32)
    scale = (safe / 7.0).astype(np.float32)
    return pack_int4(np.round(w / scale).clip(-8, 7).astype(np.int8)), scale


def dequantize_int8(q, scale):
    return np.asarray(q).astype(np.float32) * scale


def dequantize_int4(packed, scale, shape):
    return unpack_int4(packed, shape).astype(np.float32) * scale


def matmul_int4(x, packed, scale, shape):
    q = unpack_int4(packed, shape).astype(np.float32)
    x2 = np.asarray(x, dtype=np.float32).reshape(-1, shape[1])
    out = x2 @ q.T
    out *= np.asarray(scale, np.float32).reshape(-1)
    return out.reshape(*np.shape(x)[:-1], shape[0])


def quantize_int4_g(w, group: int = 128):
    """(N, K) fp32 -> (packed (N, K/2) uint8, scales (N, K/group) fp16)."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    if K % group:
        raise ValueError(f"K={K} is not a multiple of the group size {group}")
    wg = w.reshape(N, K // group, group)
    max_abs = np.max(np.abs(wg), axis=-1)
    safe = np.where(max_abs > 0, max_abs, np.float32(1.0)).astype(np.float32)
    s16 = (safe / np.float32(7.0)).astype(np.float32).astype(np.float16)
    if np.any(s16 == 0):
        raise ValueError("a group scale underflows fp16")
    s32 = s16.astype(np.float32)[..., None]
    q = np.round(wg / s32).clip(-8, 7).astype(np.int8).reshape(N, K)
    return pack_int4(q), s16


def dequantize_int4_g(packed, scales16, shape, group: int = 128):
    N, K = shape
    q = unpack_int4(packed, shape).astype(np.float32).reshape(N, K // group, group)
    return (q * np.asarray(scales16, np.float16).astype(np.float32)[..., None]).reshape(N, K)


def gemv_ref(x, w_deq):
    """y = x @ w_deq.T in fp64 (the exact value the kernels approximate in fp32)."""
    return np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64).T


def gemv_abs(x, w_deq):
    """sum_k |x_k * w_k| per output, the scale of the fp32 rounding error."""
    return np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(w_deq, np.float64)).T

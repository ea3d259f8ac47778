"""ctypes binding of libvnx_hip.so (the C ABI declared in include/vnx.h).

The library is loaded from this package directory only.  There is no
fallback: if the library is missing or cannot be loaded, every GPU entry point
raises RuntimeError naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import threading

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libvnx_hip.so")

VNX_OK = 0
VNX_ERR_INVALID_ARG = -1
VNX_ERR_WORKSPACE = -2
VNX_ERR_UNSUPPORTED = -3
VNX_ERR_HIP = -4
VNX_ERR_NO_DEVICE = -5
VNX_ERR_TOO_LARGE = -6

VNX_EPI_NONE, VNX_EPI_SWIGLU = 0, 1
VNX_F32 = 0
VNX_BF16 = 1
VNX_F16 = 2

try:
    import torch as _torch
    DTYPE_CODES = {_torch.float32: VNX_F32, _torch.bfloat16: VNX_BF16, _torch.float16: VNX_F16}
except Exception:  # the CPU-only ABI tests do not need torch dtypes
    DTYPE_CODES = {}

FLAG_NEAR_TIE = 1
FLAG_LSE_EDGE = 2
FLAG_CDF_EDGE = 4
FLAG_ZERO_RESIDUAL = 8
FLAG_BAD_ID = 16

SAMPLE_EXACT_K = 1
SAMPLE_CALIBRATE = 2
SAMPLE_UNIFORM_F64 = 4

_c_i64 = ctypes.c_int64
_c_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/vnx.h
SIGNATURES = {
    "vnx_version": (_int, []),
    "vnx_status_string": (ctypes.c_char_p, [_int]),
    "vnx_last_hip_error": (ctypes.c_char_p, []),
    "vnx_init": (_int, [_int]),
    "vnx_profile_begin": (_int, [_int]),
    "vnx_profile_end": (_int, [_vp, _int, _vp]),
    "vnx_row_lse_workspace": (_c_sz, [_c_i64, _c_i64]),
    "vnx_row_lse": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _f32, _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "vnx_row_argmax": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_sz, _vp]),
    "vnx_softmax_workspace": (_c_sz, [_c_i64, _c_i64]),
    "vnx_softmax": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _f32, _vp, _vp, _c_i64, _vp, _c_sz, _vp]),
    "vnx_spec_accept_workspace": (_c_sz, [_c_i64, _int, _c_i64]),
    "vnx_spec_accept": (_int, [_vp, _vp, _int, _c_i64, _int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                               _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "vnx_spec_accept_draft_lse": (_int, [_vp, _vp, _int, _c_i64, _int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _vp, _vp, _f32, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "vnx_sampler_workspace": (_c_sz, [_c_i64, _c_i64, _int]),
    "vnx_sampler_sample": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _f32, _c_i64, _f32, _int, _f32, _f32,
                                  _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "vnx_logit_calibrate": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _f32, _f32, _vp, _c_i64, _vp, _vp]),
    "vnx_spec_accept_noalloc_max_bytes": (_c_sz, []),
    "vnx_spec_accept_noalloc": (_int, [_vp, _vp, _int, _c_i64, _int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vnx_gemv_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "vnx_quantize_w4_g": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _int, _vp, _c_i64, _vp, _c_i64, _vp, _vp]),
    "vnx_gemv_w4": (_int, [_vp, _c_i64, _vp, _c_i64, _vp, _int, _c_i64, _c_i64, _c_i64, _c_i64, _int,
                           _vp, _c_i64, _vp, _c_sz, _vp]),
    "vnx_w4_tiles_bytes": (_c_sz, [_c_i64, _c_i64]),
    "vnx_pack_w4_tiles": (_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp]),
    "vnx_gemv_w4_tiles": (_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp]),
    "vnx_gemv_w4_tiles_out": (_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _int, _c_i64, _vp]),
    "vnx_gemv_w4_swiglu": (_int, [_vp, _c_i64, _vp, _f32, _vp, _c_i64, _vp, _int, _c_i64, _c_i64, _c_i64, _c_i64,
                                  _int, _vp, _c_i64, _vp]),
    "vnx_gemv_w4_residual": (_int, [_vp, _c_i64, _vp, _c_i64, _vp, _int, _c_i64, _c_i64, _c_i64, _c_i64, _int,
                                    _vp, _c_i64, _vp]),
    "vnx_gemv_w8": (_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64,
                           _vp, _c_sz, _vp]),
    "vnx_dequant_w4": (_int, [_vp, _c_i64, _vp, _int, _c_i64, _c_i64, _c_i64, _int, _vp, _c_i64, _vp]),
    "vnx_dequant_w8": (_int, [_vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp]),
    "vnx_sample_workspace": (_c_sz, [_c_i64, _c_i64]),
    "vnx_sample": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "vnx_greedy_verify_workspace": (_c_sz, [_c_i64, _int, _c_i64]),
    "vnx_greedy_verify": (_int, [_vp, _int, _c_i64, _int, _int, _c_i64, _c_i64, _c_i64, _vp,
                                 _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
}



class TreeAttnArgs(ctypes.Structure):
    """vnx_tree_attn_args (include/vnx.h)."""
    _fields_ = [
        ("q", _vp), ("q_strides", _c_i64 * 3),
        ("k_cache", _vp), ("v_cache", _vp), ("cache_strides", _c_i64 * 3),
        ("k_tree", _vp), ("v_tree", _vp), ("tree_strides", _c_i64 * 3),
        ("anc", _vp), ("anc_batch_stride", _c_i64),
        ("out", _vp), ("out_dtype", _int), ("out_strides", _c_i64 * 3),
        ("B", _int), ("H", _int), ("Hkv", _int), ("Tp", _int), ("N", _int), ("d", _int),
        ("scale", _f32), ("tp_batch", _vp), ("tree_follows_prefix", _int),
        ("k_seg2", _vp), ("v_seg2", _vp), ("seg2_strides", _c_i64 * 3), ("T2", _int), ("gates", _vp),
        ("qkv", _vp), ("qkv_ld", _c_i64), ("cos_table", _vp), ("sin_table", _vp), ("table_rows", _c_i64),
        ("rope", _int), ("cap", _c_i64),
        ("window", _int), ("alibi_slopes", _vp), ("alibi_max_keys", _int),
        ("force_splits", _int), ("force_waves", _int), ("f32_rows", _int),
    ]


class RopeKvArgs(ctypes.Structure):
    """vnx_rope_kv_args (include/vnx.h)."""
    _fields_ = [
        ("lens", _vp), ("n", _int), ("H", _int), ("Hkv", _int), ("d", _int),
        ("cos_table", _vp), ("sin_table", _vp), ("table_rows", _c_i64), ("rope", _int),
        ("q_out", _vp), ("k_cache", _vp), ("v_cache", _vp),
        ("c_sb", _c_i64), ("c_sh", _c_i64), ("c_sr", _c_i64), ("cap", _c_i64),
    ]


SIGNATURES.update({
    "vnx_gemv_w4_rope_kv": (_int, [_vp, _c_i64, _vp, _f32, _vp, _c_i64, _vp, _int, _c_i64, _c_i64, _c_i64, _c_i64,
                                   _int, ctypes.POINTER(RopeKvArgs), _vp]),
    "vnx_gemv_w4_rope_kv_embed": (_int, [_vp, _vp, _int, _c_i64, _c_i64, _f32, _vp, _c_i64, _vp, _f32, _vp, _c_i64,
                                         _vp, _int, _c_i64, _c_i64, _c_i64, _c_i64, _int, ctypes.POINTER(RopeKvArgs),
                                         _vp]),
    "vnx_tree_attn_workspace": (_c_sz, [_int, _int, _int, _int, _int, _int]),
    "vnx_tree_attn_workspace_args": (_c_sz, [ctypes.POINTER(TreeAttnArgs)]),
    "vnx_tree_attn": (_int, [ctypes.POINTER(TreeAttnArgs), _vp, _c_sz, _vp]),
    "vnx_tree_attn_plan": (_int, [_int, _int, _int, _int, _int, _int, _vp, _vp, _vp]),
    "vnx_tree_greedy_workspace": (_c_sz, [_c_i64, _int, _c_i64]),
    "vnx_tree_greedy": (_int, [_vp, _int, _c_i64, _int, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp,
                               _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "vnx_row_topk_workspace": (_c_sz, [_c_i64, _c_i64, _int]),
    "vnx_row_topk": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _int, _vp, _vp, _c_i64, _vp, _c_sz, _vp]),
    "vnx_lm_head": (_int, [_vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _int, _c_i64, _vp]),
    "vnx_rmsnorm": (_int, [_vp, _c_i64, _vp, _int, _c_i64, _vp, _f32, _c_i64, _c_i64, _vp, _c_i64, _vp, _int,
                           _c_i64, _vp]),
    "vnx_rope_kv": (_int, [_vp, _int, _c_i64, _c_i64, _int, _int, _int, _int, _vp, _vp, _vp, _c_i64, _int,
                           _vp, _vp, _vp, _int, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
    "vnx_embed_rmsnorm": (_int, [_vp, _vp, _int, _c_i64, _c_i64, _f32, _vp, _f32, _c_i64, _c_i64, _vp, _c_i64,
                                 _vp, _int, _c_i64, _vp]),
    "vnx_swiglu": (_int, [_vp, _int, _c_i64, _c_i64, _c_i64, _vp, _int, _c_i64, _vp]),
    "vnx_axpby": (_int, [_vp, _vp, _vp, _c_i64, _vp, _int, _vp]),
    "vnx_spec_commit": (_int, [_vp, _vp, _c_i64, _int, _int, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vnx_pack_bf16_size": (_c_sz, [_c_i64, _c_i64]),
    "vnx_pack_bf16": (_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp]),
    "vnx_gemm_bf16": (_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _int, _int, _vp,
                             _c_i64, _vp, _int, _c_i64, _c_i64, _vp]),
    "vnx_mod_route_x": (_int, [_vp, _c_i64, _vp, _f32, _vp, _c_i64, _c_i64, _c_i64, _int, _int, _int, _vp, _c_i64,
                               _vp, _c_i64, _c_i64, _int, _vp]),
    "vnx_gemm_bf16_norm": (_int, [_vp, _c_i64, _vp, _f32, _vp, _c_i64, _c_i64, _c_i64, _int, _vp, _c_i64, _vp]),
    "vnx_gemm_bf16_norm_embed": (_int, [_vp, _vp, _int, _c_i64, _c_i64, _f32, _vp, _c_i64, _vp, _f32, _vp, _c_i64,
                                        _c_i64, _c_i64, _vp, _c_i64, _vp]),
    "vnx_gemm_bf16_residual": (_int, [_vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp]),
    "vnx_mod_route": (_int, [_vp, _c_i64, _c_i64, _int, _int, _int, _vp, _c_i64, _vp]),
    "vnx_mod_swiglu": (_int, [_vp, _int, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _int, _c_i64, _vp, _int, _c_i64,
                              _c_i64, _vp]),
    "vnx_sum_experts": (_int, [_vp, _int, _c_i64, _int, _c_i64, _vp, _vp]),
    "vnx_sum_expert_rows": (_int, [_vp, _int, _c_i64, _c_i64, _vp, _c_i64, _int, _c_i64, _vp, _c_i64, _int, _vp]),
    "vnx_expert_gemm_bf16": (_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _int, _int, _vp,
                                    _c_i64, _int, _vp, _vp, _vp, _vp, _int, _c_i64, _c_i64, _vp]),
})

_lib = None
_lock = threading.Lock()


class VnxError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Loads libvnx_hip.so (raises RuntimeError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"vnx HIP library not found at {LIB_PATH}; build it with "
                    "`python -m versenext_amd.build` (hipcc, gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def check(status: int, what: str = "vnx call") -> None:
    """Maps a vnx_status to the reference's error conventions
    (ValueError for arguments, RuntimeError for the device; speculative.py:188-196,
    device.py:371-378)."""
    if status == VNX_OK:
        return
    L = lib()
    text = L.vnx_status_string(status).decode()
    if status in (VNX_ERR_INVALID_ARG, VNX_ERR_WORKSPACE, VNX_ERR_UNSUPPORTED, VNX_ERR_TOO_LARGE):
        raise ValueError(f"{what}: {text} (status {status})")
    if status == VNX_ERR_HIP:
        raise VnxError(f"{what}: {text}: {L.vnx_last_hip_error().decode()}")
    raise VnxError(f"{what}: {text} (status {status})")

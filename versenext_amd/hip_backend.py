"""HipBackend: the "rocm" DeviceBackend, backed by libvnx_hip.so (gfx950 kernels).

Interface parity with packages/verse_torch/verse_torch/backend_torch.py:246-379
(`TorchBackend`): same constructor argument, `device_type` keeps the caller's
prefix ("rocm" for "rocm:0"), `torch_device`, `from_numpy`, `to_numpy`, and
the DeviceBackend operators.  Operators on the speculative-verification path
(`softmax`, `row_lse`, `argmax`, `spec_accept`, `greedy_verify`) run the
hand-written kernels; `matmul` / `linear` use PyTorch's rocBLAS GEMM and
`layernorm` / `rmsnorm` / `rope` PyTorch elementwise ops (not on the hot path).

Tensors: inputs may be torch tensors (any device; moved to this one) or
numpy arrays; outputs are torch tensors on this device.  Kernels run on the
current PyTorch stream of the device.  Each (device, stream) pair owns one
zero-initialised workspace that the kernels leave zeroed after every call.
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from . import _lib
from .device import DeviceBackend, _device_index, _parse_device, _to_torch_device_str


def _to_tensor(x, device, dtype=None) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        t = x
    elif isinstance(x, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(x))
    elif hasattr(x, "data") and not isinstance(x, (list, tuple)):
        return _to_tensor(x.data, device, dtype)  # verse_torch.Tensor-like objects
    else:
        t = torch.as_tensor(x)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    if t.device != device:
        t = t.to(device)
    return t


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


_LOGIT_DTYPES = {torch.float32: _lib.VNX_F32, torch.bfloat16: _lib.VNX_BF16}


class HipBackend(DeviceBackend):
    def __init__(self, device: str = "rocm"):
        self._device_str = str(device).lower()
        if _parse_device(self._device_str) not in ("rocm", "cuda"):
            raise RuntimeError(f"HipBackend serves rocm/cuda devices, got {device!r}")
        if not torch.cuda.is_available():
            raise RuntimeError(f"no ROCm GPU visible; device '{device}' is unavailable")
        idx = _device_index(self._device_str)
        self._torch_device = torch.device(_to_torch_device_str(self._device_str if ":" in self._device_str
                                                               else self._device_str + f":{idx}"))
        self._index = idx
        L = _lib.lib()
        with torch.cuda.device(idx):
            _lib.check(L.vnx_init(idx), "vnx_init")
        self._L = L
        self._ws = {}
        self._ws_lock = threading.Lock()

    # ---- identity -------------------------------------------------------
    @property
    def device_type(self) -> str:
        return self._device_str.split(":")[0]

    @property
    def torch_device(self):
        return self._torch_device

    @property
    def torch_device_str(self) -> str:
        return self._device_str

    def from_numpy(self, x):
        return _to_tensor(x, self._torch_device)

    def to_numpy(self, t):
        return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)

    # ---- plumbing -------------------------------------------------------
    def _stream(self):
        return torch.cuda.current_stream(self._torch_device)

    def _workspace(self, nbytes: int) -> torch.Tensor:
        """Zeroed scratch for the current stream, grown on demand."""
        st = self._stream().cuda_stream
        with self._ws_lock:
            buf = self._ws.get(st)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=self._torch_device)
                self._ws[st] = buf
            return buf

    def _logits(self, x) -> torch.Tensor:
        t = _to_tensor(x, self._torch_device)
        if t.dtype not in _LOGIT_DTYPES:
            t = t.to(torch.float32)
        return t

    @staticmethod
    def _vec_ok(t: torch.Tensor) -> bool:
        ve = 4 if t.dtype == torch.float32 else 8
        if t.stride(-1) != 1 or t.data_ptr() % 16:
            return False
        return all(s % ve == 0 for s in t.stride()[:-1])

    def _rows2d(self, x):
        """(..., V) logits -> (rows, V) view with 16-byte aligned rows."""
        t = self._logits(x)
        V = t.shape[-1]
        t2 = t.reshape(-1, V) if t.dim() != 2 else t
        if not self._vec_ok(t2) or (t2.shape[0] > 1 and t2.stride(0) < V):
            t2 = t2.contiguous()
            if not self._vec_ok(t2):  # V not a multiple of the vector width: pad rows
                ve = 4 if t2.dtype == torch.float32 else 8
                ld = (V + ve - 1) // ve * ve
                padded = torch.empty((t2.shape[0], ld), dtype=t2.dtype, device=t2.device)
                padded[:, :V] = t2
                t2 = padded[:, :V]
        return t2

    def _rows3d(self, x, nrows: int):
        """(B, nrows, V) view usable with (ld, sb) strides."""
        t = self._logits(x)
        if t.dim() != 3 or t.shape[1] != nrows:
            raise ValueError(f"expected logits of shape (B, {nrows}, V), got {tuple(t.shape)}")
        V = t.shape[-1]
        ok = self._vec_ok(t) and t.stride(1) >= V and t.stride(0) >= (nrows - 1) * t.stride(1) + V
        if not ok:
            t = t.contiguous()
            if not self._vec_ok(t):
                ve = 4 if t.dtype == torch.float32 else 8
                ld = (V + ve - 1) // ve * ve
                padded = torch.empty((t.shape[0], nrows, ld), dtype=t.dtype, device=t.device)
                padded[..., :V] = t
                t = padded[..., :V]
        return t

    # ---- DeviceBackend operators -------------------------------------------
    def matmul(self, a, b):
        return torch.matmul(_to_tensor(a, self._torch_device), _to_tensor(b, self._torch_device))

    def linear(self, x, weight, bias=None):
        x = _to_tensor(x, self._torch_device)
        w = _to_tensor(weight, self._torch_device, x.dtype)
        bb = None if bias is None else _to_tensor(bias, self._torch_device, x.dtype)
        return torch.nn.functional.linear(x, w, bb)

    def softmax(self, x, dim: int = -1, temperature: float = 1.0, thresholds=None):
        t = self._logits(x)
        moved = dim not in (-1, t.dim() - 1)
        if moved:
            t = t.movedim(dim, -1)
        shape = t.shape
        x2 = self._rows2d(t)
        R, V = x2.shape
        out = torch.empty((R, V), dtype=torch.float32, device=self._torch_device)
        thr = None if thresholds is None else _to_tensor(thresholds, self._torch_device, torch.float32).contiguous()
        ws = self._workspace(self._L.vnx_softmax_workspace(R, V))
        _lib.check(self._L.vnx_softmax(_ptr(x2), _LOGIT_DTYPES[x2.dtype], R, V, x2.stride(0), float(temperature),
                                       _ptr(thr), _ptr(out), V, _ptr(ws), ws.numel(),
                                       ctypes.c_void_p(self._stream().cuda_stream)), "softmax")
        out = out.reshape(shape)
        return out.movedim(-1, dim) if moved else out

    def layernorm(self, x, weight, bias, eps: float = 1e-5):
        x = _to_tensor(x, self._torch_device)
        w = _to_tensor(weight, self._torch_device, x.dtype)
        bb = _to_tensor(bias, self._torch_device, x.dtype)
        return torch.nn.functional.layer_norm(x, tuple(w.shape), w, bb, eps)

    def rmsnorm(self, x, weight, eps: float = 1e-6):
        x = _to_tensor(x, self._torch_device)
        w = _to_tensor(weight, self._torch_device, x.dtype)
        return x / torch.sqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w

    def rope(self, x, cos=None, sin=None):
        if cos is None or sin is None:
            return x
        x = _to_tensor(x, self._torch_device)
        cos = _to_tensor(cos, self._torch_device, x.dtype)
        sin = _to_tensor(sin, self._torch_device, x.dtype)
        d = x.shape[-1]
        half = d // 2
        x1, x2 = x[..., :half], x[..., half:]
        cos_b = cos[..., :half] if cos.shape[-1] >= d else cos
        sin_b = sin[..., :half] if sin.shape[-1] >= d else sin
        return torch.cat([x1 * cos_b - x2 * sin_b, x1 * sin_b + x2 * cos_b], dim=-1)

    # ---- verification operators -------------------------------------------
    def row_lse(self, x, temperature: float = 1.0, thresholds=None, want_max: bool = False,
                want_argmax: bool = False):
        """Per-row log-sum-exp of RN(x / T) in fp64 (+ optional fp32 max, int64 raw argmax)."""
        x2 = self._rows2d(x)
        R, V = x2.shape
        dev = self._torch_device
        lse = torch.empty(R, dtype=torch.float64, device=dev)
        mx = torch.empty(R, dtype=torch.float32, device=dev) if want_max else None
        am = torch.empty(R, dtype=torch.int64, device=dev) if want_argmax else None
        thr = None if thresholds is None else _to_tensor(thresholds, dev, torch.float32).contiguous()
        ws = self._workspace(self._L.vnx_row_lse_workspace(R, V))
        _lib.check(self._L.vnx_row_lse(_ptr(x2), _LOGIT_DTYPES[x2.dtype], R, V, x2.stride(0), float(temperature),
                                       _ptr(thr), _ptr(lse), _ptr(mx), _ptr(am), _ptr(ws), ws.numel(),
                                       ctypes.c_void_p(self._stream().cuda_stream)), "row_lse")
        return lse, mx, am

    def argmax(self, x) -> torch.Tensor:
        """numpy.argmax over the last axis (first maximal index)."""
        t = self._logits(x)
        lead = t.shape[:-1]
        x2 = self._rows2d(t)
        R, V = x2.shape
        am = torch.empty(R, dtype=torch.int64, device=self._torch_device)
        ws = self._workspace(self._L.vnx_row_lse_workspace(R, V))
        _lib.check(self._L.vnx_row_argmax(_ptr(x2), _LOGIT_DTYPES[x2.dtype], R, V, x2.stride(0), _ptr(am),
                                          _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)),
                   "argmax")
        return am.reshape(lead)

    def spec_accept(self, target, draft, draft_ids, uniforms, temperature: float = 1.0,
                    thr_t=None, thr_d=None, lse_d_in=None, flags_d_in=None):
        """Stochastic acceptance (see vnx_spec_accept in include/vnx.h).
        target (B,k+1,V), draft (B,k,V) fp32/bf16; draft_ids (B,k); uniforms (B,k+1).
        lse_d_in (k, B) fp32 with flags_d_in (k, B) uint8: the draft rows'
        LSEs and flags as the draws produced them (vnx_spec_accept_draft_lse:
        the draft rows are then read only at the draft ids; no thresholds).
        Returns dict of device tensors: accept_len (B,) int32, out_ids (B,k+1)
        int64, flags (B,k+1) uint8, lse_t (B,k+1) f32, lse_d (B,k) f32."""
        dev = self._torch_device
        ids = _to_tensor(draft_ids, dev, torch.int64).contiguous()
        if ids.dim() != 2:
            raise ValueError("draft_ids must be (B, k)")
        B, k = ids.shape
        tg = self._rows3d(target, k + 1)
        df = self._rows3d(draft, k)
        if df.dtype != tg.dtype:
            df = df.to(tg.dtype)
        if tg.shape[0] != B or df.shape[0] != B or tg.shape[2] != df.shape[2]:
            raise ValueError("target / draft / draft_ids shapes disagree")
        V = tg.shape[2]
        u = _to_tensor(uniforms, dev, torch.float32).contiguous()
        if tuple(u.shape) != (B, k + 1):
            raise ValueError(f"uniforms must be (B, k+1) = ({B}, {k + 1})")
        tt = None if thr_t is None else _to_tensor(thr_t, dev, torch.float32).contiguous()
        td = None if thr_d is None else _to_tensor(thr_d, dev, torch.float32).contiguous()
        alen = torch.empty(B, dtype=torch.int32, device=dev)
        out = torch.empty((B, k + 1), dtype=torch.int64, device=dev)
        flags = torch.empty((B, k + 1), dtype=torch.uint8, device=dev)
        lse_t = torch.empty((B, k + 1), dtype=torch.float32, device=dev)
        lse_d = torch.empty((B, k), dtype=torch.float32, device=dev)
        ws = self._workspace(self._L.vnx_spec_accept_workspace(B, k, V))
        if lse_d_in is not None:
            if tt is not None or td is not None:
                raise ValueError("draft LSEs from the draws exclude per-row thresholds")
            ld = _to_tensor(lse_d_in, dev, torch.float32)
            if tuple(ld.shape) != (k, B) or ld.stride(1) != 1:
                raise ValueError(f"lse_d_in must be (k, B) = ({k}, {B}) with unit column stride")
            fd = None
            if flags_d_in is not None:
                fd = _to_tensor(flags_d_in, dev, torch.uint8)
                if tuple(fd.shape) != (k, B) or fd.stride(1) != 1 or fd.stride(0) != ld.stride(0):
                    raise ValueError("flags_d_in must match lse_d_in's layout")
            _lib.check(self._L.vnx_spec_accept_draft_lse(
                _ptr(tg), _ptr(df), _LOGIT_DTYPES[tg.dtype], B, k, V,
                tg.stride(1), tg.stride(0), df.stride(1), df.stride(0),
                _ptr(ids), _ptr(u), float(temperature), _ptr(ld), _ptr(fd), ld.stride(0),
                _ptr(alen), _ptr(out), _ptr(flags), _ptr(lse_t),
                _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)), "spec_accept_draft_lse")
            return dict(accept_len=alen, out_ids=out, flags=flags, lse_t=lse_t, lse_d=ld.t())
        _lib.check(self._L.vnx_spec_accept(
            _ptr(tg), _ptr(df), _LOGIT_DTYPES[tg.dtype], B, k, V,
            tg.stride(1), tg.stride(0), df.stride(1), df.stride(0),
            _ptr(ids), _ptr(u), float(temperature), _ptr(tt), _ptr(td),
            _ptr(alen), _ptr(out), _ptr(flags), _ptr(lse_t), _ptr(lse_d),
            _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)), "spec_accept")
        return dict(accept_len=alen, out_ids=out, flags=flags, lse_t=lse_t, lse_d=lse_d)

    def sample(self, logits, uniforms, temperature: float = 1.0, thresholds=None, out=None,
               return_all: bool = False, lse_out=None, flags_out=None):
        """Inverse-CDF draw per row from softmax(logits / T) with the given
        uniforms (vnx_sample).  logits (B, V) (strided rows allowed);
        returns ids (B,) int64 (written into `out` when given), or with
        return_all a dict with ids, flags and the fp32 row LSEs.  lse_out /
        flags_out: (B,) contiguous tensors the row LSEs and flags are written
        into (for vnx_spec_accept_draft_lse)."""
        dev = self._torch_device
        lg = self._rows2d(logits)
        B, V = lg.shape
        u = _to_tensor(uniforms, dev, torch.float32).reshape(-1).contiguous()
        if u.numel() != B:
            raise ValueError(f"uniforms must have {B} entries")
        thr = None if thresholds is None else _to_tensor(thresholds, dev, torch.float32).contiguous()
        ids = out if out is not None else torch.empty(B, dtype=torch.int64, device=dev)
        flags = flags_out if flags_out is not None else (
            torch.empty(B, dtype=torch.uint8, device=dev) if return_all else None)
        lse = lse_out if lse_out is not None else (
            torch.empty(B, dtype=torch.float32, device=dev) if return_all else None)
        for t_, dt_ in ((flags, torch.uint8), (lse, torch.float32)):
            if t_ is not None and (t_.dtype != dt_ or t_.numel() != B or not t_.is_contiguous()):
                raise ValueError("lse_out / flags_out must be contiguous (B,) float32 / uint8 tensors")
        ws = self._workspace(self._L.vnx_sample_workspace(B, V))
        _lib.check(self._L.vnx_sample(
            _ptr(lg), _LOGIT_DTYPES[lg.dtype], B, V, lg.stride(0), _ptr(u), float(temperature), _ptr(thr),
            _ptr(ids), _ptr(flags), _ptr(lse), _ptr(ws), ws.numel(),
            ctypes.c_void_p(self._stream().cuda_stream)), "sample")
        if return_all:
            return dict(ids=ids, flags=flags, lse=lse)
        return ids

    def sampler_sample(self, logits, uniforms, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0,
                       return_all: bool = False, exact_k: bool = False, calib_factor=None, calib_eps: float = 1e-8):
        """Sampler.sample for every row of logits (B, V) (vnx_sampler_sample):
        temperature / top_k / top_p with the reference's semantics, one host
        uniform per row in place of the RNG.  exact_k takes CometSpark's
        exactly-k top-k (argpartition, ties by lower id); calib_factor (not
        None) first applies its logit calibration with eps calib_eps.  Returns
        ids (B,) int64, or with return_all a dict with ids, flags, lse, kth,
        p_star, j_star, k_star.  Float64 uniforms (numpy's Generator.random
        values) are used as drawn (VNX_SAMPLE_UNIFORM_F64); others as float32."""
        if temperature < 0.0:
            raise ValueError(f"temperature must be >= 0, got {temperature}")
        if top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {top_k}")
        if not 0.0 < top_p <= 1.0:
            raise ValueError(f"top_p must be in (0, 1], got {top_p}")
        mode = (_lib.SAMPLE_EXACT_K if exact_k else 0) | (_lib.SAMPLE_CALIBRATE if calib_factor is not None else 0)
        dev = self._torch_device
        lg = self._rows2d(logits)
        B, V = lg.shape
        u64 = getattr(uniforms, "dtype", None) in (np.float64, torch.float64)
        if u64:
            mode |= _lib.SAMPLE_UNIFORM_F64
        u = _to_tensor(uniforms, dev, torch.float64 if u64 else torch.float32).reshape(-1).contiguous()
        if u.numel() != B:
            raise ValueError(f"uniforms must have {B} entries")
        ids = torch.empty(B, dtype=torch.int64, device=dev)
        extra = None
        if return_all:
            extra = dict(flags=torch.empty(B, dtype=torch.uint8, device=dev),
                         lse=torch.empty(B, dtype=torch.float32, device=dev),
                         kth=torch.empty(B, dtype=torch.float32, device=dev),
                         p_star=torch.empty(B, dtype=torch.float32, device=dev),
                         j_star=torch.empty(B, dtype=torch.int64, device=dev),
                         k_star=torch.empty(B, dtype=torch.int64, device=dev))
        g = (lambda k: _ptr(extra[k])) if extra else (lambda k: None)
        dt = _LOGIT_DTYPES[lg.dtype]
        ws = self._workspace(self._L.vnx_sampler_workspace(B, V, dt))
        _lib.check(self._L.vnx_sampler_sample(
            _ptr(lg), dt, B, V, lg.stride(0), float(temperature), int(top_k), float(top_p),
            mode, float(calib_factor if calib_factor is not None else 1.0), float(calib_eps),
            _ptr(u), _ptr(ids), g("flags"), g("lse"), g("kth"), g("p_star"), g("j_star"), g("k_star"),
            _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)), "sampler_sample")
        if return_all:
            return dict(ids=ids, **extra)
        return ids

    def logit_calibrate(self, logits, calib_factor: float, eps: float = 1e-8, return_var: bool = False):
        """CometSparkNexLM._apply_logit_calibration along the last axis
        (vnx_logit_calibrate): logits / sqrt(var + eps) * calib_factor, fp32."""
        t = self._logits(logits)
        shape = t.shape
        x2 = self._rows2d(t)
        R, V = x2.shape
        out = torch.empty((R, V), dtype=torch.float32, device=self._torch_device)
        var = torch.empty(R, dtype=torch.float64, device=self._torch_device)
        _lib.check(self._L.vnx_logit_calibrate(_ptr(x2), _LOGIT_DTYPES[x2.dtype], R, V, x2.stride(0),
                                               float(calib_factor), float(eps), _ptr(out), V, _ptr(var),
                                               ctypes.c_void_p(self._stream().cuda_stream)), "logit_calibrate")
        out = out.reshape(shape)
        return (out, var) if return_var else out

    # ---- weight-only quantized GEMV -------------------------------------------
    def _acts(self, x, K: int) -> torch.Tensor:
        """(..., K) activations -> contiguous (B, K) fp16 on this device."""
        t = _to_tensor(x, self._torch_device)
        if t.shape[-1] != K:
            raise ValueError(f"activations have {t.shape[-1]} features, the weight expects {K}")
        return t.reshape(-1, K).to(torch.float16).contiguous()

    @staticmethod
    def _rows16(w: torch.Tensor) -> torch.Tensor:
        """2-D byte weights whose rows start 16-byte aligned (pads the row pitch)."""
        w = w.contiguous()
        if w.stride(0) % 16 == 0 and w.data_ptr() % 16 == 0:
            return w
        ld = (w.shape[1] + 15) // 16 * 16
        out = torch.zeros((w.shape[0], ld), dtype=w.dtype, device=w.device)
        out[:, :w.shape[1]] = w
        return out[:, :w.shape[1]]

    def gemv_w4(self, x, wq, scales, group: int) -> torch.Tensor:
        """y = x @ (q * s)^T for packed int4 wq (N, K/2) and scales (N, K/group)
        (fp16 or fp32); returns (..., N) fp32 (vnx_gemv_w4)."""
        dev = self._torch_device
        w = self._rows16(_to_tensor(wq, dev, torch.uint8))
        sc = _to_tensor(scales, dev)
        if sc.dtype not in (torch.float16, torch.float32):
            sc = sc.to(torch.float32)
        sc = sc.reshape(w.shape[0], -1).contiguous()
        N, K = w.shape[0], 2 * w.shape[1]
        lead = _to_tensor(x, dev).shape[:-1]
        x2 = self._acts(x, K)
        B = x2.shape[0]
        y = torch.empty((B, N), dtype=torch.float32, device=dev)
        sdt = _lib.VNX_F16 if sc.dtype == torch.float16 else _lib.VNX_F32
        ws = self._workspace(self._L.vnx_gemv_workspace(B, N, K))
        _lib.check(self._L.vnx_gemv_w4(_ptr(x2), K, _ptr(w), w.stride(0), _ptr(sc), sdt, sc.stride(0), B, N, K,
                                       int(group), _ptr(y), N, _ptr(ws), ws.numel(),
                                       ctypes.c_void_p(self._stream().cuda_stream)), "gemv_w4")
        return y.reshape(*lead, N)

    def pack_w4_tiles(self, wq, K: int) -> torch.Tensor:
        """The tiled copy (vnx_pack_w4_tiles: 16-row tiles of 1 KB pieces,
        nibbles in offset form) of packed int4 wq (N, K/2); returns a uint8
        tensor of vnx_w4_tiles_bytes(N, K) bytes."""
        dev = self._torch_device
        w = self._rows16(_to_tensor(wq, dev, torch.uint8))
        N = w.shape[0]
        out = torch.empty(self._L.vnx_w4_tiles_bytes(N, K), dtype=torch.uint8, device=dev)
        _lib.check(self._L.vnx_pack_w4_tiles(_ptr(w), w.stride(0), N, K, _ptr(out),
                                             ctypes.c_void_p(self._stream().cuda_stream)), "pack_w4_tiles")
        return out

    def gemv_w4_tiles(self, x, wt, scales, N: int, K: int, out_dtype=torch.float32) -> torch.Tensor:
        """y = x @ (q * s)^T from the tiled copy wt (pack_w4_tiles) and fp16
        group-128 scales (N, K/128); returns (..., N) fp32 (vnx_gemv_w4_tiles)
        or bf16 (vnx_gemv_w4_tiles_out: the fp32 sums rounded once)."""
        dev = self._torch_device
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("out_dtype must be torch.float32 or torch.bfloat16")
        sc = _to_tensor(scales, dev, torch.float16).reshape(N, -1).contiguous()
        lead = _to_tensor(x, dev).shape[:-1]
        x2 = self._acts(x, K)
        B = x2.shape[0]
        y = torch.empty((B, N), dtype=out_dtype, device=dev)
        _lib.check(self._L.vnx_gemv_w4_tiles_out(_ptr(x2), K, _ptr(wt), _ptr(sc), sc.stride(0), B, N, K, _ptr(y),
                                                 _LOGIT_DTYPES[out_dtype], N,
                                                 ctypes.c_void_p(self._stream().cuda_stream)), "gemv_w4_tiles")
        return y.reshape(*lead, N)

    def gemv_w8(self, x, wq, scale) -> torch.Tensor:
        """y = x @ (q * s)^T for int8 wq (N, K) and per-row fp32 scale (N,)."""
        dev = self._torch_device
        w = self._rows16(_to_tensor(wq, dev, torch.int8))
        sc = _to_tensor(scale, dev, torch.float32).reshape(-1).contiguous()
        N, K = w.shape
        lead = _to_tensor(x, dev).shape[:-1]
        x2 = self._acts(x, K)
        B = x2.shape[0]
        y = torch.empty((B, N), dtype=torch.float32, device=dev)
        ws = self._workspace(self._L.vnx_gemv_workspace(B, N, K))
        _lib.check(self._L.vnx_gemv_w8(_ptr(x2), K, _ptr(w), w.stride(0), _ptr(sc), B, N, K, _ptr(y), N,
                                       _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)),
                   "gemv_w8")
        return y.reshape(*lead, N)

    def dequant_w4(self, wq, scales, K: int, group: int) -> torch.Tensor:
        dev = self._torch_device
        w = _to_tensor(wq, dev, torch.uint8).contiguous()
        sc = _to_tensor(scales, dev)
        if sc.dtype not in (torch.float16, torch.float32):
            sc = sc.to(torch.float32)
        sc = sc.reshape(w.shape[0], -1).contiguous()
        N = w.shape[0]
        out = torch.empty((N, K), dtype=torch.float32, device=dev)
        sdt = _lib.VNX_F16 if sc.dtype == torch.float16 else _lib.VNX_F32
        _lib.check(self._L.vnx_dequant_w4(_ptr(w), w.stride(0), _ptr(sc), sdt, sc.stride(0), N, K, int(group),
                                          _ptr(out), K, ctypes.c_void_p(self._stream().cuda_stream)),
                   "dequant_w4")
        return out

    def dequant_w8(self, wq, scale) -> torch.Tensor:
        dev = self._torch_device
        w = _to_tensor(wq, dev, torch.int8).contiguous()
        sc = _to_tensor(scale, dev, torch.float32).reshape(-1).contiguous()
        N, K = w.shape
        out = torch.empty((N, K), dtype=torch.float32, device=dev)
        _lib.check(self._L.vnx_dequant_w8(_ptr(w), w.stride(0), _ptr(sc), N, K, _ptr(out), K,
                                          ctypes.c_void_p(self._stream().cuda_stream)), "dequant_w8")
        return out

    # ---- tree-verify attention ------------------------------------------------
    def _heads_bf16(self, x, name: str, dtype=torch.bfloat16) -> torch.Tensor:
        """(B, heads, rows, d) view in dtype (bf16, or fp32 for the fp32-rows
        path) with the head dimension contiguous and 16-byte aligned strides
        (copied when it is not)."""
        t = _to_tensor(x, self._torch_device, dtype)
        if t.dim() != 4:
            raise ValueError(f"{name} must be (B, heads, rows, d), got shape {tuple(t.shape)}")
        unit = 16 // t.element_size()
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any(st % unit for st in t.stride()[:3]):
            t = t.contiguous()
        return t

    def tree_attention(self, q, k_cache, v_cache, k_tree, v_tree, anc, scale: float | None = None,
                       out_dtype=torch.float32, seg2=None, gates=None, tp=None, window: int = 0,
                       alibi_slopes=None, alibi_max_keys: int = 1024, force_splits: int = 0,
                       force_waves: int = 0, fp32_rows: bool = False) -> torch.Tensor:
        """Tree-verify attention (vnx_tree_attn).

        q (B, H, N, d); k_cache / v_cache (B, Hkv, Tp, d) or None (Tp = 0);
        k_tree / v_tree (B, Hkv, N, d); anc (N,) or (B, N) ancestor words
        (tree.ancestor_words).  Inputs are read as bf16; returns (B, H, N, d)
        in out_dtype (torch.float32, torch.bfloat16 or torch.float16).
        seg2 = (k2, v2), each (B or 1, Hkv, T2, d), with gates (2,) adds
        TriSparse's gated global path: out = gates[0] * (the tree attention)
        + gates[1] * (attention over the T2 rows, all visible).  tp (B,)
        int32: per-row prefix lengths (ragged caches).  window > 0 keeps
        keys less than window positions behind each node; alibi_slopes (H,)
        with gates (3,) adds the ALiBi path as gates[2] * it for rows with
        tp_b + N <= alibi_max_keys.  force_splits / force_waves pin the launch
        shape (tuning and tests).  fp32_rows: inputs read as fp32 (d in 8 /
        16 / 32, the fp32 models' path), and anc may be None for a chain of
        any length N."""
        dev = self._torch_device
        rows = torch.float32 if fp32_rows else torch.bfloat16
        qt = self._heads_bf16(q, "q", rows)
        kt = self._heads_bf16(k_tree, "k_tree", rows)
        vt = self._heads_bf16(v_tree, "v_tree", rows)
        B, H, N, d = qt.shape
        if kt.shape != vt.shape or kt.shape[0] != B or kt.shape[2] != N or kt.shape[3] != d:
            raise ValueError(f"tree rows {tuple(kt.shape)} / {tuple(vt.shape)} do not match q {tuple(qt.shape)}")
        Hkv = kt.shape[1]
        if kt.stride() != vt.stride():
            kt, vt = kt.contiguous(), vt.contiguous()
        if k_cache is None or v_cache is None:
            if (k_cache is None) != (v_cache is None):
                raise ValueError("pass both k_cache and v_cache, or neither")
            kc = vc = None
            Tp = 0
            cstr = (0, 0, 0)
        else:
            kc = self._heads_bf16(k_cache, "k_cache", rows)
            vc = self._heads_bf16(v_cache, "v_cache", rows)
            if kc.shape != vc.shape or kc.shape[0] != B or kc.shape[1] != Hkv or kc.shape[3] != d:
                raise ValueError(f"cache {tuple(kc.shape)} / {tuple(vc.shape)} does not match the tree rows")
            if kc.stride() != vc.stride():
                kc, vc = kc.contiguous(), vc.contiguous()
            Tp = kc.shape[2]
            cstr = kc.stride()[:3]
            if Tp == 0:
                kc = vc = None
        if anc is None:
            if not fp32_rows:
                raise ValueError("anc=None (a chain) needs fp32_rows")
            a = anc_t = None
        else:
            a = anc.detach().cpu().numpy() if isinstance(anc, torch.Tensor) else np.asarray(anc)
            a = np.ascontiguousarray(a.astype(np.uint64) if a.dtype != np.uint64 else a)
            if a.shape not in ((N,), (B, N)):
                raise ValueError(f"anc must be ({N},) or ({B}, {N}), got {a.shape}")
            anc_t = torch.from_numpy(a.view(np.int64)).to(dev)
        if out_dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise ValueError("out_dtype must be torch.float32, torch.bfloat16 or torch.float16")
        out = torch.empty((B, H, N, d), dtype=out_dtype, device=dev)
        sc = float(scale) if scale is not None else 1.0 / float(np.sqrt(d))
        args = _lib.TreeAttnArgs()
        args.q = qt.data_ptr()
        args.q_strides[:] = list(qt.stride()[:3])
        args.k_cache = kc.data_ptr() if kc is not None else None
        args.v_cache = vc.data_ptr() if vc is not None else None
        args.cache_strides[:] = list(cstr)
        args.k_tree = kt.data_ptr()
        args.v_tree = vt.data_ptr()
        args.tree_strides[:] = list(kt.stride()[:3])
        args.anc = anc_t.data_ptr() if anc_t is not None else None
        args.anc_batch_stride = N if a is not None and a.ndim == 2 else 0
        args.f32_rows = int(fp32_rows)
        args.out = out.data_ptr()
        args.out_dtype = _lib.DTYPE_CODES[out_dtype]
        args.out_strides[:] = list(out.stride()[:3])
        args.B, args.H, args.Hkv, args.Tp, args.N, args.d = B, H, Hkv, Tp, N, d
        args.scale = sc
        keep = []
        if tp is not None:
            tpt = _to_tensor(tp, dev, torch.int32).reshape(-1).contiguous()
            if tpt.numel() != B:
                raise ValueError(f"tp must have {B} entries")
            keep.append(tpt)
            args.tp_batch = tpt.data_ptr()
        args.window = int(window)
        args.force_splits, args.force_waves = int(force_splits), int(force_waves)
        if alibi_slopes is not None:
            sl = _to_tensor(alibi_slopes, dev, torch.float32).reshape(-1).contiguous()
            if sl.numel() != H:
                raise ValueError(f"alibi_slopes must have {H} entries")
            if gates is None:
                raise ValueError("the ALiBi path needs three gates")
            g3 = _to_tensor(gates, dev, torch.float32).reshape(-1).contiguous()
            if g3.numel() < 3:
                raise ValueError("gates must hold three values with ALiBi")
            keep += [sl, g3]
            args.alibi_slopes = sl.data_ptr()
            args.alibi_max_keys = int(alibi_max_keys)
            args.gates = g3.data_ptr()
        if seg2 is not None:
            k2 = self._heads_bf16(seg2[0], "k_seg2", rows)
            v2 = self._heads_bf16(seg2[1], "v_seg2", rows)
            if k2.shape != v2.shape or k2.shape[0] not in (1, B) or k2.shape[1] != Hkv or k2.shape[3] != d:
                raise ValueError(f"second segment {tuple(k2.shape)} / {tuple(v2.shape)} does not match")
            if k2.stride() != v2.stride():
                k2, v2 = k2.contiguous(), v2.contiguous()
            if gates is None:
                raise ValueError("a second segment needs the two gates")
            g = _to_tensor(gates, dev, torch.float32).reshape(-1).contiguous()
            if g.numel() < 2:
                raise ValueError("gates must hold two values")
            keep += [k2, v2, g]
            args.k_seg2, args.v_seg2 = k2.data_ptr(), v2.data_ptr()
            args.seg2_strides[:] = [0 if k2.shape[0] == 1 else k2.stride(0), k2.stride(1), k2.stride(2)]
            args.T2 = k2.shape[2]
            args.gates = g.data_ptr()
        ws = self._workspace(self._L.vnx_tree_attn_workspace_args(ctypes.byref(args)))
        _lib.check(self._L.vnx_tree_attn(ctypes.byref(args), _ptr(ws), ws.numel(),
                                         ctypes.c_void_p(self._stream().cuda_stream)), "tree_attn")
        del keep
        return out

    def attention(self, q, k, v, mask=None):
        """DeviceBackend.attention (device.py:260-270; TorchBackend's SDPA call,
        backend_torch.py:356-379).  bf16 (B, H, Nq, d) queries over (B, Hkv, T, d)
        keys with mask None, or an additive (Nq, T) token-tree mask (the first
        T - Nq columns visible, the last Nq x Nq block 0 / -inf; see
        tree.words_from_mask), run the tree-verify kernel and return bf16, as
        SDPA does for bf16 inputs.  Anything else takes the generic composition
        (matmul, vnx softmax, matmul)."""
        from . import tree as _tree
        words = None
        if (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor)
                and q.dtype == k.dtype == v.dtype == torch.bfloat16 and q.dim() == k.dim() == v.dim() == 4
                and k.shape == v.shape and q.shape[-1] in (64, 128) and q.shape[-1] == k.shape[-1]
                and q.shape[0] == k.shape[0] and q.shape[1] % k.shape[1] == 0):
            nq, T = q.shape[2], k.shape[2]
            if 1 <= nq <= _tree.MAX_NODES and T >= nq:
                if mask is None:
                    words = np.full(nq, (1 << nq) - 1, dtype=np.uint64)
                else:
                    m = mask.detach().float().cpu().numpy() if isinstance(mask, torch.Tensor) else np.asarray(mask)
                    while m.ndim > 2 and m.shape[0] == 1:
                        m = m[0]
                    words = _tree.words_from_mask(m, T - nq)
        if words is None:
            return super().attention(q, k, v, mask)
        Tp = k.shape[2] - q.shape[2]
        kc, vc = (k[:, :, :Tp], v[:, :, :Tp]) if Tp else (None, None)
        return self.tree_attention(q, kc, vc, k[:, :, Tp:], v[:, :, Tp:], words, out_dtype=torch.bfloat16)

    def greedy_verify(self, target, draft_ids, rows_t: int | None = None):
        """Greedy verify of every batch row (see vnx_greedy_verify).
        target (B, rows_t, V) (may be a strided slice of (B, T, V) logits).
        Returns (accepted (B,k) bool, main_pred (B,rows_t), accept_len (B,), out_ids (B,k+1))."""
        dev = self._torch_device
        ids = _to_tensor(draft_ids, dev, torch.int64).contiguous()
        if ids.dim() != 2:
            raise ValueError("draft_ids must be (B, k)")
        B, k = ids.shape
        rows_t = k if rows_t is None else int(rows_t)
        tg = self._rows3d(target, rows_t)
        if tg.shape[0] != B:
            raise ValueError(f"batch mismatch: logits {tg.shape[0]} vs draft {B}")
        V = tg.shape[2]
        acc = torch.empty((B, k), dtype=torch.uint8, device=dev)
        pred = torch.empty((B, rows_t), dtype=torch.int64, device=dev)
        alen = torch.empty(B, dtype=torch.int32, device=dev)
        out = torch.empty((B, k + 1), dtype=torch.int64, device=dev)
        ws = self._workspace(self._L.vnx_greedy_verify_workspace(B, rows_t, V))
        _lib.check(self._L.vnx_greedy_verify(
            _ptr(tg), _LOGIT_DTYPES[tg.dtype], B, k, rows_t, V, tg.stride(1), tg.stride(0), _ptr(ids),
            _ptr(acc), _ptr(pred), _ptr(alen), _ptr(out), _ptr(ws), ws.numel(),
            ctypes.c_void_p(self._stream().cuda_stream)), "greedy_verify")
        return acc.bool(), pred, alen, out

    def lm_head(self, x, weight, out=None, out_dtype=torch.float32) -> torch.Tensor:
        """Verify-pass LM head (vnx_lm_head): x (..., K) . weight (V, K)^T on the
        matrix cores, bf16 in, fp32 accumulate; returns (..., V) in out_dtype
        (or writes `out`, a (rows, V) view with unit last stride)."""
        dev = self._torch_device
        xt = _to_tensor(x, dev, torch.bfloat16)
        lead = tuple(xt.shape[:-1])
        K = xt.shape[-1]
        x2 = xt.reshape(-1, K)
        if x2.stride(1) != 1 or x2.data_ptr() % 16 or x2.stride(0) % 8:
            x2 = x2.contiguous()
        wt = _to_tensor(weight, dev, torch.bfloat16)
        if wt.dim() != 2 or wt.shape[1] != K:
            raise ValueError(f"weight must be (V, {K}), got {tuple(wt.shape)}")
        if wt.stride(1) != 1 or wt.data_ptr() % 16 or wt.stride(0) % 8:
            wt = wt.contiguous()
        M, V = x2.shape[0], wt.shape[0]
        if out is None:
            if out_dtype not in (torch.float32, torch.bfloat16):
                raise ValueError("out_dtype must be torch.float32 or torch.bfloat16")
            ldo = (V + 3) // 4 * 4
            buf = torch.empty((M, ldo), dtype=out_dtype, device=dev)
            o = buf[:, :V]
        else:
            o = out
            if o.dim() != 2 or tuple(o.shape) != (M, V) or o.stride(1) != 1:
                raise ValueError(f"out must be a ({M}, {V}) view with unit last stride")
        _lib.check(self._L.vnx_lm_head(
            _ptr(x2), x2.stride(0), _ptr(wt), wt.stride(0), M, K, V, _ptr(o),
            _LOGIT_DTYPES[o.dtype], o.stride(0), ctypes.c_void_p(self._stream().cuda_stream)), "lm_head")
        return o.reshape(*lead, V) if out is None else o

    def tree_greedy(self, target, tokens, parent):
        """Greedy tree verification (vnx_tree_greedy) of every batch row.

        target (B, N+1, V) logits (row 0: after the last committed token,
        row 1+n: after node n; may be a strided slice); tokens (B, N) node
        tokens; parent (N,) BFS parent array (tree.tree_from_branching).
        Returns (accept_len (B,) int32, best (B,) int32, out_ids (B, N+1) int64,
        pred (B, N+1) int64); out_ids holds the accepted root path, the bonus
        argmax, then -1."""
        from . import tree as _tree
        dev = self._torch_device
        par = np.ascontiguousarray(_tree.check_parents(parent), dtype=np.int32)
        N = par.size
        tok = _to_tensor(tokens, dev, torch.int64)
        if tok.dim() != 2 or tok.shape[1] != N:
            raise ValueError(f"tokens must be (B, {N}), got {tuple(tok.shape)}")
        if tok.stride(1) != 1:
            tok = tok.contiguous()
        B = tok.shape[0]
        tg = self._rows3d(target, N + 1)
        if tg.shape[0] != B:
            raise ValueError(f"batch mismatch: logits {tg.shape[0]} vs tokens {B}")
        V = tg.shape[2]
        alen = torch.empty(B, dtype=torch.int32, device=dev)
        best = torch.empty(B, dtype=torch.int32, device=dev)
        out = torch.empty((B, N + 1), dtype=torch.int64, device=dev)
        pred = torch.empty((B, N + 1), dtype=torch.int64, device=dev)
        ws = self._workspace(self._L.vnx_tree_greedy_workspace(B, N, V))
        _lib.check(self._L.vnx_tree_greedy(
            _ptr(tg), _LOGIT_DTYPES[tg.dtype], B, N, V, tg.stride(1), tg.stride(0), _ptr(tok),
            tok.stride(0), par.ctypes.data_as(ctypes.c_void_p), _ptr(alen), _ptr(best), _ptr(out),
            _ptr(pred), _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)), "tree_greedy")
        return alen, best, out, pred

    def topk(self, x, b: int):
        """(ids, vals): the b best ids of each row (vnx_row_topk; value
        descending, ties to the lower id, NaN first), shapes (..., b)."""
        t = self._rows2d(x)
        rows, V = t.shape
        lead = tuple(self._logits(x).shape[:-1])
        ids = torch.empty((rows, b), dtype=torch.int64, device=self._torch_device)
        vals = torch.empty((rows, b), dtype=torch.float32, device=self._torch_device)
        ws = self._workspace(self._L.vnx_row_topk_workspace(rows, V, b))
        _lib.check(self._L.vnx_row_topk(
            _ptr(t), _LOGIT_DTYPES[t.dtype], rows, V, t.stride(0), int(b), _ptr(ids),
            _ptr(vals), b, _ptr(ws), ws.numel(), ctypes.c_void_p(self._stream().cuda_stream)), "row_topk")
        return ids.reshape(*lead, b), vals.reshape(*lead, b)

    def expand_tree(self, draft, parent):
        """Node tokens (B, N) of a token tree: node n takes the r-th best id
        of its parent's draft row (row 0 for the root, 1 + parent otherwise),
        r = the number of earlier siblings of n.  draft (B, R, V)."""
        from . import tree as _tree
        par = _tree.check_parents(parent)
        rows = np.where(par < 0, 0, par + 1)
        rank = np.zeros(par.size, np.int64)
        seen: dict = {}
        for i, p in enumerate(par):
            rank[i] = seen.get(int(p), 0)
            seen[int(p)] = rank[i] + 1
        ids, _ = self.topk(draft, int(rank.max()) + 1)
        dev = self._torch_device
        return ids[:, torch.from_numpy(rows).to(dev), torch.from_numpy(rank).to(dev)]


__all__ = ["HipBackend"]

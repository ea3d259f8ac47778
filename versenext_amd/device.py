"""Device backends: the VerseTorch `DeviceBackend` interface with a HIP "rocm" device.

Mirrors packages/verse_torch/verse_torch/device.py:
- `_parse_device` (:171-188), `_to_torch_device_str` (:191-206), `is_cpu_device`,
  `DEFAULT_DEVICE`;
- the `DeviceBackend` ABC with the same abstract methods and the default
  `attention` (:219-270);
- `NumpyBackend` for the "cpu" device (:285-335);
- the `get_backend` factory with its per-device-string cache and
  `clear_backend_cache` (:343-391).

Difference: "rocm" / "rocm:N" (and "cuda" / "cuda:N", the same AMD GPU under
PyTorch-ROCm) return `HipBackend`, whose softmax and verification operators
are the hand-written gfx950 kernels of libvnx_hip.so (the reference returns a
`TorchBackend` that delegates to PyTorch, backend_torch.py:246-379).  There is
no fallback: without the library or a GPU, `get_backend("rocm")` raises
RuntimeError.
"""
from __future__ import annotations

import abc
import threading
from typing import Optional

import numpy as np

try:  # PyTorch is plumbing for device memory and streams
    import torch as _torch
except Exception:  # pragma: no cover - torch is present in this image
    _torch = None


DEFAULT_DEVICE = "cpu"


def has_torch() -> bool:
    return _torch is not None


def _parse_device(device) -> str:
    """'rocm' / 'rocm:0' / 'ROCM:2' -> 'rocm'; None / unknown -> 'cpu' (device.py:171-188)."""
    if device is None:
        return "cpu"
    s = str(device).lower()
    if s.startswith(("cuda", "npu", "mps", "rocm")):
        return s.split(":")[0]
    return "cpu"


def _to_torch_device_str(device) -> str:
    """'rocm' -> 'cuda', 'rocm:N' -> 'cuda:N' (device.py:191-206)."""
    s = str(device).lower()
    if s == "rocm":
        return "cuda"
    if s.startswith("rocm:"):
        return "cuda:" + s.split(":", 1)[1]
    return s


def is_cpu_device(device) -> bool:
    return _parse_device(device) == "cpu"


def _device_index(device) -> int:
    s = str(device).lower()
    if ":" in s:
        try:
            return int(s.split(":", 1)[1])
        except ValueError as e:
            raise ValueError(f"bad device string {device!r}") from e
    return 0


class DeviceBackend(abc.ABC):
    """Operator interface (device.py:219-270)."""

    @property
    @abc.abstractmethod
    def device_type(self) -> str:
        """'cpu' / 'rocm' / 'cuda'."""

    @abc.abstractmethod
    def matmul(self, a, b):
        """a @ b."""

    @abc.abstractmethod
    def linear(self, x, weight, bias=None):
        """y = x @ weight.T + bias."""

    @abc.abstractmethod
    def softmax(self, x, dim: int = -1):
        """Numerically stable softmax along dim."""

    @abc.abstractmethod
    def layernorm(self, x, weight, bias, eps: float = 1e-5):
        """LayerNorm over the last axis, then affine."""

    @abc.abstractmethod
    def rmsnorm(self, x, weight, eps: float = 1e-6):
        """x / sqrt(mean(x^2) + eps) * weight."""

    @abc.abstractmethod
    def rope(self, x, cos=None, sin=None):
        """GPT-NeoX rotate-half RoPE; identity when cos or sin is None."""

    def attention(self, q, k, v, mask=None):
        """softmax(q @ k^T / sqrt(d) + mask) @ v with an additive mask (device.py:260-270)."""
        d = q.shape[-1]
        scores = self.matmul(q, _swap_last_two(k)) / (d ** 0.5)
        if mask is not None:
            scores = scores + mask
        attn = self.softmax(scores, dim=-1)
        return self.matmul(attn, v)


def _swap_last_two(x):
    if _torch is not None and isinstance(x, _torch.Tensor):
        return x.transpose(-1, -2)
    return np.swapaxes(x, -1, -2)


class NumpyBackend(DeviceBackend):
    """The "cpu" device of the interface: numpy operators (device.py:285-335).
    Never used for "rocm"."""

    @property
    def device_type(self) -> str:
        return "cpu"

    def matmul(self, a, b):
        return np.matmul(a, b)

    def linear(self, x, weight, bias=None):
        out = np.matmul(x, np.swapaxes(weight, -1, -2))
        if bias is not None:
            out = out + bias
        return out

    def softmax(self, x, dim: int = -1):
        x_max = np.max(x, axis=dim, keepdims=True)
        e = np.exp(x - x_max)
        return e / np.sum(e, axis=dim, keepdims=True)

    def layernorm(self, x, weight, bias, eps: float = 1e-5):
        mean = x.mean(axis=-1, keepdims=True)
        var = x.var(axis=-1, keepdims=True)
        return (x - mean) / np.sqrt(var + eps) * weight + bias

    def rmsnorm(self, x, weight, eps: float = 1e-6):
        ms = np.mean(x * x, axis=-1, keepdims=True)
        return x / np.sqrt(ms + eps) * weight

    def rope(self, x, cos=None, sin=None):
        if cos is None or sin is None:
            return x
        d = x.shape[-1]
        half = d // 2
        x1, x2 = x[..., :half], x[..., half:]
        cos_b = cos[..., :half] if cos.shape[-1] >= d else cos
        sin_b = sin[..., :half] if sin.shape[-1] >= d else sin
        return np.concatenate([x1 * cos_b - x2 * sin_b, x1 * sin_b + x2 * cos_b], axis=-1)


_BACKEND_CACHE: dict = {}
_CACHE_LOCK = threading.Lock()


def get_backend(device=None) -> DeviceBackend:
    """None / 'cpu' -> cached NumpyBackend; 'rocm[:N]' / 'cuda[:N]' -> cached
    HipBackend (device.py:346-386).  RuntimeError if PyTorch, the GPU or the
    HIP library is unavailable, or for 'npu' / 'mps'."""
    dtype = _parse_device(device)
    if dtype == "cpu":
        with _CACHE_LOCK:
            if "cpu" not in _BACKEND_CACHE:
                _BACKEND_CACHE["cpu"] = NumpyBackend()
            return _BACKEND_CACHE["cpu"]
    if not has_torch():
        raise RuntimeError(f"PyTorch is not installed; device '{device}' is unavailable (CPU only)")
    if dtype in ("npu", "mps"):
        raise RuntimeError(f"device '{device}' is not provided by the MI355X backend (rocm only)")
    key = str(device).lower()
    with _CACHE_LOCK:
        if key not in _BACKEND_CACHE:
            from .hip_backend import HipBackend
            _BACKEND_CACHE[key] = HipBackend(device=key)
        return _BACKEND_CACHE[key]


def clear_backend_cache() -> None:
    with _CACHE_LOCK:
        _BACKEND_CACHE.clear()


__all__ = [
    "DEFAULT_DEVICE", "DeviceBackend", "NumpyBackend", "get_backend", "clear_backend_cache",
    "is_cpu_device", "has_torch", "_parse_device", "_to_torch_device_str",
]

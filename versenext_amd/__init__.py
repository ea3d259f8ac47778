"""versenext_amd — MI355X-native speculative-decoding verification for VerseNext.

Entry points (reference names):
- `SpeculativeDecoder` (packages/verse_nex/verse_nex/speculative.py:55)
- `DeviceBackend`, `NumpyBackend`, `get_backend`, `clear_backend_cache`
  (packages/verse_torch/verse_torch/device.py:219-391); `get_backend("rocm")`
  returns `HipBackend`, backed by libvnx_hip.so (include/vnx.h).
"""
from .device import (  # noqa: F401
    DEFAULT_DEVICE,
    DeviceBackend,
    NumpyBackend,
    _parse_device,
    _to_torch_device_str,
    clear_backend_cache,
    get_backend,
    has_torch,
    is_cpu_device,
)

__version__ = "0.1.0"


def __getattr__(name):
    # GPU-side modules import torch.cuda state lazily.
    if name == "SpeculativeDecoder":
        from .speculative import SpeculativeDecoder
        return SpeculativeDecoder
    if name == "HipBackend":
        from .hip_backend import HipBackend
        return HipBackend
    raise AttributeError(name)

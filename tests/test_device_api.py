"""Host-side boundary: device-string parsing, the backend factory and the "cpu"
NumpyBackend, with the vectors of tests/test_rocm_npu_compat.py:56-90, :455-503
and tests/test_device_backend.py:56-210."""
import numpy as np
import pytest

from conftest import gpu_available
from versenext_amd import (DeviceBackend, NumpyBackend, _parse_device, _to_torch_device_str,
                           clear_backend_cache, get_backend, is_cpu_device)


def test_parse_device_vectors():
    assert _parse_device("rocm") == "rocm"
    assert _parse_device("rocm:0") == "rocm"
    assert _parse_device("ROCM:2") == "rocm"
    for s, e in [("cpu", "cpu"), ("cuda", "cuda"), ("cuda:0", "cuda"), ("CUDA:1", "cuda"),
                 ("npu", "npu"), ("npu:1", "npu"), ("mps", "mps")]:
        assert _parse_device(s) == e
    assert _parse_device(None) == "cpu"
    assert _parse_device("foo") == "cpu" and _parse_device("") == "cpu"
    assert _to_torch_device_str("rocm") == "cuda" and _to_torch_device_str("rocm:3") == "cuda:3"
    assert is_cpu_device(None) and not is_cpu_device("rocm:1")


def test_cpu_backend_factory_and_cache():
    clear_backend_cache()
    b = get_backend("cpu")
    assert isinstance(b, NumpyBackend) and isinstance(b, DeviceBackend)
    assert get_backend(None) is b and get_backend("cpu") is b
    assert b.device_type == "cpu"


def test_npu_mps_unavailable():
    clear_backend_cache()
    for dev in ("npu", "npu:0", "mps"):
        with pytest.raises(RuntimeError):
            get_backend(dev)


@pytest.mark.skipif(gpu_available(), reason="checks the no-GPU error path")
def test_rocm_without_gpu_raises_runtime_error():
    clear_backend_cache()
    with pytest.raises(RuntimeError):
        get_backend("rocm")


def test_numpy_backend_ops():
    rng = np.random.RandomState(42)
    b = NumpyBackend()
    a, m = rng.randn(2, 3).astype(np.float32), rng.randn(3, 4).astype(np.float32)
    np.testing.assert_allclose(b.matmul(a, m), a @ m, atol=1e-5)
    x, w, bias = rng.randn(4, 3).astype(np.float32), rng.randn(2, 3).astype(np.float32), rng.randn(2)
    np.testing.assert_allclose(b.linear(x, w, bias), x @ w.T + bias, atol=1e-5)
    np.testing.assert_allclose(b.linear(x, w), x @ w.T, atol=1e-5)
    s = b.softmax(rng.randn(3, 5).astype(np.float32))
    np.testing.assert_allclose(s.sum(-1), 1.0, atol=1e-6)
    assert np.all(np.isfinite(b.softmax(np.array([[1000.0, 1001.0, 1002.0]], np.float32))))
    ln = b.layernorm(rng.randn(4, 8), np.full(8, 2.0), np.full(8, 1.0))
    np.testing.assert_allclose(ln.var(-1), 4.0, atol=0.1)
    r = b.rmsnorm(rng.randn(4, 8).astype(np.float32), np.ones(8, np.float32))
    np.testing.assert_allclose(np.sqrt((r * r).mean(-1)), 1.0, atol=1e-4)
    xr = rng.randn(2, 4, 8).astype(np.float32)
    np.testing.assert_allclose(b.rope(xr), xr)
    cos, sin = rng.randn(2, 4, 4).astype(np.float32), rng.randn(2, 4, 4).astype(np.float32)
    out = b.rope(xr, cos, sin)
    x1, x2 = xr[..., :4], xr[..., 4:]
    np.testing.assert_allclose(out, np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos], -1), atol=1e-5)
    q = rng.randn(2, 4, 8).astype(np.float32)
    assert b.attention(q, q, q).shape == (2, 4, 8)

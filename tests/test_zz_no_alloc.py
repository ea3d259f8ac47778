"""vnx_spec_accept_noalloc (the allocation-free acceptance entry point, with
its scratch in a fixed static device array) against vnx_spec_accept (the
same kernels, caller-supplied workspace), through the C ABI: identical
outputs on two calls in a row, the second with a smaller input, and sizes
past the fixed scratch rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from versenext_amd import _lib

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _inputs(dev, B, k, V, seed, dtype):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    tgt = torch.randn((B, k + 1, V), generator=g, device=dev) * 2.0
    dft = tgt[:, :k] + torch.randn((B, k, V), generator=g, device=dev) * 0.5
    ids = torch.randint(0, V, (B, k), generator=g, device=dev)
    ids[:, ::2] = torch.argmax(dft[:, ::2], -1)          # some drafts the target likes
    u = torch.rand((B, k + 1), generator=g, device=dev)
    return tgt.to(dtype).contiguous(), dft.to(dtype).contiguous(), ids.contiguous(), u.contiguous()


def _outs(dev, B, k):
    return (torch.full((B,), -7, dtype=torch.int32, device=dev),
            torch.full((B, k + 1), -7, dtype=torch.int64, device=dev),
            torch.full((B, k + 1), 99, dtype=torch.uint8, device=dev),
            torch.zeros((B, k + 1), dtype=torch.float32, device=dev),
            torch.zeros((B, k), dtype=torch.float32, device=dev))


def _call(L, noalloc, tgt, dft, ids, u, T, outs, stream):
    B, k1, V = tgt.shape
    k = k1 - 1
    dt = _lib.VNX_F32 if tgt.dtype == torch.float32 else _lib.VNX_BF16
    head = (P(tgt.data_ptr()), P(dft.data_ptr()), dt, B, k, V, tgt.stride(1), tgt.stride(0), dft.stride(1),
            dft.stride(0), P(ids.data_ptr()), P(u.data_ptr()), float(T), None, None) + \
        tuple(P(o.data_ptr()) for o in outs)
    if noalloc:
        return L.vnx_spec_accept_noalloc(*head, P(stream))
    ws = torch.zeros(L.vnx_spec_accept_workspace(B, k, V), dtype=torch.uint8, device=tgt.device)
    return L.vnx_spec_accept(*head, P(ws.data_ptr()), ws.numel(), P(stream))


def test_noalloc_matches_workspace_entry_point(hip):
    L = _lib.lib()
    dev = hip.torch_device
    stream = torch.cuda.current_stream(dev).cuda_stream
    # two calls in a row, the second smaller (the scratch keeps the first
    # call's contents), then the first shape again in bf16
    for (B, k, V, T, dtype, seed) in ((48, 8, 248320, 0.8, torch.float32, 1),
                                      (5, 3, 50000, 1.0, torch.float32, 2),
                                      (48, 8, 248320, 0.7, torch.bfloat16, 3)):
        print(f"noalloc vs workspace: B={B} k={k} V={V} T={T} {dtype}", flush=True)
        tgt, dft, ids, u = _inputs(dev, B, k, V, seed, dtype)
        ref, got = _outs(dev, B, k), _outs(dev, B, k)
        assert _call(L, False, tgt, dft, ids, u, T, ref, stream) == _lib.VNX_OK
        assert _call(L, True, tgt, dft, ids, u, T, got, stream) == _lib.VNX_OK
        torch.cuda.synchronize()
        for r, g in zip(ref, got):
            assert torch.equal(r, g)
        n = ref[0].cpu().numpy()
        assert n.min() >= 0 and n.max() <= k
        print(f"  accept_len {n.tolist()[:12]} ...", flush=True)


def test_noalloc_rejects_sizes_past_its_scratch(hip):
    """Host-side checks: nothing is launched, so no device memory is touched
    (the pointers are never dereferenced)."""
    L = _lib.lib()
    mx = L.vnx_spec_accept_noalloc_max_bytes()
    assert mx == 8 << 20
    B, k, V = 4096, 8, 248320
    assert L.vnx_spec_accept_workspace(B, k, V) > mx
    dummy = torch.zeros(16, dtype=torch.float32, device=hip.torch_device)
    p = P(dummy.data_ptr())
    st = L.vnx_spec_accept_noalloc(p, p, _lib.VNX_F32, B, k, V, V, (k + 1) * V, V, k * V, p, p, 0.8, None, None,
                                   p, p, None, None, None, None)
    assert st == _lib.VNX_ERR_TOO_LARGE
    with pytest.raises(ValueError, match="fixed scratch"):
        _lib.check(st, "spec_accept_noalloc")

"""GPU parity of the routed MoD expert products (vnx_expert_gemm_bf16) and the
expert sum over compact rows (vnx_sum_expert_rows).

The row lists are integers and must match exactly: expert z's rows are the m
with comb[m, z] != 0, ascending, and slots is their inverse.  The products are
held to the bar of the dense GEMM test: |y - ref| <= RTOL * sum_k |x_k w_k| +
one rounding of the output type (plus half the spacing of its subnormals),
against the fp64 product of the same bf16
inputs (SwiGLU propagated as in the dense test).  The sum over compact rows
must equal vnx_sum_experts of the dense (zero-filled) outputs bit for bit."""
import ctypes

import pytest
import torch

from versenext_amd import _lib

pytestmark = pytest.mark.gpu

RTOL = 1e-5
VP = ctypes.c_void_p


def _say(*a):
    print(*a, flush=True)


def _st():
    return VP(torch.cuda.current_stream().cuda_stream)


def _rnd(dtype):
    return {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]


def _sub(dtype):
    """Absolute rounding error of the output type's subnormals (half their spacing)."""
    return {torch.float32: 2.0 ** -150, torch.bfloat16: 2.0 ** -134, torch.float16: 2.0 ** -25}[dtype]


def _packed(w):
    """(E, N, K) bf16 -> packed (E, elems) bf16."""
    L = _lib.lib()
    E, N, K = w.shape
    el = L.vnx_pack_bf16_size(N, K) // 2
    out = torch.empty((E, el), dtype=torch.bfloat16, device=w.device)
    for z in range(E):
        _lib.check(L.vnx_pack_bf16(VP(w[z].data_ptr()), K, N, K, VP(out[z].data_ptr()), _st()), "pack")
    return out


def _routing(dev, M, E, frac, seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    comb = torch.rand((M, E), generator=g) + 0.05
    comb[torch.rand((M, E), generator=g) >= frac] = 0.0
    return comb.to(dev)


def _lists(comb):
    c = comb.cpu()
    M, E = c.shape
    rows = [torch.nonzero(c[:, z] != 0).flatten() for z in range(E)]
    slots = torch.full((M, E), -1, dtype=torch.int32)
    for z in range(E):
        slots[rows[z], z] = torch.arange(rows[z].numel(), dtype=torch.int32)
    return rows, slots


@pytest.mark.parametrize("M,N,K,E,frac,epi,route,dtype", [
    (224, 5376, 1024, 16, 0.5, 1, 1, torch.bfloat16),   # the mate MoD gate|up
    (224, 1024, 2688, 16, 0.5, 0, 0, torch.bfloat16),   # its down product shape, all rows
    (224, 1024, 2688, 16, 0.5, 0, 1, torch.float32),
    (256, 96, 128, 3, 0.9, 0, 1, torch.float32),        # more than one 128-row pass
    (256, 64, 128, 3, 1.0, 1, 0, torch.bfloat16),
    (37, 64, 64, 9, 0.3, 1, 1, torch.float16),          # a ragged tail, experts not a multiple of 8
    (5, 32, 192, 2, 0.0, 1, 1, torch.float32)])         # no routed rows at all
def test_routed_products(hip, M, N, K, E, frac, epi, route, dtype):
    _say(f"expert_gemm M={M} N={N} K={K} E={E} frac={frac} epi={epi} route={route} out={dtype}")
    dev = hip.torch_device
    g = torch.Generator(device=dev)
    g.manual_seed(M + N + K)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((E, N, K), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    comb = _routing(dev, M, E, frac, seed=E + K)
    wp = _packed(w)
    ncols = N // 2 if epi else N
    y = torch.full((E, M, ncols), float("nan"), dtype=dtype, device=dev)
    rows = torch.full((E, M), -7, dtype=torch.int32, device=dev)
    counts = torch.full((E,), -7, dtype=torch.int32, device=dev)
    slots = torch.full((M, E), -7, dtype=torch.int32, device=dev)
    L = _lib.lib()
    if route:
        rc = L.vnx_expert_gemm_bf16(VP(x.data_ptr()), K, 0, VP(wp.data_ptr()), wp.stride(0), M, N, K, E, epi,
                                    VP(comb.data_ptr()), E, 1, VP(rows.data_ptr()), VP(counts.data_ptr()),
                                    VP(slots.data_ptr()), VP(y.data_ptr()), _lib.DTYPE_CODES[dtype], ncols, M * ncols,
                                    _st())
    else:
        # every expert on all M rows of a shared x; SwiGLU weights by comb[j, z]
        comb.fill_(0.75)
        rc = L.vnx_expert_gemm_bf16(VP(x.data_ptr()), K, 0, VP(wp.data_ptr()), wp.stride(0), M, N, K, E, epi,
                                    VP(comb.data_ptr()) if epi else None, E, 0, None, None, None, VP(y.data_ptr()),
                                    _lib.DTYPE_CODES[dtype], ncols, M * ncols, _st())
    _lib.check(rc, "expert_gemm")
    torch.cuda.synchronize()
    xd, wd = x.double().cpu(), w.double().cpu()
    if route:
        ref_rows, ref_slots = _lists(comb)
        assert counts.cpu().tolist() == [r.numel() for r in ref_rows]
        assert torch.equal(slots.cpu(), ref_slots)
        for z in range(E):
            assert torch.equal(rows.cpu()[z, :ref_rows[z].numel()].long(), ref_rows[z])
    else:
        ref_rows = [torch.arange(M) for _ in range(E)]
    cd = comb.double().cpu()
    worst = 0.0
    for z in range(E):
        rl = ref_rows[z]
        n = rl.numel()
        if n == 0:
            continue
        acc = xd[rl] @ wd[z].t()
        mag = xd[rl].abs() @ wd[z].abs().t()
        got = y[z, :n].double().cpu()
        if epi:
            blk = torch.arange(N).view(-1, 32)
            gi, ui = blk[:, :16].reshape(-1), blk[:, 16:].reshape(-1)
            g_, u_ = acc[:, gi], acc[:, ui]
            silu = g_ * torch.sigmoid(g_)
            cw = cd[rl, z].unsqueeze(1)
            ref = cw * silu * u_
            bound = (cw * RTOL * (1.1 * mag[:, gi] * u_.abs() + silu.abs() * mag[:, ui]) + _rnd(dtype) * ref.abs()
                     + _sub(dtype))
        else:
            ref = acc
            bound = RTOL * mag + _rnd(dtype) * ref.abs() + _sub(dtype)
        err = (got - ref).abs()
        worst = max(worst, float((err / (bound + 1e-300)).max()))
        assert bool((err <= bound + 1e-30).all()), f"expert {z}: worst err / bound = {worst:.3e}"
    _say(f"  worst err / bound = {worst:.2e}")


def test_compact_second_product_and_sum(hip):
    """route=0 with counts: rows past counts[z] are left alone; the compact
    sum equals the dense sum of the zero-filled outputs exactly."""
    dev = hip.torch_device
    M, N, K, E = 224, 1024, 2688, 16
    _say(f"expert_gemm compact M={M} N={N} K={K} E={E}")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    comb = _routing(dev, M, E, 0.5, seed=3)
    ref_rows, ref_slots = _lists(comb)
    cnt = torch.tensor([r.numel() for r in ref_rows], dtype=torch.int32, device=dev)
    act = torch.randn((E, M, K), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((E, N, K), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wp = _packed(w)
    y = torch.full((E, M, N), 3.0, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    _lib.check(L.vnx_expert_gemm_bf16(VP(act.data_ptr()), K, M * K, VP(wp.data_ptr()), wp.stride(0), M, N, K, E, 0,
                                      None, 0, 0, None, VP(cnt.data_ptr()), None, VP(y.data_ptr()), _lib.VNX_BF16, N,
                                      M * N, _st()), "expert_gemm")
    torch.cuda.synchronize()
    yc = y.cpu()
    for z in range(E):
        n = ref_rows[z].numel()
        assert bool((yc[z, n:] == 3.0).all()), f"expert {z} wrote past its count"
        ref = act[z, :n].double().cpu() @ w[z].double().cpu().t()
        mag = act[z, :n].double().cpu().abs() @ w[z].double().cpu().abs().t()
        err = (yc[z, :n].double() - ref).abs()
        assert bool((err <= RTOL * mag + 2.0 ** -8 * ref.abs() + 1e-30).all()), f"expert {z}"
    # dense zero-filled outputs for vnx_sum_experts vs the compact sum
    dense = torch.zeros((E, M, N), dtype=torch.bfloat16)
    for z in range(E):
        dense[z, ref_rows[z]] = yc[z, :ref_rows[z].numel()]
    dense = dense.to(dev)
    out_dense = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.check(L.vnx_sum_experts(VP(dense.data_ptr()), _lib.VNX_BF16, M, E, N, VP(out_dense.data_ptr()), _st()), "sum")
    slots = ref_slots.to(dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.check(L.vnx_sum_expert_rows(VP(y.data_ptr()), _lib.VNX_BF16, N, M * N, VP(slots.data_ptr()), M, E, N,
                                     VP(out.data_ptr()), N, 0, _st()), "sum_rows")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out_dense.cpu())
    # accumulate: res + the sum, as the residual add rounds it
    res = torch.randn((M, N), generator=g, device=dev)
    res0 = res.clone()
    _lib.check(L.vnx_sum_expert_rows(VP(y.data_ptr()), _lib.VNX_BF16, N, M * N, VP(slots.data_ptr()), M, E, N,
                                     VP(res.data_ptr()), N, 1, _st()), "sum_rows accumulate")
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), (res0 + out_dense).cpu())


def test_rejects(hip):
    dev = hip.torch_device
    x = torch.zeros((300, 64), dtype=torch.bfloat16, device=dev)
    w = _packed(torch.zeros((2, 32, 64), dtype=torch.bfloat16, device=dev))
    comb = torch.zeros((300, 2), dtype=torch.float32, device=dev)
    i32 = torch.zeros(600, dtype=torch.int32, device=dev)
    y = torch.zeros((2, 300, 32), dtype=torch.float32, device=dev)
    L = _lib.lib()
    args = lambda M, route, sxb=0: (VP(x.data_ptr()), 64, sxb, VP(w.data_ptr()), w.stride(0), M, 32, 64, 2, 1,
                                    VP(comb.data_ptr()), 2, route, VP(i32.data_ptr()), VP(i32.data_ptr()),
                                    VP(i32.data_ptr()), VP(y.data_ptr()), _lib.VNX_F32, 16, 300 * 32, _st())
    assert L.vnx_expert_gemm_bf16(*args(300, 1)) == _lib.VNX_ERR_UNSUPPORTED      # routing needs M <= 256
    assert L.vnx_expert_gemm_bf16(*args(200, 1, sxb=64)) == _lib.VNX_ERR_INVALID_ARG  # routed x is shared
    assert L.vnx_expert_gemm_bf16(*args(200, 0)) == _lib.VNX_OK
    torch.cuda.synchronize()

"""GPU parity of the fused per-layer kernels of layer.hip against a torch
fp32 (CPU) reference of the same op on the same rounded inputs.

Bars: fp32 outputs within 2e-6 relative (+ 1e-6 absolute) of the reference
(fp32 arithmetic in a possibly different order; exp via the hardware
exp2); 16-bit outputs within one rounding of their type (2^-8 relative for
bf16, 2^-11 for fp16) on top of that.  Sizes cover the 4-wide vector paths
(column counts and strides multiples of 4) and the scalar paths (odd sizes),
the config-5 shapes (D 1024, expert hidden 2688, 16 experts, 224 rows)
included."""
import ctypes

import numpy as np
import pytest
import torch

from versenext_amd import _lib

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _say(*a):
    print(*a, flush=True)


def _tol(dtype):
    return {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]


def _close(out, ref, dtype, rtol=2e-6, atol=1e-6):
    o = out.float().cpu()
    r = ref.float()
    err = (o - r).abs()
    bound = (rtol + _tol(dtype)) * r.abs() + atol
    worst = float((err / (r.abs() + 1e-6)).max())
    assert bool((err <= bound).all()), f"worst rel err {worst:.3e}"


def _st():
    return P(torch.cuda.current_stream().cuda_stream)


def _gen(hip, seed):
    g = torch.Generator(device=hip.torch_device)
    g.manual_seed(seed)
    return g


@pytest.mark.parametrize("M,D,res_dtype,y_dtype", [(224, 1024, torch.bfloat16, torch.bfloat16),
                                                   (7, 1000, None, torch.float32),
                                                   (5, 37, torch.float16, torch.float16),
                                                   (3, 4096, torch.float32, torch.float32)])
def test_rmsnorm(hip, M, D, res_dtype, y_dtype):
    _say(f"rmsnorm M={M} D={D} res={res_dtype} y={y_dtype}")
    dev = hip.torch_device
    g = _gen(hip, M + D)
    x = torch.randn((M, D), generator=g, device=dev)
    res = torch.randn((M, D), generator=g, device=dev).to(res_dtype) if res_dtype else None
    w = torch.rand((D,), generator=g, device=dev) + 0.5
    xo = torch.empty_like(x)
    y = torch.empty((M, D), dtype=y_dtype, device=dev)
    eps = 1e-6
    _lib.check(_lib.lib().vnx_rmsnorm(P(x.data_ptr()), D, P(res.data_ptr()) if res is not None else None,
                                      _lib.DTYPE_CODES[res_dtype] if res_dtype else 0, D, P(w.data_ptr()), eps, M, D,
                                      P(xo.data_ptr()), D, P(y.data_ptr()), _lib.DTYPE_CODES[y_dtype], D, _st()),
               "rmsnorm")
    torch.cuda.synchronize()
    s = x.cpu() + (res.float().cpu() if res is not None else 0.0)
    ref = s / torch.sqrt((s * s).mean(dim=-1, keepdim=True) + eps) * w.cpu()
    _close(xo, s, torch.float32)
    _close(y, ref, y_dtype, rtol=2e-5)


@pytest.mark.parametrize("B,n,H,Hkv,d,rope", [(32, 7, 16, 8, 64, 1), (3, 1, 4, 2, 10, 1), (2, 5, 4, 4, 64, 0)])
def test_rope_kv(hip, B, n, H, Hkv, d, rope):
    _say(f"rope_kv B={B} n={n} H={H} Hkv={Hkv} d={d} rope={rope}")
    dev = hip.torch_device
    g = _gen(hip, B * n + d)
    cap, T = 64, 80
    heads = H + 2 * Hkv
    qkv = torch.randn((B * n, heads * d), generator=g, device=dev).to(torch.bfloat16)
    lens = torch.randint(0, cap - n + 2, (B,), generator=g, device=dev, dtype=torch.int32)
    lens[0] = cap - n + 1          # its last row falls past the cache and is skipped
    ang = torch.rand((T, d), generator=g, device=dev) * 6.0
    cos, sin = torch.cos(ang), torch.sin(ang)
    q = torch.zeros((B, H, n, d), dtype=torch.bfloat16, device=dev)
    kc = torch.zeros((B, Hkv, cap, d), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    _lib.check(_lib.lib().vnx_rope_kv(
        P(qkv.data_ptr()), _lib.VNX_BF16, qkv.stride(0), B, n, H, Hkv, d, P(lens.data_ptr()), P(cos.data_ptr()),
        P(sin.data_ptr()), T, rope, P(q.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()), _lib.VNX_BF16,
        kc.stride(0), kc.stride(1), kc.stride(2), cap, _st()), "rope_kv")
    torch.cuda.synchronize()
    x = qkv.float().cpu().view(B, n, heads, d)
    L = lens.long().cpu()
    pos = (L.view(B, 1) + torch.arange(n).view(1, n))                        # (B, n)
    ok = pos < cap
    pc = pos.clamp(max=T - 1)
    c, s_ = cos.cpu()[pc].unsqueeze(2), sin.cpu()[pc].unsqueeze(2)           # (B, n, 1, d)
    half = d // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    xr = x * c + rot * s_ if rope else x
    ref_q = xr[:, :, :H].permute(0, 2, 1, 3)
    qm = ok.view(B, 1, n, 1).expand(B, H, n, d)
    _close(q.cpu()[qm].view(-1), torch.where(qm, ref_q, torch.zeros(()))[qm].view(-1), torch.bfloat16, rtol=2e-6)
    ref_k = torch.zeros((B, Hkv, cap, d))
    ref_v = torch.zeros((B, Hkv, cap, d))
    for b in range(B):
        for i in range(n):
            if ok[b, i]:
                ref_k[b, :, pos[b, i]] = xr[b, i, H:H + Hkv]
                ref_v[b, :, pos[b, i]] = x[b, i, H + Hkv:]
    _close(kc, ref_k, torch.bfloat16)
    _close(vc, ref_v, torch.bfloat16)


@pytest.mark.parametrize("M,Hf,dt,odt", [(224, 2752, torch.bfloat16, torch.bfloat16),
                                         (32, 4096, torch.float16, torch.float16),
                                         (9, 37, torch.bfloat16, torch.float32),
                                         (4, 100, torch.float32, torch.bfloat16)])
def test_swiglu(hip, M, Hf, dt, odt):
    _say(f"swiglu M={M} Hf={Hf} {dt}->{odt}")
    dev = hip.torch_device
    g = _gen(hip, M + Hf)
    gu = (torch.randn((M, 2 * Hf), generator=g, device=dev) * 3).to(dt)
    out = torch.empty((M, Hf), dtype=odt, device=dev)
    _lib.check(_lib.lib().vnx_swiglu(P(gu.data_ptr()), _lib.DTYPE_CODES[dt], gu.stride(0), M, Hf, P(out.data_ptr()),
                                     _lib.DTYPE_CODES[odt], Hf, _st()), "swiglu")
    torch.cuda.synchronize()
    a, u = gu.float().cpu()[:, :Hf], gu.float().cpu()[:, Hf:]
    _close(out, torch.nn.functional.silu(a) * u, odt, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M,PE,He,layout,odt", [(224, 16, 2688, "expert", torch.bfloat16),
                                                (6, 8, 37, "expert", torch.float32),
                                                (5, 4, 64, "row", torch.float16),
                                                (3, 6, 30, "row", torch.bfloat16)])
def test_mod_swiglu_and_sum(hip, M, PE, He, layout, odt):
    _say(f"mod_swiglu M={M} PE={PE} He={He} layout={layout} out={odt}")
    dev = hip.torch_device
    g = _gen(hip, M * PE + He)
    comb = torch.rand((M, PE), generator=g, device=dev)
    comb[torch.rand((M, PE), generator=g, device=dev) < 0.5] = 0.0   # unselected experts
    if layout == "expert":
        gu = (torch.randn((PE, M, 2 * He), generator=g, device=dev) * 2).to(torch.bfloat16)
        ldg, sxg = 2 * He, M * 2 * He
        out = torch.empty((PE, M, He), dtype=odt, device=dev)
        ldo, sxo = He, M * He
        gm = gu.float().cpu().permute(1, 0, 2)                           # (M, PE, 2He)
    else:
        gu = (torch.randn((M, PE * 2 * He), generator=g, device=dev) * 2).to(torch.bfloat16)
        ldg, sxg = PE * 2 * He, 2 * He
        out = torch.empty((M, PE * He), dtype=odt, device=dev)
        ldo, sxo = PE * He, He
        gm = gu.float().cpu().view(M, PE, 2 * He)
    _lib.check(_lib.lib().vnx_mod_swiglu(P(gu.data_ptr()), _lib.VNX_BF16, ldg, sxg, P(comb.data_ptr()), PE, M, PE,
                                         He, P(out.data_ptr()), _lib.DTYPE_CODES[odt], ldo, sxo, _st()), "mod_swiglu")
    torch.cuda.synchronize()
    ref = comb.cpu().unsqueeze(-1) * torch.nn.functional.silu(gm[..., :He]) * gm[..., He:]   # (M, PE, He)
    got = out.float().cpu().permute(1, 0, 2) if layout == "expert" else out.float().cpu().view(M, PE, He)
    _close(got, ref, odt, rtol=1e-5, atol=1e-6)
    assert bool((got[comb.cpu() == 0] == 0).all())
    if layout == "expert":
        y = out.contiguous()
        s = torch.empty((M, He), dtype=torch.float32, device=dev)
        _lib.check(_lib.lib().vnx_sum_experts(P(y.data_ptr()), _lib.DTYPE_CODES[odt], M, PE, He, P(s.data_ptr()),
                                              _st()), "sum_experts")
        torch.cuda.synchronize()
        ref_s = torch.zeros((M, He))
        for x in range(PE):   # fp32 accumulation in expert order
            ref_s = ref_s + y.float().cpu()[x]
        _close(s, ref_s, torch.float32, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("M,D,NP,NE,topk", [(224, 1024, 4, 4, 2), (5, 100, 2, 3, 1), (33, 64, 1, 8, 3)])
def test_mod_route_from_hidden(hip, M, D, NP, NE, topk, norm):
    """vnx_mod_route_x (router products + routing) against torch fp32
    logits and the reference rule: softmax over all part logits, per part the
    top-k expert logits (ties to the lower index) re-softmaxed.  norm: the
    input is the raw row and the kernel applies RMSNorm (fp64 reference of
    x * rstd * w; the bf16 copies within one rounding)."""
    _say(f"mod_route_x M={M} D={D} P={NP} E={NE} topk={topk} norm={norm}")
    dev = hip.torch_device
    g = _gen(hip, M + D + NP * NE)
    h = torch.randn((M, D), generator=g, device=dev) * (3.0 if norm else 1.0)
    nw = torch.rand((D,), generator=g, device=dev) + 0.5
    eps = 1e-6
    R = NP + NP * NE
    wr = torch.randn((R, D), generator=g, device=dev) * 0.02   # router init scale: logits of order 1
    comb = torch.empty((M, NP * NE), dtype=torch.float32, device=dev)
    copies = 3
    xo = torch.empty((copies, M, D), dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.lib().vnx_mod_route_x(P(h.data_ptr()), D, P(nw.data_ptr()) if norm else None, eps,
                                          P(wr.data_ptr()), D, M, D, NP, NE, topk, P(comb.data_ptr()), NP * NE,
                                          P(xo.data_ptr()), D, M * D, copies, _st()), "mod_route_x")
    torch.cuda.synchronize()
    hd = h.double().cpu()
    if norm:
        hd = hd / torch.sqrt((hd * hd).mean(dim=1, keepdim=True) + eps) * nw.double().cpu()
        err = (xo.double().cpu() - hd.unsqueeze(0)).abs()
        assert bool((err <= 2.0 ** -8 * hd.abs().unsqueeze(0) + 1e-6 * hd.abs().unsqueeze(0) + 1e-30).all())
    else:
        assert torch.equal(xo.cpu(), h.to(torch.bfloat16).cpu().unsqueeze(0).expand(copies, M, D))
    lg = (hd @ wr.double().cpu().t())                                      # (M, R)
    pw = torch.softmax(lg[:, :NP], dim=-1)
    ref = torch.zeros((M, NP * NE), dtype=torch.float64)
    for p_ in range(NP):
        le = lg[:, NP + p_ * NE:NP + (p_ + 1) * NE]
        idx = torch.argsort(-le, dim=-1, stable=True)[:, :topk]
        sel = torch.gather(le, 1, idx)
        w = torch.softmax(sel, dim=-1) * pw[:, p_:p_ + 1]
        ref[:, p_ * NE:(p_ + 1) * NE].scatter_(1, idx, w)
    got = comb.double().cpu()
    assert bool(((got > 0) == (ref > 0)).all()), "selected experts differ"
    assert float((got - ref).abs().max()) < 2e-5

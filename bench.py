"""Benchmark: fused speculative acceptance on one MI355X.

One step = one vnx_spec_accept call over B=64 rows, k=8 draft positions,
V=248,320 (target logits (64,9,V) fp32 ~ N(0,2), draft = target[:, :8] +
N(0,0.5), T=0.8, no top-k, draft ids drawn from q, uniforms U(0,1)); inputs
are resident in HBM before the timed region.

value = algorithmic bytes per step / mean step time, with
  bytes = 4*V*[B*(2k+1) + sum_b r_b], r_b = 2 if row b rejects (p_n and q_n
  re-read by the residual draw) else 1 (p_k re-read by the bonus draw).
roofline = the acceptance path's kernel, k_spec_stage: one call is a
  pipeline of P+2 launches of it (the row LSE streaming of part s beside the
  accept + mass of part s-1 and the draw of part s-2); achieved = the call's
  algorithmic bytes / the summed duration of its launches, timed with HIP
  events the library records on the launch stream (vnx_profile_begin /
  vnx_profile_end).  traffic = HBM bytes per call from the committed
  rocprofv3 FETCH_SIZE / WRITE_SIZE summary, when present.
The CPU baseline is the numpy/C checker (oracle/) on a bounded sample of the
same workload, timed on the host's cores (threads over batch rows).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
B, K, V, T = 64, 8, 248320, 0.8
MAX_PHASES = 7  # kMaxPhases of the library's profiler
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_spec_stage_config2_pmc.md")


def make_inputs_gpu(device):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(0)
    tgt = torch.randn((B, K + 1, V), generator=g, device=device) * 2.0
    dft = tgt[:, :K] + torch.randn((B, K, V), generator=g, device=device) * 0.5
    q = torch.softmax(dft / T, dim=-1).reshape(B * K, V)
    ids = torch.multinomial(q, 1, generator=g).reshape(B, K)
    u = torch.rand((B, K + 1), generator=g, device=device)
    return tgt.contiguous(), dft.contiguous(), ids.contiguous(), u.contiguous()


def algorithmic_bytes(accept_len):
    r = sum(2 if int(n) < K else 1 for n in accept_len)
    return 4 * V * (B * (2 * K + 1) + r)


def traffic_from_profile():
    """HBM bytes per vnx_spec_accept call (all its k_spec_stage launches) from
    the committed PMC summary (the line `traffic_bytes_per_call: N`), or None."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_call:\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


def cpu_baseline(tgt, dft, ids, u, budget_s: float = 12.0):
    """Times the CPU checker on a bounded sample: whole config-2 batches, rows
    split over the host's cores, repeated until about budget_s of CPU work."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle.speculative import spec_accept

    cores = max(1, min(16, os.cpu_count() or 1))
    tgt, dft, ids, u = tgt.cpu().numpy(), dft.cpu().numpy(), ids.cpu().numpy(), u.cpu().numpy()
    chunks = np.array_split(np.arange(B), cores)

    def part(idx):
        return spec_accept(tgt[idx], dft[idx], ids[idx], u[idx], T)

    reps, total_t, total_bytes = 0, 0.0, 0
    while True:
        t0 = time.perf_counter()
        with ThreadPoolExecutor(max_workers=cores) as ex:
            outs = list(ex.map(part, [c for c in chunks if len(c)]))
        dt = time.perf_counter() - t0
        alen = np.concatenate([o["accept_len"] for o in outs])
        total_t += dt
        total_bytes += algorithmic_bytes(alen)
        reps += 1
        if total_t > budget_s or reps >= 200:
            break
    return dict(value=round(total_bytes / total_t / 1e9, 3), unit="GB/s", cores=cores, kind="port",
                sample=f"{reps} full config-2 batches (B={B}, k={K}, V={V}) through oracle.speculative."
                       f"spec_accept (numpy fp64 LSE + C canonical draw), {cores} threads over batch rows; "
                       f"{total_t / reps:.3f} s per batch")


GEMV_SHAPES = (("tied_head", 248320, 1024), ("w_gate_up", 4096, 1024), ("w_down", 1024, 4096))


def bench_gemv(args):
    """weight-only INT4 (group 128, fp16 scales) and INT8
    (per-channel) GEMV, weights N(0, 0.02), fp16 activations N(0, 1), B in
    {1, 8, 32}.  bytes per launch = weight + scales + 2*B*K (fp16 x) + 4*B*N
    (fp32 y).  Time: the C entry point is called `steps` times back to back on
    preallocated buffers, between two HIP events on its stream, so the small
    FFN layers are timed on the GPU rather than on the Python launch path."""
    import ctypes
    import numpy as np
    import torch
    from versenext_amd import get_backend
    from versenext_amd import quant as VQ
    from versenext_amd import _lib

    hip = get_backend("rocm:0")
    L = _lib.lib()
    dev = hip.torch_device
    g = torch.Generator(device=dev)
    g.manual_seed(20)
    rows = []
    for name, N, K in GEMV_SHAPES:
        w = torch.randn((N, K), generator=g, device=dev) * 0.02
        packed = {"int4_g128": VQ.quantize_int4_g(w, 128), "int8": VQ.quantize_int8(w)}
        del w
        for qtype in ("int4_g128", "int8"):
            wq, sc = packed[qtype]
            for B in (1, 8, 32):
                x = (torch.randn((B, K), generator=g, device=dev)).to(torch.float16)
                y = torch.empty((B, N), dtype=torch.float32, device=dev)
                ws = torch.zeros(max(256, L.vnx_gemv_workspace(B, N, K)), dtype=torch.uint8, device=dev)
                stream = torch.cuda.current_stream(dev)
                st = ctypes.c_void_p(stream.cuda_stream)
                P = ctypes.c_void_p
                if qtype == "int8":
                    call, argv = L.vnx_gemv_w8, (P(x.data_ptr()), K, P(wq.data_ptr()), wq.stride(0),
                                                 P(sc.data_ptr()), B, N, K, P(y.data_ptr()), N,
                                                 P(ws.data_ptr()), ws.numel(), st)
                else:
                    call, argv = L.vnx_gemv_w4, (P(x.data_ptr()), K, P(wq.data_ptr()), wq.stride(0),
                                                 P(sc.data_ptr()), _lib.VNX_F16, sc.stride(0), B, N, K, 128,
                                                 P(y.data_ptr()), N, P(ws.data_ptr()), ws.numel(), st)
                _lib.check(call(*argv), "gemv")
                for _ in range(args.warmup):
                    call(*argv)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(args.steps):
                    call(*argv)
                e1.record(stream)
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / args.steps
                nbytes = VQ.weight_bytes(qtype, N, K) + 2 * B * K + 4 * B * N
                gbs = nbytes / (us * 1e-6) / 1e9
                rows.append({"shape": name, "N": N, "K": K, "qtype": qtype, "B": B, "us": round(us, 2),
                             "bytes": nbytes, "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                             "TFLOP/s": round(2 * B * N * K / (us * 1e-6) / 1e12, 2)})
    head = [r for r in rows if r["shape"] == "tied_head" and r["qtype"] == "int4_g128"]
    best = max(head, key=lambda r: r["GB/s"])
    out = {"metric": "quantized GEMV HBM GB/s (config 4, INT4 g128 tied head, B=1)",
           "value": [r for r in head if r["B"] == 1][0]["GB/s"], "unit": "GB/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "higher_is_better": True, "dtype": "int4/int8 x fp16",
           "data": "synthetic", "config": {"workload": "BASELINE config 4: weight-only dequant-GEMV"},
           "roofline": {"bound": "hbm", "achieved": best["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": best["frac"], "traffic": None, "kernel": "k_qgemv_stream<*, 8, 2> (tied head)"},
           "results": rows}
    print(json.dumps(out), flush=True)


def _timed(call, argv, steps, warmup, stream):
    """Mean microseconds of `call(*argv)` issued back to back on `stream`
    between two HIP events (torch's events on the library's launch stream)."""
    import torch
    from versenext_amd import _lib
    _lib.check(call(*argv), call.__name__)
    for _ in range(warmup):
        call(*argv)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        call(*argv)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


def bench_tree(args):
    """tree verification.  B = 16, tree (4,3,2) = 40 nodes,
    16 heads x 64 over a 2048-token bf16 KV prefix (N(0,1)); target logits
    (16, 41, V) and draft logits (16, 17, V) fp32 N(0, 2).  Three kernels,
    each timed alone with the C entry point called back to back on
    preallocated buffers:
      vnx_row_topk    expansion: node tokens = top-b of the parent's draft row,
                      bytes 4*V*B*17;
      vnx_tree_attn   ancestor-masked attention, bytes = K/V prefix 2*B*Hkv*Tp*d*2
                      + q, out, tree K/V 4*B*H*N*d*2 (bf16 out);
      vnx_tree_greedy argmax of the 41 target rows + longest accepted path,
                      bytes 4*V*B*41."""
    import numpy as np
    import torch
    from versenext_amd import get_backend, _lib
    from versenext_amd import tree as TR

    hip = get_backend("rocm:0")
    L = _lib.lib()
    dev = hip.torch_device
    Bt, H, Hkv, d, Tp = 16, 16, 16, 64, 2048
    par = TR.tree_from_branching((4, 3, 2))
    N = par.size
    g = torch.Generator(device=dev)
    g.manual_seed(10)
    q = torch.randn((Bt, H, N, d), generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn((Bt, Hkv, Tp, d), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((Bt, Hkv, Tp, d), generator=g, device=dev).to(torch.bfloat16)
    kt = torch.randn((Bt, Hkv, N, d), generator=g, device=dev).to(torch.bfloat16)
    vt = torch.randn((Bt, Hkv, N, d), generator=g, device=dev).to(torch.bfloat16)
    tgt = torch.randn((Bt, N + 1, V), generator=g, device=dev) * 2.0
    dft = torch.randn((Bt, 17, V), generator=g, device=dev) * 2.0
    stream = torch.cuda.current_stream(dev)
    st = ctypes.c_void_p(stream.cuda_stream)
    P = ctypes.c_void_p
    rows = []

    # expansion: top-b of the 17 parent draft rows (b = 4, the widest level)
    tok = hip.expand_tree(dft, par).contiguous()
    ids = torch.empty((Bt * 17, 4), dtype=torch.int64, device=dev)
    ws_k = torch.zeros(L.vnx_row_topk_workspace(Bt * 17, V, 4), dtype=torch.uint8, device=dev)
    us = _timed(L.vnx_row_topk, (P(dft.data_ptr()), _lib.VNX_F32, Bt * 17, V, V, 4, P(ids.data_ptr()), None, 4,
                                 P(ws_k.data_ptr()), ws_k.numel(), st), args.steps, args.warmup, stream)
    nb = 4 * V * Bt * 17
    rows.append({"kernel": "vnx_row_topk (b=4)", "us": round(us, 2), "bytes": nb,
                 "GB/s": round(nb / us / 1e3, 1), "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)})

    # attention
    words = torch.from_numpy(TR.ancestor_words(par).view(np.int64)).to(dev)
    out = torch.empty((Bt, H, N, d), dtype=torch.bfloat16, device=dev)
    a = _lib.TreeAttnArgs()
    a.q = q.data_ptr(); a.q_strides[:] = list(q.stride()[:3])
    a.k_cache = kc.data_ptr(); a.v_cache = vc.data_ptr(); a.cache_strides[:] = list(kc.stride()[:3])
    a.k_tree = kt.data_ptr(); a.v_tree = vt.data_ptr(); a.tree_strides[:] = list(kt.stride()[:3])
    a.anc = words.data_ptr(); a.anc_batch_stride = 0
    a.out = out.data_ptr(); a.out_dtype = _lib.VNX_BF16; a.out_strides[:] = list(out.stride()[:3])
    a.B, a.H, a.Hkv, a.Tp, a.N, a.d = Bt, H, Hkv, Tp, N, d
    a.scale = 1.0 / float(np.sqrt(d))
    ws_a = torch.zeros(max(256, L.vnx_tree_attn_workspace(Bt, H, Hkv, N, Tp, d)), dtype=torch.uint8, device=dev)
    us = _timed(L.vnx_tree_attn, (ctypes.byref(a), P(ws_a.data_ptr()), ws_a.numel(), st), args.steps,
                args.warmup, stream)
    nb = 2 * Bt * Hkv * Tp * d * 2 + 4 * Bt * H * N * d * 2
    flop = 4 * Bt * H * N * (Tp + N) * d
    attn = {"kernel": "vnx_tree_attn", "us": round(us, 2), "bytes": nb, "GB/s": round(nb / us / 1e3, 1),
            "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4), "TFLOP/s": round(flop / us / 1e6, 2)}
    rows.append(attn)

    # greedy path over the target rows
    alen = torch.empty(Bt, dtype=torch.int32, device=dev)
    best = torch.empty(Bt, dtype=torch.int32, device=dev)
    oids = torch.empty((Bt, N + 1), dtype=torch.int64, device=dev)
    ws_g = torch.zeros(L.vnx_tree_greedy_workspace(Bt, N, V), dtype=torch.uint8, device=dev)
    parc = np.ascontiguousarray(par, dtype=np.int32)
    us = _timed(L.vnx_tree_greedy, (P(tgt.data_ptr()), _lib.VNX_F32, Bt, N, V, V, (N + 1) * V, P(tok.data_ptr()), N,
                                    parc.ctypes.data_as(P), P(alen.data_ptr()), P(best.data_ptr()),
                                    P(oids.data_ptr()), None, P(ws_g.data_ptr()), ws_g.numel(), st),
                args.steps, args.warmup, stream)
    nb = 4 * V * Bt * (N + 1)
    greedy = {"kernel": "vnx_tree_greedy", "us": round(us, 2), "bytes": nb, "GB/s": round(nb / us / 1e3, 1),
              "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    rows.append(greedy)
    total_us = sum(r["us"] for r in rows)
    total_b = sum(r["bytes"] for r in rows)
    out_line = {"metric": "tree verification HBM GB/s (config 3: expansion + attention + greedy path)",
                "value": round(total_b / total_us / 1e3, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": round(total_us / 1e3, 4), "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "bf16 attention / f32 logits",
                "data": "synthetic",
                "config": {"workload": "BASELINE config 3: tree verification", "batch": Bt, "tree": [4, 3, 2],
                           "nodes": N, "heads": H, "kv_heads": Hkv, "head_dim": d, "kv_prefix": Tp, "vocab": V},
                "roofline": {"bound": "hbm", "achieved": greedy["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": greedy["frac"], "traffic": None, "kernel": "vnx_tree_greedy"},
                "accept_len": alen.cpu().tolist(), "results": rows}
    print(json.dumps(out_line), flush=True)


def bench_lmhead(args):
    """Verify-pass LM head (vnx_lm_head): logits (M, V) = x (M, 1024) . W^T with
    M = B*(k+1) = 32*7 = 224 (config 5's verify batch), W the 248,320 x 1024
    bf16 tied embedding (N(0, 0.02)), x bf16 N(0, 1).  bytes = 2*V*K (W) +
    2*M*K (x) + out_bytes*M*V; flop = 2*M*V*K.  Timed back to back on
    preallocated buffers; torch.matmul (hipBLASLt, bf16 out) on the same
    operands is timed beside it."""
    import torch
    from versenext_amd import get_backend, _lib

    hip = get_backend("rocm:0")
    L = _lib.lib()
    dev = hip.torch_device
    M, Kd, Vh = 224, 1024, V
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    x = torch.randn((M, Kd), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((Vh, Kd), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    st = ctypes.c_void_p(stream.cuda_stream)
    P = ctypes.c_void_p
    rows = []
    flop = 2 * M * Vh * Kd
    for name, dt, esz in (("f32", _lib.VNX_F32, 4), ("bf16", _lib.VNX_BF16, 2)):
        out = torch.empty((M, Vh), dtype=torch.float32 if esz == 4 else torch.bfloat16, device=dev)
        us = _timed(L.vnx_lm_head, (P(x.data_ptr()), Kd, P(w.data_ptr()), Kd, M, Kd, Vh, P(out.data_ptr()), dt, Vh,
                                    st), args.steps, args.warmup, stream)
        nb = 2 * Vh * Kd + 2 * M * Kd + esz * M * Vh
        rows.append({"kernel": f"vnx_lm_head ({name} out)", "us": round(us, 2), "bytes": nb,
                     "GB/s": round(nb / us / 1e3, 1), "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
                     "TFLOP/s": round(flop / us / 1e6, 1), "frac_mfma": round(flop / us / 1e6 / 2500.0, 4)})
    # hipBLASLt reference point (bf16 out)
    for _ in range(args.warmup):
        torch.matmul(x, w.t())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        torch.matmul(x, w.t())
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    nb = 2 * Vh * Kd + 2 * M * Kd + 2 * M * Vh
    rows.append({"kernel": "torch.matmul bf16 (hipBLASLt)", "us": round(us, 2), "bytes": nb,
                 "GB/s": round(nb / us / 1e3, 1), "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
                 "TFLOP/s": round(flop / us / 1e6, 1), "frac_mfma": round(flop / us / 1e6 / 2500.0, 4)})
    main_row = rows[0]
    print(json.dumps({"metric": "verify LM head HBM GB/s (M=224, K=1024, V=248,320, fp32 logits)",
                      "value": main_row["GB/s"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
                      "warmup": args.warmup, "ms_per_step": round(main_row["us"] / 1e3, 4),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                      "data": "synthetic",
                      "config": {"workload": "config 5 verify pass: tied LM head over B*(k+1) = 224 rows"},
                      "roofline": {"bound": "hbm", "achieved": main_row["GB/s"], "peak": HBM_PEAK_GBS,
                                   "unit": "GB/s", "frac": main_row["frac_hbm"], "traffic": None,
                                   "kernel": "k_lm_head<14, false>"},
                      "results": rows}), flush=True)


E2E_B, E2E_K, E2E_T0, E2E_NEW, E2E_TEMP = 32, 6, 512, 256, 0.8


def build_e2e(hip, B=E2E_B, k=E2E_K, T0=E2E_T0, n_new=E2E_NEW, draft_layers=2, seed=0):
    """BASELINE config 5 models on the GPU: the CometSparkV05 mate target
    (random init, bf16) and a 2-layer mate-width draft with INT4 group-128
    weights and head, caches for T0 + n_new + 2(k+1) positions."""
    import torch
    from versenext_amd import model as VM
    dev = hip.torch_device
    cap = T0 + n_new + 2 * (k + 1) + 16
    tcfg, dcfg = VM.mate_target(), VM.mate_draft(draft_layers)
    Wt = VM.init_weights(tcfg, seed=seed, device=dev)
    target = VM.CometSparkGPU(tcfg, Wt, hip, batch=B, capacity=cap, dtype=torch.bfloat16)
    del Wt
    Wd = VM.init_weights(dcfg, seed=seed + 1, device=dev)
    draft = VM.CometSparkGPU(dcfg, Wd, hip, batch=B, capacity=cap, dtype=torch.bfloat16, int4=True)
    del Wd
    torch.cuda.empty_cache()
    return target, draft


def cpu_baseline_e2e(Wt, Wd, prompt, budget_s: float = 15.0):
    """The reference's CPU verify path restated in numpy (oracle/model.py:
    full re-forward of [context, drafts] per round with no KV cache, head read
    at the k+1 verified positions; draft re-forwarded per token; canonical
    acceptance), timed on one sequence of the config-5 workload for about
    budget_s of host time, BLAS threads limited to the box's CPU share."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import model as OM
    from versenext_amd import model as VM

    cores = max(1, min(16, os.cpu_count() or 1))
    ct, cd = VM.mate_target(), VM.mate_draft(2)
    rng = np.random.default_rng(31)
    seq = [int(t) for t in prompt]
    rounds, toks, tsum = 0, 0, 0.0
    with threadpool_limits(limits=cores):
        while rounds < 1 or (tsum < budget_s and rounds < 8):
            ud = rng.random(E2E_K).astype(np.float32)
            ua = rng.random(E2E_K + 1).astype(np.float32)
            t0 = time.perf_counter()
            acc = OM.spec_round_cpu(Wt, ct, Wd, cd, seq, E2E_K, E2E_TEMP, ud, ua)
            tsum += time.perf_counter() - t0
            seq += acc
            toks += len(acc)
            rounds += 1
    return dict(value=round(toks / tsum, 3), unit="tokens/s", cores=cores, kind="port",
                sample=f"{rounds} speculative rounds (k={E2E_K}, T={E2E_TEMP}) of one config-5 sequence "
                       f"(512-token prompt) through oracle.model.spec_round_cpu: numpy fp32 re-forward of the "
                       f"CometSparkV05 target and the 2-layer draft (fp32 weights), {toks} tokens committed, "
                       f"{tsum / rounds:.2f} s per round, {cores} BLAS threads")


def trace_summary(d: str, top: int = 40) -> None:
    """Per-round GPU time by kernel between the two marker kernels of an
    --e2e-mark run (rocprofv3 --kernel-trace --output-format csv): the decode
    rounds of the last run only (no prefill, capture or warm-up)."""
    import collections
    import csv
    import glob
    path = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))[0]
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if "scan" in r["Kernel_Name"].lower()]
    if len(marks) < 2:
        raise SystemExit("no marker kernels in the trace (run bench.py --workload e2e --e2e-mark)")
    win = rows[marks[-2] + 1:marks[-1]]
    lm = sum(1 for r in win if "k_lm_head" in r["Kernel_Name"])  # one verify head per round
    rounds = max(1, lm)
    agg = collections.defaultdict(lambda: [0, 0.0])
    busy = 0.0
    for r in win:
        du = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        agg[r["Kernel_Name"][:110]][0] += 1
        agg[r["Kernel_Name"][:110]][1] += du
        busy += du
    span = (int(win[-1]["End_Timestamp"]) - int(win[0]["Start_Timestamp"])) / 1e3
    print(f"rounds {rounds}; window {span / rounds:.1f} us/round, kernels {len(win) / rounds:.1f}/round, "
          f"kernel time {busy / rounds:.1f} us/round")
    for name, (c, t) in sorted(agg.items(), key=lambda x: -x[1][1])[:top]:
        print(f"{t / rounds:9.1f} us/round {c / rounds:6.1f} calls {t / c:8.1f} us  {name}")


def bench_e2e(args):
    """end-to-end speculative decode.  Target CometSparkV05
    (D 1024, 20 layers = 5 MoD + 15 TriSparse, tied 248,320 head, random init,
    bf16); draft: 2 mate-width TriSparse layers (D 1024, ffn 4096) with INT4
    group-128 weights and tied head; k = 6, batch 32, 512-token uniform-random
    prompts, 256 new tokens per sequence, temperature 0.8.  Each decode round
    is one HIP graph replay.
    value = verified tokens / s = 32 * 256 committed tokens / wall time of the
    decode rounds (prefill timed and reported separately).
    The accept-kernel half of the metric is measured in
    the same run after the models are freed: its k_spec_lse launch is the
    roofline object, and its CPU leg rides along as cpu_baseline_accept."""
    import numpy as np
    import torch
    from versenext_amd import get_backend
    from versenext_amd import model as VM
    from versenext_amd.e2e import SpecDecodeEngine

    hip = get_backend("rocm:0")
    dev = hip.torch_device
    t_build = time.perf_counter()
    Wt_host = Wd_host = None
    if not args.no_cpu:
        Wt_host = {k: v.cpu().numpy() for k, v in VM.init_weights(VM.mate_target(), seed=0, device=dev).items()}
        Wd_host = {k: v.cpu().numpy() for k, v in VM.init_weights(VM.mate_draft(2), seed=1, device=dev).items()}
    target, draft = build_e2e(hip)
    build_s = time.perf_counter() - t_build
    g = torch.Generator(device=dev)
    g.manual_seed(30)
    prompts = torch.randint(0, V, (E2E_B, E2E_T0), generator=g, device=dev)
    eng = SpecDecodeEngine(target, draft, hip, k=E2E_K, temperature=E2E_TEMP, seed=31,
                           use_graph=not args.e2e_eager)
    runs = []
    nruns = max(1, args.e2e_runs)
    mark = torch.ones(64, dtype=torch.int16, device=dev) if args.e2e_mark else None
    if mark is not None:
        # marker kernels (an int16 scan, used nowhere else) bracket the last
        # run's decode rounds in a kernel trace: one after its prefill, one
        # after its last round (see --trace-summary)
        fill = eng._fill_uniforms
        armed = {"on": False}

        def fill_marked():
            if armed["on"]:
                torch.cumsum(mark, 0)
                armed["on"] = False
            fill()
        eng._fill_uniforms = fill_marked
    for r in range(nruns):
        if mark is not None and r == nruns - 1:
            armed["on"] = True
        toks, st = eng.generate(prompts, E2E_NEW)
        if mark is not None and r == nruns - 1:
            torch.cumsum(mark, 0)
            torch.cuda.synchronize()
        runs.append(st)
        print(json.dumps({"e2e_run": r, "rounds": st.rounds, "decode_s": round(st.decode_s, 4),
                          "prefill_s": round(st.prefill_s, 4), "tokens_per_s": round(st.tokens_per_s, 1),
                          "graph": eng.graph is not None}), flush=True)
    timed = runs[-1]
    graphed = eng.graph is not None
    tcfg_name, dcfg_name = target.cfg.name, draft.cfg.name
    prompt0 = prompts[0].cpu().numpy()
    mean_tokens_round = float(np.mean(timed.per_round_tokens)) / E2E_B
    del eng, target, draft, toks
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    acc = bench_accept(args, emit=False)
    out = {"metric": "verified tokens/s (mate target, k=6, bs32)", "value": round(timed.tokens_per_s, 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": timed.rounds, "warmup": len(runs) - 1,
           "ms_per_step": round(timed.decode_s * 1e3 / timed.rounds, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16 target / int4 draft / f32 logits",
           "data": "synthetic (random-init weights, uniform-random prompts)",
           "config": {"workload": "BASELINE config 5: end-to-end speculative decode", "batch": E2E_B, "k": E2E_K,
                      "rounds_as": "HIP graph replays" if graphed else "eager launches",
                      "prompt": E2E_T0, "new_tokens": E2E_NEW, "temperature": E2E_TEMP,
                      "target": tcfg_name, "draft": dcfg_name + ", INT4 g128",
                      "step": "one speculative round: 7 draft forwards + 6 draws, one 7-token target verify "
                              "+ LM head, acceptance, commit"},
           "prefill_s": round(timed.prefill_s, 4), "build_s": round(build_s, 2),
           "mean_tokens_per_round_per_seq": round(mean_tokens_round, 3),
           "roofline": acc["roofline"],
           "accept_kernel": {"metric": acc["metric"], "value": acc["value"], "unit": acc["unit"],
                             "workload": acc["config"]["workload"], "frac_of_hbm_peak":
                             acc["config"]["frac_of_hbm_peak"], "ms_per_call": acc["config"]["event_ms_mean"]}}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_e2e(Wt_host, Wd_host, prompt0)
        out["cpu_baseline_accept"] = acc.get("cpu_baseline")
    print(json.dumps(out), flush=True)


def bench_accept(args, emit=True):
    """one vnx_spec_accept call per step (module docstring)."""
    import numpy as np
    import torch
    from versenext_amd import get_backend
    from versenext_amd import _lib

    hip = get_backend("rocm:0")
    dev = hip.torch_device
    tgt, dft, ids, u = make_inputs_gpu(dev)
    L = _lib.lib()
    # the C entry point on preallocated buffers, issued back to back on one
    # stream, so the timed region holds the library's launches only
    alen = torch.empty(B, dtype=torch.int32, device=dev)
    out_ids = torch.empty((B, K + 1), dtype=torch.int64, device=dev)
    flags = torch.empty((B, K + 1), dtype=torch.uint8, device=dev)
    lse_t = torch.empty((B, K + 1), dtype=torch.float32, device=dev)
    lse_d = torch.empty((B, K), dtype=torch.float32, device=dev)
    ws = torch.zeros(L.vnx_spec_accept_workspace(B, K, V), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    P = ctypes.c_void_p
    argv = (P(tgt.data_ptr()), P(dft.data_ptr()), _lib.VNX_F32, B, K, V, tgt.stride(1), tgt.stride(0),
            dft.stride(1), dft.stride(0), P(ids.data_ptr()), P(u.data_ptr()), T, None, None,
            P(alen.data_ptr()), P(out_ids.data_ptr()), P(flags.data_ptr()), P(lse_t.data_ptr()),
            P(lse_d.data_ptr()), P(ws.data_ptr()), ws.numel(), P(stream.cuda_stream))

    def step():
        return L.vnx_spec_accept(*argv)

    _lib.check(step(), "vnx_spec_accept")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res = {"accept_len": alen}
    # Per-launch times from a second pass of the same steps with the library's
    # stage events (kept out of the timed pass above).
    L = _lib.lib()
    _lib.check(L.vnx_profile_begin(args.steps), "vnx_profile_begin")
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    phase = (ctypes.c_double * MAX_PHASES)()
    ncalls = ctypes.c_int(0)
    _lib.check(L.vnx_profile_end(ctypes.cast(phase, ctypes.c_void_p), MAX_PHASES,
                                 ctypes.cast(ctypes.pointer(ncalls), ctypes.c_void_p)), "vnx_profile_end")
    stage_ms = [float(phase[i]) / max(1, ncalls.value) for i in range(MAX_PHASES) if phase[i] > 0.0]
    alen = res["accept_len"].cpu().numpy()
    nbytes = algorithmic_bytes(alen)
    mean_ms = e0.elapsed_time(e1) / args.steps
    gbs = nbytes / (mean_ms * 1e-3) / 1e9
    call_kernel_ms = sum(stage_ms)
    stage_gbs = nbytes / (call_kernel_ms * 1e-3) / 1e9
    emitted = int(alen.sum()) + B

    if args.calib_copy:
        n = 1 << 28  # 1 GiB of fp32
        src = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    out = {
        "metric": "accept-kernel HBM GB/s",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 2: fused stochastic acceptance (vnx_spec_accept)",
                   "batch": B, "k": K, "vocab": V, "temperature": T, "top_k": None,
                   "logits": "fp32 target N(0,2), draft = target + N(0,0.5)",
                   "bytes_per_step": nbytes, "event_ms_mean": round(mean_ms, 4),
                   "timing": "HIP events around the back-to-back calls of the C entry point",
                   "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(stage_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(stage_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
                     "kernel": "k_spec_stage", "launches_per_call": len(stage_ms),
                     "bytes_per_call": nbytes, "kernel_ms_per_call": round(call_kernel_ms, 4),
                     "timing": "HIP events recorded by the library before each launch and after the last, "
                               "on its stream (each interval includes the gap before the next launch)",
                     "stage_ms_mean": [round(v, 4) for v in stage_ms],
                     "profiled_calls": ncalls.value},
        "emitted_tokens_per_s": round(emitted / (mean_ms * 1e-3), 1),
        "mean_accept_len": round(float(alen.mean()), 3),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(tgt, dft, ids, u)
    if emit:
        print(json.dumps(out), flush=True)
    return out



def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--e2e-runs", type=int, default=2, help="e2e: decode runs (the last is reported)")
    ap.add_argument("--e2e-eager", action="store_true", help="e2e: launch every round eagerly (no HIP graph)")
    ap.add_argument("--e2e-mark", action="store_true",
                    help="e2e: bracket the last run's decode rounds with marker kernels for a kernel trace")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print the per-round kernel table of a rocprofv3 kernel trace of an --e2e-mark run "
                         "(DIR holds *kernel_trace.csv) and exit")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 1 GiB device copy (the known-size kernel that scales PMC counters)")
    ap.add_argument("--workload", default="e2e", choices=("e2e", "accept", "gemv", "tree", "lmhead"),
                    help="e2e: BASELINE config 5 verified tokens/s with the config-2 accept-kernel roofline "
                         "(the bench line); accept: config 2 alone; gemv: config 4; tree: config 3; "
                         "lmhead: the verify-pass LM head")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (one MI355X per box); "
                                   "run with --gpus 1", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.workload == "gemv":
        bench_gemv(args)
        return
    if args.workload == "tree":
        bench_tree(args)
        return
    if args.workload == "lmhead":
        bench_lmhead(args)
        return
    if args.workload == "e2e":
        bench_e2e(args)
        return

    bench_accept(args)

if __name__ == "__main__":
    main()

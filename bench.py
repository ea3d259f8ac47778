"""Benchmark of the MI355X speculative-decoding verification path.

Default line (python bench.py): BASELINE.json's metric, both halves.
- value = verified tokens/s of config 5 (end-to-end speculative decode, the
  mate target with an INT4 draft, B = 32, k = 6, T = 0.8): one step is one
  speculative round (a HIP graph replay); W warm-up rounds, then exactly K
  timed rounds of one generation; value = tokens committed in the K rounds /
  their wall time.
- roofline = the acceptance path of config 2 (vnx_spec_accept, B = 64, k = 8,
  V = 248,320, fp32 logits): its two kernels' launches per call, algorithmic
  bytes 4*V*[B*(2k+1) + sum_b r_b] (r_b = 2 when row b rejects: p_n and q_n
  re-read by the residual draw, else 1: p_k for the bonus draw) over the
  summed launch time, timed with HIP events the library records on its
  stream; accept_kernel = the same bytes over back-to-back calls of the C
  entry point.
- Extra keys carry config 1 (greedy spec decode of the small models), config
  3 (tree verification kernels) and config 4 (INT4 / INT8 GEMV), each with
  its CPU baseline, and a config-5 leg with the VerseNex draft (no embedding
  scale), whose drafts the target mostly rejects.
CPU baselines are the numpy/C restatement of the reference path (oracle/, or
numpy written in the reference's semantics here) on a bounded sample, timed
on the host's cores; each states its core count, CPU model and BLAS.

--workload accept / tree / gemv / lmhead / config1 print one config alone.
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
CPU_THREADS = max(1, min(16, os.cpu_count() or 1))  # the box's CPU share


def cpu_env(threads: int) -> dict:
    """Host facts every CPU number states: threads used, os.cpu_count(), the
    CPU model and numpy's BLAS."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas = ""
    try:
        import numpy as np
        info = np.show_config(mode="dicts")["Build Dependencies"]["blas"]
        blas = f"{info.get('name', '')} {info.get('version', '')}".strip()
    except Exception:
        pass
    return {"cores": threads, "cpu_count": os.cpu_count(), "cpu_model": model, "blas": blas}


def _median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]
MAX_PHASES = 7  # kMaxPhases of the library's profiler
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "vnx_spec_accept_config2.md")


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


def cpu_gemv(packed, qtype, x_list, reps_head: int = 3, reps: int = 5):
    """The reference's QuantizedLinear.forward, path B (quantize.py:467-504:
    int8 weights unpacked once at load, per call cast to fp32, GEMM, scale),
    with the group-128 INT4 format applied as its extension: per call the
    cached int8 q times the fp16 group scales in fp32, then x @ W^T.  Median
    of `reps` calls per batch size (reps_head for the tied head)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import quant as OQ

    wq, sc = packed
    N = wq.shape[0]
    if qtype == "int8":
        q8, s = wq, sc.reshape(-1).astype(np.float32)
        K = q8.shape[1]
    else:
        K = wq.shape[1] * 2
        q8 = OQ.unpack_int4(wq, (N, K))                         # load time, not timed
        s = sc.astype(np.float32)                              # (N, K/128)
    out = {}
    with threadpool_limits(limits=CPU_THREADS):
        for x in x_list:
            ts = []
            for _ in range(reps_head if N > 100000 else reps):
                t0 = time.perf_counter()
                if qtype == "int8":
                    y = x @ q8.astype(np.float32).T
                    y *= s
                else:
                    w = (q8.reshape(N, K // 128, 128).astype(np.float32) * s[:, :, None]).reshape(N, K)
                    y = x @ w.T
                ts.append(time.perf_counter() - t0)
            out[x.shape[0]] = _median(ts)
    return out


def bench_gemv(args, emit=True):
    """weight-only INT4 (group 128, fp16 scales) and INT8
    (per-channel) GEMV, weights N(0, 0.02), fp16 activations N(0, 1), B in
    {1, 8, 32}; the INT4 tied head (N >= 32,768) through vnx_gemv_w4_tiles on
    its tiled copy, the layout the draft model keeps for its head.  bytes per launch = weight + scales + 2*B*K (fp16 x) + 4*B*N
    (fp32 y).  Time: the C entry point is called `steps` times back to back on
    preallocated buffers, between two HIP events on its stream, so the small
    FFN layers are timed on the GPU rather than on the Python launch path.
    The CPU leg (cpu_gemv) runs on the same quantized weights and activations."""
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
    cpu_rows = []
    for name, N, K in GEMV_SHAPES:
        w = torch.randn((N, K), generator=g, device=dev) * 0.02
        packed = {"int4_g128": VQ.quantize_int4_g(w, 128), "int8": VQ.quantize_int8(w)}
        del w
        for qtype in ("int4_g128", "int8"):
            wq, sc = packed[qtype]
            wt = None
            if qtype == "int4_g128" and N >= 32768 and K in (512, 1024):
                wt = hip.pack_w4_tiles(wq, K)   # vnx_gemv_w4_tiles' layout (the tied head's copy)
            xs = []
            for B in (1, 8, 32):
                x = (torch.randn((B, K), generator=g, device=dev)).to(torch.float16)
                xs.append(x)
                y = torch.empty((B, N), dtype=torch.float32, device=dev)
                ws = torch.zeros(max(256, L.vnx_gemv_workspace(B, N, K)), dtype=torch.uint8, device=dev)
                stream = torch.cuda.current_stream(dev)
                st = ctypes.c_void_p(stream.cuda_stream)
                P = ctypes.c_void_p
                if qtype == "int8":
                    call, argv = L.vnx_gemv_w8, (P(x.data_ptr()), K, P(wq.data_ptr()), wq.stride(0),
                                                 P(sc.data_ptr()), B, N, K, P(y.data_ptr()), N,
                                                 P(ws.data_ptr()), ws.numel(), st)
                elif wt is not None:
                    # the tied head as the draft runs it: the tiled copy
                    call, argv = L.vnx_gemv_w4_tiles, (P(x.data_ptr()), K, P(wt.data_ptr()), P(sc.data_ptr()),
                                                       sc.stride(0), B, N, K, P(y.data_ptr()), N, st)
                else:
                    call, argv = L.vnx_gemv_w4, (P(x.data_ptr()), K, P(wq.data_ptr()), wq.stride(0),
                                                 P(sc.data_ptr()), _lib.VNX_F16, sc.stride(0), B, N, K, 128,
                                                 P(y.data_ptr()), N, P(ws.data_ptr()), ws.numel(), st)
                us = _timed(call, argv, args.steps, args.warmup, stream)
                nbytes = VQ.weight_bytes(qtype, N, K) + 2 * B * K + 4 * B * N
                gbs = nbytes / (us * 1e-6) / 1e9
                rows.append({"shape": name, "N": N, "K": K, "qtype": qtype, "B": B, "us": round(us, 2),
                             "entry": call.__name__,
                             "bytes": nbytes, "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                             "TFLOP/s": round(2 * B * N * K / (us * 1e-6) / 1e12, 2)})
            if not args.no_cpu:
                xs_h = [x.float().cpu().numpy() for x in xs]
                t_cpu = cpu_gemv((wq.cpu().numpy(), sc.cpu().numpy()), qtype, xs_h)
                for x in xs_h:
                    Bx = x.shape[0]
                    nbytes = VQ.weight_bytes(qtype, N, K) + 2 * Bx * K + 4 * Bx * N
                    gpu = [r for r in rows if r["shape"] == name and r["qtype"] == qtype and r["B"] == Bx][0]
                    cpu_rows.append({"shape": name, "qtype": qtype, "B": Bx, "ms": round(t_cpu[Bx] * 1e3, 3),
                                     "GB/s": round(nbytes / t_cpu[Bx] / 1e9, 2),
                                     "gpu_speedup": round(t_cpu[Bx] * 1e6 / gpu["us"], 1)})
    head = [r for r in rows if r["shape"] == "tied_head" and r["qtype"] == "int4_g128"]
    best = max(head, key=lambda r: r["GB/s"])
    out = {"metric": "quantized GEMV HBM GB/s (config 4, INT4 g128 tied head, B=1)",
           "value": [r for r in head if r["B"] == 1][0]["GB/s"], "unit": "GB/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "higher_is_better": True, "dtype": "int4/int8 x fp16",
           "data": "synthetic", "config": {"workload": "BASELINE config 4: weight-only dequant-GEMV"},
           "roofline": {"bound": "hbm", "achieved": best["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": best["frac"], "traffic": None,
                        "kernel": "k_qgemv_tiles (vnx_gemv_w4_tiles, tied head)"},
           "results": rows}
    if cpu_rows:
        out["cpu_baseline"] = dict(cpu_env(CPU_THREADS), kind="port", results=cpu_rows,
                                   sample="QuantizedLinear.forward path B semantics (int8 cached at load; per call "
                                          "cast, group-128 scale, BLAS GEMM): median of 5 calls (3 for the tied "
                                          "head) per batch size, fp32 activations")
    if emit:
        print(json.dumps(out), flush=True)
    return out


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


def bench_tree(args, emit=True):
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
    if not args.no_cpu:
        host = dict(q=q.float().cpu().numpy(), kc=kc.float().cpu().numpy(), vc=vc.float().cpu().numpy(),
                    kt=kt.float().cpu().numpy(), vt=vt.float().cpu().numpy(), tgt=tgt.cpu().numpy(),
                    dft=dft.cpu().numpy(), tok=tok.cpu().numpy())
        t_cpu = cpu_tree(host, par)
        cpu_rows = []
        for r in rows:
            key = r["kernel"].split()[0]
            t = t_cpu[key]
            cpu_rows.append({"kernel": key, "ms": round(t * 1e3, 3), "GB/s": round(r["bytes"] / t / 1e9, 2),
                             "gpu_speedup": round(t * 1e6 / r["us"], 1)})
        out_line["cpu_baseline"] = dict(cpu_env(CPU_THREADS), kind="port", results=cpu_rows,
                                        sample="numpy fp32, median of 5: top-b expansion by argpartition, "
                                               "DeviceBackend.attention semantics (softmax(q k^T / sqrt(d) + "
                                               "ancestor mask) v, device.py:260-270), oracle.tree.tree_greedy")
    if emit:
        print(json.dumps(out_line), flush=True)
    return out_line


def cpu_tree(h, par, reps: int = 5):
    """Config 3 on the host, each part timed alone (median of reps): the
    expansion (top-4 ids of the 17 parent draft rows), the ancestor-masked
    attention in the reference's DeviceBackend.attention semantics
    (device.py:260-270, fp32, additive 0 / -inf mask), and the greedy longest
    accepted path (argmax of the 41 target rows + the path rule)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import tree as OT
    from versenext_amd import tree as TR

    B_, H_, N_, d_ = h["q"].shape
    Tp_ = h["kc"].shape[2]
    words = TR.ancestor_words(par)
    bits = ((words[:, None] >> np.arange(N_, dtype=np.uint64)[None, :]) & np.uint64(1)).astype(bool)
    mask = np.zeros((N_, Tp_ + N_), np.float32)
    mask[:, Tp_:][~bits] = -np.inf
    K_ = np.concatenate([h["kc"], h["kt"]], axis=2)
    V_ = np.concatenate([h["vc"], h["vt"]], axis=2)
    res = {}

    def timeit(fn):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return _median(ts)

    def expand():
        x = h["dft"].reshape(-1, h["dft"].shape[-1])
        cand = np.argpartition(x, -4, axis=-1)[:, -4:]
        vals = np.take_along_axis(x, cand, axis=-1)
        order = np.lexsort((cand, -vals), axis=-1)
        return np.take_along_axis(cand, order, axis=-1)

    def attend():
        s_ = np.matmul(h["q"], K_.transpose(0, 1, 3, 2)) * np.float32(1.0 / np.sqrt(d_)) + mask
        s_ = np.exp(s_ - s_.max(axis=-1, keepdims=True))
        s_ /= s_.sum(axis=-1, keepdims=True)
        return np.matmul(s_, V_)

    with threadpool_limits(limits=CPU_THREADS):
        res["vnx_row_topk"] = timeit(expand)
        reps = min(reps, 3)  # ~1-2 s per call
        res["vnx_tree_attn"] = timeit(attend)
        res["vnx_tree_greedy"] = timeit(lambda: OT.tree_greedy(h["tgt"], h["tok"], par))
    return res


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
                                   "kernel": "k_lm_head<7, 4, false, 8, 1>"},
                      "results": rows}), flush=True)


E2E_B, E2E_K, E2E_T0, E2E_NEW, E2E_TEMP = 32, 6, 512, 256, 0.8
# final-norm weight scale of the partial-acceptance draft: its logits shrink
# by this factor, so it puts about 0.7 of its mass on the token both random-
# init models favour (repeating the current one) instead of ~1.0
PARTIAL_ALPHA = 0.6


def build_e2e(hip, B=E2E_B, k=E2E_K, T0=E2E_T0, n_new=E2E_NEW, draft_layers=2, seed=0, versenex=False):
    """BASELINE config 5 models on the GPU: the CometSparkV05 mate target
    (random init, bf16) and a 2-layer mate-width draft with INT4 group-128
    weights and head, caches for T0 + n_new + 2(k+1) positions.  versenex:
    also a second draft of the same shape without the x sqrt(D) embedding
    scale (CometSparkNexLM.forward, cometspark.py:670-690), and a third whose
    final-norm weight is scaled by PARTIAL_ALPHA (a flatter draft, so
    acceptance is partial)."""
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
    draft2 = None
    if versenex:
        dcfg2 = VM.mate_draft(draft_layers)
        dcfg2.embedding_scale = False
        dcfg2.name = dcfg.name.replace("VerseNex draft", "VerseNex draft without the embedding scale")
        draft2 = VM.CometSparkGPU(dcfg2, Wd, hip, batch=B, capacity=cap, dtype=torch.bfloat16, int4=True)
        dcfg3 = VM.mate_draft(draft_layers)
        dcfg3.name = dcfg.name.replace("VerseNex draft", f"VerseNex draft, final norm x {PARTIAL_ALPHA}")
        Wd["norm.weight"] = Wd["norm.weight"] * PARTIAL_ALPHA
        draft3 = VM.CometSparkGPU(dcfg3, Wd, hip, batch=B, capacity=cap, dtype=torch.bfloat16, int4=True)
    del Wd
    torch.cuda.empty_cache()
    return (target, draft, draft2, draft3) if versenex else (target, draft)


def round_floor_bytes(target, draft, B: int, k: int, ctx: float) -> dict:
    """Algorithmic HBM bytes of one speculative round at mean context ctx
    (committed cache rows per sequence): every weight read once per forward
    that uses it, each cache read once per forward, the logits written once
    and read by the kernels that need them.
      target (one (k+1)-token forward): bf16 weights incl. the tied head,
        fp32 router weights; K/V of ctx + k+1 rows per layer;
      draft (k+1 one-token forwards, the last one cache-only): INT4 g128
        linears every forward, the INT4 head k times; its K/V per forward;
      logits: p (B, k+1, V) and q (B, k, V) fp32 written once; each of the k
        draft draws reads its q row twice (row LSE, then the draw mass); the
        acceptance reads p and q once and re-reads p_n and q_n (2 rows)."""
    tc, dc = target.cfg, draft.cfg
    V, D = tc.vocab_size, tc.dim

    def attn_params(c):
        return (c.n_head + 2 * c.n_kv_head) * c.head_dim * c.dim + c.dim * c.n_head * c.head_dim

    tw = V * D * 2
    for kind in tc.layer_pattern:
        tw += attn_params(tc) * 2
        if kind == "mod":
            P, E = tc.num_dense_parts, tc.num_experts_per_part
            tw += P * E * 3 * tc.expert_hidden_eff * D * 2 + (P + P * E) * D * 4
        else:
            tw += 3 * tc.ffn_hidden * D * 2
    kv_t = tc.n_layer * B * (ctx + k + 1) * tc.n_kv_head * tc.head_dim * 2 * 2

    def int4(n, kk):
        return n * kk // 2 + 2 * n * (kk // 128)

    dw_layers = dc.n_layer * (int4((dc.n_head + 2 * dc.n_kv_head) * dc.head_dim, dc.dim)
                              + int4(dc.dim, dc.n_head * dc.head_dim) + int4(2 * dc.ffn_hidden, dc.dim)
                              + int4(dc.dim, dc.ffn_hidden))
    dw = (k + 1) * dw_layers + k * int4(V, D)
    kv_d = (k + 1) * dc.n_layer * B * (ctx + k) * dc.n_kv_head * dc.head_dim * 2 * 2
    logits = 4 * V * B * ((k + 1) + k + 2 * k + (2 * k + 1) + 2)
    total = tw + kv_t + dw + kv_d + logits
    return {"bytes": int(total), "target_weights": int(tw), "target_kv": int(kv_t), "draft_weights": int(dw),
            "draft_kv": int(kv_d), "logits": int(logits), "floor_ms_at_peak": round(total / HBM_PEAK_GBS / 1e6, 4)}


def e2e_rounds(eng, prompts, n_new, steps, warmup, mark=None):
    """Prefill, `warmup` untimed rounds (the first captures the round's HIP
    graph), then exactly `steps` timed rounds of the same generation (mark(),
    when given, runs right before and right after them), each enqueued
    before the previous round's info is read (SpecDecodeEngine.run_rounds).
    Returns (seconds, tokens committed in the timed rounds, per-round token
    counts, prefill seconds)."""
    import torch
    B = eng.B
    prefill_s = eng.prefill(prompts, n_new)
    if eng.use_graph and eng.graph is None:
        eng._capture()
    for _ in range(warmup):
        eng.step()
    torch.cuda.synchronize(eng.dev)
    if mark:
        mark()
    t0 = time.perf_counter()
    per = [int(info[3]) + B for info in eng.run_rounds(steps)]
    torch.cuda.synchronize(eng.dev)
    dt = time.perf_counter() - t0
    if mark:
        mark()
        torch.cuda.synchronize(eng.dev)
    return dt, sum(per), per, prefill_s


def cpu_baseline_e2e(Wt, Wd, prompt, budget_s: float = 15.0):
    """The reference's CPU verify path restated in numpy (oracle/model.py:
    full re-forward of [context, drafts] per round with no KV cache, head read
    at the k+1 verified positions; draft re-forwarded per token; canonical
    acceptance), timed on one sequence of the config-5 workload for about
    budget_s of host time, BLAS threads limited to the box's CPU share.  One
    sequence, not the batch of 32: the reference's verify_then_commit
    commits batch row 0 only (speculative.py:262-268), so its decode loop
    serves one sequence per call, and a 32-row round of this numpy path
    (one (32, 518)-token target re-forward and six draft re-forwards) takes
    about a minute of host time, past the bench's bounded CPU sample."""
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
    """Per-round GPU time by kernel between the first two marker kernels of
    an --e2e-mark run (rocprofv3 --kernel-trace --output-format csv): the
    timed rounds only (no prefill, capture or warm-up)."""
    import collections
    import csv
    import glob
    path = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))[0]
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if "scan" in r["Kernel_Name"].lower()]
    if len(marks) < 2:
        raise SystemExit("no marker kernels in the trace (run bench.py --workload e2e --e2e-mark)")
    win = rows[marks[0] + 1:marks[1]]
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


def bench_e2e(args, full: bool = True):
    """end-to-end speculative decode.  Target CometSparkV05
    (D 1024, 20 layers = 5 MoD + 15 TriSparse, tied 248,320 head, random init,
    bf16); draft: 2 mate-width TriSparse layers (D 1024, ffn 4096) with INT4
    group-128 weights and tied head; k = 6, batch 32, 512-token uniform-random
    prompts, T = 0.8.  One step = one speculative round (a HIP graph replay):
    `warmup` rounds, then `steps` timed rounds of one generation of at least
    256 new tokens per sequence; value = tokens committed in the timed rounds
    / their wall time (prefill reported separately).  The accept-kernel half
    of the metric is measured in the same run after the
    models are freed, then configs 3, 4 and 1."""
    import numpy as np
    import torch
    from versenext_amd import get_backend
    from versenext_amd import model as VM
    from versenext_amd.e2e import SpecDecodeEngine

    hip = get_backend("rocm:0")
    dev = hip.torch_device
    # config 2's 1.2 GB of logits are allocated first, while device memory is
    # unfragmented, and stay resident until their measurement
    acc_inputs = make_inputs_gpu(dev)
    n_new = max(E2E_NEW, (args.warmup + args.steps + 2) * (E2E_K + 1))
    t_build = time.perf_counter()
    Wt_host = Wd_host = None
    if not args.no_cpu:
        Wt_host = {k: v.cpu().numpy() for k, v in VM.init_weights(VM.mate_target(), seed=0, device=dev).items()}
        Wd_host = {k: v.cpu().numpy() for k, v in VM.init_weights(VM.mate_draft(2), seed=1, device=dev).items()}
    target, draft, draft2, draft3 = build_e2e(hip, n_new=n_new, versenex=True)
    build_s = time.perf_counter() - t_build
    g = torch.Generator(device=dev)
    g.manual_seed(30)
    prompts = torch.randint(0, V, (E2E_B, E2E_T0), generator=g, device=dev)
    eng = SpecDecodeEngine(target, draft, hip, k=E2E_K, temperature=E2E_TEMP, seed=31,
                           use_graph=not args.e2e_eager)
    mark = None
    if args.e2e_mark:
        # marker kernels (an int16 scan, used nowhere else) bracket the timed
        # rounds in a kernel trace (see --trace-summary)
        mvec = torch.ones(64, dtype=torch.int16, device=dev)

        def mark():
            torch.cumsum(mvec, 0)
    dt, toks, per, prefill_s = e2e_rounds(eng, prompts, n_new, args.steps, args.warmup, mark)
    graphed = eng.graph is not None
    ms_round = dt * 1e3 / args.steps
    ctx = E2E_T0 + (args.warmup + args.steps / 2) * float(np.mean(per)) / E2E_B
    floor = round_floor_bytes(target, draft, E2E_B, E2E_K, ctx)
    floor["frac_of_round"] = round(floor["floor_ms_at_peak"] / ms_round, 4)
    floor["mean_context"] = round(ctx, 1)
    # the whole 256-token generation, for continuity with earlier runs
    toks_gen, st = eng.generate(prompts, E2E_NEW)
    gen = {"tokens_per_s": round(st.tokens_per_s, 1), "rounds": st.rounds, "decode_s": round(st.decode_s, 4),
           "new_tokens_per_seq": E2E_NEW}
    del toks_gen
    # the same round with the VerseNex draft (no embedding scale)
    eng2 = SpecDecodeEngine(target, draft2, hip, k=E2E_K, temperature=E2E_TEMP, seed=31,
                            use_graph=not args.e2e_eager)
    dt2, toks2, per2, _ = e2e_rounds(eng2, prompts, n_new, args.steps, args.warmup)
    versenex = {"draft": draft2.cfg.name + ", INT4 g128", "tokens_per_s": round(toks2 / dt2, 1),
                "ms_per_round": round(dt2 * 1e3 / args.steps, 3),
                "mean_tokens_per_round_per_seq": round(toks2 / args.steps / E2E_B, 3)}
    # and with the flatter draft: acceptance between none and all
    eng3 = SpecDecodeEngine(target, draft3, hip, k=E2E_K, temperature=E2E_TEMP, seed=31,
                            use_graph=not args.e2e_eager)
    dt3, toks3, per3, _ = e2e_rounds(eng3, prompts, n_new, args.steps, args.warmup)
    partial = {"draft": draft3.cfg.name + ", INT4 g128", "tokens_per_s": round(toks3 / dt3, 1),
               "ms_per_round": round(dt3 * 1e3 / args.steps, 3),
               "mean_tokens_per_round_per_seq": round(toks3 / args.steps / E2E_B, 3),
               "acceptance_rate": round((toks3 / args.steps / E2E_B - 1) / E2E_K, 4),
               "tokens_per_round_min_max": [min(per3), max(per3)]}
    tcfg_name, dcfg_name = target.cfg.name, draft.cfg.name
    prompt0 = prompts[0].cpu().numpy()
    del eng, eng2, eng3, target, draft, draft2, draft3
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    if not full:
        print(json.dumps({"metric": "verified tokens/s (mate target, k=6, bs32)", "value": round(toks / dt, 1),
                          "unit": "tokens/s", "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": round(ms_round, 3),
                          "mean_tokens_per_round_per_seq": round(toks / args.steps / E2E_B, 3),
                          "round_floor": floor, "e2e_versenex_draft": versenex,
                          "e2e_partial_accept": partial}), flush=True)
        return
    acc = bench_accept(args, emit=False, inputs=acc_inputs, calls=max(args.steps, 100), warm=max(args.warmup, 50))
    del acc_inputs
    tree = bench_tree(args, emit=False)
    gemv = bench_gemv(args, emit=False)
    c1 = bench_config1(args, emit=False)
    samp = bench_sampler(args, emit=False)
    out = {"metric": "verified tokens/s (mate target, k=6, bs32)", "value": round(toks / dt, 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms_round, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16 target / int4 draft / f32 logits",
           "data": "synthetic (random-init weights, uniform-random prompts)",
           "config": {"workload": "BASELINE config 5: end-to-end speculative decode", "batch": E2E_B, "k": E2E_K,
                      "rounds_as": "HIP graph replays" if graphed else "eager launches",
                      "prompt": E2E_T0, "new_tokens": n_new, "temperature": E2E_TEMP,
                      "target": tcfg_name, "draft": dcfg_name + ", INT4 g128",
                      "step": "one speculative round: 7 draft forwards + 6 draws, one 7-token target verify "
                              "+ LM head, acceptance, commit"},
           "prefill_s": round(prefill_s, 4), "build_s": round(build_s, 2),
           "mean_tokens_per_round_per_seq": round(toks / args.steps / E2E_B, 3),
           "acceptance_rate": round((toks / args.steps / E2E_B - 1) / E2E_K, 4),
           "round_floor": floor, "generation_256": gen, "e2e_versenex_draft": versenex,
           "e2e_partial_accept": partial,
           "roofline": acc["roofline"],
           "accept_kernel": {"metric": acc["metric"], "value": acc["value"], "unit": acc["unit"],
                             "workload": acc["config"]["workload"], "frac_of_hbm_peak":
                             acc["config"]["frac_of_hbm_peak"], "ms_per_call": acc["config"]["event_ms_mean"],
                             "calls_timed": acc["steps"], "warmup_calls": acc["warmup"]},
           "config3_tree": {k: tree.get(k) for k in ("value", "unit", "ms_per_step", "results", "cpu_baseline")},
           "config4_gemv": {k: gemv.get(k) for k in ("value", "unit", "results", "cpu_baseline")},
           "config1": c1,
           "sampler": {k: samp.get(k) for k in ("value", "unit", "results", "cpu_baseline")}}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_e2e(Wt_host, Wd_host, prompt0)
        out["cpu_baseline_accept"] = acc.get("cpu_baseline")
    print(json.dumps(out), flush=True)


def bench_sampler(args, emit=True):
    """Sampler.sample on the GPU (vnx_sampler_sample), config-5 batch: 32 rows
    of 248,320 fp32 logits N(0, 2), T 0.8, three settings: top-k 50 (the
    radix select), top-p 0.9 (the nucleus), top-k 50 + top-p 0.9; and the
    CometSpark step (calibration + exactly-k 50).  Each row is split over
    32 workgroups: with top-k one read of the row and a per-row candidate
    search (2 launches, 4 with the calibration sums); top-p alone 7 launches,
    the passes after the first mostly from the L2 / MALL; bytes = the row
    read once, 4 V per row.  CPU: the reference's
    numpy Sampler (partition, exp / sum, argsort / cumsum / searchsorted,
    choice) per row, restated in oracle/sampler.py, all 32 rows on the host's
    cores (up to 16 threads)."""
    import numpy as np
    import torch
    from versenext_amd import get_backend, _lib
    from oracle import sampler as OS

    hip = get_backend("rocm:0")
    L = _lib.lib()
    dev = hip.torch_device
    Bs = E2E_B
    g = torch.Generator(device=dev)
    g.manual_seed(41)
    x = torch.randn((Bs, V), generator=g, device=dev) * 2.0
    u = torch.rand((Bs,), generator=g, device=dev)
    ids = torch.empty(Bs, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    st = ctypes.c_void_p(stream.cuda_stream)
    P = ctypes.c_void_p
    rows = []
    nb = 4 * V * Bs
    settings = [("top_k 50", 50, 1.0, 0), ("top_p 0.9", 0, 0.9, 0), ("top_k 50 + top_p 0.9", 50, 0.9, 0),
                ("CometSpark: calibrate + exactly-k 50", 50, 1.0, _lib.SAMPLE_EXACT_K | _lib.SAMPLE_CALIBRATE)]
    ws = torch.empty(L.vnx_sampler_workspace(Bs, V, _lib.VNX_F32), dtype=torch.uint8, device=dev)
    for name, k, p, mode in settings:
        us = _timed(L.vnx_sampler_sample, (P(x.data_ptr()), _lib.VNX_F32, Bs, V, V, 0.8, k, p, mode, 1.2, 1e-8,
                                           P(u.data_ptr()), P(ids.data_ptr()), None, None, None, None, None, None,
                                           P(ws.data_ptr()), ws.numel(), st), args.steps, args.warmup, stream)
        rows.append({"setting": name, "us": round(us, 2), "rows_per_s": round(Bs / us * 1e6, 1),
                     "GB/s": round(nb / us / 1e3, 1), "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)})
    out = {"metric": "sampled rows/s (config-5 batch, V=248320)", "value": rows[2]["rows_per_s"],
           "unit": "rows/s", "steps": args.steps, "warmup": args.warmup, "results": rows,
           "config": {"workload": "Sampler.sample, 32 x 248320 fp32 rows, T 0.8", "bytes_per_call": nb}}
    if not args.no_cpu:
        from concurrent.futures import ThreadPoolExecutor
        xs = x.cpu().numpy()
        us_ = u.cpu().numpy()
        threads = max(1, min(16, os.cpu_count() or 1))
        cpu_rows = []
        with ThreadPoolExecutor(max_workers=threads) as ex:
            for name, k, p, mode in settings[:3]:
                t0 = time.perf_counter()
                list(ex.map(lambda b: OS.sample(xs[b], 0.8, k, p, us_[b]), range(Bs)))
                dt = time.perf_counter() - t0
                cpu_rows.append({"setting": name, "rows_per_s": round(Bs / dt, 2)})
        out["cpu_baseline"] = dict(cpu_env(threads), kind="port", value=cpu_rows[2]["rows_per_s"], unit="rows/s",
                                   results=cpu_rows,
                                   sample=f"all {Bs} rows, one row per task on {threads} threads (numpy releases "
                                          f"the GIL in its partition, sort, exp and cumsum)")
    if emit:
        print(json.dumps(out), flush=True)
    return out


def bench_config1(args, emit=True):
    """greedy speculative decode of the CometSparkV05Small
    target (V 256, D 64, 2 layers) with the 1-layer D = 32 draft, k = 4, one
    sequence, the 16-token prompt and 128 new tokens, with the weights the
    reference itself wrote (tests/golden/cometspark_small.npz, np.random.seed
    (0) construction).  GPU: SpecDecodeEngine, fp32, greedy verify, rounds as
    graph replays; CPU: the reference's loop restated in numpy
    (oracle.model.spec_decode_greedy: draft argmax by re-forward, full
    re-forward verify, speculative.py:230-310), the full 128 tokens."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits
    from oracle import model as OM
    from versenext_amd import get_backend
    from versenext_amd import model as VM
    from versenext_amd.e2e import SpecDecodeEngine

    hip = get_backend("rocm:0")
    z = np.load(os.path.join(ROOT, "tests", "golden", "cometspark_small.npz"))
    gold = {k: z[k] for k in z.files}

    def w(prefix):
        return {k[len(prefix):]: v for k, v in gold.items() if k.startswith(prefix) and not k.endswith("head.weight")}

    Wt, Wd = w("t/"), w("d/")
    ct, cd = VM.small_target(), VM.small_draft()
    torch.backends.cuda.matmul.allow_tf32 = False
    t = VM.CometSparkGPU(ct, Wt, hip, batch=1, capacity=256, dtype=torch.float32)
    d = VM.CometSparkGPU(cd, Wd, hip, batch=1, capacity=256, dtype=torch.float32)
    eng = SpecDecodeEngine(t, d, hip, k=4, temperature=0.0, use_graph=True)
    prompt = torch.from_numpy(gold["prompt"][None].astype(np.int64)).to(hip.torch_device)
    eng.generate(prompt, 128)                                   # captures the graph
    runs = [eng.generate(prompt, 128) for _ in range(3)]
    toks, st = runs[-1]
    ok = bool(np.array_equal(toks.cpu().numpy()[0], gold["greedy128"]))
    out = {"workload": "BASELINE config 1: greedy spec decode, CometSparkV05Small target + 1-layer draft, k=4, "
                       "128 tokens", "gpu_tokens_per_s": round(_median([r[1].tokens_per_s for r in runs]), 1),
           "gpu_rounds": st.rounds, "gpu_stream_equals_reference_greedy128": ok}
    if not args.no_cpu:
        with threadpool_limits(limits=CPU_THREADS):
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                ctoks, steps = OM.spec_decode_greedy(Wt, ct, Wd, cd, gold["prompt"], 128, 4)
                ts.append(time.perf_counter() - t0)
        tc = _median(ts)
        out["cpu_baseline"] = dict(cpu_env(CPU_THREADS), kind="port", value=round(128 / tc, 2), unit="tokens/s",
                                   sample=f"the full 128-token run (median of 3), {steps} verify rounds, "
                                          f"stream equals greedy128: {bool(np.array_equal(ctoks, gold['greedy128']))}")
        out["gpu_speedup"] = round(out["gpu_tokens_per_s"] / out["cpu_baseline"]["value"], 2)
    if emit:
        print(json.dumps(out), flush=True)
    return out


def bench_accept(args, emit=True, inputs=None, calls=None, warm=None):
    """one vnx_spec_accept call per step (module docstring).
    inputs: (target, draft, ids, uniforms) already on the device (make_inputs_gpu).
    calls / warm: timed and warm-up calls (default --steps / --warmup); the
    default run's accept leg times more of these 0.2 ms calls than it runs
    rounds, after a longer warm-up, so the figure is the steady clock's."""
    calls = args.steps if calls is None else calls
    warm = args.warmup if warm is None else warm
    import numpy as np
    import torch
    from versenext_amd import get_backend
    from versenext_amd import _lib

    hip = get_backend("rocm:0")
    dev = hip.torch_device
    tgt, dft, ids, u = inputs if inputs is not None else make_inputs_gpu(dev)
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
    for _ in range(warm):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(calls):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res = {"accept_len": alen}
    # Per-launch times from a second pass of the same steps with the library's
    # stage events (kept out of the timed pass above).
    L = _lib.lib()
    _lib.check(L.vnx_profile_begin(calls), "vnx_profile_begin")
    for _ in range(calls):
        step()
    torch.cuda.synchronize()
    phase = (ctypes.c_double * MAX_PHASES)()
    ncalls = ctypes.c_int(0)
    _lib.check(L.vnx_profile_end(ctypes.cast(phase, ctypes.c_void_p), MAX_PHASES,
                                 ctypes.cast(ctypes.pointer(ncalls), ctypes.c_void_p)), "vnx_profile_end")
    stage_ms = [float(phase[i]) / max(1, ncalls.value) for i in range(MAX_PHASES) if phase[i] > 0.0]
    alen = res["accept_len"].cpu().numpy()
    nbytes = algorithmic_bytes(alen)
    mean_ms = e0.elapsed_time(e1) / calls
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
        "steps": calls,
        "warmup": warm,
        "ms_per_step": round(wall * 1e3 / calls, 4),
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
                     "kernel": "k_spec_lse + k_spec_mass_draw", "launches_per_call": len(stage_ms),
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
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--e2e-eager", action="store_true", help="e2e: launch every round eagerly (no HIP graph)")
    ap.add_argument("--e2e-mark", action="store_true",
                    help="e2e: bracket the last run's decode rounds with marker kernels for a kernel trace")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print the per-round kernel table of a rocprofv3 kernel trace of an --e2e-mark run "
                         "(DIR holds *kernel_trace.csv) and exit")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 1 GiB device copy (the known-size kernel that scales PMC counters)")
    ap.add_argument("--workload", default="all",
                    choices=("all", "e2e", "accept", "gemv", "tree", "lmhead", "config1", "sampler"),
                    help="all: the bench line (config 5 verified tokens/s, the config-2 accept-kernel "
                         "roofline, configs 1, 3 and 4 as extra keys); e2e: config 5 alone; accept: config 2; "
                         "gemv: config 4; tree: config 3; config1: config 1; lmhead: the verify-pass LM head")
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
    if args.workload == "sampler":
        bench_sampler(args)
        return
    if args.workload == "config1":
        bench_config1(args)
        return
    if args.workload in ("all", "e2e"):
        bench_e2e(args, full=args.workload == "all")
        return

    bench_accept(args)

if __name__ == "__main__":
    main()

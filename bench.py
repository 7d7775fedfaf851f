#!/usr/bin/env python3
"""bench.py — INT8 transformer-inference kernels on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload all]

The default run (`--workload all`) measures every BASELINE configuration:
  * the headline, config 2: decode attention over a contiguous INT8 KV cache,
    B=32 H=32 D=128 ctx=8192 (2 GiB of K+V), 1% of channels x8 before
    per-token quantization.  One step = one decode call over the whole batch
    (one kernel launch: 8 chunks per (b,h) merged in LDS), inputs already
    resident in HBM.  Its
    effective KV-read bandwidth (2*B*H*S*D bytes / step time, TB/s) is the
    line's `value`;
  * under `configs`: config 1 (B1 H12 D64 ctx 1K), config 3 (B8 H32 D64 ctx
    32K) with its ctx sweep 2K..16K, config 4 (the INT8 MLP, T=4096
    4096->16384->4096), config 5 (causal prefill B4 H32 S4096 D128) and the
    end-to-end pre-LN block, INT8 against FP16 (block.py).
Every figure is the median of 5 windows of `--steps` steps after `--warmup`
untimed steps (config 1 and the sweep points: enough steps for ~2 ms windows,
`steps_per_window`), timed with HIP events on the launch stream; every config has
its own `roofline` and an oracle parity check (all rows for decode).  Decode
steps shorter than 50 us also report `graph_us`: the same steps captured in a
HIP graph and replayed, the device time per step without the host's per-call
issue (config 1's step is otherwise set by one ctypes call and one launch).
`cpu_baseline` times this repo's torch-CPU fp32 restatement of the reference's
CPU path (dequantize, then common/baseline.py's math) on a bounded sample of
the same workload on this host.  Prints ONE JSON line; details go to stderr.
`--workload decode|decode-sweep|mlp|prefill|decode-paged|gemm|block` runs one
part alone (the profiling commands under profiles/ use these).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

REPO_DIR = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO_DIR, "int8-transformer-kernels_amd")
sys.path.insert(0, REPO_DIR)
sys.path.insert(0, PKG_DIR)

HBM_PEAK_GBS = 8000.0
METRIC = ("decode attn µs + effective KV-read TB/s (% HBM peak), "
          "B=32 H=32 D=128 8K ctx")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_steps(fn, steps, warmup, stream):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


WINDOWS = 5
GRAPH_BELOW_MS = 0.05  # decode steps shorter than this are also timed from a captured graph


def time_graph(step_on, n_steps, stream, windows=WINDOWS):
    """Device time per step with the host's launch issue taken out: `n_steps` steps are
    captured in one HIP graph (step_on(handle) returns a step that launches on the stream
    with that handle, here the capture stream) and the graph is replayed in `windows` timed
    windows on `stream`.  Returns the median window's ms per step."""
    import ctypes

    import torch

    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.graph(graph, stream=cap):
        fn = step_on(ctypes.c_void_p(cap.cuda_stream))
        for _ in range(n_steps):
            fn()
    torch.cuda.synchronize()
    graph.replay()
    runs = [time_steps(graph.replay, 1, 0, stream) / n_steps for _ in range(windows)]
    del graph
    return statistics.median(runs)


def time_windows(fn, steps, warmup, stream, windows=WINDOWS):
    """`warmup` untimed steps, then `windows` timed windows of exactly `steps` steps, each
    bracketed by a device synchronisation and timed with HIP events on `stream` (the stream
    the kernels are launched on).  Returns (median window's ms per step, every window's)."""
    for _ in range(warmup):
        fn()
    runs = [time_steps(fn, steps, 0, stream) for _ in range(windows)]
    return statistics.median(runs), [round(r, 5) for r in runs]


def calibrate(dev):
    """On-box ceilings: non-temporal chunked streaming read, vector copy, i8 MFMA."""
    import ctypes

    import torch

    L = ctypes.CDLL(os.path.join(PKG_DIR, "libint8k_calib.so"))
    stream = torch.cuda.current_stream(dev)
    st = ctypes.c_void_p(stream.cuda_stream)
    nbytes = 4 << 30
    buf = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.empty(1 << 22, dtype=torch.int32, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    ms = time_steps(lambda: L.int8k_calib_stream_chunk_nt(P(buf), ctypes.c_size_t(nbytes),
                                                          P(sink), 4096, st), 10, 2, stream)
    read_tbs = nbytes / (ms * 1e-3) / 1e12
    half = nbytes // 2
    ms = time_steps(lambda: L.int8k_calib_copy(P(buf), ctypes.c_void_p(buf.data_ptr() + half),
                                               ctypes.c_size_t(half), 8192, st), 10, 2, stream)
    copy_tbs = 2 * half / (ms * 1e-3) / 1e12
    blocks, iters = 4096, 2000
    ms = time_steps(lambda: L.int8k_calib_mfma_i8(blocks, iters, P(sink), st), 5, 1, stream)
    mfma_tops = blocks * 4 * iters * 4 * 32768 / (ms * 1e-3) / 1e12
    del buf
    torch.cuda.empty_cache()
    sustained = mfma_sustained(L, dev)
    return {"hbm_stream_read_TBps": round(read_tbs, 3), "hbm_copy_rw_TBps": round(copy_tbs, 3),
            "mfma_i8_16x16x64_TOPS": round(mfma_tops, 1), **sustained,
            "copy_kernel_bytes": {"read": half, "write": half}}


def mfma_sustained(L, dev, steps=10):
    """Back-to-back v_mfma_i32_32x32x32_i8 (one wave per SIMD, ~0.3 ms launches) with
    operands drawn from uniform random int8 and from zeros: the part's sustained clock,
    and so its MFMA rate, depends on the operand bits toggled."""
    import ctypes

    import torch

    stream = torch.cuda.current_stream(dev)
    st = ctypes.c_void_p(stream.cuda_stream)
    blocks, iters = 256, 1000
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(7)
    out = {}
    for name, src in (("random", torch.randint(-128, 128, (blocks * 8192,), dtype=torch.int8,
                                               device=dev, generator=g)),
                      ("zero", torch.zeros(blocks * 8192, dtype=torch.int8, device=dev))):
        ms = time_steps(lambda: L.int8k_calib_mfma_i8_32_src(
            ctypes.c_void_p(src.data_ptr()), blocks, iters, ctypes.c_void_p(sink.data_ptr()), st),
            steps, 2, stream)
        out[f"mfma_i8_32x32x32_sustained_{name}_TOPS"] = round(
            blocks * 4 * iters * 16 * 65536 / (ms * 1e-3) / 1e12, 1)
    return out


def _threads_info():
    import torch

    return f"os.cpu_count()={os.cpu_count()}, torch.get_num_threads()={torch.get_num_threads()}"


def torch_cpu_decode(Q, K, V, sQ, sK, sV):
    """The reference's CPU/PyTorch path for decode, restated: dequantize with
    int8.float() * per-token scale, then fp32 attention exactly as
    common/baseline.py:18-22 with Q.unsqueeze(2) (validation/check_decode.py:68).
    Q [n,D] int8, K/V [n,S,D] int8, sQ [n], sK/sV [n,S] fp32 (CPU tensors) -> [n,D] fp32."""
    import torch

    D = Q.shape[-1]
    q = (Q.float() * sQ[:, None]).unsqueeze(1)
    k = K.float() * sK[..., None]
    v = V.float() * sV[..., None]
    w = torch.matmul(q, k.transpose(-2, -1)) * D ** -0.5
    w = torch.softmax(w, dim=-1)
    return torch.matmul(w, v).squeeze(1)


def cpu_baseline_decode(host, D, S, budget_s=10.0, one_thread_s=2.0, gpu_out=None):
    """torch-CPU fp32 restatement of the reference path (torch_cpu_decode) timed on this
    host over (b,h) heads of the workload, in chunks, passing over the heads again until
    `budget_s` of wall time is spent; then one thread for `one_thread_s`.  `host` holds the
    workload's CPU tensors (Q [BH,D], K/V [BH,S,D], sQ [BH], sK/sV [BH,S])."""
    import torch

    Q, K, V, sQ, sK, sV = host
    BH = Q.shape[0]
    chunk = max(1, min(BH, (64 << 20) // (S * D * 4)))  # ~64 MB of fp32 K per chunk
    err = None
    if gpu_out is not None:
        n = min(chunk, BH)
        ref = torch_cpu_decode(Q[:n], K[:n], V[:n], sQ[:n], sK[:n], sV[:n])
        err = float((ref - gpu_out[:n].float().cpu()).abs().max())

    def run(budget, step):
        heads, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget:
            lo = heads % BH
            hi = min(BH, lo + step)
            torch_cpu_decode(Q[lo:hi], K[lo:hi], V[lo:hi], sQ[lo:hi], sK[lo:hi], sV[lo:hi])
            heads += hi - lo
        return heads, time.perf_counter() - t0

    threads = torch.get_num_threads()
    heads, dt = run(budget_s, chunk)
    torch.set_num_threads(1)
    try:
        h1, dt1 = run(one_thread_s, max(1, chunk // 8))
    finally:
        torch.set_num_threads(threads)
    per = 2 * S * D
    return dict(value=heads * per / dt / 1e12, unit="TB/s", cores=threads, kind="port",
                sample=f"torch-CPU fp32 restatement of common/baseline.py:18-22 (dequantize, "
                       f"matmul, softmax, matmul) on {heads} (b,h) heads ({heads / BH:.2f} "
                       f"passes over the {BH} heads of this workload, {chunk} per call) in "
                       f"{dt:.1f} s; {_threads_info()}; 1 thread: "
                       f"{h1 * per / dt1 / 1e9:.2f} GB/s ({h1} heads in {dt1:.1f} s)"
                       + (f"; max |cpu - gpu| on the first {min(chunk, BH)} heads {err:.1e}"
                          if err is not None else ""),
                one_thread_GBps=round(h1 * per / dt1 / 1e9, 3))


def measured_traffic(key):
    """HBM bytes per launch of the dominant kernel, from the committed PMC summary."""
    try:
        with open(os.path.join(REPO_DIR, "profiles", "traffic.json")) as f:
            t = json.load(f).get(key)
    except (OSError, ValueError):
        return None
    return None if t is None else int(t["read_bytes"]) + int(t["write_bytes"])


def hbm_roofline(nbytes, ms, kernel, traffic_key=None, ceiling=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    r = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(gbs / HBM_PEAK_GBS, 4),
         "traffic": measured_traffic(traffic_key) if traffic_key else None, "kernel": kernel}
    if ceiling:
        r["measured_ceiling"] = ceiling
    return r


def decode_kernel_label(nsplit):
    """The kernels one contiguous decode step launches for a plan of `nsplit` chunks per
    (b,h): up to 16 chunks run as one block each (merged in LDS), unless
    INT8K_DECODE_BLOCK=0 turns that off."""
    if nsplit <= 16 and os.environ.get("INT8K_DECODE_BLOCK", "1") != "0":
        return "decode_block_kernel (one launch per step)"
    return "decode_split_kernel + decode_combine_kernel (one step)"


def measure_decode(B, H, D, S, outlier_frac, args, dev, stream, keep_host=False,
                   min_window_ms=0.0):
    """One decode configuration: seeded inputs, `--warmup` untimed steps, then the median of
    5 windows of `--steps` steps.  Cases whose K+V (+ scales) are under
    512 MB cycle through enough copies of the cache (at least 3, 768 MB in total) that the
    256 MB Infinity Cache cannot serve a step from the previous one.  Every (b,h) row of
    the output is checked against the C oracle."""
    import ctypes

    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import oracle_c

    BH = B * H
    case = workloads.decode_case(B, H, D, S, seed=args.seed, outlier_frac=outlier_frac,
                                 device=dev)
    Q = case["Qi"].reshape(BH, D)
    sQ = case["sQ"].reshape(-1)
    kv = (case["Ki"].reshape(BH, S, D), case["Vi"].reshape(BH, S, D), case["sK"].reshape(-1),
          case["sV"].reshape(-1))
    del case
    kv_bytes = 2 * BH * S * D
    total = kv_bytes + 2 * BH * S * 4
    n_copies = 1 if total >= (512 << 20) else max(3, -(-(768 << 20) // total))
    copies = [kv] + [tuple(t.clone() for t in kv) for _ in range(n_copies - 1)]
    out = torch.empty((BH, D), dtype=torch.float16, device=dev)
    ws = torch.empty(max(capi.decode_workspace_bytes(BH, S, D, args.nsplit), 1),
                     dtype=torch.uint8, device=dev)
    # A step is one call of the C ABI entry point with its arguments built once per
    # cache copy, as a serving loop holds them: the Python wrapper's per-call checks
    # would otherwise set the time of the short steps (config 1's kernel takes ~6 us).
    fn = capi.load().int8k_decode_attention_forward
    Pt = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(stream.cuda_stream)
    def step_on(handle):
        calls = [(Pt(Q), Pt(K), Pt(V), Pt(out), Pt(sQ), Pt(sK), Pt(sV), BH, S, D, args.nsplit,
                  Pt(ws), ws.numel(), handle) for (K, V, sK, sV) in copies]
        it = [0]

        def step():
            a = calls[it[0] % n_copies]
            it[0] += 1
            rc = fn(*a)
            if rc != 0:
                capi.check("int8k_decode_attention_forward", rc)
        return step

    # a window of a few microsecond-steps is at the mercy of host jitter: the short configs
    # (min_window_ms > 0) take enough steps per window to last about that long, estimated
    # from their bytes at 5 TB/s plus ~6 us per launch
    est_ms = total / 5e12 * 1e3 + 0.006
    steps = max(args.steps, math.ceil(min_window_ms / est_ms))
    # every cache copy is touched before the first timed window
    ms, windows = time_windows(step_on(st), steps, max(args.warmup, 2 * n_copies), stream)
    # a short step can be set by the host's issue rate (one ctypes call and one launch per
    # step): its device time is also taken from a captured graph of steps over the copies
    graph_ms = (time_graph(step_on, n_copies * max(1, 40 // n_copies), stream)
                if ms < GRAPH_BELOW_MS else None)
    K, V, sK, sV = kv
    out.zero_()
    capi.decode_attention(Q, K, V, sQ, sK, sV, nsplit=args.nsplit, out=out, workspace=ws)
    torch.cuda.synchronize()
    host = (Q.cpu(), K.cpu(), V.cpu(), sQ.cpu(), sK.reshape(BH, S).cpu(),
            sV.reshape(BH, S).cpu())
    ref = oracle_c.decode_attention(*(t.numpy() for t in host))
    got = out.float().cpu().numpy()
    err = float(np.abs(got - ref).max())
    cos = float((got * ref).sum() / max(np.linalg.norm(got) * np.linalg.norm(ref), 1e-30))
    if not (err <= 2e-2 and cos >= 0.9999):
        raise SystemExit(f"decode B{B} H{H} D{D} S{S} does not match the oracle "
                         f"(max_abs={err}, cos={cos})")
    tbs = kv_bytes / (ms * 1e-3) / 1e12
    row = {"B": B, "H": H, "D": D, "ctx": S,
           "nsplit": capi.decode_num_splits(BH, S, D, args.nsplit),
           "us": round(ms * 1e3, 2), "TBps": round(tbs, 4),
           "pct_hbm_peak": round(tbs * 1e3 / HBM_PEAK_GBS * 100, 2),
           "windows_ms": windows, "steps_per_window": steps, "cache_copies": n_copies,
           "parity": {"rows_checked": BH, "max_abs": err, "cos": round(cos, 7)}}
    if graph_ms is not None:
        row["graph_us"] = round(graph_ms * 1e3, 2)
        row["graph_pct_hbm_peak"] = round(kv_bytes / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBS * 100,
                                          2)
    log(f"[bench] decode B{B} H{H} D{D} ctx{S}: {ms * 1e3:.1f} us {tbs:.3f} TB/s "
        f"({row['pct_hbm_peak']:.1f}% of 8 TB/s), {n_copies} cache copies, "
        f"all {BH} rows vs oracle: max_abs {err:.1e} cos {cos:.6f}"
        + (f"; from a captured graph {graph_ms * 1e3:.1f} us per step" if graph_ms else ""))
    return row, (host if keep_host else None), (out if keep_host else None)


def bench_decode(args):
    """The headline alone: decode B32 H32 D128 ctx 8192."""
    import torch

    B, H, D, S = args.batch, args.heads, args.head_dim, args.ctx
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    ceilings = None if args.no_calibrate else calibrate(dev)
    if ceilings:
        log(f"[bench] on-box ceilings: {ceilings}")
    log(f"[bench] decode inputs B{B} H{H} D{D} S{S} (outliers 1% x8)")
    row, host, out = measure_decode(B, H, D, S, 0.01, args, dev, stream,
                                    keep_host=not args.no_cpu_baseline)
    ms = row["us"] / 1e3
    kv_bytes = 2 * B * H * S * D
    res = {
        "metric": METRIC,
        "value": row["TBps"],
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": row["us"],
        "pct_hbm_peak": row["pct_hbm_peak"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1), 1% channels x8, per-token int8)",
        "config": {"workload": f"int8-kv decode attention B={B} H={H} D={D} ctx={S}",
                   "batch": B, "heads": H, "head_dim": D, "ctx": S, "nsplit": row["nsplit"],
                   "kv_bytes": kv_bytes, "scale_bytes": 2 * B * H * S * 4,
                   "timing": f"median of {WINDOWS} windows of {args.steps} steps",
                   "windows_ms": row["windows_ms"], "parity": row["parity"]},
        "roofline": hbm_roofline(kv_bytes, ms, decode_kernel_label(row["nsplit"]),
                                 f"decode_b{B}h{H}d{D}_s{S}",
                                 round(ceilings["hbm_stream_read_TBps"] * 1e3, 1)
                                 if ceilings else None),
        "ceilings": ceilings,
    }
    res["cpu_baseline"] = None
    if not args.no_cpu_baseline:
        cb = cpu_baseline_decode(host, D, S, budget_s=args.cpu_budget, gpu_out=out)
        log(f"[bench] cpu baseline: {cb['value'] * 1e3:.3f} GB/s on {cb['cores']} threads; "
            f"{cb['sample']}")
        res["cpu_baseline"] = cb
    return res


def cpu_baseline_cfg1(host, reps=50):
    """Config 1 (the reference's CPU-runnable decode case) through the torch-CPU path, whole:
    median of `reps` calls, all threads and one thread."""
    import torch

    def med(n):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            torch_cpu_decode(*host)
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    threads = torch.get_num_threads()
    t_all = med(reps)
    torch.set_num_threads(1)
    try:
        t_one = med(reps)
    finally:
        torch.set_num_threads(threads)
    nbytes = 2 * host[1].numel()
    return dict(value=nbytes / t_all / 1e12, unit="TB/s", cores=threads, kind="port",
                us=round(t_all * 1e6, 1), one_thread_us=round(t_one * 1e6, 1),
                sample=f"the whole config-1 call, median of {reps}; {_threads_info()}")


def bench_decode_sweep(args):
    """BASELINE config 3 (B8 H32 D64, ctx 32K) with the ctx sweep 2K..32K at B=8, and config 1
    (B1 H12 D64 ctx 1K)."""
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    rows, cfg1_host = sweep_rows(args, dev, stream)
    head = rows[-1]
    achieved = head["TBps"] * 1e3
    res = {
        "metric": "decode attn us + effective KV-read TB/s, B=8 H=32 D=64 ctx 32K (config 3), "
                  "ctx sweep 2K-32K and config 1",
        "value": head["TBps"], "unit": "TB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["us"] / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1), 1% channels x8 (none for config 1), per-token int8)",
        "config": {"workload": "int8-kv decode attention B=8 H=32 D=64 ctx=32768; sweep and "
                               "config 1 in rows", "rows": rows},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("decode_b8h32d64_s32768"),
                     "kernel": decode_kernel_label(head["nsplit"])},
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_cfg1(cfg1_host),
    }
    return res


def sweep_rows(args, dev, stream):
    """Config 1, then config 3's ctx sweep at B8 H32 D64 (ending with config 3 itself)."""
    import torch

    rows, cfg1_host = [], None
    for B, H, D, S, outl in [(1, 12, 64, 1024, 0.0)] + [(8, 32, 64, S, 0.01) for S in (
            2048, 4096, 8192, 16384, 32768)]:
        row, host, _ = measure_decode(B, H, D, S, outl, args, dev, stream,
                                      keep_host=(B, H, S) == (1, 12, 1024), min_window_ms=2.0)
        if host is not None:
            cfg1_host = host
        row["roofline"] = hbm_roofline(2 * B * H * S * D, row["us"] / 1e3,
                                       decode_kernel_label(row["nsplit"]),
                                       "decode_b8h32d64_s32768" if S == 32768 else None)
        rows.append(row)
        torch.cuda.empty_cache()
    return rows, cfg1_host


def bench_decode_paged(args):
    """The headline decode over a paged copy of the same cache: pages of --page positions in
    a seeded random physical order, one block table row per sequence, all lengths = ctx."""
    import ctypes

    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads

    B, H, D, S, P = args.batch, args.heads, args.head_dim, args.ctx, args.page
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"[bench] generating paged decode inputs B{B} H{H} D{D} S{S} page {P}")
    case = workloads.decode_case(B, H, D, S, seed=args.seed, outlier_frac=0.01, device=dev)
    npp = -(-S // P)
    NP = B * npp
    perm = torch.randperm(NP, generator=torch.Generator().manual_seed(args.seed)).to(dev)

    def to_pages(x):  # [B, H, S, ...] -> [NP, H, P, ...], page (b, i) stored at perm[b*npp + i]
        tail = tuple(x.shape[3:])
        pad = torch.zeros((B, H, npp * P) + tail, dtype=x.dtype, device=dev)
        pad[:, :, :S] = x
        pg = pad.reshape((B, H, npp, P) + tail).movedim(2, 1).reshape((NP, H, P) + tail)
        out = torch.empty_like(pg)
        out[perm] = pg
        return out

    Kp, Vp = to_pages(case["Ki"]), to_pages(case["Vi"])
    sKp, sVp = to_pages(case["sK"]), to_pages(case["sV"])
    del case["Ki"], case["Vi"]
    tables = perm.to(torch.int32).reshape(B, npp).contiguous()
    lens = torch.full((B,), S, dtype=torch.int32, device=dev)
    out = torch.empty((B, H, D), dtype=torch.float16, device=dev)
    ws = torch.empty(max(capi.decode_paged_workspace_bytes(B, H, S, D, args.nsplit), 1),
                     dtype=torch.uint8, device=dev)
    lib = capi.load()
    stream = torch.cuda.current_stream(dev)
    Pt = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(stream.cuda_stream)

    def step():
        rc = lib.int8k_decode_attention_forward_paged(
            Pt(case["Qi"]), Pt(Kp), Pt(Vp), Pt(out), Pt(case["sQ"]), Pt(sKp), Pt(sVp),
            Pt(tables), Pt(lens), B, H, D, NP, P, npp, S, args.nsplit, Pt(ws), ws.numel(), st)
        if rc != 0:
            raise SystemExit(f"paged decode failed: status {rc}")

    ms = time_steps(step, args.steps, args.warmup, stream)
    kv_bytes = 2 * B * H * S * D
    achieved_gbs = kv_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] paged decode page={P}: {ms * 1e3:.1f} us  {achieved_gbs / 1e3:.3f} TB/s "
        f"({achieved_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    from oracle import int8_oracle
    rows = [0, B - 1]
    ref = int8_oracle.decode_attention_paged(
        case["Qi"][rows].cpu().numpy(), Kp.cpu().numpy(), Vp.cpu().numpy(),
        case["sQ"][rows].cpu().numpy(), sKp.cpu().numpy(), sVp.cpu().numpy(),
        tables[rows].cpu().numpy(), lens[rows].cpu().numpy())
    err = float(np.abs(out[rows].float().cpu().numpy() - ref).max())
    log(f"[bench] parity sample (sequences {rows}): max_abs={err:.2e}")
    if not (err <= 2e-2):
        raise SystemExit(f"paged decode output does not match the oracle (max_abs={err})")
    nsplit = capi.decode_paged_num_splits(B, H, S, D, args.nsplit)
    one_launch = (nsplit <= 8 and npp * 4 <= (48 << 10)
                  and os.environ.get("INT8K_DECODE_BLOCK", "1") != "0")
    return {
        "metric": f"paged decode attn effective KV-read TB/s, B={B} H={H} D={D} ctx={S}",
        "value": round(achieved_gbs / 1e3, 4), "unit": "TB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1), 1% channels x8, per-token int8), shuffled pages",
        "config": {"workload": f"int8-kv paged decode B={B} H={H} D={D} ctx={S} page={P}",
                   "pages": NP},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None, "nsplit": nsplit,
                     "kernel": ("decode_paged_block_kernel (one launch per step)" if one_launch
                                else "decode_paged_kernel + decode_combine_kernel (one step)")},
        "cpu_baseline": None,
    }


def measure_paged(B, H, D, S, pages, args, dev, stream):
    """Paged decode at one shape for each page size in `pages`: the contiguous case's data
    (same seed) cut into pages stored in a seeded random physical order, one block-table row
    per sequence, every length = S.  Windows of `--steps` paged steps alternate with windows
    of the contiguous kernel on the same data (5 each, medians reported), so the paging tax
    is measured under the same clock; cases under 512 MB cycle through cache copies.  Every
    (b,h) row of the paged output is checked against the C oracle."""
    import ctypes

    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import oracle_c

    BH = B * H
    case = workloads.decode_case(B, H, D, S, seed=args.seed, outlier_frac=0.01, device=dev)
    host = [case[k].cpu().numpy() for k in ("Qi", "Ki", "Vi", "sQ", "sK", "sV")]
    ref = oracle_c.decode_attention(host[0].reshape(BH, D), host[1].reshape(BH, S, D),
                                    host[2].reshape(BH, S, D), host[3].reshape(BH),
                                    host[4].reshape(BH, S), host[5].reshape(BH, S))
    del host
    lib = capi.load()
    Pt = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(stream.cuda_stream)
    kv_bytes = 2 * BH * S * D
    total = kv_bytes + 2 * BH * S * 4
    n_copies = 1 if total >= (512 << 20) else max(3, -(-(768 << 20) // total))
    Q, sQ = case["Qi"], case["sQ"]
    flat = (case["Ki"].reshape(BH, S, D), case["Vi"].reshape(BH, S, D), case["sK"].reshape(-1),
            case["sV"].reshape(-1))
    ccopies = [flat] + [tuple(t.clone() for t in flat) for _ in range(n_copies - 1)]
    cout = torch.empty((BH, D), dtype=torch.float16, device=dev)
    cws = torch.empty(max(capi.decode_workspace_bytes(BH, S, D, args.nsplit), 1),
                      dtype=torch.uint8, device=dev)
    ccalls = [(Pt(Q), Pt(K), Pt(V), Pt(cout), Pt(sQ), Pt(sK), Pt(sV), BH, S, D, args.nsplit,
               Pt(cws), cws.numel(), st) for (K, V, sK, sV) in ccopies]

    def check(out, what):
        got = out.float().reshape(BH, D).cpu().numpy()
        err = float(np.abs(got - ref).max())
        cos = float((got * ref).sum() / max(np.linalg.norm(got) * np.linalg.norm(ref), 1e-30))
        if not (err <= 2e-2 and cos >= 0.9999):
            raise SystemExit(f"{what} does not match the oracle (max_abs={err}, cos={cos})")
        return {"rows_checked": BH, "max_abs": err, "cos": round(cos, 7)}

    def runner(fn, calls):
        it = [0]

        def step():
            a = calls[it[0] % len(calls)]
            it[0] += 1
            rc = fn(*a)
            if rc != 0:
                capi.check("decode", rc)
        return step

    cstep = runner(lib.int8k_decode_attention_forward, ccalls)
    rows = []
    for P in pages:
        npp = -(-S // P)
        NP = B * npp
        perm = torch.randperm(NP, generator=torch.Generator().manual_seed(args.seed)).to(dev)

        def to_pages(x):  # [B, H, S, ...] -> [NP, H, P, ...]; page (b, i) at perm[b*npp + i]
            tail = tuple(x.shape[3:])
            pad = torch.zeros((B, H, npp * P) + tail, dtype=x.dtype, device=dev)
            pad[:, :, :S] = x
            pg = pad.reshape((B, H, npp, P) + tail).movedim(2, 1).reshape((NP, H, P) + tail)
            o = torch.empty_like(pg)
            o[perm] = pg
            return o

        cache = tuple(to_pages(case[k]) for k in ("Ki", "Vi", "sK", "sV"))
        copies = [cache] + [tuple(t.clone() for t in cache) for _ in range(n_copies - 1)]
        tables = perm.to(torch.int32).reshape(B, npp).contiguous()
        lens = torch.full((B,), S, dtype=torch.int32, device=dev)
        out = torch.empty((B, H, D), dtype=torch.float16, device=dev)
        ws = torch.empty(max(capi.decode_paged_workspace_bytes(B, H, S, D, args.nsplit), 1),
                         dtype=torch.uint8, device=dev)
        pstep = runner(lib.int8k_decode_attention_forward_paged,
                       [(Pt(Q), Pt(Kp), Pt(Vp), Pt(out), Pt(sQ), Pt(sKp), Pt(sVp), Pt(tables),
                         Pt(lens), B, H, D, NP, P, npp, S, args.nsplit, Pt(ws), ws.numel(), st)
                        for (Kp, Vp, sKp, sVp) in copies])
        for _ in range(max(args.warmup, 2 * n_copies)):
            cstep()
            pstep()
        pw, cw = [], []
        for _ in range(WINDOWS):
            cw.append(time_steps(cstep, args.steps, 0, stream))
            pw.append(time_steps(pstep, args.steps, 0, stream))
        ms, cms = statistics.median(pw), statistics.median(cw)
        out.zero_()
        pstep()
        torch.cuda.synchronize()
        parity = check(out, f"paged decode B{B} H{H} D{D} S{S} page {P}")
        tbs = kv_bytes / (ms * 1e-3) / 1e12
        rows.append({"B": B, "H": H, "D": D, "ctx": S, "page": P,
                     "nsplit": capi.decode_paged_num_splits(B, H, S, D, args.nsplit),
                     "us": round(ms * 1e3, 2), "TBps": round(tbs, 4),
                     "pct_hbm_peak": round(tbs * 1e3 / HBM_PEAK_GBS * 100, 2),
                     "contiguous_us": round(cms * 1e3, 2),
                     "vs_contiguous": round(ms / cms, 4),
                     "windows_ms": [round(w, 5) for w in pw], "cache_copies": n_copies,
                     "parity": parity})
        log(f"[bench] paged decode B{B} H{H} D{D} ctx{S} page {P}: {ms * 1e3:.1f} us "
            f"{tbs:.3f} TB/s ({ms / cms:.3f}x the contiguous {cms * 1e3:.1f} us in alternate "
            f"windows), all {BH} rows vs oracle: max_abs {parity['max_abs']:.1e}")
        del copies, cache, ws
        torch.cuda.empty_cache()
    return rows


INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0
BLENDED_PEAK = 1.0 / (0.5 / INT8_PEAK_TOPS + 0.5 / FP16_PEAK_TFLOPS)  # i8 QK^T + fp16 PV


def torch_cpu_mlp(x, sx, W1d, W2d):
    """The reference's CPU/PyTorch MLP path, restated: dequantize the int8 tokens with their
    per-token scales, then fp32 Linear -> GELU(tanh) -> Linear as common/baseline.py:36-37.
    W1d/W2d are the weights dequantized once (fp32, per output channel)."""
    import torch
    import torch.nn.functional as F

    xd = x.float() * sx[:, None]
    return F.gelu(xd @ W1d, approximate="tanh") @ W2d


def measure_mlp(args, dev, stream, cpu_budget=None):
    """T=4096, 4096 -> 16384 -> 4096, per-token x, per-channel W,
    prepacked weights; the unpacked path (per-call weight transposes) beside it."""
    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import int8_oracle, oracle_c

    T, dm, dff = 4096, 4096, 16384
    log(f"[bench] MLP inputs T={T} {dm}->{dff}->{dm}")
    c = workloads.mlp_case(T, dm, dff, seed=args.seed, device=dev)
    x = c["x"].reshape(T, dm)
    W1T, W2T = capi.transpose_int8_weights(c["W1"], c["W2"])
    out = torch.empty(T, dm, dtype=torch.int8, device=dev)
    osc = torch.empty(T, dtype=torch.float32, device=dev)
    ops = 4 * T * dm * dff
    times = {}
    for name, flags, w1, w2 in (("prepacked", capi.MLP_WEIGHTS_PREPACKED, W1T, W2T),
                                ("unpacked", 0, c["W1"], c["W2"]),
                                ("separate", capi.MLP_WEIGHTS_PREPACKED |
                                 capi.MLP_SEPARATE_REQUANT, W1T, W2T)):
        ws = torch.empty(capi.mlp_workspace_bytes(T, dm, dff, flags), dtype=torch.uint8,
                         device=dev)

        def step():
            capi.mlp_forward(x, w1, w2, c["sx"], c["sW1"], c["sW2"], flags=flags, out=out,
                             out_scale=osc, workspace=ws)

        times[name] = time_windows(step, args.steps, args.warmup, stream)
        log(f"[bench] MLP {name}: {times[name][0] * 1e3:.1f} us  "
            f"{ops / (times[name][0] * 1e-3) / 1e12:.1f} TOPS")
        del ws
    # the output of the prepacked path, parity on 64 rows (8 in each 512-row block)
    capi.mlp_forward(x, W1T, W2T, c["sx"], c["sW1"], c["sW2"], flags=capi.MLP_WEIGHTS_PREPACKED,
                     out=out, out_scale=osc)
    rows = np.arange(0, T, T // 64) + np.arange(64) % 7
    W1n, W2n = c["W1"].cpu().numpy(), c["W2"].cpu().numpy()
    sW1n, sW2n = c["sW1"].cpu().numpy(), c["sW2"].cpu().numpy()
    xn, sxn = x.cpu().numpy(), c["sx"].cpu().numpy()
    ref, rsc = int8_oracle.mlp_forward(xn[rows], W1n, W2n, sxn[rows], sW1n, sW2n,
                                       gemm=oracle_c.gemm_i8_i32)
    got = out.cpu().numpy()[rows].astype(np.int32)
    diff = np.abs(got - ref.astype(np.int32))
    log(f"[bench] MLP parity ({len(rows)} rows): max |int8 diff| = {diff.max()}, "
        f"{(diff != 0).mean():.4f} of codes off by one")
    if diff.max() > 1 or (diff != 0).mean() > 0.02:
        raise SystemExit("MLP output does not match the oracle within 1 LSB")
    ms, windows = times["prepacked"]
    tops = ops / (ms * 1e-3) / 1e12
    r = {"workload": "int8 MLP T=4096 d_model=4096 d_ff=16384 GELU, per-token x, per-channel "
                     "W, prepacked weights",
         "us": round(ms * 1e3, 2), "TOPS": round(tops, 1), "windows_ms": windows,
         "unpacked_us": round(times["unpacked"][0] * 1e3, 2),
         "separate_requant_us": round(times["separate"][0] * 1e3, 2),
         "sync_timeouts": capi.mlp_sync_timeouts(),
         "parity": {"rows_checked": len(rows), "max_lsb": int(diff.max()),
                    "frac_off_by_one": round(float((diff != 0).mean()), 5)},
         "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                      "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                      "traffic": measured_traffic("mlp_t4096_d4096_f16384"),
                      "kernel": "whole MLP step (GEMM1 + GEMM2 and their epilogues, requant)"}}
    if cpu_budget:
        import torch as th
        W1d = th.from_numpy(W1n).float() * th.from_numpy(sW1n)[None, :]
        W2d = th.from_numpy(W2n).float() * th.from_numpy(sW2n)[None, :]
        xt, sxt = th.from_numpy(xn), th.from_numpy(sxn)
        blk, n, t0 = 256, 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_budget:
            lo = n % T
            torch_cpu_mlp(xt[lo:lo + blk], sxt[lo:lo + blk], W1d, W2d)
            n += blk
        dt = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": 4 * n * dm * dff / dt / 1e12, "unit": "TOPS",
                             "cores": th.get_num_threads(), "kind": "port",
                             "sample": f"torch-CPU fp32 restatement of common/baseline.py:36-37 "
                                       f"(per-token dequant, Linear, GELU tanh, Linear; weights "
                                       f"dequantized once) on {n} tokens in blocks of {blk}, "
                                       f"{dt:.1f} s; {_threads_info()}"}
    return r


def bench_mlp(args):
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    r = measure_mlp(args, dev, torch.cuda.current_stream(dev),
                    None if args.no_cpu_baseline else min(args.cpu_budget, 6.0))
    res = {
        "metric": "fused INT8 MLP TOPS (% dense INT8 MFMA peak), T=4096 4096->16384->4096",
        "value": r["TOPS"], "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["us"] / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) x, N(0,0.02) W, per-token/per-channel int8)",
        "config": {k: v for k, v in r.items() if k not in ("roofline", "cpu_baseline")},
        "roofline": r["roofline"], "cpu_baseline": r.get("cpu_baseline"),
    }
    if not args.no_calibrate:
        import ctypes
        res["ceilings"] = mfma_sustained(ctypes.CDLL(os.path.join(PKG_DIR, "libint8k_calib.so")),
                                         dev)
    return res


def torch_cpu_prefill(Q, K, V, sQ, sK, sV, causal):
    """The reference's CPU/PyTorch attention path, restated for one (b,h): dequantize, then
    fp32 attention as common/baseline.py:18-22, with the causal mask this build adds."""
    import torch

    S, D = Q.shape
    q, k, v = Q.float() * sQ[:, None], K.float() * sK[:, None], V.float() * sV[:, None]
    w = torch.matmul(q, k.transpose(-2, -1)) * D ** -0.5
    if causal:
        w.masked_fill_(torch.ones(S, S, dtype=torch.bool).triu_(1), float("-inf"))
    return torch.matmul(torch.softmax(w, dim=-1), v)


def measure_prefill(args, dev, stream, cpu_budget=None, extras=True):
    """B=4 H=32 S=4096 D=128, causal (non-causal beside it)."""
    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import oracle_c

    B, H, S, D = 4, 32, 4096, 128
    log(f"[bench] prefill inputs B{B} H{H} S{S} D{D}")
    c = workloads.prefill_case(B, H, S, D, seed=args.seed, device=dev)
    out = torch.empty(B, H, S, D, dtype=torch.float16, device=dev)
    times = {}
    for causal in (True, False):
        def step():
            capi.attention_forward(c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"],
                                   causal=causal, out=out)
        times[causal] = time_windows(step, args.steps, args.warmup, stream)
        ops = 2 * B * H * D * S * (S + 1) if causal else 4 * B * H * S * S * D
        log(f"[bench] prefill causal={causal}: {times[causal][0] * 1e3:.1f} us  "
            f"{ops / (times[causal][0] * 1e-3) / 1e12:.1f} TOPS")
    capi.attention_forward(c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"], causal=True,
                           out=out)
    torch.cuda.synchronize()
    heads = [(0, 0), (B - 1, H - 1)]
    errs = []
    for b, hh in heads:
        args_h = [c[k][b, hh:hh + 1].cpu().numpy() for k in ("Qi", "Ki", "Vi", "sQ", "sK", "sV")]
        ref = oracle_c.prefill_attention(*args_h, causal=True)[0]
        errs.append(float(np.abs(out[b, hh].float().cpu().numpy() - ref).max()))
    log(f"[bench] prefill parity (heads {heads}): max_abs {max(errs):.1e}")
    if max(errs) > 2e-2:
        raise SystemExit(f"prefill output does not match the oracle ({errs})")
    r = {"workload": "int8 causal prefill attention B=4 H=32 S=4096 D=128",
         "us": round(times[True][0] * 1e3, 2), "windows_ms": times[True][1],
         "noncausal_us": round(times[False][0] * 1e3, 2),
         "noncausal_TOPS": round(4 * B * H * S * S * D / (times[False][0] * 1e-3) / 1e12, 1),
         "parity": {"heads_checked": [list(h) for h in heads], "max_abs": max(errs)},
         "blended_peak_TOPS": round(BLENDED_PEAK, 1)}
    ms = times[True][0]
    tops = 2 * B * H * D * S * (S + 1) / (ms * 1e-3) / 1e12
    r["TOPS"] = round(tops, 1)
    r["roofline"] = {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "frac_of_blended_i8_f16": round(tops / BLENDED_PEAK, 4),
                     "traffic": measured_traffic("prefill_b4h32s4096d128"),
                     "kernel": "prefill_kernel<128, causal>"}
    if extras:
        # the attention output emitted as per-token int8 (fused) against the fp16 output
        # followed by a separate per-token quantization pass
        q8 = torch.empty(B, H, S, D, dtype=torch.int8, device=dev)
        s8 = torch.empty(B, H, S, dtype=torch.float32, device=dev)
        lib = capi.load()
        P = capi._ptr

        def fused():
            capi.check("int8k_attention_forward_quant", lib.int8k_attention_forward_quant(
                P(c["Qi"]), P(c["Ki"]), P(c["Vi"]), P(q8), P(s8), P(c["sQ"]), P(c["sK"]),
                P(c["sV"]), B, H, S, D, 1, capi._stream(q8)))

        def two_pass():
            capi.attention_forward(c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"],
                                   causal=True, out=out)
            capi.check("int8k_quantize_per_token", lib.int8k_quantize_per_token(
                P(out), capi.DTYPE_F16, P(q8), P(s8), B * H * S, D, capi._stream(out)))

        r["int8_output_fused_us"] = round(time_windows(fused, args.steps, args.warmup,
                                                       stream)[0] * 1e3, 2)
        r["int8_output_two_pass_us"] = round(time_windows(two_pass, args.steps, args.warmup,
                                                          stream)[0] * 1e3, 2)
        log(f"[bench] prefill causal, int8 output: fused {r['int8_output_fused_us']} us, "
            f"fp16 + quantize_per_token {r['int8_output_two_pass_us']} us")
    if cpu_budget:
        done, t0 = 0, time.perf_counter()
        host = {k: c[k].cpu() for k in ("Qi", "Ki", "Vi", "sQ", "sK", "sV")}
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < cpu_budget:
            b, hh = divmod(done % (B * H), H)
            torch_cpu_prefill(*(host[k][b, hh] for k in ("Qi", "Ki", "Vi", "sQ", "sK", "sV")),
                              causal=True)
            done += 1
        dt = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": 2 * done * D * S * (S + 1) / dt / 1e12, "unit": "TOPS",
                             "cores": torch.get_num_threads(), "kind": "port",
                             "sample": f"torch-CPU fp32 restatement of common/baseline.py:18-22 "
                                       f"with a causal mask on {done} of {B * H} heads x {S} "
                                       f"tokens, {dt:.1f} s; {_threads_info()}"}
    return r


def bench_prefill(args):
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    r = measure_prefill(args, dev, torch.cuda.current_stream(dev),
                        None if args.no_cpu_baseline else min(args.cpu_budget, 6.0))
    return {
        "metric": "INT8 causal prefill attention TOPS, B=4 H=32 S=4096 D=128",
        "value": r["TOPS"], "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["us"] / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1), per-token int8)",
        "config": {k: v for k, v in r.items() if k not in ("roofline", "cpu_baseline")},
        "roofline": r["roofline"], "cpu_baseline": r.get("cpu_baseline"),
    }


def bench_all(args):
    """The default run: the headline (config 2) as the line's value, then configs 1, 3 (with
    the ctx sweep), 4 and 5 under `configs`, each with its own roofline and parity check."""
    import torch

    res = bench_decode(args)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    torch.cuda.empty_cache()
    rows, cfg1_host = sweep_rows(args, dev, stream)
    cfg1, sweep = rows[0], rows[1:]
    if not args.no_cpu_baseline:
        cfg1["cpu_baseline"] = cpu_baseline_cfg1(cfg1_host)
        log(f"[bench] cfg1 torch-CPU: {cfg1['cpu_baseline']['us']} us "
            f"(1 thread {cfg1['cpu_baseline']['one_thread_us']} us)")
    torch.cuda.empty_cache()
    paged = (measure_paged(args.batch, args.heads, args.head_dim, args.ctx, (16, 256), args, dev,
                           stream)
             + measure_paged(8, 32, 64, 32768, (16, 256), args, dev, stream))
    torch.cuda.empty_cache()
    cfg4 = measure_mlp(args, dev, stream, None if args.no_cpu_baseline else 5.0)
    torch.cuda.empty_cache()
    cfg5 = measure_prefill(args, dev, stream, None if args.no_cpu_baseline else 5.0,
                           extras=False)
    torch.cuda.empty_cache()
    blk = bench_block(args)
    res["configs"] = {
        "cfg1_decode_b1h12d64_s1024": cfg1,
        "cfg3_decode_b8h32d64_s32768": sweep[-1],
        "cfg3_ctx_sweep_b8h32d64": sweep[:-1],
        "paged_decode": paged,
        "cfg4_mlp_t4096_d4096_f16384": cfg4,
        "cfg5_prefill_causal_b4h32s4096d128": cfg5,
        "block_d1024_h16_dff4096": {"metric": blk["metric"], "value": blk["value"],
                                    "unit": blk["unit"], "rows": blk["config"]["rows"]},
    }
    return res


def bench_gemm(args):
    """The MLP's GEMM1 shape alone (4096 x 16384 x 4096, int32 out): our gemm core on uniform
    random and on all-zero operands, and hipBLASLt (torch._int_mm) on the random operands.
    Shows how far the sustained MFMA rate depends on the operand data on this part."""
    import ctypes

    import torch

    import int8k_capi as capi

    M, N, K = 4096, 16384, 4096
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    A = torch.randint(-128, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    Bt = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    C = torch.empty(M, N, dtype=torch.int32, device=dev)
    ops = 2 * M * N * K
    ms_rand = time_steps(lambda: capi.gemm_i8_i32(A, Bt, out=C), args.steps, args.warmup, stream)
    ref = A[:64].double().cpu() @ Bt.double().cpu().t()
    if not torch.equal(C[:64].cpu().double(), ref):
        raise SystemExit("gemm_i8_i32 does not match the exact int32 product")
    ms_lib = time_steps(lambda: torch._int_mm(A, Bt.t()), args.steps, args.warmup, stream)
    # the MLP's own operands: config 4's per-token x and per-channel W1 codes (Gaussian data)
    import workloads

    c = workloads.mlp_case(M, K, N, seed=args.seed, device=dev)
    Am = c["x"].reshape(M, K).contiguous()
    Bm = c["W1"].t().contiguous()  # [N][K]
    del c
    ms_mlp = time_steps(lambda: capi.gemm_i8_i32(Am, Bm, out=C), args.steps, args.warmup, stream)
    ref = Am[:64].double().cpu() @ Bm.double().cpu().t()
    if not torch.equal(C[:64].cpu().double(), ref):
        raise SystemExit("gemm_i8_i32 does not match the exact int32 product (MLP operands)")
    ms_lib_mlp = time_steps(lambda: torch._int_mm(Am, Bm.t()), args.steps, args.warmup, stream)
    del Am, Bm
    A.zero_()
    Bt.zero_()
    ms_zero = time_steps(lambda: capi.gemm_i8_i32(A, Bt, out=C), args.steps, args.warmup, stream)
    tops = ops / (ms_rand * 1e-3) / 1e12
    for name, ms in (("random", ms_rand), ("zero", ms_zero), ("hipblaslt random", ms_lib),
                     ("mlp operands", ms_mlp), ("hipblaslt mlp operands", ms_lib_mlp)):
        log(f"[bench] gemm {name}: {ms * 1e3:.1f} us  {ops / (ms * 1e-3) / 1e12:.1f} TOPS")
    L = ctypes.CDLL(os.path.join(PKG_DIR, "libint8k_calib.so"))
    return {
        "metric": "INT8 GEMM TOPS, 4096x16384x4096 (the MLP's GEMM1 shape), int32 out",
        "value": round(tops, 1), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_rand, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic uniform random int8 (and all-zero for the comparison)",
        "config": {"workload": "int8 GEMM M=4096 N=16384 K=4096",
                   "zero_operands_TOPS": round(ops / (ms_zero * 1e-3) / 1e12, 1),
                   "hipblaslt_int_mm_random_TOPS": round(ops / (ms_lib * 1e-3) / 1e12, 1),
                   "mlp_operands_us": round(ms_mlp * 1e3, 2),
                   "hipblaslt_int_mm_mlp_operands_us": round(ms_lib_mlp * 1e3, 2)},
        "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "traffic": None, "kernel": "gemm_i8_kernel<0>"},
        "ceilings": mfma_sustained(L, dev),
    }


def bench_block(args):
    """End-to-end pre-LN transformer block, INT8 vs FP16 (the reference's bench/bench_block.py:
    h = x + Wo.Attn(split_heads(LN1(x).Wqkv)); y = h + MLP(LN2(h))).  The INT8 block runs
    the attention core and the MLP on this library, with its producer-fused quantizers
    (split-heads+quant of the QKV projection, LN2+quant of the MLP input) and the MLP output's
    dequantization fused with the second residual add; LayerNorm1, the QKV/output projections
    and the first residual add stay FP16 in both paths, as in the reference.
    Reports ms per block forward for both paths, the speedup and the cosine of the outputs."""
    import torch
    import torch.nn.functional as F

    import int8_ext as ext
    from block import TransformerBlock

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    def cos(a, b):
        return F.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0).item()

    rows = []
    H, Dh, dff = 16, 64, 4096
    d = H * Dh
    blk = TransformerBlock(d, H, dff, dev)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    for S in (512, 1024, 2048):
        x = torch.randn(8, S, d, generator=g, device=dev, dtype=torch.float16)
        c = cos(blk.prefill(x, True), blk.prefill(x, False))
        ms8 = time_steps(lambda: blk.prefill(x, True), args.steps, args.warmup, stream)
        ms16 = time_steps(lambda: blk.prefill(x, False), args.steps, args.warmup, stream)
        rows.append({"regime": "prefill", "B": 8, "seq": S, "int8_ms": round(ms8, 4),
                     "fp16_ms": round(ms16, 4), "speedup": round(ms16 / ms8, 3),
                     "cos": round(c, 5)})
        log(f"[bench] block prefill B8 S{S}: int8 {ms8:.3f} ms fp16 {ms16:.3f} ms "
            f"speedup {ms16 / ms8:.2f}x cos {c:.5f}")
    B = 128
    x = torch.randn(B, 1, d, generator=g, device=dev, dtype=torch.float16)
    for Skv in (2048, 4096, 8192, 16384, 32768):
        Kf = torch.randn(B, H, Skv, Dh, generator=g, device=dev, dtype=torch.float16)
        Vf = torch.randn(B, H, Skv, Dh, generator=g, device=dev, dtype=torch.float16)
        Ki, sK = ext.quantize_per_token(Kf)
        Vi, sV = ext.quantize_per_token(Vf)
        c = cos(blk.decode(x, (Ki, Vi, sK, sV), True), blk.decode(x, (Kf, Vf), False))
        ms8 = time_steps(lambda: blk.decode(x, (Ki, Vi, sK, sV), True), args.steps, args.warmup,
                         stream)
        ms16 = time_steps(lambda: blk.decode(x, (Kf, Vf), False), args.steps, args.warmup, stream)
        rows.append({"regime": "decode", "B": B, "seq": Skv, "int8_ms": round(ms8, 4),
                     "fp16_ms": round(ms16, 4), "speedup": round(ms16 / ms8, 3),
                     "cos": round(c, 5)})
        log(f"[bench] block decode B{B} Skv{Skv}: int8 {ms8:.3f} ms fp16 {ms16:.3f} ms "
            f"speedup {ms16 / ms8:.2f}x cos {c:.5f}")
        del Kf, Vf, Ki, Vi, sK, sV
        torch.cuda.empty_cache()
    head = next(r for r in rows if r["regime"] == "decode" and r["seq"] == 8192)
    return {
        "metric": "transformer block INT8/FP16 speedup, decode B=128 H=16 Dh=64 d_ff=4096 Skv=8192",
        "value": head["speedup"], "unit": "x", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["int8_ms"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations and KV, random-init weights)",
        "config": {"workload": "pre-LN transformer block d_model=1024 H=16 d_ff=4096; prefill "
                               "B=8 S=512..2048 and decode B=128 Skv=2K..32K", "rows": rows},
        "roofline": None, "cpu_baseline": None,
    }


def trace_summary(path):
    """Per-kernel dispatch statistics from a rocprofv3 `--kernel-trace --output-format csv`
    file: calls, the median and mean duration with the first dispatch of each kernel
    excluded (it carries the code-object load and cold caches), min and max.  Prints a
    markdown table."""
    import csv

    durs = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name") or row.get("KernelName") or row.get("Name")
            t0 = int(row.get("Start_Timestamp") or row["BeginNs"])
            t1 = int(row.get("End_Timestamp") or row["EndNs"])
            durs.setdefault(name, []).append((t0, (t1 - t0) / 1e3))
    print("| kernel | calls | median µs (first excluded) | mean µs (first excluded) | min µs | "
          "max µs |")
    print("|---|---|---|---|---|---|")
    for name, v in sorted(durs.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        d = [x for _, x in sorted(v)]
        rest = d[1:] or d
        short = name.replace("(anonymous namespace)::", "").replace("void ", "")
        short = short.split("(")[0] if "int8k::" in short else short[:60] + "..."
        print(f"| `{short}` | {len(d)} | {statistics.median(rest):.2f} | "
              f"{statistics.fmean(rest):.2f} | {min(d):.2f} | {max(d):.2f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="all",
                    choices=["all", "decode", "decode-sweep", "decode-paged", "mlp", "prefill",
                             "gemm", "block"])
    ap.add_argument("--page", type=int, default=16, help="page size for --workload decode-paged")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--nsplit", type=int, default=0)
    ap.add_argument("--seed", type=int, default=20241201)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-calibrate", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU time for the headline's CPU baseline")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise a rocprofv3 kernel-trace CSV (no GPU work) and exit")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode and prefill would shard over (b,h) with no exchange, the MLP over "
              "d_ff with an all-reduce of the row maxima and of the output)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "mlp":
        res = bench_mlp(args)
    elif args.workload == "prefill":
        res = bench_prefill(args)
    elif args.workload == "gemm":
        res = bench_gemm(args)
    elif args.workload == "decode-paged":
        res = bench_decode_paged(args)
    elif args.workload == "decode-sweep":
        res = bench_decode_sweep(args)
    elif args.workload == "block":
        res = bench_block(args)
    elif args.workload == "decode":
        res = bench_decode(args)
    else:
        res = bench_all(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

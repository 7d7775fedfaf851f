#!/usr/bin/env python3
"""bench.py — INT8-KV split-KV decode attention on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload decode]

Default workload is the BASELINE headline: decode attention over a contiguous
INT8 KV cache, B=32 H=32 D=128 ctx=8192 (2 GiB of K+V), 1% of channels x8
before per-token quantization.  One step = one decode call over the whole
batch (split kernel + combine kernel), inputs already resident in HBM.

Prints ONE JSON line (rank 0).  `value` is the effective KV-read bandwidth
(2*B*H*S*D bytes / step time) in TB/s; `roofline` prices the same bytes
against the 8 TB/s HBM peak; `cpu_baseline` is the CPU oracle (C, OpenMP)
timed on a bounded sample of the same heads on this host.
Everything else (per-config details) goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
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


def cpu_baseline_decode(case, B, H, D, S, budget_s=12.0):
    """Time the C oracle (all host cores) on (b,h) heads of the workload, in slices of
    growing size, passing over all heads again until `budget_s` of CPU time is spent
    (the inputs are copied to host memory once, outside the timed calls)."""
    from oracle import oracle_c

    BH = B * H
    host = [t.reshape((BH,) + shape).cpu().numpy() for t, shape in (
        (case["Qi"], (D,)), (case["Ki"], (S, D)), (case["Vi"], (S, D)), (case["sQ"], ()),
        (case["sK"], (S,)), (case["sV"], (S,)))]
    threads = oracle_c.max_threads()
    n, spent, done_bytes, heads = 4, 0.0, 0, 0
    while spent < budget_s:
        start = heads % BH
        n = min(n, BH - start)
        args = [a[start:start + n] for a in host]
        t0 = time.perf_counter()
        oracle_c.decode_attention(*args, threads=threads)
        spent += time.perf_counter() - t0
        done_bytes += 2 * n * S * D
        heads += n
        n = min(2 * n, BH)
    tbs = done_bytes / spent / 1e12
    # one thread on the first head, for the per-core figure
    args = [a[0:1] for a in host]
    t0 = time.perf_counter()
    oracle_c.decode_attention(*args, threads=1)
    one = 2 * S * D / (time.perf_counter() - t0) / 1e9
    return dict(value=tbs, unit="TB/s", cores=threads, kind="port",
                sample=f"C oracle (float64, OpenMP) on {heads} (b,h) heads "
                       f"({heads / BH:.1f} passes over the {BH} heads) of the same "
                       f"B{B} H{H} D{D} S{S} inputs; {spent:.1f} s of CPU time; "
                       f"host os.cpu_count()={os.cpu_count()}; 1 thread: {one:.2f} GB/s",
                seconds=spent, heads=heads)


def measured_traffic(key):
    """HBM bytes per launch of the dominant kernel, from the committed PMC summary."""
    try:
        with open(os.path.join(REPO_DIR, "profiles", "traffic.json")) as f:
            t = json.load(f).get(key)
    except (OSError, ValueError):
        return None
    return None if t is None else int(t["read_bytes"]) + int(t["write_bytes"])


def bench_decode(args):
    import torch

    import int8k_capi as capi
    import workloads

    B, H, D, S = args.batch, args.heads, args.head_dim, args.ctx
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ceilings = None if args.no_calibrate else calibrate(dev)
    if ceilings:
        log(f"[bench] on-box ceilings: {ceilings}")
    log(f"[bench] generating decode inputs B{B} H{H} D{D} S{S} (outliers 1% x8)")
    case = workloads.decode_case(B, H, D, S, seed=args.seed, outlier_frac=0.01, device=dev)
    BH = B * H
    Q = case["Qi"].reshape(BH, D)
    K = case["Ki"].reshape(BH, S, D)
    V = case["Vi"].reshape(BH, S, D)
    sQ, sK, sV = case["sQ"].reshape(-1), case["sK"].reshape(-1), case["sV"].reshape(-1)
    out = torch.empty((BH, D), dtype=torch.float16, device=dev)
    ws = torch.empty(max(capi.decode_workspace_bytes(BH, S, D, args.nsplit), 1),
                     dtype=torch.uint8, device=dev)
    nsplit = capi.decode_num_splits(BH, S, D, args.nsplit)
    stream = torch.cuda.current_stream(dev)

    def step():
        capi.decode_attention(Q, K, V, sQ, sK, sV, nsplit=args.nsplit, out=out, workspace=ws)

    ms = time_steps(step, args.steps, args.warmup, stream)
    kv_bytes = 2 * BH * S * D
    scale_bytes = 2 * BH * S * 4
    tbs = kv_bytes / (ms * 1e-3) / 1e12
    achieved_gbs = kv_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] nsplit={nsplit} units={BH * nsplit} step={ms * 1e3:.1f} us "
        f"KV-read {tbs:.3f} TB/s ({achieved_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s); "
        f"scale-inclusive {(kv_bytes + scale_bytes) / (ms * 1e-3) / 1e12:.3f} TB/s")

    # sanity: a few heads against the oracle (cheap, untimed)
    import numpy as np
    from oracle import oracle_c
    rows = np.arange(0, BH, max(1, BH // 8))
    ref = oracle_c.decode_attention(Q[rows].cpu().numpy(), K[rows].cpu().numpy(),
                                    V[rows].cpu().numpy(), sQ.reshape(BH)[rows].cpu().numpy(),
                                    sK.reshape(BH, S)[rows].cpu().numpy(),
                                    sV.reshape(BH, S)[rows].cpu().numpy())
    err = float(np.abs(out[rows].float().cpu().numpy() - ref).max())
    log(f"[bench] parity sample ({len(rows)} heads): max_abs={err:.2e}")
    if not (err <= 2e-2):
        raise SystemExit(f"decode output does not match the oracle (max_abs={err})")

    res = {
        "metric": METRIC,
        "value": round(tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_hbm_peak": round(achieved_gbs / HBM_PEAK_GBS * 100, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1), 1% channels x8, per-token int8)",
        "config": {"workload": f"int8-kv decode attention B={B} H={H} D={D} ctx={S}",
                   "batch": B, "heads": H, "head_dim": D, "ctx": S, "nsplit": nsplit,
                   "kv_bytes": kv_bytes, "scale_bytes": scale_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(f"decode_b{B}h{H}d{D}_s{S}"),
                     "kernel": "decode_split_kernel + decode_combine_kernel (one step)",
                     "measured_ceiling": (round(ceilings["hbm_stream_read_TBps"] * 1e3, 1)
                                          if ceilings else None)},
        "ceilings": ceilings,
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline_decode(case, B, H, D, S, budget_s=args.cpu_budget)
        log(f"[bench] cpu baseline: {cb['value'] * 1e3:.3f} GB/s on {cb['cores']} threads "
            f"({cb['heads']} heads, {cb['seconds']:.1f} s)")
        res["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    else:
        res["cpu_baseline"] = None
    return res


def bench_decode_sweep(args):
    """BASELINE config 3 (B8 H32 D64, ctx 32K) with the ctx sweep 2K..32K at B=8, and config 1
    (B1 H12 D64 ctx 1K).  Cases whose K+V (+ scales) are under 512 MB cycle through enough copies
    of the cache (at least 3, 768 MB in total) that the 256 MB Infinity Cache cannot serve a step
    from the previous one.  Each case: `--warmup` untimed steps, then 5 runs of `--steps` steps;
    the median run's mean per step is reported, with a parity sample against the C oracle."""
    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import oracle_c

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    cases = [(1, 12, 64, 1024, 0.0)] + [(8, 32, 64, S, 0.01) for S in (2048, 4096, 8192, 16384,
                                                                        32768)]
    rows, last = [], None
    for B, H, D, S, outl in cases:
        BH = B * H
        case = workloads.decode_case(B, H, D, S, seed=args.seed, outlier_frac=outl, device=dev)
        Q = case["Qi"].reshape(BH, D)
        sQ = case["sQ"].reshape(-1)
        kv = (case["Ki"].reshape(BH, S, D), case["Vi"].reshape(BH, S, D),
              case["sK"].reshape(-1), case["sV"].reshape(-1))
        kv_bytes = 2 * BH * S * D
        total = kv_bytes + 2 * BH * S * 4
        n_copies = 1 if total >= (512 << 20) else max(3, -(-(768 << 20) // total))
        copies = [kv] + [tuple(t.clone() for t in kv) for _ in range(n_copies - 1)]
        out = torch.empty((BH, D), dtype=torch.float16, device=dev)
        ws = torch.empty(max(capi.decode_workspace_bytes(BH, S, D, 0), 1), dtype=torch.uint8,
                         device=dev)
        it = [0]

        def step():
            K, V, sK, sV = copies[it[0] % n_copies]
            it[0] += 1
            capi.decode_attention(Q, K, V, sQ, sK, sV, out=out, workspace=ws)

        for _ in range(args.warmup):
            step()
        runs = sorted(time_steps(step, args.steps, 0, stream) for _ in range(5))
        ms = runs[2]
        tbs = kv_bytes / (ms * 1e-3) / 1e12
        K, V, sK, sV = kv
        sel = np.arange(0, BH, max(1, BH // 8))
        step_out = out.clone()
        capi.decode_attention(Q, K, V, sQ, sK, sV, out=step_out, workspace=ws)
        ref = oracle_c.decode_attention(Q[sel].cpu().numpy(), K[sel].cpu().numpy(),
                                        V[sel].cpu().numpy(), sQ[sel].cpu().numpy(),
                                        sK.reshape(BH, S)[sel].cpu().numpy(),
                                        sV.reshape(BH, S)[sel].cpu().numpy())
        err = float(np.abs(step_out[sel].float().cpu().numpy() - ref).max())
        if not (err <= 2e-2):
            raise SystemExit(f"decode B{B} H{H} D{D} S{S} does not match the oracle ({err})")
        row = {"B": B, "H": H, "D": D, "ctx": S, "nsplit": capi.decode_num_splits(BH, S, D, 0),
               "us": round(ms * 1e3, 2), "TBps": round(tbs, 4),
               "pct_hbm_peak": round(tbs * 1e3 / HBM_PEAK_GBS * 100, 2),
               "cache_copies": n_copies, "max_abs_err_sample": err}
        rows.append(row)
        log(f"[bench] decode B{B} H{H} D{D} ctx{S}: {ms * 1e3:.1f} us {tbs:.3f} TB/s "
            f"({row['pct_hbm_peak']:.1f}% of 8 TB/s), {n_copies} cache copies, max_abs {err:.1e}")
        last = (case, B, H, D, S) if S == 32768 else last
        if (B, H, S) == (1, 12, 1024):
            cfg1 = (case, B, H, D, S)
        del copies, kv
        if S != 32768:
            del case
        torch.cuda.empty_cache()
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
                     "kernel": "decode_split_kernel + decode_combine_kernel (one step)"},
    }
    if not args.no_cpu_baseline:
        case, B, H, D, S = cfg1
        cb = cpu_baseline_decode(case, B, H, D, S, budget_s=args.cpu_budget)
        log(f"[bench] cpu baseline (config 1): {cb['value'] * 1e3:.3f} GB/s on {cb['cores']} "
            f"threads")
        res["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    else:
        res["cpu_baseline"] = None
    return res


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
    return {
        "metric": "paged decode attn effective KV-read TB/s, B=32 H=32 D=128 8K ctx",
        "value": round(achieved_gbs / 1e3, 4), "unit": "TB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1), 1% channels x8, per-token int8), shuffled pages",
        "config": {"workload": f"int8-kv paged decode B={B} H={H} D={D} ctx={S} page={P}",
                   "pages": NP},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": "decode_paged_kernel + decode_combine_kernel (one step)"},
        "cpu_baseline": None,
    }


INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0
BLENDED_PEAK = 1.0 / (0.5 / INT8_PEAK_TOPS + 0.5 / FP16_PEAK_TFLOPS)  # i8 QK^T + fp16 PV


def bench_mlp(args):
    """T=4096, 4096 -> 16384 -> 4096, per-token x, per-channel W."""
    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import int8_oracle, oracle_c

    T, dm, dff = 4096, 4096, 16384
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"[bench] generating MLP inputs T={T} {dm}->{dff}->{dm}")
    c = workloads.mlp_case(T, dm, dff, seed=args.seed, device=dev)
    x = c["x"].reshape(T, dm)
    W1T, W2T = capi.transpose_int8_weights(c["W1"], c["W2"])
    out = torch.empty(T, dm, dtype=torch.int8, device=dev)
    osc = torch.empty(T, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    ops = 4 * T * dm * dff
    res_lines = {}
    for name, flags, w1, w2 in (("prepacked", capi.MLP_WEIGHTS_PREPACKED, W1T, W2T),
                                ("unpacked", 0, c["W1"], c["W2"])):
        ws = torch.empty(capi.mlp_workspace_bytes(T, dm, dff, flags), dtype=torch.uint8,
                         device=dev)

        def step():
            capi.mlp_forward(x, w1, w2, c["sx"], c["sW1"], c["sW2"], flags=flags, out=out,
                             out_scale=osc, workspace=ws)

        ms = time_steps(step, args.steps, args.warmup, stream)
        res_lines[name] = ms
        log(f"[bench] MLP {name}: {ms * 1e3:.1f} us  {ops / (ms * 1e-3) / 1e12:.1f} TOPS")
        del ws
    rows = np.arange(0, T, T // 8)
    ref, rsc = int8_oracle.mlp_forward(x[rows].cpu().numpy(), c["W1"].cpu().numpy(),
                                       c["W2"].cpu().numpy(), c["sx"][rows].cpu().numpy(),
                                       c["sW1"].cpu().numpy(), c["sW2"].cpu().numpy(),
                                       gemm=oracle_c.gemm_i8_i32)
    diff = np.abs(out[rows].cpu().numpy().astype(np.int32) - ref.astype(np.int32)).max()
    log(f"[bench] parity sample ({len(rows)} rows): max |int8 diff| = {diff}")
    if diff > 1:
        raise SystemExit("MLP output does not match the oracle within 1 LSB")
    ms = res_lines["prepacked"]
    tops = ops / (ms * 1e-3) / 1e12
    res = {
        "metric": "fused INT8 MLP TOPS (% dense INT8 MFMA peak), T=4096 4096->16384->4096",
        "value": round(tops, 1), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) x, N(0,0.02) W, per-token/per-channel int8)",
        "config": {"workload": "int8 MLP T=4096 d_model=4096 d_ff=16384 GELU, prepacked weights",
                   "unpacked_ms_per_step": round(res_lines["unpacked"], 5)},
        "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "traffic": measured_traffic("mlp_t4096_d4096_f16384"),
                     "kernel": "whole MLP step (2 GEMMs + requant kernels)"},
    }
    if not args.no_calibrate:
        import ctypes
        res["ceilings"] = mfma_sustained(ctypes.CDLL(os.path.join(PKG_DIR, "libint8k_calib.so")),
                                         dev)
    if not args.no_cpu_baseline:
        # The oracle MLP on token blocks of the same workload, as many as fit in the CPU budget.
        threads = oracle_c.max_threads()
        W1n, W2n = c["W1"].cpu().numpy(), c["W2"].cpu().numpy()
        sW1n, sW2n = c["sW1"].cpu().numpy(), c["sW2"].cpu().numpy()
        xn, sxn = x.cpu().numpy(), c["sx"].cpu().numpy()
        n, blk, t0 = 0, 128, time.perf_counter()
        while n < T:
            t1 = time.perf_counter()
            int8_oracle.mlp_forward(xn[n:n + blk], W1n, W2n, sxn[n:n + blk], sW1n, sW2n,
                                    gemm=oracle_c.gemm_i8_i32)
            n += blk
            if (time.perf_counter() - t0) + (time.perf_counter() - t1) > args.cpu_budget:
                break
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": 4 * n * dm * dff / dt / 1e12, "unit": "TOPS",
                               "cores": threads, "kind": "port",
                               "sample": f"oracle MLP (C int8 GEMMs, numpy epilogue) on {n} of "
                                         f"{T} tokens; {dt:.1f} s"}
    return res


def bench_prefill(args):
    """B=4 H=32 S=4096 D=128, causal."""
    import numpy as np
    import torch

    import int8k_capi as capi
    import workloads
    from oracle import oracle_c

    B, H, S, D = 4, 32, 4096, 128
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"[bench] generating prefill inputs B{B} H{H} S{S} D{D}")
    c = workloads.prefill_case(B, H, S, D, seed=args.seed, device=dev)
    out = torch.empty(B, H, S, D, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)
    res_ms = {}
    for causal in (True, False):
        def step():
            capi.attention_forward(c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"],
                                   causal=causal, out=out)
        res_ms[causal] = time_steps(step, args.steps, args.warmup, stream)
        ops = 2 * B * H * D * S * (S + 1) if causal else 4 * B * H * S * S * D
        log(f"[bench] prefill causal={causal}: {res_ms[causal] * 1e3:.1f} us  "
            f"{ops / (res_ms[causal] * 1e-3) / 1e12:.1f} TOPS")
    # the attention output emitted as per-token int8 (fused) against the fp16 output
    # followed by a separate per-token quantization pass
    q8 = torch.empty(B, H, S, D, dtype=torch.int8, device=dev)
    s8 = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    lib = capi.load()
    P = capi._ptr

    def fused():
        capi.check("int8k_attention_forward_quant", lib.int8k_attention_forward_quant(
            P(c["Qi"]), P(c["Ki"]), P(c["Vi"]), P(q8), P(s8), P(c["sQ"]), P(c["sK"]), P(c["sV"]),
            B, H, S, D, 1, capi._stream(q8)))

    def two_pass():
        capi.attention_forward(c["Qi"], c["Ki"], c["Vi"], c["sQ"], c["sK"], c["sV"],
                               causal=True, out=out)
        capi.check("int8k_quantize_per_token", lib.int8k_quantize_per_token(
            P(out), capi.DTYPE_F16, P(q8), P(s8), B * H * S, D, capi._stream(out)))

    ms_fused = time_steps(fused, args.steps, args.warmup, stream)
    ms_two = time_steps(two_pass, args.steps, args.warmup, stream)
    log(f"[bench] prefill causal, int8 output: fused {ms_fused * 1e3:.1f} us, "
        f"fp16 + quantize_per_token {ms_two * 1e3:.1f} us")
    ms = res_ms[True]
    ops = 2 * B * H * D * S * (S + 1)
    tops = ops / (ms * 1e-3) / 1e12
    res = {
        "metric": "INT8 causal prefill attention TOPS, B=4 H=32 S=4096 D=128",
        "value": round(tops, 1), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1), per-token int8)",
        "config": {"workload": "int8 causal prefill attention B=4 H=32 S=4096 D=128",
                   "noncausal_ms_per_step": round(res_ms[False], 5),
                   "int8_output_fused_ms_per_step": round(ms_fused, 5),
                   "int8_output_two_pass_ms_per_step": round(ms_two, 5),
                   "blended_peak_TOPS": round(BLENDED_PEAK, 1)},
        "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "frac_of_blended_i8_f16": round(tops / BLENDED_PEAK, 4),
                     "traffic": measured_traffic("prefill_b4h32s4096d128"),
                     "kernel": "prefill_kernel<128, causal>"},
    }
    if not args.no_cpu_baseline:
        # The C oracle (float64, all host threads) on whole heads of the same workload, as many
        # as fit in the CPU budget (one head of S=4096 is ~0.2 s).
        threads = oracle_c.max_threads()
        heads = [(b, hh) for b in range(B) for hh in range(H)]
        done, t0 = 0, time.perf_counter()
        for b, hh in heads:
            q = c["Qi"][b, hh:hh + 1].cpu().numpy()
            k = c["Ki"][b, hh:hh + 1].cpu().numpy()
            v = c["Vi"][b, hh:hh + 1].cpu().numpy()
            sq, sk, sv = (c[n][b, hh:hh + 1].cpu().numpy() for n in ("sQ", "sK", "sV"))
            t1 = time.perf_counter()
            oracle_c.prefill_attention(q, k, v, sq, sk, sv, causal=True, threads=threads)
            done += 1
            elapsed = time.perf_counter() - t0
            if elapsed + (time.perf_counter() - t1) > args.cpu_budget:
                break
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": 2 * done * D * S * (S + 1) / dt / 1e12, "unit": "TOPS",
                               "cores": threads, "kind": "port",
                               "sample": f"C oracle causal attention (float64) on {done} of "
                                         f"{B * H} heads x {S} tokens; {dt:.1f} s"}
    _ = np
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
    A.zero_()
    Bt.zero_()
    ms_zero = time_steps(lambda: capi.gemm_i8_i32(A, Bt, out=C), args.steps, args.warmup, stream)
    tops = ops / (ms_rand * 1e-3) / 1e12
    for name, ms in (("random", ms_rand), ("zero", ms_zero), ("hipblaslt random", ms_lib)):
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
                   "hipblaslt_int_mm_random_TOPS": round(ops / (ms_lib * 1e-3) / 1e12, 1)},
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
    import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    class Block:
        def __init__(self, d, H, dff):
            self.d, self.H, self.Dh, self.dff = d, H, d // H, dff
            g = torch.Generator(device=dev).manual_seed(0)
            rn = lambda *sh: torch.randn(*sh, generator=g, device=dev, dtype=torch.float16)  # noqa: E731
            self.Wqkv = rn(d, 3 * d) * (d ** -0.5)
            self.Wo = rn(d, d) * (d ** -0.5)
            self.W1 = rn(d, dff) * (d ** -0.5)
            self.W2 = rn(dff, d) * (dff ** -0.5)
            w1i, self.sW1 = workloads.quantize_per_channel_w(self.W1)
            w2i, self.sW2 = workloads.quantize_per_channel_w(self.W2)
            self.W1T, self.W2T = ext.transpose_int8_weights(w1i, w2i)

        def mlp_int8_residual(self, h):
            # h + MLP(LN2(h)); the int8 output's dequantization and the residual add are
            # one pass (the reference: h + (out.float() * out_scale).half())
            B, S, d = h.shape
            xi, sx = ext.layernorm_quantize_per_token(h)
            o, so = ext.int8_mlp_forward_prepacked(xi.view(B, S, d), self.W1T, self.W2T,
                                                   sx.reshape(-1), self.sW1, self.sW2)
            return ext.dequantize_per_token(o.view(B, S, d), so.view(B, S), residual=h)

        def mlp_fp16(self, h):
            return F.gelu(F.layer_norm(h, (self.d,)) @ self.W1, approximate="tanh") @ self.W2

        def prefill(self, x, int8):
            B, S, _ = x.shape
            qkv = F.layer_norm(x, (self.d,)) @ self.Wqkv
            if int8:
                qi, sq, ki, sk, vi, sv = ext.quantize_heads(qkv, self.H)
                # rows come out as [B, S, H, Dh], the projection's order: no transpose copy
                a = ext.int8_attention_forward(qi, ki, vi, sq, sk, sv, out_bshd=True)
                a = a.view(B, S, self.d)
            else:
                q, k, v = (t.view(B, S, self.H, self.Dh).transpose(1, 2).contiguous()
                           for t in qkv.split(self.d, dim=-1))
                a = F.scaled_dot_product_attention(q, k, v)
                a = a.transpose(1, 2).contiguous().view(B, S, self.d)
            h = x + a @ self.Wo
            return self.mlp_int8_residual(h) if int8 else h + self.mlp_fp16(h)

        def decode(self, x, kv, int8):
            B = x.size(0)
            q = (F.layer_norm(x, (self.d,)) @ self.Wqkv)[..., :self.d]
            if int8:
                Ki, Vi, sK, sV = kv
                qi, sq = ext.quantize_per_token(q.reshape(B, self.H, self.Dh))
                a = ext.int8_decode_attention_forward(qi, Ki, Vi, sq, sK, sV).view(B, 1, self.d)
            else:
                Kf, Vf = kv
                a = F.scaled_dot_product_attention(q.view(B, self.H, 1, self.Dh), Kf, Vf)
                a = a.transpose(1, 2).contiguous().view(B, 1, self.d)
            h = x + a @ self.Wo
            return self.mlp_int8_residual(h) if int8 else h + self.mlp_fp16(h)

    def cos(a, b):
        return F.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0).item()

    rows = []
    H, Dh, dff = 16, 64, 4096
    d = H * Dh
    blk = Block(d, H, dff)
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "decode-sweep", "decode-paged", "mlp", "prefill", "gemm",
                             "block"])
    ap.add_argument("--page", type=int, default=16, help="page size for --workload decode-paged")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--nsplit", type=int, default=0)
    ap.add_argument("--seed", type=int, default=20241201)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-calibrate", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode shards over (b,h) with no exchange; see DESIGN.md)", file=sys.stderr)
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
    else:
        res = bench_decode(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""MLA decode benchmark on one MI355X.

Metric: microseconds per MLA decode call + achieved HBM TB/s,
n_h = 128, N = 4096, fp16 -- the reference's `-k fused` fp16 path
(mla_decode_split, csrc/mla_api.cpp:86-113), here through the C ABI of
libmla_mi355x.so.

A step is one decode call (split-KV kernel + LSE combine) over one
synthetic (Q*, C) pair. Inputs are resident in HBM before timing starts;
each step uses the next pair of a pool of distinct buffers totalling
--flush-mb (default 1024 MB > the 256 MB MALL + 32 MB of L2), so no step
finds its C in a cache. Timing is HIP events on the launch stream: one pair
around all K steps (value, us/call) and one pair around K back-to-back
split-kernel launches (roofline.achieved for the dominant kernel).

Prints ONE JSON line. --workload picks another configuration (n65536, nh16,
batched, paged, block, bf16, the fp8 cache workloads, fp32 and fp32_n4096) for
measurement runs; the default is the headline one.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ada-mla_amd"))
sys.path.insert(0, ROOT)

METRIC = "µs per MLA decode call + achieved HBM TB/s, n_h=128 N=4096 fp16"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA
MFMA_F32_PEAK_TFS = 157.3   # MI355X dense fp32 MFMA

FP8_KINDS = ("fp8", "fp8_batched")
BATCHED_KINDS = ("batched", "paged", "block", "fp8_batched")

WORKLOADS = {
    "n4096": dict(kind="fp16", n_h=128, n=4096, desc="fp16 single sequence, n_h=128, N=4096 (BASELINE config 2)"),
    "n65536": dict(kind="fp16", n_h=128, n=65536, desc="fp16 split-KV, n_h=128, N=65536 (BASELINE config 3)"),
    "nh16": dict(kind="fp16", n_h=16, n=32768, desc="fp16 low-head, n_h=16, N=32768 (BASELINE config 4)"),
    "batched": dict(kind="batched", n_h=128, batch=32,
                    desc="fp16 batched, B=32, N_b ~ U[512,16384] seed 42 (BASELINE config 5)"),
    "fp32": dict(kind="fp32", n_h=128, n=1024, desc="fp32 path, n_h=128, N=1024 (BASELINE config 1 shape on GPU)"),
    "fp32_n4096": dict(kind="fp32", n_h=128, n=4096,
                       desc="fp32 path, n_h=128, N=4096 (the length of the reference's --fp32 worklog figure)"),
    "paged": dict(kind="paged", n_h=128, batch=32, page=64,
                  desc="fp16 paged KV cache (64-token pages, shuffled), B=32, N_b ~ U[512,16384] seed 42 "
                       "(config 5 through a block table)"),
    "block": dict(kind="block", n_h=128, batch=32, d_model=5120,
                  desc="fp16 MLA block decode step: query absorption (W_UK) + config-5 batched decode + value "
                       "and output projections (W_UV, W_O; d_model 5120), B=32"),
    "fp8": dict(kind="fp8", n_h=128, n=4096, desc="fp8 (E4M3FN, per-tensor scale) KV cache, fp16 query/output, "
                                                 "n_h=128, N=4096 (fp8 variant of config 2)"),
    "fp8_n65536": dict(kind="fp8", n_h=128, n=65536, desc="fp8 (E4M3FN, per-tensor scale) KV cache, fp16 "
                                                          "query/output, n_h=128, N=65536 (fp8 variant of config 3)"),
    "fp8_batched": dict(kind="fp8_batched", n_h=128, batch=32,
                        desc="fp8 (E4M3FN, per-tensor scale) KV cache, fp16 query/output, batched B=32, "
                             "N_b ~ U[512,16384] seed 42 (fp8 variant of config 5)"),
    "bf16": dict(kind="bf16", n_h=128, n=4096, desc="bf16 KV cache, n_h=128, N=4096 (bf16 variant of config 2)"),
}


def algorithmic(kind, n_h, total_tokens, batch=1, d_model=0):
    """Bytes and flops of one call: e*(n_h*576 + N*576 + n_h*512), 2*n_h*N*1088; for the block
    step also the weights W_UK, W_UV [n_h,128,512], W_O [d_model, n_h*128], the query halves and
    the output read or written once, and their GEMM flops."""
    e = 4 if kind == "fp32" else 2
    ec = 1 if kind in FP8_KINDS else e  # cache bytes per value
    bytes_ = e * (batch * n_h * 576 + batch * n_h * 512) + ec * total_tokens * 576
    flops = 2 * n_h * total_tokens * (576 + 512)
    if kind == "block":
        bytes_ += e * (2 * n_h * 128 * 512 + d_model * n_h * 128 + batch * n_h * 192 + batch * d_model)
        flops += 2 * batch * (2 * n_h * 128 * 512 + n_h * 128 * d_model)
    return bytes_, flops


def roof_kernel_key(kind):
    return "mla::splitkv_fp32_kernel" if kind == "fp32" else "mla::splitkv_fp16_kernel"


def hbm_traffic(workload, kernel):
    """HBM bytes per launch of the dominant kernel (FETCH_SIZE + WRITE_SIZE, each
    scaled by its reading for a known-size device copy), from the committed
    rocprofv3 --pmc summary profiles/hbm_traffic.json, or None when that file has
    no entry for this workload."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f)["workloads"][workload][kernel]
    except (OSError, KeyError, ValueError):
        return None, None
    return entry["fetch_bytes"] + entry["write_bytes"], "profiles/hbm_traffic_fetch_write.txt"


def cpu_info():
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, os.cpu_count()


def cpu_baseline(n_h, n, reps=5):
    """The oracle's C restatement of run_mla_decode_cpu (cpu.cpp:5-61), contract
    form (scale 1/sqrt(192), 512 value columns), fp32, one thread pinned to one
    core: 1 warm-up + median of `reps` calls on the workload's shape."""
    import numpy as np
    from oracle import mla_oracle
    from ada_mla import synthetic
    q, c = synthetic.decode_inputs(n_h, n, seed=42, dtype=np.float32)
    old = os.sched_getaffinity(0)
    core = min(old)
    os.sched_setaffinity(0, {core})
    try:
        mla_oracle.naive_cpu(q, c)
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            mla_oracle.naive_cpu(q, c)
            times.append(time.perf_counter() - t0)
        ref_us = None
        if mla_oracle.reference_cpu_available():
            mla_oracle.reference_cpu(q, c)
            rt = []
            for _ in range(3):
                t0 = time.perf_counter()
                mla_oracle.reference_cpu(q, c)
                rt.append(time.perf_counter() - t0)
            ref_us = statistics.median(rt) * 1e6
    finally:
        os.sched_setaffinity(0, old)
    model, ncpu = cpu_info()
    return {
        "value": statistics.median(times) * 1e6,
        "unit": "us/call",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle/mla_naive_cpu.c (restatement of run_mla_decode_cpu, cpu.cpp:5-61), fp32, "
                   f"n_h={n_h}, N={n}, scale 1/sqrt(192), 512 value columns; gcc -O2; 1 thread pinned to "
                   f"core {core}; 1 warm-up + median of {reps} calls; host: {model}, {ncpu} logical CPUs"),
        "reference_binary_us": ref_us,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--spinup-ms", type=float, default=300.0,
                    help="untimed decode calls for at least this long before the warm-up steps, so that "
                         "the GPU's clocks are at their steady state (a cold start reads up to 15%% slower)")
    ap.add_argument("--workload", default="n4096", choices=sorted(WORKLOADS))
    ap.add_argument("--num-splits", type=int, default=0)
    ap.add_argument("--partials", choices=("auto", "fp16", "fp32"), default="auto",
                    help="fp16 single-sequence workloads: precision of the split partials (auto: fp32 for "
                         "n65536, whose BASELINE config names fp32 partials, else fp16); the other precision "
                         "is timed too and reported as alt_partials")
    ap.add_argument("--no-alt", action="store_true",
                    help="skip the timing with the other partial precision (profiling runs: one kernel variant)")
    ap.add_argument("--flush-mb", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="run 10 plain device-to-device copies of MB MiB instead of the decode: the "
                         "known-size kernel that scales rocprof's FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the decode path is built and measured on "
              "one MI355X; a multi-GPU figure is not produced). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from ada_mla import capi

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        n = args.calibrate_copy * 2**20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(10):
            dst.copy_(src)
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 100.0
        print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "us_per_copy": us,
                          "GBps_read_plus_write": 2 * n / (us * 1e-6) / 1e9}), flush=True)
        return
    lib = capi.load()
    wl = WORKLOADS[args.workload]
    kind, n_h = wl["kind"], wl["n_h"]
    stream = torch.cuda.current_stream(dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)

    is_fp8 = kind in FP8_KINDS
    c_dtype = torch.float8_e4m3fn if is_fp8 else None
    if kind in BATCHED_KINDS:
        from ada_mla import synthetic
        seqlens = synthetic.batched_seqlens(wl["batch"], seed=42)
        batch = wl["batch"]
        total = int(seqlens.sum())
        cu = torch.zeros(batch + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.from_numpy(seqlens), 0)
        cu_d = cu.to(dev)
        q_shape, c_shape = (batch, n_h, 576), (total, 576)
        dtype = torch.float16
        if kind == "paged":
            page = wl["page"]
            need = [-(-int(n) // page) for n in seqlens]
            n_pages = sum(need)
            perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(42)).to(torch.int32)
            bt = torch.zeros(batch, max(need), dtype=torch.int32)
            k = 0
            for b, nb in enumerate(need):
                bt[b, :nb] = perm[k:k + nb]
                k += nb
            bt_d = bt.to(dev)
            c_shape = (n_pages, page, 576)
        if kind == "block":
            d_model = wl["d_model"]
            gw = torch.Generator(device=dev)
            gw.manual_seed(7)
            mk = lambda *shape, sc=1.0: (torch.randn(shape, generator=gw, device=dev) * sc).to(dtype)
            q_nope, q_rope = mk(batch, n_h, 128), mk(batch, n_h, 64)
            w_uk, w_uv = mk(n_h, 128, 512, sc=128 ** -0.5), mk(n_h, 128, 512, sc=512 ** -0.5)
            w_o = mk(d_model, n_h * 128, sc=(n_h * 128) ** -0.5)
            q_star = torch.empty(batch, n_h, 576, device=dev, dtype=dtype)
            o_star = torch.empty(batch, n_h, 512, device=dev, dtype=dtype)
            y = torch.empty(batch, d_model, device=dev, dtype=dtype)
            pws_bytes = lib.mla_project_output_workspace_size(batch, n_h)
            pws = torch.empty(pws_bytes, dtype=torch.uint8, device=dev)
    else:
        batch, total = 1, wl["n"]
        q_shape, c_shape = (n_h, 576), (total, 576)
        dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}.get(kind, torch.float16)
    esz = 4 if dtype == torch.float32 else 2
    pair_bytes = (math.prod(q_shape) + math.prod(c_shape)) * esz
    pool = max(2, math.ceil(args.flush_mb * 2**20 / pair_bytes))
    if is_fp8:
        pair_bytes = math.prod(q_shape) * esz + math.prod(c_shape)
        pool = max(2, math.ceil(args.flush_mb * 2**20 / pair_bytes))
    qs = [torch.randn(q_shape, generator=gen, device=dev, dtype=dtype) for _ in range(pool)]
    cs = [torch.randn(c_shape, generator=gen, device=dev, dtype=torch.float32).to(c_dtype) if is_fp8 else
          torch.randn(c_shape, generator=gen, device=dev, dtype=dtype) for _ in range(pool)]
    out = torch.empty((batch, n_h, 512) if kind in BATCHED_KINDS else (n_h, 512), device=dev, dtype=dtype)

    splits = args.num_splits
    if kind in ("fp16", "bf16"):
        ws_bytes = lib.mla_decode_split_workspace_size(n_h, total, splits)
        eff_splits = lib.mla_decode_split_num_splits(
            n_h, total, splits, capi.FLAG_FP32_PARTIALS if args.partials == "fp32" or
            (args.partials == "auto" and args.workload == "n65536") else 0)
    elif kind == "fp32":
        ws_bytes = lib.mla_decode_fused_workspace_size(n_h, total, splits)
        eff_splits = None
    elif kind == "paged":
        ws_bytes = lib.mla_decode_paged_workspace_size(batch, n_h, total, splits)
        eff_splits = None
    elif is_fp8:
        ws_bytes = lib.mla_decode_split_fp8_workspace_size(batch, n_h, total, splits)
        eff_splits = None
    elif kind == "block":
        ws_bytes = lib.mla_decode_split_batched_workspace_size(batch, n_h, total, splits)
        eff_splits = None
    else:
        ws_bytes = lib.mla_decode_split_batched_workspace_size(batch, n_h, total, splits)
        eff_splits = None
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

    def check(st, fn):
        if st != 0:
            raise capi.MlaError(fn, st)

    partials = args.partials
    if partials == "auto":
        partials = "fp32" if args.workload == "n65536" else "fp16"
    pflags = [capi.FLAG_FP32_PARTIALS if partials == "fp32" else 0]

    def phase1(i):
        q, c = qs[i % pool], cs[i % pool]
        if kind == "fp16":
            check(lib.mla_decode_split_fp16_partials(q.data_ptr(), c.data_ptr(), ws.data_ptr(), ws_bytes,
                                                     n_h, total, splits, pflags[0], sptr), "partials")
        elif kind == "fp8":
            check(lib.mla_decode_split_fp8(q.data_ptr(), c.data_ptr(), 1.0, out.data_ptr(), ws.data_ptr(), ws_bytes,
                                           n_h, total, splits, sptr), "fp8")
        elif kind == "fp8_batched":
            check(lib.mla_decode_split_batched_fp8(q.data_ptr(), c.data_ptr(), 1.0, cu_d.data_ptr(), out.data_ptr(),
                                                   ws.data_ptr(), ws_bytes, batch, n_h, total, splits, sptr),
                  "fp8_batched")
        elif kind == "bf16":
            check(lib.mla_decode_split_bf16(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
                                            n_h, total, splits, sptr), "bf16")
        elif kind == "block":
            check(lib.mla_absorb_query_fp16(q_nope.data_ptr(), q_rope.data_ptr(), w_uk.data_ptr(),
                                            q_star.data_ptr(), batch, n_h, sptr), "absorb")
            check(lib.mla_decode_split_batched_fp16(q_star.data_ptr(), c.data_ptr(), cu_d.data_ptr(),
                                                    o_star.data_ptr(), ws.data_ptr(), ws_bytes, batch, n_h, total,
                                                    splits, sptr), "batched")
            check(lib.mla_project_output_fp16(o_star.data_ptr(), w_uv.data_ptr(), w_o.data_ptr(), y.data_ptr(),
                                              pws.data_ptr(), pws_bytes, batch, n_h, d_model, sptr), "project")
        elif kind == "paged":
            check(lib.mla_decode_paged_fp16(q.data_ptr(), c.data_ptr(), bt_d.data_ptr(), cu_d.data_ptr(),
                                            out.data_ptr(), ws.data_ptr(), ws_bytes, batch, n_h, total, page,
                                            c.shape[0], bt_d.shape[1], splits, sptr), "paged")
        elif kind == "fp32":
            check(lib.mla_decode_fused_fp32(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
                                            n_h, 576, total, splits, sptr), "fused_fp32")
        else:
            check(lib.mla_decode_split_batched_fp16(q.data_ptr(), c.data_ptr(), cu_d.data_ptr(), out.data_ptr(),
                                                    ws.data_ptr(), ws_bytes, batch, n_h, total, splits, sptr),
                  "batched")

    def phase2():
        if kind == "fp16":
            check(lib.mla_decode_split_fp16_combine(ws.data_ptr(), ws_bytes, out.data_ptr(), n_h, total, splits,
                                                    pflags[0], sptr), "combine")

    t_end = time.perf_counter() + args.spinup_ms * 1e-3
    while time.perf_counter() < t_end:
        for i in range(50):
            phase1(i)
            phase2()
        torch.cuda.synchronize()
    for i in range(args.warmup):
        phase1(i)
        phase2()
    torch.cuda.synchronize()

    K = args.steps
    # (1) the timed region: exactly K steps, nothing but the decode calls
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(K):
        phase1(args.warmup + i)
        phase2()
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    us_call = total_ms * 1000.0 / K

    # (2) the dominant kernel alone, K launches back to back between one event
    # pair on the launch stream: the mean launch-to-launch time, which is what
    # rocprofv3's kernel trace reports as the kernel's duration (an event pair
    # around every single launch would add the events' own ~3.5 us each)
    torch.cuda.synchronize()
    ka = torch.cuda.Event(enable_timing=True)
    kb = torch.cuda.Event(enable_timing=True)
    ka.record(stream)
    for i in range(K):
        phase1(args.warmup + K + i)
    kb.record(stream)
    torch.cuda.synchronize()
    k_us = ka.elapsed_time(kb) * 1000.0 / K
    # (3) for reference: an event pair around each split launch (combine outside)
    pa = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    pb = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    for i in range(K):
        pa[i].record(stream)
        phase1(args.warmup + 2 * K + i)
        pb[i].record(stream)
        phase2()
    torch.cuda.synchronize()
    k_pair_us = statistics.median(a.elapsed_time(b) * 1000.0 for a, b in zip(pa, pb))

    # (4) fp16 single sequence: the same K calls with the other partial precision
    alt = None
    if kind == "fp16" and not args.no_alt:
        pflags[0] ^= capi.FLAG_FP32_PARTIALS
        for i in range(args.warmup):
            phase1(i)
            phase2()
        torch.cuda.synchronize()
        start.record(stream)
        for i in range(K):
            phase1(args.warmup + i)
            phase2()
        end.record(stream)
        torch.cuda.synchronize()
        alt = {"partials": "fp16" if partials == "fp32" else "fp32", "us_per_call": start.elapsed_time(end) * 1000.0 / K}
        pflags[0] ^= capi.FLAG_FP32_PARTIALS

    alg_bytes, alg_flops = algorithmic(kind, n_h, total, batch, wl.get("d_model", 0))
    achieved = alg_bytes / (k_us * 1e-6) / 1e9
    mfma_peak = MFMA_F32_PEAK_TFS if kind == "fp32" else MFMA_F16_PEAK_TFS
    tflops = alg_flops / (k_us * 1e-6) / 1e12
    bound_hbm = alg_bytes / HBM_PEAK_GBS / 1e3  # us
    bound_mfma = alg_flops / mfma_peak / 1e6    # us
    if bound_hbm >= bound_mfma:
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS}
    else:
        roof = {"bound": "mfma", "achieved": tflops, "peak": mfma_peak, "unit": "TFLOP/s",
                "frac": tflops / mfma_peak}
    traffic, traffic_src = hbm_traffic(args.workload, roof_kernel_key(kind))
    roof.update({
        "traffic": traffic,
        "traffic_source": traffic_src,
        "kernel": ("splitkv_fp32_kernel" if kind == "fp32" else
                   "absorb GEMM + splitkv_fp16_kernel + combine + projection GEMMs" if kind == "block" else
                   "splitkv_fp16_kernel"),
        "kernel_us": k_us,
        "kernel_us_event_pair_median": k_pair_us,
        "algorithmic_bytes": alg_bytes,
        "algorithmic_flops": alg_flops,
        "mfma_tflops": tflops,
        "mfma_frac": tflops / mfma_peak,
        "roofline_time_us": max(bound_hbm, bound_mfma),
        "call_frac": max(bound_hbm, bound_mfma) / us_call,
    })
    if kind in ("batched", "bf16", "paged", "block") + FP8_KINDS:
        roof["note"] = f"{kind} has no phase split: kernel_us is the whole call"

    res = {
        "metric": METRIC,
        "value": us_call,
        "unit": "us/call",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "spinup_ms": args.spinup_ms,
        "ms_per_step": total_ms / K,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp8 E4M3FN cache)" if is_fp8 else {"fp32": "fp32", "bf16": "bf16"}.get(kind, "fp16"),
        "data": "synthetic (N(0,1), torch generator seed 42, resident in HBM)",
        "config": {
            "workload": wl["desc"],
            "num_heads": n_h,
            "seq_len": total if kind not in BATCHED_KINDS else None,
            "total_tokens": total,
            "batch": batch,
            "num_splits": eff_splits,
            "partials": partials if kind == "fp16" else ("fp32" if kind == "fp32" else "fp16"),
            "cache_flush": f"{pool} distinct (Q*, C) buffers, {pool * pair_bytes / 2**20:.0f} MB, rotated per step",
            "parallelism": "single GPU",
        },
        "tbps": alg_bytes / (us_call * 1e-6) / 1e12,
        "roofline": roof,
    }
    if alt is not None:
        res["alt_partials"] = alt
    if not args.no_cpu:
        cn = 1024 if kind == "fp32" else (total if kind == "fp16" else 4096)
        res["cpu_baseline"] = cpu_baseline(n_h, cn)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

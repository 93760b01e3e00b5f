#!/usr/bin/env python3
"""MLA decode benchmark on one MI355X.

Metric: microseconds per MLA decode call + achieved HBM TB/s,
n_h = 128, N = 4096, fp16 -- the reference's `-k fused` fp16 path
(mla_decode_split, csrc/mla_api.cpp:86-113), here through the C ABI of
libmla_mi355x.so.

A step is one decode call over one synthetic input set (Q*, C, and for the
block workload the weights). Inputs are resident in HBM before timing starts.

Cache-cold by construction: every call the process makes -- spin-up, warm-up,
timed, the split-kernel-only loop, the other-precision loop -- takes the next
input set of one pool in strict round-robin order (one cursor per workload),
so between two uses of any buffer every other set of the pool is used once.
The pool is sized so that this reuse distance is at least --flush-mb
(default 1024 MB, four times the 256 MB MALL and far above the 4 MB L2s);
the script asserts >= 512 MB for every workload. The reference flushes its L2
by zeroing a 256 MB buffer before each timed call (mla.py:122-130).

Timing is HIP events on the launch stream: one pair around all K calls
(`value`, us/call), one pair around K back-to-back split-kernel launches
(`roofline.kernel_us`, the dominant kernel alone: single sequences and
batches). `roofline.frac` is over the whole call (algorithmic bytes / call
time / 8 TB/s); `roofline.kernel_frac` over the split kernel alone.
`roofline.traffic` is the split kernel's HBM bytes per launch and
`roofline.traffic_call` the whole call's (every kernel), both from the
committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary, with their ratios to the
algorithmic bytes.

Prints ONE JSON line. With the default workload the line also carries
`other_configs`: BASELINE configs 3, 4 and 5 (N = 65536 with fp32 partials,
n_h = 16, batched B = 32) measured the same way in the same run. --workload
picks another configuration (n65536, nh16, batched, paged, block, bf16, the fp8
cache workloads, fp32, fp32_n4096, n256, a short sequence on the one-launch
path, and n32, the shortest call: the library's fixed cost) as the main line.
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
MIN_REUSE_MB = 512          # bytes of other inputs between two uses of one buffer (> 256 MB MALL)

FP8_KINDS = ("fp8", "fp8_batched")
BATCHED_KINDS = ("batched", "paged", "block", "fp8_batched")

WORKLOADS = {
    "n4096": dict(kind="fp16", n_h=128, n=4096, desc="fp16 single sequence, n_h=128, N=4096 (BASELINE config 2)"),
    "n65536": dict(kind="fp16", n_h=128, n=65536, desc="fp16 split-KV, n_h=128, N=65536 (BASELINE config 3)"),
    "nh16": dict(kind="fp16", n_h=16, n=32768, desc="fp16 low-head, n_h=16, N=32768 (BASELINE config 4)"),
    "n256": dict(kind="fp16", n_h=128, n=256, desc="fp16 short sequence, n_h=128, N=256 (one split: the one-launch "
                                                  "path, no combine)"),
    "n32": dict(kind="fp16", n_h=128, n=32, desc="fp16 shortest call, n_h=128, N=32 (one 32-token block, one launch, "
                                                "no combine): the library's fixed cost per call"),
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

# measured beside the default (headline) workload
OTHER_CONFIGS = ("n65536", "nh16", "batched")


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
    """HBM bytes per launch of the dominant kernel and per whole call (every
    kernel of the call: FETCH_SIZE + WRITE_SIZE, each scaled by its reading for
    a known-size device copy), from the committed rocprofv3 --pmc summary
    profiles/hbm_traffic.json, or None when that file has no entry for this
    workload."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            entries = json.load(f)["workloads"][workload]
        entry = entries[kernel]
    except (OSError, KeyError, ValueError):
        return None, None, None
    call = sum(e["fetch_bytes"] + e["write_bytes"] for e in entries.values())
    return entry["fetch_bytes"] + entry["write_bytes"], call, "profiles/hbm_traffic_fetch_write.txt"


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


def _timed_reps(fn, budget_s, min_reps=3, max_reps=200):
    """1 warm-up call, then calls until budget_s has passed (at least min_reps):
    the list of per-call seconds."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def cpu_baseline(n_h, n, budget_s=7.0):
    """The oracle's C restatement of run_mla_decode_cpu (cpu.cpp:5-61), contract
    form (scale 1/sqrt(192), 512 value columns), fp32, one thread pinned to one
    core, on the workload's shape: 1 warm-up, then calls for about budget_s
    seconds, median. Beside it: the reference's own CPU kernel (oracle/_ref,
    built from /root/reference where that exists) on the same inputs, and the
    restatement at BASELINE config 1's shape (n_h = 128, N = 1024)."""
    import numpy as np
    from oracle import mla_oracle
    from ada_mla import synthetic
    q, c = synthetic.decode_inputs(n_h, n, seed=42, dtype=np.float32)
    q1, c1 = synthetic.decode_inputs(128, 1024, seed=42, dtype=np.float32)
    old = os.sched_getaffinity(0)
    core = min(old)
    os.sched_setaffinity(0, {core})
    try:
        times = _timed_reps(lambda: mla_oracle.naive_cpu(q, c), budget_s)
        ref_us = ref_reps = None
        if mla_oracle.reference_cpu_available():
            rt = _timed_reps(lambda: mla_oracle.reference_cpu(q, c), 2.0)
            ref_us, ref_reps = statistics.median(rt) * 1e6, len(rt)
        t1 = _timed_reps(lambda: mla_oracle.naive_cpu(q1, c1), 2.0)
    finally:
        os.sched_setaffinity(0, old)
    model, ncpu = cpu_info()
    return {
        "value": statistics.median(times) * 1e6,
        "unit": "us/call",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle/mla_naive_cpu.c (restatement of run_mla_decode_cpu, cpu.cpp:5-61), fp32, "
                   f"n_h={n_h}, N={n} (this line's workload), scale 1/sqrt(192), 512 value columns; gcc -O2; "
                   f"1 thread pinned to core {core}; 1 warm-up + median of {len(times)} calls "
                   f"({sum(times):.1f} s of CPU work); host: {model}, {ncpu} logical CPUs"),
        "reference_binary_us": ref_us,
        "reference_binary_calls": ref_reps,
        "config1_n1024_us": statistics.median(t1) * 1e6,
        "config1_calls": len(t1),
    }


class Runner:
    """One workload's input pool, workspace and call functions. Every call
    (call() or split_only()) takes the next pool entry in round-robin order."""

    def __init__(self, lib, capi, torch, name, dev, stream, flush_mb, partials="auto", num_splits=0):
        wl = WORKLOADS[name]
        self.name, self.wl = name, wl
        self.kind, self.n_h = wl["kind"], wl["n_h"]
        kind, n_h = self.kind, self.n_h
        self.lib, self.capi, self.torch = lib, capi, torch
        self.sptr = ctypes.c_void_p(stream.cuda_stream)
        self.splits = num_splits
        self.cursor = 0
        gen = torch.Generator(device=dev)
        gen.manual_seed(42)
        is_fp8 = kind in FP8_KINDS
        self.is_fp8 = is_fp8
        dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}.get(kind, torch.float16)
        self.dtype = dtype
        esz = 4 if dtype == torch.float32 else 2
        self.batch, self.page = 1, None
        if kind in BATCHED_KINDS:
            from ada_mla import synthetic
            seqlens = synthetic.batched_seqlens(wl["batch"], seed=42)
            self.batch = wl["batch"]
            self.total = int(seqlens.sum())
            cu = torch.zeros(self.batch + 1, dtype=torch.int32)
            cu[1:] = torch.cumsum(torch.from_numpy(seqlens), 0)
            self.cu_d = cu.to(dev)
            q_shape, c_shape = (self.batch, n_h, 576), (self.total, 576)
            if kind == "paged":
                self.page = wl["page"]
                need = [-(-int(n) // self.page) for n in seqlens]
                n_pages = sum(need)
                perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(42)).to(torch.int32)
                bt = torch.zeros(self.batch, max(need), dtype=torch.int32)
                k = 0
                for b, nb in enumerate(need):
                    bt[b, :nb] = perm[k:k + nb]
                    k += nb
                self.bt_d = bt.to(dev)
                c_shape = (n_pages, self.page, 576)
        else:
            self.total = wl["n"]
            q_shape, c_shape = (n_h, 576), (self.total, 576)
        self.q_shape, self.c_shape = q_shape, c_shape
        c_esz = 1 if is_fp8 else esz
        set_bytes = math.prod(q_shape) * esz + math.prod(c_shape) * c_esz
        if kind == "block":
            d_model = self.d_model = wl["d_model"]
            # the weights of a layer rotate with the cache: a decode loop reads each layer's
            # weights once per step, so they are not cache-resident either
            set_bytes += esz * (self.batch * n_h * 192 + 2 * n_h * 128 * 512 + d_model * n_h * 128)
        pool = max(2, math.ceil(flush_mb * 2**20 / set_bytes) + 1)
        self.pool, self.set_bytes = pool, set_bytes
        self.reuse_bytes = (pool - 1) * set_bytes
        assert self.reuse_bytes >= MIN_REUSE_MB * 2**20, (name, pool, set_bytes)

        self.qs = [torch.randn(q_shape, generator=gen, device=dev, dtype=dtype) for _ in range(pool)]
        self.cs = [torch.randn(c_shape, generator=gen, device=dev, dtype=torch.float32).to(torch.float8_e4m3fn)
                   if is_fp8 else torch.randn(c_shape, generator=gen, device=dev, dtype=dtype) for _ in range(pool)]
        self.out = torch.empty((self.batch, n_h, 512) if kind in BATCHED_KINDS else (n_h, 512), device=dev,
                               dtype=dtype)
        if kind == "block":
            gw = torch.Generator(device=dev)
            gw.manual_seed(7)
            mk = lambda *shape, sc=1.0: (torch.randn(shape, generator=gw, device=dev) * sc).to(dtype)
            self.q_nope = [mk(self.batch, n_h, 128) for _ in range(pool)]
            self.q_rope = [mk(self.batch, n_h, 64) for _ in range(pool)]
            self.w_uk = [mk(n_h, 128, 512, sc=128 ** -0.5) for _ in range(pool)]
            self.w_uv = [mk(n_h, 128, 512, sc=512 ** -0.5) for _ in range(pool)]
            self.w_o = [mk(d_model, n_h * 128, sc=(n_h * 128) ** -0.5) for _ in range(pool)]
            self.q_star = torch.empty(self.batch, n_h, 576, device=dev, dtype=dtype)
            self.o_star = torch.empty(self.batch, n_h, 512, device=dev, dtype=dtype)
            self.y = torch.empty(self.batch, d_model, device=dev, dtype=dtype)
            self.pws_bytes = lib.mla_project_output_workspace_size(self.batch, n_h, self.d_model)
            self.pws = torch.empty(self.pws_bytes, dtype=torch.uint8, device=dev)

        if partials == "auto":
            partials = "fp32" if name == "n65536" else "fp16"
        self.partials = partials if kind == "fp16" else ("fp32" if kind == "fp32" else "fp16")
        self.pflags = capi.FLAG_FP32_PARTIALS if (kind == "fp16" and partials == "fp32") else 0
        total, s = self.total, self.splits
        if kind in ("fp16", "bf16"):
            self.ws_bytes = lib.mla_decode_split_workspace_size(n_h, total, s)
        elif kind == "fp32":
            self.ws_bytes = lib.mla_decode_fused_workspace_size(n_h, total, s)
        elif kind == "paged":
            self.ws_bytes = lib.mla_decode_paged_workspace_size(self.batch, n_h, total, s)
        elif is_fp8:
            self.ws_bytes = lib.mla_decode_split_fp8_workspace_size(self.batch, n_h, total, s)
        else:
            self.ws_bytes = lib.mla_decode_split_batched_workspace_size(self.batch, n_h, total, s)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=dev)
        # device addresses of the pool, read once: a call's two launches take
        # ~8 us of host time (HIP's own launch path, ~3.3 us each) against
        # ~11 us of GPU time at N = 4096, and four tensor.data_ptr() calls per
        # call cost a further 1.2-1.4 us of Python (0.5 us with the addresses
        # cached), which narrows the host's lead over the GPU
        self.qp = [t.data_ptr() for t in self.qs]
        self.cp = [t.data_ptr() for t in self.cs]
        self.outp, self.wsp = self.out.data_ptr(), self.ws.data_ptr()

    def num_splits(self):
        if self.kind in ("fp16", "bf16"):
            return self.lib.mla_decode_split_num_splits(self.n_h, self.total, self.splits, self.pflags)
        return None

    def _check(self, st, fn):
        if st != 0:
            raise self.capi.MlaError(fn, st)

    def _next(self):
        i = self.cursor % self.pool
        self.cursor += 1
        return i

    def split_only(self):
        """The split kernel alone (fp16 single sequence or fp16 batch); the whole call otherwise."""
        if self.kind == "batched":
            i = self._next()
            self._check(self.lib.mla_decode_split_batched_fp16_partials(
                self.qs[i].data_ptr(), self.cs[i].data_ptr(), self.cu_d.data_ptr(), self.ws.data_ptr(), self.ws_bytes,
                self.batch, self.n_h, self.total, self.splits, self.sptr), "batched partials")
            return
        if self.kind != "fp16":
            return self.call()
        i = self.cursor % self.pool
        self.cursor += 1
        st = self.lib.mla_decode_split_fp16_partials(self.qp[i], self.cp[i], self.wsp, self.ws_bytes, self.n_h,
                                                     self.total, self.splits, self.pflags, self.sptr)
        if st:
            self._check(st, "partials")

    def call(self):
        """One whole decode call (for the block workload: the whole block step)."""
        if self.kind == "fp16":
            i = self.cursor % self.pool
            self.cursor += 1
            st = self.lib.mla_decode_split_fp16_ex(self.qp[i], self.cp[i], self.outp, self.wsp, self.ws_bytes,
                                                   self.n_h, self.total, self.splits, self.pflags, self.sptr)
            if st:
                self._check(st, "split_fp16")
            return
        i = self._next()
        lib, sp, n_h, total, s = self.lib, self.sptr, self.n_h, self.total, self.splits
        q, c, out, ws, wsb, kind = self.qs[i], self.cs[i], self.out, self.ws, self.ws_bytes, self.kind
        if kind == "bf16":
            self._check(lib.mla_decode_split_bf16(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(), wsb,
                                                  n_h, total, s, sp), "bf16")
        elif kind == "fp8":
            self._check(lib.mla_decode_split_fp8(q.data_ptr(), c.data_ptr(), 1.0, out.data_ptr(), ws.data_ptr(), wsb,
                                                 n_h, total, s, sp), "fp8")
        elif kind == "fp8_batched":
            self._check(lib.mla_decode_split_batched_fp8(q.data_ptr(), c.data_ptr(), 1.0, self.cu_d.data_ptr(),
                                                         out.data_ptr(), ws.data_ptr(), wsb, self.batch, n_h, total,
                                                         s, sp), "fp8_batched")
        elif kind == "fp32":
            self._check(lib.mla_decode_fused_fp32(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(), wsb,
                                                  n_h, 576, total, s, sp), "fused_fp32")
        elif kind == "paged":
            self._check(lib.mla_decode_paged_fp16(q.data_ptr(), c.data_ptr(), self.bt_d.data_ptr(),
                                                  self.cu_d.data_ptr(), out.data_ptr(), ws.data_ptr(), wsb,
                                                  self.batch, n_h, total, self.page, c.shape[0],
                                                  self.bt_d.shape[1], s, sp), "paged")
        elif kind == "block":
            self._check(lib.mla_absorb_query_fp16(self.q_nope[i].data_ptr(), self.q_rope[i].data_ptr(),
                                                  self.w_uk[i].data_ptr(), self.q_star.data_ptr(), self.batch, n_h,
                                                  sp), "absorb")
            self._check(lib.mla_decode_split_batched_fp16(self.q_star.data_ptr(), c.data_ptr(),
                                                          self.cu_d.data_ptr(), self.o_star.data_ptr(),
                                                          ws.data_ptr(), wsb, self.batch, n_h, total, s, sp),
                        "batched")
            self._check(lib.mla_project_output_fp16(self.o_star.data_ptr(), self.w_uv[i].data_ptr(),
                                                    self.w_o[i].data_ptr(), self.y.data_ptr(), self.pws.data_ptr(),
                                                    self.pws_bytes, self.batch, n_h, self.d_model, sp), "project")
        else:
            self._check(lib.mla_decode_split_batched_fp16(q.data_ptr(), c.data_ptr(), self.cu_d.data_ptr(),
                                                          out.data_ptr(), ws.data_ptr(), wsb, self.batch, n_h, total,
                                                          s, sp), "batched")

    def release(self):
        for k in ("qs", "cs", "q_nope", "q_rope", "w_uk", "w_uv", "w_o", "ws", "out"):
            if hasattr(self, k):
                setattr(self, k, None)


def time_loop(torch, stream, fn, k):
    """k calls of fn between one pair of HIP events on the launch stream: us per call."""
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(k):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1000.0 / k


def spin_up(torch, r, seconds):
    """Untimed calls for about `seconds`, so that the clocks reach their steady state."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(20):
            r.call()
        torch.cuda.synchronize()


def roofline(r, us_call, k_us):
    alg_bytes, alg_flops = algorithmic(r.kind, r.n_h, r.total, r.batch, r.wl.get("d_model", 0))
    mfma_peak = MFMA_F32_PEAK_TFS if r.kind == "fp32" else MFMA_F16_PEAK_TFS
    bound_hbm = alg_bytes / HBM_PEAK_GBS / 1e3  # us
    bound_mfma = alg_flops / mfma_peak / 1e6    # us
    hbm = bound_hbm >= bound_mfma
    per_us = (alg_bytes / 1e3) if hbm else (alg_flops / 1e6)  # GB/s or TFLOP/s per (1/us)
    peak = HBM_PEAK_GBS if hbm else mfma_peak
    roof = {"bound": "hbm" if hbm else "mfma", "achieved": per_us / us_call, "peak": peak,
            "unit": "GB/s" if hbm else "TFLOP/s", "frac": per_us / us_call / peak,
            "frac_over": "whole call (every kernel of one decode call, back to back)"}
    traffic, traffic_call, src = hbm_traffic(r.name, roof_kernel_key(r.kind))
    roof.update({
        "traffic": traffic,
        "traffic_of": "the split kernel alone (FETCH + WRITE, HBM side)",
        "traffic_over_algorithmic": (traffic / alg_bytes) if traffic else None,
        "traffic_call": traffic_call,
        "traffic_call_of": "every kernel of the call (split partials written and read back included)",
        "traffic_call_over_algorithmic": (traffic_call / alg_bytes) if traffic_call else None,
        "traffic_source": src,
        "kernel": ("splitkv_fp32_kernel + combine" if r.kind == "fp32" else
                   "absorb + splitkv_fp16_kernel + combine + projections" if r.kind == "block" else
                   "splitkv_fp16_kernel + combine"),
        "call_us": us_call,
        "kernel_us": k_us,
        "kernel_frac": (per_us / k_us / peak) if k_us else None,
        "kernel_frac_of": "splitkv_fp16_kernel alone (K launches back to back)" if k_us else None,
        "algorithmic_bytes": alg_bytes,
        "algorithmic_flops": alg_flops,
        "mfma_tflops": alg_flops / (us_call * 1e-6) / 1e12,
        "mfma_frac": alg_flops / (us_call * 1e-6) / 1e12 / mfma_peak,
        "roofline_time_us": max(bound_hbm, bound_mfma),
    })
    return roof, alg_bytes


def measure(torch, stream, r, steps, warmup, spinup_s):
    spin_up(torch, r, spinup_s)
    for _ in range(warmup):
        r.call()
    torch.cuda.synchronize()
    us_call = time_loop(torch, stream, r.call, steps)
    k_us = time_loop(torch, stream, r.split_only, steps) if r.kind in ("fp16", "batched") else None
    return us_call, k_us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 2000 calls: the steady back-to-back rate (one box, three processes each,
    # N = 4096: 2000 calls 10.97-11.00 us, 200 calls 11.63-12.33, 20 calls 10.96-11.23)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--spinup-ms", type=float, default=1000.0,
                    help="untimed decode calls for at least this long before the warm-up steps, so that "
                         "the GPU's clocks are at their steady state (a cold start reads up to 15%% slower; "
                         "after 300 ms the first N = 4096 measurement of a process still read 12.4-12.9 "
                         "instead of 11.8 us on some boxes)")
    ap.add_argument("--workload", default="n4096", choices=sorted(WORKLOADS))
    ap.add_argument("--num-splits", type=int, default=0)
    ap.add_argument("--partials", choices=("auto", "fp16", "fp32"), default="auto",
                    help="fp16 single-sequence workloads: precision of the split partials (auto: fp32 for "
                         "n65536, whose BASELINE config names fp32 partials, else fp16); the other precision "
                         "is timed too and reported as alt_partials")
    ap.add_argument("--no-alt", action="store_true",
                    help="skip the timing with the other partial precision (profiling runs: one kernel variant)")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the other BASELINE configs measured beside the default workload")
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
    stream = torch.cuda.current_stream(dev)
    K, W = args.steps, args.warmup

    r = Runner(lib, capi, torch, args.workload, dev, stream, args.flush_mb, args.partials, args.num_splits)
    us_call, k_us = measure(torch, stream, r, K, W, args.spinup_ms * 1e-3)
    roof, alg_bytes = roofline(r, us_call, k_us)
    if r.kind in ("bf16", "paged", "block") + FP8_KINDS:
        roof["note"] = f"{r.kind} has no phase split: kernel_us is not measured separately"

    # the same K calls with the other partial precision (fresh buffers: the cursor runs on)
    alt = None
    if r.kind == "fp16" and not args.no_alt:
        r.pflags ^= capi.FLAG_FP32_PARTIALS
        for _ in range(W):
            r.call()
        alt = {"partials": "fp16" if r.partials == "fp32" else "fp32",
               "us_per_call": time_loop(torch, stream, r.call, K)}
        r.pflags ^= capi.FLAG_FP32_PARTIALS

    res = {
        "metric": METRIC,
        "value": us_call,
        "unit": "us/call",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "spinup_ms": args.spinup_ms,
        "ms_per_step": us_call / 1000.0,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp8 E4M3FN cache)" if r.is_fp8 else {"fp32": "fp32", "bf16": "bf16"}.get(r.kind, "fp16"),
        "data": "synthetic (N(0,1), torch generator seed 42, resident in HBM)",
        "config": {
            "workload": r.wl["desc"],
            "num_heads": r.n_h,
            "seq_len": r.total if r.kind not in BATCHED_KINDS else None,
            "total_tokens": r.total,
            "batch": r.batch,
            "num_splits": r.num_splits(),
            "partials": r.partials,
            "cache_flush": (f"{r.pool} distinct input sets of {r.set_bytes / 2**20:.1f} MB used round-robin by "
                            f"every call of the run (spin-up, warm-up, timed, kernel-only, alt): "
                            f"{r.reuse_bytes / 2**20:.0f} MB of other inputs between two uses of any buffer"),
            "reuse_distance_mb": r.reuse_bytes / 2**20,
            "parallelism": "single GPU",
        },
        "tbps": alg_bytes / (us_call * 1e-6) / 1e12,
        "roofline": roof,
    }
    if alt is not None:
        res["alt_partials"] = alt
    r.release()
    del r
    torch.cuda.empty_cache()

    if args.workload == "n4096" and not args.no_others:
        others = {}
        for name in OTHER_CONFIGS:
            o = Runner(lib, capi, torch, name, dev, stream, args.flush_mb)
            o_us, o_k = measure(torch, stream, o, K, W, 0.1)
            o_roof, o_bytes = roofline(o, o_us, o_k)
            others[name] = {
                "workload": o.wl["desc"],
                "us_per_call": o_us,
                "kernel_us": o_k,
                "frac": o_roof["frac"],
                "kernel_frac": o_roof["kernel_frac"],
                "tbps": o_bytes / (o_us * 1e-6) / 1e12,
                "num_splits": o.num_splits(),
                "partials": o.partials,
                "algorithmic_bytes": o_bytes,
                "reuse_distance_mb": o.reuse_bytes / 2**20,
            }
            o.release()
            del o
            torch.cuda.empty_cache()
        res["other_configs"] = others

    if not args.no_cpu:
        wl = WORKLOADS[args.workload]
        # the workload's own shape for single sequences; N = 4096 stands in for the batched ones
        cn = wl["n"] if "n" in wl else 4096
        res["cpu_baseline"] = cpu_baseline(wl["n_h"], cn)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

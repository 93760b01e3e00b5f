"""Per-workgroup timeline of the fp16 split kernel on the GPU.

Loads ada_mla/libmla_mi355x_timeline.so (python ada-mla_amd/build.py
--timeline: the library built with -DMLA_TIMELINE, in which every workgroup
of the split kernel records the phase boundaries of its last piece) and, for
each case, after a 1 s spin-up, times K back-to-back split-kernel launches
(mla_decode_split_fp16_partials: the split kernel alone) between two HIP
events and reads the stamps of the last launch. Times are s_memrealtime
(100 MHz, one clock for the whole GPU) relative to the first workgroup's
entry; the shader clock is s_memtime cycles over s_memrealtime time around
the block loop.

Phases (median / min / max over the workgroups, us):
  entry      wave 0 starts
  landed     wave 0's own prologue loads (Q* rows, block 0) have landed
  barrier_a  every wave's have: the block loop can start
  barrier_b  the S waves hold Q* in registers
  loop_end   the last block step ends (S and O waves)
  s_done     the S waves' m and l are stored (stores complete)
  o_done     the O waves' partial O is stored (stores complete)
  step       (loop_end - barrier_b) / (blocks + 1): one block step

A sweep over the sequence length at a fixed split count (--sweep) gives the
step cost with every CU busy as the slope of the launch time over blocks per
workgroup, and the fixed cost per launch as its intercept.

--combine times whole calls (split kernel, then combine) and reads, besides the
split kernel's stamps, the combine's per-wave stamps of the last call: entry,
slots merged (every load landed), before the store, store complete; gap_us is
the time from the split kernel's last partial store to the first combine
wave's entry.

--fp32 reads the fp32 kernel's stamps instead (calls through
mla_decode_fused_fp32, so call_us includes the combine): entry, first
block, loop end and partials stored, and per step (one 16-token block of
each role: the S waves' block t, the O waves' block t - 1) the shader cycles
of wave 0 (an S wave) in its three phases -- the partial first product (to
barrier X), the softmax (to the wait for the next block's loads) and that
wait with barrier Y.

Usage (single sequences, inputs rotated over >= 1 GB so that C comes from HBM):
  python ada-mla_amd/timeline.py --heads 128 --tokens 65536 --splits 128 --head-tile 64
  python ada-mla_amd/timeline.py --heads 128 --tokens 16384,32768,65536,131072 --splits 128 --head-tile 64 --sweep
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "ada_mla", "libmla_mi355x_timeline.so")
SLOTS = 16
FLAG_FP32_PARTIALS = 4
NAMES = [("entry", 0), ("landed", 1), ("barrier_a", 2), ("barrier_b", 3), ("loop_end", 4), ("s_done", 5),
         ("o_done", 10)]


def run_case(lib, torch, n_h, n, splits, flags, k, spin_s):
    vp = ctypes.c_void_p
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = vp(stream.cuda_stream)
    set_bytes = n * 576 * 2 + n_h * 576 * 2
    pool = min(64, max(2, math.ceil(1024 * 2**20 / set_bytes) + 1))
    qs = [torch.randn(n_h, 576, device=dev, dtype=torch.float16) for _ in range(pool)]
    cs = [torch.randn(n, 576, device=dev, dtype=torch.float16) for _ in range(pool)]
    wsb = lib.mla_decode_split_workspace_size(n_h, n, splits)
    if wsb == 0:
        raise SystemExit(f"invalid sizes: heads {n_h}, tokens {n}, splits {splits}")
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ht = lib.mla_decode_split_head_tile(n_h, n, splits, flags)
    ns = lib.mla_decode_split_num_splits(n_h, n, splits, flags)
    n_wg = ((ns + 7) // 8 * 8) * (n_h // ht)
    cursor = [0]

    def launch():
        i = cursor[0] % pool
        cursor[0] += 1
        st = lib.mla_decode_split_fp16_partials(qs[i].data_ptr(), cs[i].data_ptr(), ws.data_ptr(), wsb, n_h, n,
                                                splits, flags, sp)
        if st != 0:
            raise RuntimeError(f"mla_decode_split_fp16_partials: status {st}")

    t_end = time.perf_counter() + spin_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            launch()
        torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(k):
        launch()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / k
    import numpy as np
    buf = np.zeros(n_wg * SLOTS, dtype=np.uint64)
    if lib.mla_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("mla_timeline_read failed")
    x = buf.reshape(n_wg, SLOTS).astype(np.int64)
    # padding workgroups of the grid stamp their entry only (their other
    # slots keep an earlier launch's stamps)
    x = x[x[:, 10] > x[:, 0]]
    t0 = x[:, 0].min()
    phases = {}
    for name, e in NAMES:
        v = (x[:, e] - t0) * 0.01
        phases[name] = [round(float(np.median(v)), 2), round(float(v.min()), 2), round(float(v.max()), 2)]
    nblk = x[:, 11]
    steps = nblk + 1
    loop_rt = (x[:, 9] - x[:, 8]) * 0.01
    cyc = (x[:, 13] - x[:, 12]).astype(np.float64)
    clk = float(np.median(cyc / (loop_rt * 1e3)))
    step_us = float(np.median(((x[:, 4] - x[:, 3]) * 0.01) / steps))
    rec = dict(heads=n_h, tokens=n, head_tile=int(ht), splits=int(ns), workgroups=int(len(x)),
               blocks=int(np.median(nblk)), partials="fp32" if flags & FLAG_FP32_PARTIALS else "fp16",
               launch_us=round(us, 2), span_us=round(float((x[:, 10].max() - t0) * 0.01), 2),
               step_us=round(step_us, 3), step_cycles=round(float(np.median(cyc / steps))), clock_ghz=round(clk, 3),
               phases_med_min_max_us=phases)
    del qs, cs, ws
    torch.cuda.empty_cache()
    return rec


def run_case_combine(lib, torch, n_h, n, splits, flags, k, spin_s, seqlens=None):
    """Whole calls (split kernel, then the combine): the split kernel's stamps
    and the combine's per-wave stamps of the last call, both relative to the
    split kernel's first workgroup entry. With seqlens, a batch of sequences
    of those lengths (packed, mla_decode_split_batched_fp16; n is then their
    total)."""
    import numpy as np
    vp = ctypes.c_void_p
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = vp(stream.cuda_stream)
    batch = 1 if seqlens is None else len(seqlens)
    set_bytes = n * 576 * 2 + batch * n_h * 576 * 2
    pool = min(64, max(2, math.ceil(1024 * 2**20 / set_bytes) + 1))
    qs = [torch.randn(batch, n_h, 576, device=dev, dtype=torch.float16) for _ in range(pool)]
    cs = [torch.randn(n, 576, device=dev, dtype=torch.float16) for _ in range(pool)]
    out = torch.empty(batch, n_h, 512, device=dev, dtype=torch.float16)
    if seqlens is None:
        wsb = lib.mla_decode_split_workspace_size(n_h, n, splits)
        if lib.mla_decode_split_launches(n_h, n, splits, flags) != 2:
            raise SystemExit("this plan makes one launch (no combine)")
        ht = lib.mla_decode_split_head_tile(n_h, n, splits, flags)
        ns = lib.mla_decode_split_num_splits(n_h, n, splits, flags)
    else:
        cu = torch.tensor(np.concatenate([[0], np.cumsum(seqlens)]).astype(np.int32), device=dev)
        wsb = lib.mla_decode_split_batched_workspace_size(batch, n_h, n, splits)
        ht = ns = 0  # not reported for batches
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    cursor = [0]

    def launch():
        i = cursor[0] % pool
        cursor[0] += 1
        if seqlens is None:
            st = lib.mla_decode_split_fp16_ex(qs[i].data_ptr(), cs[i].data_ptr(), out.data_ptr(), ws.data_ptr(),
                                              wsb, n_h, n, splits, flags, sp)
        else:
            st = lib.mla_decode_split_batched_fp16(qs[i].data_ptr(), cs[i].data_ptr(), cu.data_ptr(),
                                                   out.data_ptr(), ws.data_ptr(), wsb, batch, n_h, n, splits, sp)
        if st != 0:
            raise RuntimeError(f"decode call: status {st}")

    t_end = time.perf_counter() + spin_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            launch()
        torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(k):
        launch()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / k
    if lib.mla_timeline_clear_combine() != 0:
        raise RuntimeError("mla_timeline_clear_combine failed")
    launch()  # the call whose stamps are read, after back-to-back ones
    launch()
    torch.cuda.synchronize()
    buf = np.zeros(8192 * SLOTS, dtype=np.uint64)
    if lib.mla_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("mla_timeline_read failed")
    x = buf.reshape(8192, SLOTS).astype(np.int64)
    bid = np.arange(len(x))  # the stamp row is the workgroup id
    keep = (x[:, 10] > x[:, 0]) & (x[:, 0] > 0)
    x, bid = x[keep], bid[keep]
    keep = x[:, 0] >= x[:, 0].max() - 100000  # the last call's workgroups (within 1 ms of its last entry)
    x, bid = x[keep], bid[keep]
    cb = np.zeros(16384 * 4, dtype=np.uint64)
    if lib.mla_timeline_read_combine(cb.ctypes.data, cb.nbytes) != 0:
        raise RuntimeError("mla_timeline_read_combine failed")
    c = cb.reshape(-1, 4).astype(np.int64)
    c = c[c[:, 0] > 0]
    t0 = x[:, 0].min()
    split_end = max(x[:, 10].max(), x[:, 5].max())

    def mmm(v):
        v = (v - t0) * 0.01
        return [round(float(np.median(v)), 2), round(float(v.min()), 2), round(float(v.max()), 2)]

    if True:
        # the split kernel's workgroups by work (blocks and pieces over the chunk) against their end time
        end = (np.maximum(x[:, 10], x[:, 5]) - t0) * 0.01
        blocks, pieces = x[:, 14], x[:, 15]
        order = np.argsort(end)
        def row(i):
            return [round(float(end[i]), 2), int(blocks[i]), int(pieces[i])]
        print(json.dumps(dict(split_end_blocks_pieces_first5=[row(i) for i in order[:5]],
                              last5=[row(i) for i in order[-5:]],
                              corr_end_blocks=round(float(np.corrcoef(end, blocks)[0, 1]), 3),
                              corr_end_pieces=round(float(np.corrcoef(end, pieces)[0, 1]), 3),
                              blocks_min_max=[int(blocks.min()), int(blocks.max())],
                              pieces_min_max=[int(pieces.min()), int(pieces.max())])), flush=True)
        # time per block from entry to the last store, by XCD (workgroup id mod 8: the dispatcher's
        # round-robin) and by the workgroup's place among its chunk's head tiles (id / 8 mod the
        # tile count, 2 at 64-head tiles of 128 heads)
        per_blk = (end - (x[:, 0] - t0) * 0.01) / np.maximum(blocks, 1)
        def by(key, n):
            return [round(float(np.median(per_blk[key == i])), 3) if np.any(key == i) else None for i in range(n)]
        n_tiles = max(1, n_h // 64)
        print(json.dumps(dict(us_per_block_median=round(float(np.median(per_blk)), 3),
                              us_per_block_min_max=[round(float(per_blk.min()), 3), round(float(per_blk.max()), 3)],
                              us_per_block_by_xcd=by(bid & 7, 8),
                              us_per_block_by_head_tile=by((bid >> 3) % n_tiles, n_tiles),
                              entry_us_min_max=[round(float((x[:, 0].min() - t0) * 0.01), 2),
                                                round(float((x[:, 0].max() - t0) * 0.01), 2)])), flush=True)
    rec = dict(heads=n_h, tokens=n, batch=batch, head_tile=int(ht), splits=int(ns),
               partials="fp32" if flags & FLAG_FP32_PARTIALS else "fp16", call_us=round(us, 2),
               split_workgroups=int(len(x)), combine_waves=int(len(c)),
               split_entry=mmm(x[:, 0]), split_stored=mmm(np.maximum(x[:, 10], x[:, 5])),
               split_end=round(float((split_end - t0) * 0.01), 2),
               combine_entry=mmm(c[:, 0]), combine_merged=mmm(c[:, 1]), combine_before_store=mmm(c[:, 2]),
               combine_stored=mmm(c[:, 3]),
               gap_us=round(float((c[:, 0].min() - split_end) * 0.01), 2),
               combine_span_us=round(float((c[:, 3].max() - c[:, 0].min()) * 0.01), 2))
    del qs, cs, ws
    torch.cuda.empty_cache()
    return rec


def run_case_f32(lib, torch, n_h, n, splits, k, spin_s):
    vp = ctypes.c_void_p
    import numpy as np
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = vp(stream.cuda_stream)
    set_bytes = (n + n_h) * 576 * 4
    pool = min(64, max(2, math.ceil(1024 * 2**20 / set_bytes) + 1))
    qs = [torch.randn(n_h, 576, device=dev) for _ in range(pool)]
    cs = [torch.randn(n, 576, device=dev) for _ in range(pool)]
    out = torch.empty(n_h, 512, device=dev)
    wsb = lib.mla_decode_fused_workspace_size(n_h, n, splits)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    cursor = [0]

    def launch():
        i = cursor[0] % pool
        cursor[0] += 1
        st = lib.mla_decode_fused_fp32(qs[i].data_ptr(), cs[i].data_ptr(), out.data_ptr(), ws.data_ptr(), wsb, n_h,
                                       576, n, splits, sp)
        if st != 0:
            raise RuntimeError(f"mla_decode_fused_fp32: status {st}")

    t_end = time.perf_counter() + spin_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            launch()
        torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(k):
        launch()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / k
    # the combine's per-wave stamps of the second of two more back-to-back calls (its split stamps are the
    # ones read below; the first call takes the GPU out of the idle that the stamp clearing leaves)
    if lib.mla_timeline_clear_combine() != 0:
        raise RuntimeError("mla_timeline_clear_combine failed")
    launch()
    launch()
    torch.cuda.synchronize()
    cb = np.zeros(16384 * 4, dtype=np.uint64)
    if lib.mla_timeline_read_combine(cb.ctypes.data, cb.nbytes) != 0:
        raise RuntimeError("mla_timeline_read_combine failed")
    c = cb.reshape(-1, 4).astype(np.int64)
    c = c[c[:, 0] > 0]
    buf = np.zeros(8192 * SLOTS, dtype=np.uint64)
    if lib.mla_timeline_read_f32(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("mla_timeline_read_f32 failed")
    x = buf.reshape(8192, SLOTS).astype(np.int64)
    x = x[(x[:, 3] > x[:, 0]) & (x[:, 0] > 0)]
    x = x[x[:, 0] >= x[:, 0].max() - 100000]  # this launch's workgroups (within 1 ms of the last entry)
    t0 = x[:, 0].min()
    phases = {}
    for name, e in (("entry", 0), ("first_block", 1), ("loop_end", 2), ("stored", 3)):
        v = (x[:, e] - t0) * 0.01
        phases[name] = [round(float(np.median(v)), 2), round(float(v.min()), 2), round(float(v.max()), 2)]
    nblk = x[:, 11].astype(np.float64)
    steps = nblk + 1  # the S waves run one block ahead of the O waves
    cyc = x[:, 6] + x[:, 7] + x[:, 8]
    clk = float(np.median(cyc / ((x[:, 2] - x[:, 1]) * 0.01 * 1e3)))
    rec = dict(path="fp32", heads=n_h, tokens=n, workgroups=int(len(x)), blocks=int(np.median(nblk)),
               call_us=round(us, 2), span_us=round(float((x[:, 3].max() - t0) * 0.01), 2), clock_ghz=round(clk, 3),
               step_cycles=round(float(np.median(cyc / steps))),
               s_product_cycles=round(float(np.median(x[:, 6] / steps))),
               s_softmax_cycles=round(float(np.median(x[:, 7] / steps))),
               wait_barrier_cycles=round(float(np.median(x[:, 8] / steps))),
               s_work_a_cycles=round(float(np.median(x[:, 4] / steps))),
               s_work_b_cycles=round(float(np.median(x[:, 5] / steps))),
               o_work_a_cycles=round(float(np.median(x[:, 9] / steps))),
               o_work_b_cycles=round(float(np.median(x[:, 10] / steps))),
               phases_med_min_max_us=phases)
    if len(c):
        def mmm(v):
            v = (v - t0) * 0.01
            return [round(float(np.median(v)), 2), round(float(v.min()), 2), round(float(v.max()), 2)]
        rec.update(combine_waves=int(len(c)), combine_entry=mmm(c[:, 0]), combine_merged=mmm(c[:, 1]),
                   combine_stored=mmm(c[:, 3]), gap_us=round(float((c[:, 0].min() - x[:, 3].max()) * 0.01), 2),
                   combine_span_us=round(float((c[:, 3].max() - c[:, 0].min()) * 0.01), 2))
    del qs, cs, ws
    torch.cuda.empty_cache()
    return rec


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--heads", type=int, default=128)
    ap.add_argument("--tokens", default="4096", help="comma-separated sequence lengths")
    ap.add_argument("--splits", type=int, default=0, help="split count (0: the planner's)")
    ap.add_argument("--head-tile", type=int, default=0, choices=(0, 16, 32, 64), help="0: the planner's")
    ap.add_argument("--partials", choices=("fp16", "fp32"), default="fp16")
    ap.add_argument("--sweep", action="store_true", help="fit launch time = fixed + blocks x step")
    ap.add_argument("--calls", type=int, default=20)
    ap.add_argument("--spin-s", type=float, default=1.0)
    ap.add_argument("--fp32", action="store_true", help="the fp32 kernel (mla_decode_fused_fp32)")
    ap.add_argument("--combine", action="store_true",
                    help="whole calls: the split kernel's end and the combine's per-wave stamps")
    ap.add_argument("--batch-config5", action="store_true",
                    help="with --combine: the batched workload (B = 32, BASELINE config-5 lengths)")
    args = ap.parse_args()
    if not os.path.exists(LIB):
        raise SystemExit(f"{LIB} is not built (python ada-mla_amd/build.py --timeline)")
    if args.head_tile:
        os.environ["MLA_TIMELINE_HEAD_TILE"] = str(args.head_tile)
    import torch
    vp, sz, i_, u_ = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint
    lib = ctypes.CDLL(LIB)
    lib.mla_decode_split_workspace_size.restype = sz
    lib.mla_decode_split_workspace_size.argtypes = [i_, i_, i_]
    lib.mla_decode_split_fp16_partials.argtypes = [vp, vp, vp, sz, i_, i_, i_, u_, vp]
    lib.mla_decode_split_head_tile.argtypes = [i_, i_, i_, u_]
    lib.mla_decode_split_num_splits.argtypes = [i_, i_, i_, u_]
    lib.mla_timeline_read.argtypes = [vp, sz]
    lib.mla_timeline_read_f32.argtypes = [vp, sz]
    lib.mla_decode_fused_workspace_size.restype = sz
    lib.mla_decode_fused_workspace_size.argtypes = [i_, i_, i_]
    lib.mla_decode_fused_fp32.argtypes = [vp, vp, vp, vp, sz, i_, i_, i_, i_, vp]
    lib.mla_decode_split_fp16_ex.argtypes = [vp, vp, vp, vp, sz, i_, i_, i_, u_, vp]
    lib.mla_decode_split_launches.argtypes = [i_, i_, i_, u_]
    lib.mla_timeline_read_combine.argtypes = [vp, sz]
    if args.fp32:
        for n in (int(t) for t in args.tokens.split(",")):
            print(json.dumps(run_case_f32(lib, torch, args.heads, n, args.splits, args.calls, args.spin_s)), flush=True)
        return 0
    flags = FLAG_FP32_PARTIALS if args.partials == "fp32" else 0
    lib.mla_decode_split_batched_workspace_size.restype = sz
    lib.mla_decode_split_batched_workspace_size.argtypes = [i_, i_, i_, i_]
    lib.mla_decode_split_batched_fp16.argtypes = [vp, vp, vp, vp, vp, sz, i_, i_, i_, i_, vp]
    if args.combine and args.batch_config5:
        sys.path.insert(0, HERE)
        from ada_mla import synthetic
        lens = synthetic.batched_seqlens(32, seed=42)
        print(json.dumps(run_case_combine(lib, torch, args.heads, int(lens.sum()), args.splits, 0, args.calls,
                                          args.spin_s, seqlens=lens)), flush=True)
        return 0
    if args.combine:
        for n in (int(t) for t in args.tokens.split(",")):
            print(json.dumps(run_case_combine(lib, torch, args.heads, n, args.splits, flags, args.calls,
                                              args.spin_s)), flush=True)
        return 0
    recs = []
    for n in (int(t) for t in args.tokens.split(",")):
        rec = run_case(lib, torch, args.heads, n, args.splits, flags, args.calls, args.spin_s)
        print(json.dumps(rec), flush=True)
        recs.append(rec)
    if args.sweep and len(recs) >= 2:
        import numpy as np
        xb = np.array([r["blocks"] for r in recs], dtype=np.float64)
        yt = np.array([r["launch_us"] for r in recs])
        slope, icpt = np.polyfit(xb, yt, 1)
        print(json.dumps(dict(fit="launch_us = fixed_us + blocks x step_us", step_us=round(float(slope), 3),
                              fixed_us=round(float(icpt), 2), head_tile=recs[0]["head_tile"],
                              splits=recs[0]["splits"], partials=recs[0]["partials"])), flush=True)


if __name__ == "__main__":
    sys.exit(main())

"""Command-line harness for the MLA decode: test, benchmark and profile runs.

Mirrors the reference's driver ``mla.py`` (mla.py:153-194): the same flags
(``--test``, ``--bench``, ``--for-ncu``, ``-s/--seq-length``, ``-k/--kernel``,
``--fp32``), the same kernel names and the same printed error line, with the
"fused" kernel bound to this library's extension (``mla_decode_split`` for
fp16, ``mla_decode_fused`` for ``--fp32``, as mla.py:182-187 binds them).

    python ada-mla_amd/mla.py --test -s 4096 -k fused
    python ada-mla_amd/mla.py --bench -k torch fused --fp32

Differences from the reference, on purpose:
  * the "torch" kernel is the closed form softmax(q c^T / sqrt(192)) c[:, :512]
    (mla.py:44-47) in eager mode, not under torch.compile;
  * ``--test`` compares every kernel against that closed form evaluated in
    fp32 on the same (already rounded) inputs, where the reference compared
    against the closed form in the input dtype (mla.py:111-120);
  * the two SDPA kernels (mla.py:49-66) are evaluated on fp32 copies of the
    inputs on a GPU: the math backend's batched products over a transposed
    operand are kept out of half precision on this platform;
  * ``--bench`` times with HIP events around each call after overwriting a
    512 MiB buffer (larger than MI355X's 256 MiB last-level cache), in place
    of triton.testing.do_bench's 256 MB L2 clear (mla.py:122-130), and takes
    the mean like do_bench does; ``--json`` also prints one JSON line per
    (sequence length, kernel) with the achieved HBM rate;
  * ``--heads`` sets the head count (the reference fixes 128, mla.py:30).
"""
from __future__ import annotations

import argparse
import json
import math
import sys

HEAD_DIM_C = 512
HEAD_DIM_ROPE = 64
HEAD_DIM_K = HEAD_DIM_C + HEAD_DIM_ROPE
NUM_HEADS = 128
SCALE = 1.0 / math.sqrt(128 + HEAD_DIM_ROPE)  # mla.py:46: (HEAD_DIM + HEAD_DIM_ROPE) ** -0.5

KERNEL_NAMES = ["torch", "sdpa-math", "sdpa-efficient", "fused"]
DEFAULT_SEQ_LENGTHS = [2048, 4096, 8192, 16384, 32768]
FLUSH_BYTES = 512 << 20


def _torch():
    import torch
    return torch


def device() -> str:
    torch = _torch()
    return "cuda" if torch.cuda.is_available() else "cpu"


def mla_decode_torch(q, c):
    """softmax(q c^T * SCALE) c[:, :512] in the inputs' dtype (mla.py:44-47)."""
    torch = _torch()
    return torch.softmax(torch.matmul(q, c.t()) * SCALE, dim=-1) @ c[:, :HEAD_DIM_C]


def _sdpa(q, c, backend):
    torch = _torch()
    from torch.nn.attention import sdpa_kernel
    from torch.nn.functional import scaled_dot_product_attention
    dt = q.dtype
    if q.is_cuda and dt != torch.float32:
        q, c = q.float(), c.float()
    with sdpa_kernel(backend):
        out = scaled_dot_product_attention(q[None, None], c[None, None],
                                           c[None, None, :, :HEAD_DIM_C], scale=SCALE)
    return out[0, 0].to(dt)


def mla_decode_sdpa_math(q, c):
    from torch.nn.attention import SDPBackend
    return _sdpa(q, c, SDPBackend.MATH)


def mla_decode_sdpa_efficient(q, c):
    from torch.nn.attention import SDPBackend
    return _sdpa(q, c, SDPBackend.EFFICIENT_ATTENTION)


def decode_funcs(fp32: bool) -> dict:
    """Kernel name -> callable(q, c), with "fused" bound as mla.py:182-187 does.
    The extension is looked up only when "fused" is called, so the other
    kernels run without it; "fused" without it raises ImportError."""
    def fused(q, c):
        import ada_mla
        return (ada_mla.mla_decode_fused if fp32 else ada_mla.mla_decode_split)(q, c)
    return {"torch": mla_decode_torch, "sdpa-math": mla_decode_sdpa_math,
            "sdpa-efficient": mla_decode_sdpa_efficient, "fused": fused}


def run_funcs(funcs: dict, names, num_heads, seq_lengths, dtype, num_iters=1):
    """Each kernel num_iters times per sequence length and nothing else, for
    profilers (mla.py:74-89, `--for-ncu`)."""
    torch = _torch()
    dev = device()
    q = torch.randn(num_heads, HEAD_DIM_K, dtype=dtype).to(dev)
    for n in seq_lengths:
        c = torch.randn(n, HEAD_DIM_K, dtype=dtype).to(dev)
        for name in names:
            for _ in range(num_iters):
                funcs[name](q, c)
    if dev == "cuda":
        torch.cuda.synchronize()


def run_test(funcs: dict, names, num_heads, seq_lengths, dtype, out=None):
    """Error of each kernel against the fp32 closed form on the same inputs,
    one line per (kernel, sequence length) as mla.py:117-120 prints them.
    Returns {(name, seq_len): (max, mean, rel)}; a kernel that raises is
    reported as unavailable."""
    torch = _torch()
    out = out or sys.stdout
    dev = device()
    q = torch.randn(num_heads, HEAD_DIM_K, dtype=dtype).to(dev)
    res = {}
    for n in seq_lengths:
        c = torch.randn(n, HEAD_DIM_K, dtype=dtype).to(dev)
        ref = mla_decode_torch(q.float(), c.float())
        for name in names:
            try:
                o = funcs[name](q, c)
            except (RuntimeError, ImportError, NotImplementedError) as e:
                print(f"[{name}] seq_len={n} unavailable: {str(e).splitlines()[0]}", file=out)
                continue
            diff = (o.float() - ref).abs()
            mx, mean = diff.max().item(), diff.mean().item()
            rel = mean / ref.abs().mean().item()
            print(f"[{name}] seq_len={n} max={mx:.6g} mean={mean:.6g} rel={rel:.6f}", file=out)
            res[(name, n)] = (mx, mean, rel)
    return res


def do_bench(fn, warmup_ms=25.0, rep_ms=100.0, flush=None):
    """Mean milliseconds per call of fn on the GPU: an estimate from 5 calls
    sets the warm-up and repeat counts for the time budgets; before every call
    the flush buffer is overwritten so inputs come from HBM."""
    torch = _torch()
    if flush is None:
        flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(5):
        flush.zero_()
        fn()
    end.record()
    torch.cuda.synchronize()
    est = max(start.elapsed_time(end) / 5, 1e-3)
    n_warm, n_rep = max(1, int(warmup_ms / est)), max(1, int(rep_ms / est))
    for _ in range(n_warm):
        fn()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_rep)]
    for s, e in evs:
        flush.zero_()
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in evs) / n_rep


def algorithmic_bytes(num_heads, seq_len, elem):
    """Bytes one call must move: Q*, C and O* once (elem bytes per value)."""
    return elem * (num_heads * HEAD_DIM_K + seq_len * HEAD_DIM_K + num_heads * HEAD_DIM_C)


def run_benchmark(funcs: dict, names, num_heads, seq_lengths, dtype, warmup_ms=25.0,
                  rep_ms=100.0, as_json=False, out=None):
    """Mean ms per call for every (sequence length, kernel), printed as a
    table like the reference's perf_report (mla.py:132-151). Inputs are drawn
    on the device, as mla.py:125-126 does. Returns {(seq_len, name): ms}."""
    torch = _torch()
    if not torch.cuda.is_available():
        raise SystemExit("mla --bench needs a GPU")
    out = out or sys.stdout
    flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    elem = torch.tensor([], dtype=dtype).element_size()
    res = {}
    for n in seq_lengths:
        q = torch.randn(num_heads, HEAD_DIM_K, dtype=dtype, device="cuda")
        c = torch.randn(n, HEAD_DIM_K, dtype=dtype, device="cuda")
        for name in names:
            try:
                ms = do_bench(lambda: funcs[name](q, c), warmup_ms, rep_ms, flush)
            except (RuntimeError, ImportError, NotImplementedError):
                ms = float("nan")
            res[(n, name)] = ms
            if as_json:
                tbps = algorithmic_bytes(num_heads, n, elem) / (ms * 1e-3) / 1e12 if ms == ms else None
                print(json.dumps({"seq_len": n, "kernel": name, "num_heads": num_heads,
                                  "dtype": str(dtype).replace("torch.", ""), "ms": ms,
                                  "us": ms * 1e3, "hbm_tbps": tbps}), file=out)
    print("mla-bench:", file=out)
    print(f"{'':>3s} {'seq_len':>10s}" + "".join(f" {nm:>15s}" for nm in names), file=out)
    for i, n in enumerate(seq_lengths):
        print(f"{i:>3d} {float(n):>10.1f}" + "".join(f" {res[(n, nm)]:>15.6f}" for nm in names),
              file=out)
    return res


def build_parser():
    p = argparse.ArgumentParser(prog="mla")
    p.add_argument("--for-ncu", "--for-profiler", dest="for_ncu", action="store_true",
                   help="run each kernel once per sequence length (for a profiler)")
    p.add_argument("--test", action="store_true", help="print each kernel's error")
    p.add_argument("--bench", action="store_true", help="time each kernel")
    p.add_argument("-s", "--seq-length", type=int, nargs="+", default=DEFAULT_SEQ_LENGTHS)
    p.add_argument("--fp32", action="store_true", help="fp32 inputs (fused = mla_decode_fused)")
    p.add_argument("-k", "--kernel", nargs="+", default=KERNEL_NAMES, choices=KERNEL_NAMES)
    p.add_argument("--heads", type=int, default=NUM_HEADS)
    p.add_argument("--json", action="store_true", help="--bench: also one JSON line per measurement")
    p.add_argument("--warmup-ms", type=float, default=25.0)
    p.add_argument("--rep-ms", type=float, default=100.0)
    return p


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)
    torch = _torch()
    torch.manual_seed(42)  # mla.py:42
    dtype = torch.float32 if args.fp32 else torch.float16
    funcs = decode_funcs(args.fp32)
    if args.for_ncu:
        run_funcs(funcs, args.kernel, args.heads, args.seq_length, dtype)
    if args.test:
        run_test(funcs, args.kernel, args.heads, args.seq_length, dtype)
    if args.bench:
        run_benchmark(funcs, args.kernel, args.heads, args.seq_length, dtype,
                      args.warmup_ms, args.rep_ms, args.json)
    return 0


if __name__ == "__main__":
    sys.exit(main())

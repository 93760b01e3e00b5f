"""Writes tests/golden/mla_ref_cpu.npz: golden vectors produced by the
reference's own CPU kernel run_mla_decode_cpu
(/root/reference/csrc/mla_decode_naive_fp32_cpu.cpp:5-61), compiled from its
unmodified source into oracle/_ref by oracle/Makefile.

The reference has no tests, fixtures or golden vectors of its own, so these
are the only vectors that come from reference code. For each case the file
holds:

  <case>/q           fp16 [n_h, 576]  seeded N(0, 1) (ada_mla.synthetic)
  <case>/c           fp16 [N, 576]
  <case>/ref_out     fp32 [n_h, 576]  run_mla_decode_cpu(q, c): scale
                                      1/sqrt(576), all 576 columns
  <case>/contract    fp32 [n_h, 512]  run_mla_decode_cpu(sqrt(3) * q, c)[:, :512]
                                      = softmax(q c^T / sqrt(192)) c[:, :512]
                                      (sqrt(3)/sqrt(576) = 1/sqrt(192)), with one
                                      extra fp32 rounding of q

Run from the repo root, in the container that holds /root/reference:
    make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "ada-mla_amd"))

from oracle import mla_oracle  # noqa: E402
from ada_mla import synthetic  # noqa: E402

CASES = {
    # name: (num_heads, seq_length, seed)
    "h16_n64": (16, 64, 7),
    "h32_n33": (32, 33, 11),
    "h16_n1": (16, 1, 13),
    "h16_n100": (16, 100, 17),
}


def main() -> None:
    if not mla_oracle.reference_cpu_available():
        raise SystemExit("oracle/_ref/libref_mla_cpu.so missing: run make -C oracle ref")
    out = {}
    sqrt3 = np.float32(math.sqrt(3.0))
    for name, (n_h, n, seed) in CASES.items():
        q, c = synthetic.decode_inputs(n_h, n, seed=seed, dtype=np.float16)
        q32 = q.astype(np.float32)
        c32 = c.astype(np.float32)
        out[f"{name}/q"] = q
        out[f"{name}/c"] = c
        out[f"{name}/ref_out"] = mla_oracle.reference_cpu(q32, c32)
        out[f"{name}/contract"] = np.ascontiguousarray(
            mla_oracle.reference_cpu(q32 * sqrt3, c32)[:, :512])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mla_ref_cpu.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()

"""CPU checks of tests/cabi/abi_client, the C++ caller of the C ABI (no
Python, no torch in that process): it links and loads the in-tree library,
reports the ABI version and status strings without a GPU call, and its
binary16 conversion helpers (which build its test inputs) agree bit for bit
with numpy's float32 -> float16 rounding."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLIENT = os.path.join(ROOT, "tests", "cabi", "abi_client")


@pytest.fixture(scope="module")
def client():
    if not os.path.exists(CLIENT):
        pytest.fail(f"{CLIENT} is not built (run __graft_entry__.build() or make -C tests/cabi)")
    return CLIENT


def test_abi_mode_without_gpu(client):
    r = subprocess.run([client, "--abi"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "abi_version 2" in r.stdout
    assert "status 3: workspace too small" in r.stdout


def test_half_conversion_matches_numpy(client):
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2**32, size=60000, dtype=np.uint64).astype(np.uint32)
    # values near binary16's range and its rounding midpoints: every half
    # pattern, and the exact midpoints between neighbours (ties to even)
    halves = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = halves.view(np.float16).astype(np.float32)
    hi = (halves + 1).view(np.float16).astype(np.float32)
    mids = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    f = np.concatenate([bits.view(np.float32), lo, mids, -mids,
                        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 6e-8, 3e-8], np.float32)])
    f = f[~np.isnan(f)]
    stdin = "\n".join(f"{b:08x}" for b in f.view(np.uint32)) + "\n"
    r = subprocess.run([client, "--to-half"], input=stdin, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.array([[int(t, 16) for t in ln.split()] for ln in r.stdout.splitlines()], dtype=np.uint64)
    assert got.shape == (f.size, 2)
    with np.errstate(over="ignore"):
        want_h = f.astype(np.float16)
    np.testing.assert_array_equal(got[:, 0].astype(np.uint16), want_h.view(np.uint16))
    np.testing.assert_array_equal(got[:, 1].astype(np.uint32), want_h.astype(np.float32).view(np.uint32))

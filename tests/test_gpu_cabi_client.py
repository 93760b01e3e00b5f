"""The C ABI driven from C++ with no Python in the calling process:
tests/cabi/abi_client allocates with hipMalloc, calls the single-sequence,
two-phase (fp32 partials), batched (with an empty sequence) and fp32 entry
points, and checks each against the CPU oracle (the restatement of the
reference's run_mla_decode_cpu, oracle/mla_naive_cpu.c, at the decode
contract's scale and 512 value columns) at atol = rtol = 1e-2 (fp16) and
1e-4 (fp32); it also checks the documented error codes."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLIENT = os.path.join(ROOT, "tests", "cabi", "abi_client")


@pytest.mark.gpu
def test_cpp_client_parity_and_errors():
    assert os.path.exists(CLIENT), "tests/cabi/abi_client is not built"
    print("running tests/cabi/abi_client", flush=True)
    r = subprocess.run([CLIENT], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, f"exit {r.returncode}\n{r.stdout}\n{r.stderr}"
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith(("PASS", "FAIL"))]
    assert len(lines) >= 12 and all(ln.startswith("PASS") for ln in lines), r.stdout

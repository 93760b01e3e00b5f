"""The mla.py-equivalent harness (ada_mla/cli.py): flags and defaults as the
reference's driver (mla.py:153-194), its printed error line (mla.py:117-120),
and the "fused" binding (mla.py:182-187). CPU tests run the torch kernels and
check that "fused" refuses CPU tensors instead of falling back; GPU tests run
the fused kernel through the harness."""
import io
import math
import re

import numpy as np
import pytest
import torch

from ada_mla import cli
from oracle import mla_oracle as O

LINE = re.compile(r"^\[(?P<name>[\w-]+)\] seq_len=(?P<n>\d+) max=(?P<max>\S+) mean=(?P<mean>\S+) rel=(?P<rel>\S+)$")


def test_flags_and_defaults_match_the_reference_driver():
    a = cli.build_parser().parse_args([])
    assert a.seq_length == [2048, 4096, 8192, 16384, 32768]      # mla.py:160-161
    assert a.kernel == ["torch", "sdpa-math", "sdpa-efficient", "fused"]  # mla.py:166
    assert not (a.test or a.bench or a.for_ncu or a.fp32)
    a = cli.build_parser().parse_args(["--test", "--fp32", "-s", "4096", "-k", "fused", "torch"])
    assert a.test and a.fp32 and a.seq_length == [4096] and a.kernel == ["fused", "torch"]
    assert cli.build_parser().parse_args(["--for-ncu"]).for_ncu
    with pytest.raises(SystemExit):
        cli.build_parser().parse_args(["-k", "naive"])


def test_scale_is_one_over_sqrt_192():
    # mla.py:46: (HEAD_DIM + HEAD_DIM_ROPE) ** 0.5 with HEAD_DIM = 128, HEAD_DIM_ROPE = 64
    assert cli.SCALE == pytest.approx(1 / math.sqrt(192), rel=0, abs=1e-15)


def test_torch_kernel_equals_the_oracle_closed_form():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((16, 576)).astype(np.float32)
    c = rng.standard_normal((77, 576)).astype(np.float32)
    got = cli.mla_decode_torch(torch.from_numpy(q).double(), torch.from_numpy(c).double()).numpy()
    np.testing.assert_allclose(got, O.closed_form(q, c), rtol=1e-12, atol=1e-12)
    got = cli.mla_decode_sdpa_math(torch.from_numpy(q).double(), torch.from_numpy(c).double()).numpy()
    np.testing.assert_allclose(got, O.closed_form(q, c), rtol=1e-10, atol=1e-10)


def test_run_test_prints_the_reference_error_line_and_fused_refuses_cpu():
    buf = io.StringIO()
    torch.manual_seed(42)
    funcs = cli.decode_funcs(fp32=True)
    res = cli.run_test(funcs, ["torch", "sdpa-math", "fused"], 16, [64, 100], torch.float32, out=buf)
    lines = buf.getvalue().splitlines()
    parsed = [LINE.match(ln) for ln in lines]
    ok = [m for m in parsed if m]
    assert {(m["name"], int(m["n"])) for m in ok} == {("torch", 64), ("sdpa-math", 64),
                                                       ("torch", 100), ("sdpa-math", 100)}
    for m in ok:
        assert float(m["max"]) < 1e-5 and float(m["rel"]) < 1e-5
    # the fused kernel has no CPU path: it reports the extension's refusal
    refused = [ln for ln in lines if ln.startswith("[fused]")]
    assert len(refused) == 2 and all("unavailable" in ln for ln in refused)
    assert set(res) == {("torch", 64), ("sdpa-math", 64), ("torch", 100), ("sdpa-math", 100)}


def test_main_runs_on_cpu_with_torch_kernels(capsys):
    assert cli.main(["--test", "-k", "torch", "-s", "32", "--heads", "16"]) == 0
    out = capsys.readouterr().out.strip().splitlines()
    assert len(out) == 1 and LINE.match(out[0])


def test_algorithmic_bytes():
    # 2 * (128*576 + 4096*576 + 128*512) = 4,997,120 B for the headline config
    assert cli.algorithmic_bytes(128, 4096, 2) == 4_997_120


@pytest.mark.gpu
@pytest.mark.parametrize("fp32,tol", [(False, 1e-2), (True, 1e-4)])
def test_fused_through_the_harness(fp32, tol):
    buf = io.StringIO()
    torch.manual_seed(42)
    dtype = torch.float32 if fp32 else torch.float16
    res = cli.run_test(cli.decode_funcs(fp32), ["fused"], 128, [1024, 4096], dtype, out=buf)
    print(buf.getvalue(), flush=True)
    assert set(res) == {("fused", 1024), ("fused", 4096)}
    for (name, n), (mx, mean, rel) in res.items():
        assert mx < tol, (n, mx)
        assert rel < (5e-3 if not fp32 else 1e-4), (n, rel)


@pytest.mark.gpu
def test_bench_mode_times_the_fused_kernel():
    buf = io.StringIO()
    res = cli.run_benchmark(cli.decode_funcs(False), ["fused"], 128, [4096], torch.float16,
                            warmup_ms=2.0, rep_ms=5.0, as_json=True, out=buf)
    ms = res[(4096, "fused")]
    assert 0 < ms < 1.0, ms
    text = buf.getvalue()
    assert "mla-bench:" in text and '"kernel": "fused"' in text

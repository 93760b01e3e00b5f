"""Pins the CPU oracle (oracle/) before anything is checked against it.

- The C restatement of run_mla_decode_cpu (cpu.cpp:5-61) is bit-identical to
  the reference kernel's own outputs (golden vectors written by the reference
  binary built from its source, and live against oracle/_ref when present).
- The float64 closed form (mla.py:44-47) agrees with the reference kernel via
  the identity 1/sqrt(192) = sqrt(3)/sqrt(576).
- Special cases fixed by the mathematics, brute force on tiny inputs, and the
  LSE merge (splitk.cuh:894-939) against the unsplit softmax.
- Planted mistakes in copies of the oracle are caught by these checks.
"""
import math

import numpy as np
import pytest

from oracle import mla_oracle as O
from ada_mla import synthetic


# ---------------------------------------------------------------- golden

def test_golden_restatement_bitexact(golden):
    for name, case in golden.items():
        q = case["q"].astype(np.float32)
        c = case["c"].astype(np.float32)
        got = O.naive_cpu(q, c, divisor=O.REF_CPU_DIVISOR, dv=576)
        assert np.array_equal(got, case["ref_out"]), name


def test_golden_closed_form_matches_reference_kernel(golden):
    for name, case in golden.items():
        q = case["q"].astype(np.float32)
        c = case["c"].astype(np.float32)
        ref = case["contract"]
        np.testing.assert_allclose(O.closed_form(q, c), ref, rtol=0, atol=2e-5,
                                   err_msg=name)
        np.testing.assert_allclose(O.naive_cpu(q, c), ref, rtol=0, atol=2e-5,
                                   err_msg=name)


@pytest.mark.skipif(not O.reference_cpu_available(),
                    reason="oracle/_ref not built (reference source absent)")
@pytest.mark.parametrize("n_h,n,seed", [(16, 48, 1), (32, 7, 2), (128, 20, 3), (48, 65, 4)])
def test_restatement_bitexact_vs_reference_binary(n_h, n, seed):
    q, c = synthetic.decode_inputs(n_h, n, seed=seed, dtype=np.float32)
    assert np.array_equal(O.naive_cpu(q, c, O.REF_CPU_DIVISOR, 576),
                          O.reference_cpu(q, c))


# ------------------------------------------------------- closed-form facts

def _qc(n_h, n, seed):
    q, c = synthetic.decode_inputs(n_h, n, seed=seed, dtype=np.float16)
    return q.astype(np.float64), c.astype(np.float64)


def test_single_token_returns_that_row():
    q, c = _qc(16, 1, 5)
    np.testing.assert_array_equal(O.closed_form(q, c), np.repeat(c[:, :512], 16, 0))


def test_equal_rows_return_the_row():
    q, c = _qc(16, 1, 6)
    cc = np.repeat(c, 37, axis=0)
    np.testing.assert_allclose(O.closed_form(q, cc), np.repeat(c[:, :512], 16, 0),
                               rtol=0, atol=1e-12)


def test_zero_query_gives_column_mean():
    _, c = _qc(16, 50, 7)
    q = np.zeros((16, 576))
    np.testing.assert_allclose(O.closed_form(q, c),
                               np.repeat(c[:, :512].mean(0, keepdims=True), 16, 0),
                               rtol=0, atol=1e-12)


def test_dominant_logit_selects_token():
    _, c = _qc(4, 30, 8)
    j = 17
    q = 40.0 * c[j:j + 1].repeat(4, 0)
    np.testing.assert_allclose(O.closed_form(q, c), np.repeat(c[j:j + 1, :512], 4, 0),
                               rtol=0, atol=1e-9)


def test_token_permutation_invariance():
    q, c = _qc(16, 40, 9)
    perm = np.random.default_rng(0).permutation(40)
    np.testing.assert_allclose(O.closed_form(q, c), O.closed_form(q, c[perm]),
                               rtol=0, atol=1e-12)


def test_shift_invariance_rope_columns():
    # Adding lambda*e to q where c.e is constant over tokens leaves softmax unchanged:
    # make the last rope column of c constant and shift q along it.
    q, c = _qc(8, 25, 10)
    c[:, -1] = 0.5
    q2 = q.copy()
    q2[:, -1] += 3.0
    np.testing.assert_allclose(O.closed_form(q, c), O.closed_form(q2, c), rtol=0, atol=1e-12)


def test_brute_force_tiny():
    q, c = _qc(2, 5, 11)
    out = np.zeros((2, 512))
    for i in range(2):
        logits = [sum(q[i, k] * c[j, k] for k in range(576)) / math.sqrt(192) for j in range(5)]
        mx = max(logits)
        w = [math.exp(x - mx) for x in logits]
        s = sum(w)
        for d in range(512):
            out[i, d] = sum(w[j] * c[j, d] for j in range(5)) / s
    np.testing.assert_allclose(O.closed_form(q, c), out, rtol=0, atol=1e-12)


def test_sdpa_math_form_matches():
    q, c = _qc(16, 70, 12)
    np.testing.assert_allclose(O.sdpa_math(q, c), O.closed_form(q, c), rtol=0, atol=1e-12)


# ---------------------------------------------------------------- LSE merge

def test_merge_every_split_point():
    q, c = _qc(16, 24, 13)
    full = O.closed_form(q, c)
    for cut in range(0, 25):
        parts = O.split_partials(q, c, [0, cut, 24])
        np.testing.assert_allclose(O.lse_merge(*parts), full, rtol=0, atol=1e-12)


def test_merge_random_splits_with_empty_and_assoc():
    q, c = _qc(16, 200, 14)
    full = O.closed_form(q, c)
    rng = np.random.default_rng(1)
    for _ in range(5):
        cuts = sorted(rng.integers(0, 201, size=6).tolist())
        bounds = [0] + cuts + [200]
        o, m, l = O.split_partials(q, c, bounds)
        np.testing.assert_allclose(O.lse_merge(o, m, l), full, rtol=0, atol=1e-12)
        # associativity: merge first half of splits into one partial, then merge
        k = len(bounds) // 2
        o1, m1, l1 = O.split_partials(q, c, [0, bounds[k], 200])
        np.testing.assert_allclose(O.lse_merge(o1, m1, l1), full, rtol=0, atol=1e-12)


def test_batched_closed_form_per_sequence_and_empty():
    seqlens = np.array([5, 0, 17, 1])
    q, c, cu = synthetic.batched_inputs(16, seqlens, seed=3)
    out = O.closed_form_batched(q, c, cu)
    for b in range(4):
        lo, hi = cu[b], cu[b + 1]
        if hi > lo:
            np.testing.assert_allclose(out[b], O.closed_form(q[b], c[lo:hi]), rtol=0, atol=0)
        else:
            assert not out[b].any()


# ------------------------------------------------------------ generator

def test_synthetic_deterministic_and_fp16_exact():
    a = synthetic.decode_inputs(16, 9, seed=5)
    b = synthetic.decode_inputs(16, 9, seed=5)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    q32, _ = synthetic.decode_inputs(16, 9, seed=5, dtype=np.float32)
    assert not np.array_equal(q32, a[0].astype(np.float32))  # fp16 path is rounded
    assert np.array_equal(a[0].astype(np.float32).astype(np.float16), a[0])
    assert abs(float(synthetic.normal((200000,), 1, np.float32).std()) - 1.0) < 0.01


def test_batched_seqlens_range():
    s = synthetic.batched_seqlens(32, seed=42)
    assert s.shape == (32,) and s.min() >= 512 and s.max() <= 16384


# ------------------------------------------------------- planted mistakes

def _fails_golden(fn, golden, atol=2e-5):
    for case in golden.values():
        q = case["q"].astype(np.float64)
        c = case["c"].astype(np.float64)
        if c.shape[0] == 1:
            continue  # a single token hides every softmax mistake
        if np.abs(fn(q, c) - case["contract"]).max() > atol:
            return True
    return False


def test_planted_wrong_scale_is_caught(golden):
    assert _fails_golden(lambda q, c: O.closed_form(q, c, scale=1 / math.sqrt(576)), golden)


def test_planted_wrong_value_slice_is_caught(golden):
    assert _fails_golden(lambda q, c: O._softmax_rows(q @ c.T * O.SCALE) @ c[:, 64:], golden)


def test_planted_softmax_over_heads_is_caught(golden):
    def bad(q, c):
        x = (q @ c.T) * O.SCALE
        e = np.exp(x - x.max(0, keepdims=True))
        return (e / e.sum(0, keepdims=True)) @ c[:, :512]
    assert _fails_golden(bad, golden)


def test_planted_merge_without_rescale_is_caught():
    q, c = _qc(16, 64, 15)
    o, m, l = O.split_partials(q, c, [0, 20, 64])
    bad = o.sum(0) / l.sum(0)[:, None]
    assert np.abs(bad - O.closed_form(q, c)).max() > 1e-3


def test_planted_restatement_divisor_is_caught(golden):
    case = golden["h16_n64"]
    q = case["q"].astype(np.float32)
    c = case["c"].astype(np.float32)
    got = O.naive_cpu(q, c, divisor=math.sqrt(192), dv=576)
    assert not np.array_equal(got, case["ref_out"])


def test_gather_paged_inverts_the_paged_layout():
    # synthetic.paged_inputs scatters a packed cache into shuffled pages; the
    # oracle's gather must return exactly the packed rows, and the paged
    # closed form must equal the packed one
    from ada_mla import synthetic
    for page in (32, 64):
        q, kv, bt, cu, c = synthetic.paged_inputs(16, [5, 0, 64, 65, 200, 1], page, seed=page)
        assert np.array_equal(O.gather_paged(kv, bt, cu), c)
        np.testing.assert_array_equal(O.closed_form_paged(q, kv, bt, cu), O.closed_form_batched(q, c, cu))
    # a wrong page order is caught
    q, kv, bt, cu, c = synthetic.paged_inputs(16, [100, 70], 32, seed=1)
    bt2 = bt.copy()
    bt2[0, [0, 1]] = bt2[0, [1, 0]]
    assert not np.array_equal(O.gather_paged(kv, bt2, cu), c)


def test_absorbed_block_equals_unabsorbed_attention():
    # the absorption identity of README.md:68-80, in float64: the absorbed
    # query against the latent cache, then the value and output projections,
    # equals per-head attention with explicit keys and values
    rng = np.random.default_rng(11)
    B, n_h, d_model = 3, 4, 40
    seqlens = np.array([7, 0, 30])
    cu = np.concatenate([[0], np.cumsum(seqlens)])
    c = rng.standard_normal((cu[-1], 576))
    q_nope = rng.standard_normal((B, n_h, 128)) * 0.1
    q_rope = rng.standard_normal((B, n_h, 64))
    w_uk = rng.standard_normal((n_h, 128, 512)) * 0.05
    w_uv = rng.standard_normal((n_h, 128, 512)) * 0.05
    w_o = rng.standard_normal((d_model, n_h * 128)) * 0.05
    qs = O.absorb_query(q_nope, q_rope, w_uk)
    assert qs.shape == (B, n_h, 576)
    got = O.project_output(O.closed_form_batched(qs, c, cu), w_uv, w_o)
    want = O.block_unabsorbed(q_nope, q_rope, c, cu, w_uk, w_uv, w_o)
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)
    # a transposed key projection is caught
    bad = O.absorb_query(q_nope, q_rope, np.ascontiguousarray(w_uk[:, :, ::-1]))
    assert not np.allclose(O.project_output(O.closed_form_batched(bad, c, cu), w_uv, w_o), want)

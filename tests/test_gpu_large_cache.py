"""GPU parity at cache offsets past 2^31 elements (3,728,271 tokens of 576
values): a batch of two sequences whose second starts there, and a first
sequence of 3.8 M tokens whose attention is carried by rows past that offset.
Batches of long sequences reach such offsets (32 sequences of 128 K tokens
hold 4.2 M tokens), so every cache address must be formed in 64 bits.

Both the 16-bit cache and the fp8 cache (one byte per value, so the same
token offset) are covered. The long sequence is all zero rows except its
first and last 4096 tokens. A zero row has logit 0 and value 0, so the
float64 closed form over the whole sequence reduces to the nonzero rows plus
Z = (number of zero rows) terms e^(0 - m) in the softmax sum (the same
formula as oracle.closed_form, mla.py:44-47, evaluated without materialising
the zero rows). The last rows are scaled so that their logits dominate, so
the output is carried by rows past the 2^31-element offset.
"""
import numpy as np
import pytest
import torch

from ada_mla import capi
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

N_BIG = 3_800_000  # > 2^31 / 576 = 3,728,270.2 tokens
N_SMALL = 3000
EDGE = 4096  # nonzero rows at each end of the long sequence
N_H = 128
# N(0, 1) rows scaled: the tail's logits dominate the head's (its largest,
# about 3.5 sigma of 1.5 * 1.73, is e^9 against e^~0.6), and stay within the
# range of the other fp8 tests, whose Q* split (about 8 significant bits)
# errs in proportion to the logits
HEAD_SCALE, TAIL_SCALE = 0.1, 1.5


def _closed_form_sparse(q, rows, n_zero):
    """softmax(scale q C^T) C[:, :512] over `rows` plus n_zero zero rows, float64."""
    s = (q @ rows.T) * O.SCALE                      # [n_h, R]
    m = np.maximum(s.max(axis=1, keepdims=True), 0.0)
    e = np.exp(s - m)
    den = e.sum(axis=1, keepdims=True) + n_zero * np.exp(-m)
    return (e @ rows[:, :512]) / den


def _check(got, want, what):
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2, err_msg=what)
    rel = np.abs(got - want).mean() / np.abs(want).mean()
    assert rel < 5e-3, f"{what}: mean relative error {rel}"


@pytest.mark.parametrize("cache", ["fp16", "fp8"])
def test_offsets_past_2_31_elements(cache):
    dev = torch.device("cuda:0")
    total = N_BIG + N_SMALL
    dt = torch.float16 if cache == "fp16" else torch.float8_e4m3fn
    print(f"large cache: {cache}, {total} tokens, {total * 576 * dt.itemsize / 2**30:.2f} GiB", flush=True)
    g = torch.Generator(device=dev).manual_seed(11)
    c = torch.zeros(total, 576, device=dev, dtype=torch.uint8).view(dt) if cache == "fp8" else \
        torch.zeros(total, 576, device=dev, dtype=dt)
    c[:EDGE] = (HEAD_SCALE * torch.randn(EDGE, 576, device=dev, generator=g)).to(dt)
    c[N_BIG - EDGE:N_BIG] = (TAIL_SCALE * torch.randn(EDGE, 576, device=dev, generator=g)).to(dt)
    c[N_BIG:] = torch.randn(N_SMALL, 576, device=dev, generator=g).to(dt)
    q = torch.randn(2, N_H, 576, device=dev, generator=g).half()
    assert (N_BIG - EDGE) * 576 > 2**31 and N_BIG * 576 > 2**31

    # the oracle sees the stored values (fp8: decoded, with scale 1)
    def host(t):  # exact: every fp16 and fp8 value is a float32 value
        return t.float().cpu().numpy().astype(np.float64)

    rows = np.concatenate([host(c[:EDGE]), host(c[N_BIG - EDGE:N_BIG])])
    q_np = host(q)
    want0 = _closed_form_sparse(q_np[0], rows, N_BIG - 2 * EDGE)
    want1 = O.closed_form(q_np[1], host(c[N_BIG:]))
    # the tail rows carry the long sequence's output
    tail_share = _closed_form_sparse(q_np[0], rows[EDGE:], N_BIG - EDGE)
    assert np.abs(want0 - tail_share).max() < 1e-3 * np.abs(want0).max()

    cu = torch.tensor([0, N_BIG, total], dtype=torch.int32, device=dev)
    if cache == "fp16":
        out = capi.decode_split_batched_fp16(q, c, cu)
    else:
        out = capi.decode_split_batched_fp8(q, c, 1.0, cu)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    _check(got[0], want0, f"{cache} batched, sequence 0 (3.8 M tokens)")
    _check(got[1], want1, f"{cache} batched, sequence 1 (starts past 2^31 elements)")

    for i, part, want in [(0, c[:N_BIG], want0), (1, c[N_BIG:], want1)]:
        if cache == "fp16":
            single = capi.decode_split_fp16(q[i].contiguous(), part)
        else:
            single = capi.decode_split_fp8(q[i].contiguous(), part, 1.0)
        torch.cuda.synchronize()
        _check(single.double().cpu().numpy(), want, f"{cache} single sequence {i}")
    del c
    torch.cuda.empty_cache()


def test_paged_pages_past_2_31_elements():
    """The paged cache: sequence 0 on the last 47 physical pages (all past
    2^31 elements) in reverse order, sequence 1 alternating between low pages
    and pages past the offset; block-table columns past a sequence's pages
    hold ids out of range."""
    dev = torch.device("cuda:0")
    page, num_pages = 64, 60_000  # 3.84 M tokens of fp16: 4.1 GiB
    lens = [3000, 1000]
    n_pg = [(n + page - 1) // page for n in lens]
    pages = [[num_pages - 1 - j for j in range(n_pg[0])],
             [j if j % 2 == 0 else num_pages - 200 - j for j in range(n_pg[1])]]
    assert min(pages[0]) * page * 576 > 2**31 and max(pages[1]) * page * 576 > 2**31
    print(f"large paged cache: {num_pages} pages of {page}", flush=True)
    g = torch.Generator(device=dev).manual_seed(12)
    kv = torch.zeros(num_pages, page, 576, device=dev, dtype=torch.float16)
    for pg in pages:
        idx = torch.tensor(pg, device=dev)
        kv[idx] = torch.randn(len(pg), page, 576, device=dev, generator=g).half()
    bt = torch.full((2, max(n_pg)), num_pages + 12345, dtype=torch.int32)
    for b, pg in enumerate(pages):
        bt[b, :len(pg)] = torch.tensor(pg, dtype=torch.int32)
    cu = torch.tensor([0, lens[0], lens[0] + lens[1]], dtype=torch.int32, device=dev)
    q = torch.randn(2, N_H, 576, device=dev, generator=g).half()
    out = capi.decode_paged(q, kv, bt.to(dev), cu, sum(lens))
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    for b, pg in enumerate(pages):
        rows = kv[torch.tensor(pg, device=dev)].reshape(-1, 576)[:lens[b]].double().cpu().numpy()
        want = O.closed_form(q[b].double().cpu().numpy(), rows)
        _check(got[b], want, f"paged sequence {b} ({lens[b]} tokens)")
    del kv
    torch.cuda.empty_cache()


def test_fp32_offsets_past_2_31_elements():
    """The fp32 path (mla_decode_fused_fp32) on the same construction: a
    3.8 M-token fp32 cache, and a sequence that starts past 2^31 elements;
    atol = rtol = 1e-4."""
    dev = torch.device("cuda:0")
    total = N_BIG + N_SMALL
    print(f"large cache: fp32, {total} tokens, {total * 576 * 4 / 2**30:.2f} GiB", flush=True)
    g = torch.Generator(device=dev).manual_seed(13)
    c = torch.zeros(total, 576, device=dev, dtype=torch.float32)
    c[:EDGE] = HEAD_SCALE * torch.randn(EDGE, 576, device=dev, generator=g)
    c[N_BIG - EDGE:N_BIG] = TAIL_SCALE * torch.randn(EDGE, 576, device=dev, generator=g)
    c[N_BIG:] = torch.randn(N_SMALL, 576, device=dev, generator=g)
    q = torch.randn(2, N_H, 576, device=dev, generator=g)
    rows = torch.cat([c[:EDGE], c[N_BIG - EDGE:N_BIG]]).double().cpu().numpy()
    q_np = q.double().cpu().numpy()
    wants = [_closed_form_sparse(q_np[0], rows, N_BIG - 2 * EDGE),
             O.closed_form(q_np[1], c[N_BIG:].double().cpu().numpy())]
    for i, part in enumerate([c[:N_BIG], c[N_BIG:]]):
        got = capi.decode_fused_fp32(q[i].contiguous(), part)
        torch.cuda.synchronize()
        np.testing.assert_allclose(got.double().cpu().numpy(), wants[i], atol=1e-4, rtol=1e-4,
                                   err_msg=f"fp32 sequence {i}")
    del c
    torch.cuda.empty_cache()

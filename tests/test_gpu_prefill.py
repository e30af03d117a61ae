"""Initial prefill (reference backend.py:175-193: the fused-infer call, causal attention of each
request over its own tokens, rows past num_actual_tokens zeroed) through
kernels.prefill_attention, on MI355X.

* Bit for bit against the general INT2 path of the same step (empty history): output, merged
  LSE and every cache byte (INT2 slots of the step's tokens, BF16 windows).
* Against the oracle's dense reference (hybrid_reference with no prefix = causal attention in
  fp64 over bf16 inputs): the reference test's atol 0.035 / rtol 0.04
  (tests/test_npu_kernels.py:194), mean-abs <= 2e-3, LSE within 2e-2.
* Padded rows past the token count: zero output, LSE -inf.
* GQA 5:1 (two KV heads) and 7:1, where the 192-row spans start and end inside a query,
  against causal attention in float64 over the same bf16 inputs.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from oscar_new_amd.config import OscarConfig, task_capacity
from oscar_new_amd import kernels
from oscar_new_amd.layout import CacheLayout
from tests._state import bits
from tests.test_gpu_fused import _case, _forward

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    ([1], 0),  # one token
    ([37, 130, 261], 0),  # ragged requests, several query tiles each
    ([1500], 0),  # one long prompt: the ring wraps in the window store
    ([3, 64, 70], 2),  # padded rows past the token count
]


@pytest.mark.parametrize("lengths,pad", CASES)
def test_prefill_matches_int2_path_and_dense_reference(lengths, pad):
    c = _case(lengths, [0] * len(lengths), seed=41, cfg=OscarConfig(sink_tokens=4,
                                                                    recent_tokens=64))
    print(f"[prefill] lengths {lengths} pad {pad}", flush=True)
    if pad:
        c.q = torch.cat([c.q, torch.randn(pad, 6, 256, device=DEV).bfloat16()])
        c.k = torch.cat([c.k, torch.randn(pad, 1, 256, device=DEV).bfloat16()])
        c.v = torch.cat([c.v, torch.randn(pad, 1, 256, device=DEV).bfloat16()])
        qt = c.layout.config.queries_per_tile
        c.meta.tasks = torch.empty((task_capacity(c.q.shape[0], c.meta.max_num_reqs, qt), 2),
                                   device=DEV, dtype=torch.int32)
        kernels.prepare_tasks(c.meta.query_start_loc, c.meta.counts, c.meta.tasks,
                              c.meta.task_count, c.meta.max_num_reqs, qt)
    n = c.q.shape[0]
    c.meta.initial_prefill = False
    want = _forward(c, "single", 1)
    c.meta.initial_prefill = True
    got = _forward(c, "single", 1)
    for a, b in zip(want, got):
        assert torch.equal(a, b)
    out = got[0].view(torch.bfloat16).float().numpy().reshape(n, 6, 256)
    lse = got[1].numpy()
    if pad:
        assert not out[n - pad:].any() and np.isneginf(lse[n - pad:]).all()
    start = 0
    for qi, ki, vi in zip(c.qs, c.ks, c.vs):
        rows = slice(start, start + qi.shape[0])
        start += qi.shape[0]
        o, l = O.hybrid_reference(bits(qi), bits(ki), bits(vi), 0, bits(c.rk), bits(c.rv),
                                  c.layout.config)
        np.testing.assert_allclose(out[rows], o, atol=0.035, rtol=0.04)
        assert np.abs(out[rows] - o).mean() <= 2e-3
        np.testing.assert_allclose(lse[rows], l, atol=2e-2, rtol=0)


@pytest.mark.parametrize("lengths,max_query_len", [
    ([2048, 1100, 9], True),  # many 32-token blocks and 192-row spans, a span crossing queries
    ([300, 5], False),  # max_query_len unknown: spans sized by the token count
])
def test_long_prefill_is_bitwise_the_int2_path(lengths, max_query_len):
    # The flash kernel's spans share K/V blocks across 192 rows; every row must still carry the
    # BF16 branch's bits (the general path runs that branch per 4-query task).
    c = _case(lengths, [0] * len(lengths), seed=43, cfg=OscarConfig(sink_tokens=4,
                                                                    recent_tokens=64))
    print(f"[prefill] lengths {lengths}", flush=True)
    if not max_query_len:
        c.meta.max_query_len = None
    c.meta.initial_prefill = False
    want = _forward(c, "single", 1)
    c.meta.initial_prefill = True
    got = _forward(c, "single", 1)
    for a, b in zip(want, got):
        assert torch.equal(a, b)
    assert torch.isfinite(got[0].view(torch.bfloat16).float()).all()


@pytest.mark.parametrize("g,kv_heads,lengths", [
    (5, 2, [300, 77, 1]),  # 192-row spans end inside a query's 5 heads, two KV heads
    (7, 1, [150, 40]),  # ... and inside a query's 7 heads
])
def test_prefill_spans_that_split_a_query(g, kv_heads, lengths):
    # With 6 query heads per KV head a 192-row span holds 32 whole queries; with 5 or 7 a
    # span starts and ends inside a query, whose heads then go to two workgroups (and two
    # workgroups copy the same K/V blocks). Checked against causal attention in float64 over
    # the same bf16 inputs: relative L2 <= 1e-2, |err| <= 2e-2 + 1e-2 |want|, LSE within 2e-2.
    print(f"[prefill] g {g} kv_heads {kv_heads} lengths {lengths}", flush=True)
    gen = torch.Generator().manual_seed(47)
    n, hq = sum(lengths), g * kv_heads
    q = torch.randn(n, hq, 256, generator=gen).bfloat16()
    k = torch.randn(n, kv_heads, 256, generator=gen).bfloat16()
    v = torch.randn(n, kv_heads, 256, generator=gen).bfloat16()
    starts = [0]
    for length in lengths:
        starts.append(starts[-1] + length)
    meta = SimpleNamespace(
        query_start_loc=torch.tensor(starts, dtype=torch.int32, device=DEV),
        seq_lens=torch.tensor(lengths, dtype=torch.int32, device=DEV),
        counts=torch.tensor([len(lengths), n], dtype=torch.int32, device=DEV),
        max_num_reqs=len(lengths), max_query_len=max(lengths))
    layout = CacheLayout(768, kv_heads=kv_heads,
                         config=OscarConfig(sink_tokens=4, recent_tokens=64))
    scale = 256 ** -0.5
    out = torch.full((n, hq * 256), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((n * hq,), float("nan"), dtype=torch.float32, device=DEV)
    kernels.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), None, meta, layout, scale, out,
                              lse)
    torch.cuda.synchronize()
    got = out.cpu().float().view(n, hq, 256).double()
    got_l = lse.cpu().view(n, hq).double()
    qf, kf, vf = q.double(), k.double(), v.double()
    for r, length in enumerate(lengths):
        rows = slice(starts[r], starts[r + 1])
        causal = torch.ones(length, length, dtype=torch.bool).tril()
        for h in range(hq):
            s = (qf[rows, h] @ kf[rows, h // g].T * scale).masked_fill(~causal, float("-inf"))
            want = torch.softmax(s, dim=1) @ vf[rows, h // g]
            o = got[rows, h]
            assert torch.isfinite(o).all(), (r, h)
            assert (o - want).norm() <= 1e-2 * want.norm(), (r, h)
            assert ((o - want).abs() <= 2e-2 + 1e-2 * want.abs()).all(), (r, h)
            assert (got_l[rows, h] - torch.logsumexp(s, dim=1)).abs().max() <= 2e-2, (r, h)


def test_prefill_rows_past_a_broken_max_query_len_are_nan():
    # A request with more query tokens than the caller's max_query_len: the grid holds
    # ceil(max_query_len * g / span) spans, the rows it covers are computed, and the rows past
    # them are NaN (output and LSE), never stale memory.
    lengths, g = [300, 40], 6
    gen = torch.Generator().manual_seed(53)
    n = sum(lengths)
    q = torch.randn(n, g, 256, generator=gen).bfloat16()
    k = torch.randn(n, 1, 256, generator=gen).bfloat16()
    v = torch.randn(n, 1, 256, generator=gen).bfloat16()
    meta = SimpleNamespace(
        query_start_loc=torch.tensor([0, 300, 340], dtype=torch.int32, device=DEV),
        seq_lens=torch.tensor(lengths, dtype=torch.int32, device=DEV),
        counts=torch.tensor([2, n], dtype=torch.int32, device=DEV),
        max_num_reqs=2, max_query_len=40)
    layout = CacheLayout(768, config=OscarConfig(sink_tokens=4, recent_tokens=64))
    scale = 256 ** -0.5
    out = torch.zeros((n, g * 256), dtype=torch.bfloat16, device=DEV)
    lse = torch.zeros((n * g,), dtype=torch.float32, device=DEV)
    print("[prefill] broken max_query_len 40 for a 300-token request", flush=True)
    kernels.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), None, meta, layout, scale, out,
                              lse)
    torch.cuda.synchronize()
    got = out.cpu().float().view(n, g, 256).double()
    got_l = lse.cpu().view(n, g).double()
    # The grid covers at least max_query_len queries of each request (spans of 192, 96 or 48
    # rows, whichever gives the launch enough workgroups): here 40 to 64 queries.
    nan_q = torch.isnan(got[:300]).any(dim=2).any(dim=1)
    covered = int((~nan_q).long().cumprod(0).sum())
    assert 40 <= covered <= 64 and (covered * g) % 48 == 0, covered
    assert torch.isnan(got[covered:300]).all() and torch.isnan(got_l[covered:300]).all()
    qf, kf, vf = q.double(), k.double(), v.double()
    for rows, length in ((slice(0, covered), covered), (slice(300, 340), 40)):
        causal = torch.ones(length, length, dtype=torch.bool).tril()
        for h in range(g):
            s = (qf[rows, h] @ kf[rows, 0].T * scale).masked_fill(~causal, float("-inf"))
            want = torch.softmax(s, dim=1) @ vf[rows, 0]
            o = got[rows, h]
            assert (o - want).norm() <= 1e-2 * want.norm(), (rows, h)

"""Device parity of attention partials, merges and the full launch order (MI355X).

Tolerances:
  * partials/LSE vs the oracle on identical packed bytes: relative L2 error <= 1e-2 and
    max-abs <= max(2e-3, 2 % of max |want|) over the live partial rows (the oracle rounds the
    dequantized K/V to bf16, which the kernel does not), LSE within 1e-2. The kernel folds scale/zero
    out of the dot products and feeds p * s_v to the PV MFMA as two FP8 terms; the oracle
    dequantizes to bf16 first (kernels.py:219) and sums in float64.
  * full step vs the cache read back (``O.cached_decode_reference``): relative L2 error
    <= 1e-2, max-abs <= max(2e-3, 2 % of max |want|), merged LSE within 1e-2;
  * full step vs the dense hybrid reference (quantization redone on the CPU): the reference
    test's atol 0.035 / rtol 0.04 (tests/test_npu_kernels.py:194), mean-abs <= 2e-3.
"""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from oscar_new_amd import _ext, kernels
from oscar_new_amd.config import OscarConfig, attention_programs
from tests._state import (assert_lse_close, assert_scaled_close, bits, check_step_against_cache,
                          make_state, oracle_geometry, prepare_prefix, run_attention)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qr(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16().to(DEV)


def _setup(lengths, prefixes, seed=42, cfg=None, max_reqs=8):
    torch.manual_seed(seed)
    layout, raw, hist, window, meta, tables = make_state(lengths, prefixes, cfg, max_reqs=max_reqs)
    rk, rv = _qr(seed), _qr(seed + 1)
    ks = [torch.randn(n, 1, 256).bfloat16() for n in lengths]
    vs = [torch.randn(n, 1, 256).bfloat16() for n in lengths]
    qs = [torch.randn(n - p, 6, 256).bfloat16() for n, p in zip(lengths, prefixes)]
    prepare_prefix(ks, vs, rk, rv, hist, window, meta, tables, layout, prefixes)
    q = torch.cat(qs).to(DEV)
    k = torch.cat([x[p:] for x, p in zip(ks, prefixes)]).to(DEV)
    v = torch.cat([x[p:] for x, p in zip(vs, prefixes)]).to(DEV)
    return layout, raw, hist, window, meta, tables, rk, rv, ks, vs, qs, q, k, v


def _oracle_partials(q, k, v, hist, window, meta, layout, splits, raw, split_tokens=0):
    counts = meta.counts.cpu().numpy()
    tasks = [tuple(t) for t in meta.tasks.cpu().tolist()]
    count = int(meta.task_count.item())
    return O.attention_partials(
        bits(q), bits(k), bits(v), hist.cpu().numpy(), bits(window), meta.query_start_loc.cpu().numpy(),
        meta.seq_lens.cpu().numpy(), meta.block_tables.cpu().numpy(), counts, tasks, count,
        oracle_geometry(layout), 1 / 16, splits, raw, layout.config.block_n,
        layout.config.queries_per_tile,
        programs=attention_programs(q.shape[0], meta.max_num_reqs, layout.config.queries_per_tile),
        split_tokens=split_tokens,
    )


@pytest.mark.parametrize(
    "lengths,prefixes,splits",
    [([1804, 2601], [1800, 2600], 8), ([1700], [800], 3), ([300, 5000, 700], [299, 4999, 699], 16)],
)
def test_history_and_raw_partials_match_oracle(lengths, prefixes, splits):
    layout, _, hist, window, meta, _, rk, rv, *_, q, k, v = _setup(lengths, prefixes)
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, layout.config.queries_per_tile)
    kr, vr = kernels.rotate(k, rk), kernels.rotate(v, rv)
    kernels.store_int2(kr, vr, hist, meta.slot_mapping, meta.counts, layout)
    qr = kernels.rotate(q, rk)
    for raw, nsplit, query in ((False, splits, qr), (True, 1, q)):
        p, l = kernels.attention_partials(query, k, v, hist, window, meta, layout, 1 / 16, nsplit,
                                          raw)
        po, lo = _oracle_partials(query, k, v, hist, window, meta, layout, nsplit, raw)
        live = ~np.isnan(lo)
        assert live.any()
        got_p, got_l = p.cpu().numpy(), l.cpu().numpy()
        assert_lse_close(got_l[live], lo[live], f"partial LSE raw={raw}")
        assert_scaled_close(got_p[live], po[live], f"partials raw={raw}")


@pytest.mark.parametrize("splits,split_tokens", [(16, 512), (40, 256)])
def test_token_bounded_splits_match_oracle_and_merge_to_one_split(splits, split_tokens):
    # Token-bounded rule: request r uses min(splits, ceil(L_r / split_tokens)) splits; the
    # other slots get LSE -inf and no partial row. 40 splits take the workgroup merge, whose
    # partial loads are gated on the LSE: the unused slots are filled with NaN to prove it.
    lengths, prefixes = [300, 5000, 700], [299, 4999, 699]
    layout, _, hist, window, meta, _, rk, rv, *_, q, k, v = _setup(lengths, prefixes)
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, layout.config.queries_per_tile)
    kernels.store_int2(kernels.rotate(k, rk), kernels.rotate(v, rv), hist, meta.slot_mapping,
                       meta.counts, layout)
    qr = kernels.rotate(q, rk)
    p, l = kernels.attention_partials(qr, k, v, hist, window, meta, layout, 1 / 16, splits,
                                      False, split_tokens=split_tokens)
    po, lo = _oracle_partials(qr, k, v, hist, window, meta, layout, splits, False, split_tokens)
    got_p, got_l = p.cpu().numpy(), l.cpu().numpy()
    written = ~np.isnan(lo)
    assert (np.isneginf(lo) & written).any()  # some slots are unused
    np.testing.assert_array_equal(np.isneginf(got_l[written]), np.isneginf(lo[written]))
    fin = written & np.isfinite(lo)
    assert_lse_close(got_l[fin], lo[fin], "token-bounded partial LSE")
    rows = ~np.isnan(po[..., 0])
    assert_scaled_close(got_p[rows], po[rows], "token-bounded partials")

    p[torch.from_numpy(~rows).to(DEV)] = float("nan")
    out, ls = kernels.merge_splits(p, l, meta.counts)
    p1, l1 = kernels.attention_partials(qr, k, v, hist, window, meta, layout, 1 / 16, 1, False)
    out1, ls1 = kernels.merge_splits(p1, l1, meta.counts)
    torch.testing.assert_close(out.float(), out1.float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(ls, ls1, atol=1e-4, rtol=0)


@pytest.mark.parametrize("splits,split_tokens", [(40, 128), (16, 512)])
def test_work_queue_is_bitwise_the_grid_form(splits, split_tokens):
    # MTP tasks of 4 query tokens x 6 heads (24 rows: the eight-wavefront kernel) with
    # token-bounded splits run as a work queue (one workgroup per CU over the units in use): the
    # same LSEs and partial rows as the grid form, call after call (the counters reset
    # themselves) and in graph replays with eager launches in between.
    lengths = [2600, 900, 5000, 300, 40]
    prefixes = [x - 4 for x in lengths]
    layout, _, hist, window, meta, _, rk, rv, *_, q, k, v = _setup(lengths, prefixes)
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, layout.config.queries_per_tile)
    kernels.store_int2(kernels.rotate(k, rk), kernels.rotate(v, rv), hist, meta.slot_mapping,
                       meta.counts, layout)
    qr = kernels.rotate(q, rk)
    assert kernels.history_rows(meta, layout, 6) == 24
    print(f"[queue] splits {splits} split_tokens {split_tokens}", flush=True)

    def run(use_queue):
        return kernels.attention_partials(qr, k, v, hist, window, meta, layout, 1 / 16, splits,
                                          False, split_tokens=split_tokens, use_queue=use_queue)

    want_p, want_l = run(False)
    fin = torch.isfinite(want_l)
    assert fin.any() and torch.isneginf(want_l).any()  # used and unused split slots

    def same(p, l, what):
        assert torch.equal(l, want_l), what + ": LSE"
        assert torch.equal(p[fin], want_p[fin]), what + ": partial rows"

    for i in range(3):
        same(*run(True), f"queue call {i}")
    counters = kernels.queue_counters(meta, qr.device)
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        gp, gl = run(True)
    torch.cuda.synchronize()
    for i in range(3):
        gp.fill_(float("nan"))
        gl.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        same(gp, gl, f"graph replay {i}")
        same(*run(True), f"eager call after replay {i}")
    assert int(counters.abs().sum()) == 0


def _abi_partials(query, meta, layout, splits, raw, hist, window, k, v, partials, lse):
    """Direct C-ABI call with caller-provided (sentinel-filled) outputs."""
    cfg = layout.config
    n, hq, _ = query.shape
    status = _ext.library().oscar_attention_partials(
        query.data_ptr(), *query.stride(), k.data_ptr(), *k.stride(), v.data_ptr(), *v.stride(),
        hist.data_ptr(), hist.numel(), window.data_ptr(), window.numel(),
        meta.query_start_loc.data_ptr(), meta.seq_lens.data_ptr(), meta.block_tables.data_ptr(),
        meta.block_tables.stride(0), meta.block_tables.shape[1], meta.counts.data_ptr(),
        meta.tasks.data_ptr(), meta.task_count.data_ptr(), n, hq,
        attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile), splits, cfg.block_n,
        cfg.queries_per_tile, 0, 1 / 16, int(raw), 0, kernels.layout_struct(layout),
        partials.data_ptr(), lse.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    _ext.check(status, "attention_partials")


@pytest.mark.parametrize("raw", [False, True])
@pytest.mark.parametrize("active", [False, True])
def test_inactive_programs_write_nothing_and_empty_history_is_zero(raw, active):
    # Reference tests/test_attention_empty_tasks.py:172-194.
    layout, _, hist, window, meta, tables = make_state([4], [0])
    q = torch.randn(4, 6, 256, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(4, 1, 256, device=DEV, dtype=torch.bfloat16)
    if not active:
        meta.counts.zero_()
        meta.query_start_loc.fill_(2**30)
        meta.seq_lens.fill_(2**30)
        meta.block_tables.fill_(2**30)
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, 4)
    partials = torch.full((4, 6, 2, 256), 123.0, device=DEV)
    lse = torch.full((4, 6, 2), 123.0, device=DEV)
    _abi_partials(q, meta, layout, 2, raw, hist, window, k, k, partials, lse)
    torch.cuda.synchronize()
    if not active:
        assert partials.eq(123).all() and lse.eq(123).all()
    elif not raw:
        assert partials.eq(0).all() and torch.isneginf(lse).all()
    else:
        # Raw: split 0 holds all 4 causal current tokens, split 1 is empty.
        assert torch.isfinite(lse[..., 0]).all() and torch.isneginf(lse[..., 1]).all()
        assert partials[..., 1, :].eq(0).all()


@pytest.mark.parametrize("n,splits", [(7, 5), (7, 16), (7, 40), (7, 130), (48, 40)])
def test_merges_match_oracle_with_empty_splits_and_padded_rows(n, splits):
    # Above 16 splits the LSEs are scanned first and only slots below the last finite one are
    # read: by a whole workgroup per row (few rows) or one wavefront per row (>= 256 rows).
    g = torch.Generator().manual_seed(5)
    hq = 6
    partials = torch.randn(n, hq, splits, 256, generator=g)
    lse = torch.randn(n, hq, splits, generator=g) * 3
    lse[0, :, 2] = -float("inf")
    lse[2, :, splits // 2:] = -float("inf")  # unwritten slots: never read
    partials[2, :, splits // 2:] = float("nan")
    lse[1] = -float("inf")
    partials[1] = float("nan")  # never read: every split of this row has zero weight
    counts = torch.tensor([3, 5], dtype=torch.int32)
    out, logsum = kernels.merge_splits(partials.to(DEV), lse.to(DEV), counts.to(DEV))
    p_clean = partials.clone()
    p_clean[1] = 0
    p_clean[2, :, splits // 2:] = 0
    want_out, want_l = O.merge_splits(p_clean.numpy(), lse.numpy(), counts.numpy())
    np.testing.assert_allclose(O.bf16_to_f32(bits(out)), O.bf16_to_f32(want_out), atol=1e-6,
                               rtol=1e-2)
    np.testing.assert_allclose(logsum.cpu().numpy(), want_l, atol=1e-5, rtol=1e-6)
    assert out[5:].float().eq(0).all() and torch.isneginf(logsum[5:]).all()

    a = torch.randn(n, hq, 256, generator=g).bfloat16()
    la = torch.randn(n, hq, generator=g)
    b = torch.randn(n, hq, 1, 256, generator=g)
    lb = torch.randn(n, hq, generator=g)
    la[2, 0] = -float("inf")
    lb[2, 1] = -float("inf")
    output = torch.full((n, hq * 256), 7.0, dtype=torch.bfloat16, device=DEV)
    merged = torch.full((n, hq), 7.0, device=DEV)
    kernels.merge_paths(a.to(DEV), la.to(DEV), b.to(DEV), lb.to(DEV), counts.to(DEV), output,
                        merged)
    want_o, want_m = O.merge_paths(bits(a), la.numpy(), b.numpy(), lb.numpy(), counts.numpy())
    np.testing.assert_allclose(O.bf16_to_f32(bits(output)), O.bf16_to_f32(want_o), atol=1e-6,
                               rtol=1e-2)
    np.testing.assert_allclose(merged.cpu().numpy()[:5], want_m[:5], atol=1e-5)
    assert output[5:].float().eq(0).all()


def _dense_expected(qs, ks, vs, prefixes, rk, rv, cfg):
    outs, lses = [], []
    for qi, ki, vi, p in zip(qs, ks, vs, prefixes):
        o, l = O.hybrid_reference(bits(qi), bits(ki), bits(vi), p, bits(rk), bits(rv), cfg)
        outs.append(o)
        lses.append(l)
    return np.concatenate(outs), np.concatenate(lses)


@pytest.mark.parametrize(
    "lengths,prefixes,splits",
    [
        ([4], [0], 32),  # empty history / all-masked splits
        ([69, 263], [65, 260], 16),  # ragged MTP, sink/recent overlap, no history
        ([1804, 2601], [1800, 2600], 8),  # non-monotonic pages, GQA + MTP
        ([1700], [800], 1),  # continuation chunk wraps the ring several times
    ],
)
def test_fused_attention_against_dense_reference(lengths, prefixes, splits):
    # Reference tests/test_npu_kernels.py:166-194.
    layout, raw, hist, window, meta, tables, rk, rv, ks, vs, qs, q, k, v = _setup(lengths, prefixes)
    merged = torch.empty(q.shape[0], 6, device=DEV)
    before = raw.clone()  # the step's window store may overwrite ring slots it read
    actual = run_attention(q, k, v, rk, rv, hist, window, meta, layout, splits, merged)
    torch.cuda.synchronize()
    # Tight: against the cache the step read, dense fp64 attention per request.
    check_step_against_cache(actual, merged, before, layout, tables, lengths, prefixes, qs, ks,
                             vs, rk, rv)
    want, want_lse = _dense_expected(qs, ks, vs, prefixes, rk.cpu(), rv.cpu(), layout.config)
    got = actual.float().cpu()
    torch.testing.assert_close(got, torch.from_numpy(want), atol=0.035, rtol=0.04)
    err = (got - torch.from_numpy(want)).abs()
    assert err.mean().item() <= 2e-3, err.mean().item()
    torch.testing.assert_close(merged.cpu(), torch.from_numpy(want_lse), atol=2e-2, rtol=0)


def test_graph_replay_changes_metadata_and_page_owners():
    # Reference tests/test_npu_kernels.py:197-245, on a HIP graph. Replayed several times
    # with eager work in between; every replay is checked.
    torch.manual_seed(10)
    layout, _, hist, window, meta, _ = make_state([4], [0], max_reqs=4)
    q = torch.randn(4, 6, 256, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(4, 1, 256, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    rk = rv = torch.eye(256, device=DEV, dtype=torch.bfloat16)
    meta.max_query_len = 4
    for _ in range(3):
        run_attention(q, k, v, rk, rv, hist, window, meta, layout, 8)
    torch.cuda.synchronize()
    meta.counts.zero_()
    before = hist.clone(), window.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        actual = run_attention(q, k, v, rk, rv, hist, window, meta, layout, 8)
    torch.cuda.synchronize()
    assert torch.equal(hist, before[0]) and torch.equal(window, before[1])
    meta.query_start_loc.copy_(torch.tensor([0, 2, 4, 0, 0], device=DEV, dtype=torch.int32))
    meta.seq_lens[:2].fill_(2)
    meta.counts[0].fill_(2)
    meta.counts[1].fill_(4)
    meta.block_tables[0, :6].copy_(torch.arange(18, 24, device=DEV, dtype=torch.int32))
    meta.block_tables[1, :6].copy_(torch.arange(36, 42, device=DEV, dtype=torch.int32))
    meta.slot_mapping.copy_(torch.tensor([18 * 128, 18 * 128 + 1, 36 * 128, 36 * 128 + 1],
                                         device=DEV))
    for replay in range(3):
        q.normal_()
        k.normal_()
        v.normal_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = torch.cat([
            torch.from_numpy(O.hybrid_reference(bits(q[i:i + 2]), bits(k[i:i + 2]),
                                                bits(v[i:i + 2]), 0, bits(rk), bits(rv),
                                                layout.config)[0])
            for i in (0, 2)
        ])
        torch.testing.assert_close(actual.float().cpu(), expected, atol=0.035, rtol=0.04)
        _ = (q * 2).sum().item()  # eager work between replays


def test_device_ring_survives_mtp_rejection_and_rewrites():
    # Reference tests/test_npu_kernels.py:248-290.
    torch.manual_seed(81)
    layout, _, hist, window, meta, tables = make_state([1500], [0], max_reqs=2)
    rk = rv = torch.eye(256, device=DEV, dtype=torch.bfloat16)
    keys = torch.randn(1500, 1, 256).bfloat16()
    values = torch.randn_like(keys)
    prepare_prefix([keys], [values], rk, rv, hist, window, meta, tables, layout, [900])
    prefix = 900
    for rejected in (3, 2, 0, 3, 1):
        keys[prefix : prefix + 4].normal_()
        values[prefix : prefix + 4].normal_()
        query = torch.randn(4, 6, 256, device=DEV, dtype=torch.bfloat16)
        meta.query_start_loc[:2].copy_(torch.tensor([0, 4], device=DEV, dtype=torch.int32))
        meta.seq_lens[0].fill_(prefix + 4)
        meta.counts.copy_(torch.tensor([1, 4], device=DEV, dtype=torch.int32))
        meta.slot_mapping = torch.tensor(
            [int(tables[0, t // 128]) * 128 + t % 128 for t in range(prefix, prefix + 4)],
            device=DEV, dtype=torch.int64)
        meta.max_query_len = 4
        actual = run_attention(query, keys[prefix : prefix + 4].to(DEV),
                               values[prefix : prefix + 4].to(DEV), rk, rv, hist, window, meta,
                               layout, 16)
        expected = O.hybrid_reference(bits(query), bits(keys[: prefix + 4]),
                                      bits(values[: prefix + 4]), prefix, bits(rk), bits(rv),
                                      layout.config)[0]
        torch.testing.assert_close(actual.float().cpu(), torch.from_numpy(expected), atol=0.035,
                                   rtol=0.04)
        prefix += 4 - rejected

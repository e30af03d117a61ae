"""The fused layer step (pre_attention, history kernel, post_attention), its two-launch form
(history + post in one launch) and the one-launch layer step against the reference order of
single launches (oscar_ascend/backend.py:171-226) and against the dense oracle.

The three- and two-launch forms run the same device code as the single entry points, so the
comparison with the single-launch path is bit for bit: attention output, merged LSE, every byte
of the K stripe (INT2 slots + untouched padding) and of the V stripe (BF16 windows). The
one-launch layer step writes the same cache bytes (bit for bit) and merges the BF16 branch
from up to four splits, so its output is checked with the scale-aware bounds against the
single-launch output and against the cache read back.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from oscar_new_amd import kernels
from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import OscarConfig
from tests._state import (assert_lse_close, assert_scaled_close, bits, check_step_against_cache,
                          make_state, prepare_prefix)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qr(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16().to(DEV)


def _case(lengths, prefixes, seed, cfg=None):
    torch.manual_seed(seed)
    layout, raw, hist, window, meta, tables = make_state(lengths, prefixes, cfg)
    rk, rv = _qr(seed), _qr(seed + 1)
    ks = [torch.randn(n, 1, 256).bfloat16() for n in lengths]
    vs = [torch.randn(n, 1, 256).bfloat16() for n in lengths]
    qs = [torch.randn(n - p, 6, 256).bfloat16() for n, p in zip(lengths, prefixes)]
    prepare_prefix(ks, vs, rk, rv, hist, window, meta, tables, layout, prefixes)
    q = torch.cat(qs).to(DEV)
    k = torch.cat([x[p:] for x, p in zip(ks, prefixes)]).to(DEV)
    v = torch.cat([x[p:] for x, p in zip(vs, prefixes)]).to(DEV)
    meta.layout = layout
    meta.num_actual_tokens = q.shape[0]
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, layout.config.queries_per_tile)
    return SimpleNamespace(layout=layout, raw=raw, meta=meta, rk=rk, rv=rv, ks=ks, vs=vs, qs=qs,
                           q=q, k=k, v=v, prefixes=prefixes, tables=tables)


def _views(raw, layout, pages=20):
    """Native (K, V) cache views of a make_state byte buffer (conv | K | V)."""
    stripe = pages * layout.stripe_page_bytes
    conv = raw.numel() - 2 * stripe
    k = raw[conv : conv + stripe].view(torch.bfloat16).view(-1, 128, 1, 256)
    v = raw[conv + stripe :].view(torch.bfloat16).view(-1, 128, 1, 256)
    return k, v


CASES = [
    ([4], [0], 32),  # empty history, all-masked splits
    ([69, 263], [65, 260], 16),  # ragged MTP, no history
    ([1804, 2601], [1800, 2600], 8),  # non-monotonic pages, GQA + MTP
    ([1700], [800], 1),  # continuation chunk wraps the ring
    ([3000, 1500, 777], [2999, 1499, 776], 16),  # decode
]


def _forward(c, form, splits, raw=None):
    """One layer step in `form` ("single"; "fused": q rotation, history launch carrying the
    BF16 branch and INT2 store, post-attention; "fused_rot": as "fused" with the q rotation
    done by the history workgroups; "fused_serial": pre-attention, history, post-attention;
    "fused1": history + post in one launch where it applies; "layer": the one-launch step
    where it applies) on a copy of the cache."""
    n = c.q.shape[0]
    raw = c.raw.clone() if raw is None else raw
    k_cache, v_cache = _views(raw, c.layout)
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, c.layout.config,
                                         fused=form != "single", one_launch_post=form == "fused1",
                                         layer_step=form == "layer", overlap=form != "fused_serial",
                                         rotate_in_history=form == "fused_rot")
    impl.set_rotations(c.rk, c.rv)
    impl.partition_for = lambda meta, tokens=None, s=splits: (s, 0)
    c.meta.merged_lse = torch.full((n, 6), 7.0, device=DEV)
    out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), c.meta, out)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu(), c.meta.merged_lse.cpu(), raw.cpu()


@pytest.mark.parametrize("lengths,prefixes,splits", CASES)
def test_fused_step_is_bitwise_the_single_launch_step(lengths, prefixes, splits):
    c = _case(lengths, prefixes, seed=7)
    want = _forward(c, "single", splits)
    for form in ("fused", "fused_rot", "fused_serial", "fused1"):
        print(f"[fused] {lengths} splits {splits} form {form}", flush=True)
        got = _forward(c, form, splits)
        for a, b in zip(want, got):
            assert torch.equal(a, b), form


@pytest.mark.parametrize("lengths,prefixes,splits", CASES + [
    ([1300, 700, 2500, 40], [1299, 699, 2499, 39], 5),  # decode, fewer splits than raw shares
    ([3000, 1500], [2999, 1499], 1),  # one split: it stores K, V and the whole BF16 branch
])
def test_layer_step_writes_the_same_cache_and_a_close_output(lengths, prefixes, splits):
    c = _case(lengths, prefixes, seed=17)
    want = _forward(c, "single", splits)
    got = _forward(c, "layer", splits)
    assert torch.equal(want[2], got[2]), "cache bytes"
    n = c.q.shape[0]
    a = want[0].view(torch.bfloat16).float().numpy()
    b = got[0].view(torch.bfloat16).float().numpy()
    assert_scaled_close(b, a, "layer step vs single launches")
    assert_lse_close(got[1].numpy(), want[1].numpy(), "layer step merged LSE", atol=1e-3)
    check_step_against_cache(got[0].view(torch.bfloat16).reshape(n, -1), got[1], c.raw,
                             c.layout, c.tables, lengths, prefixes, c.qs, c.ks, c.vs, c.rk, c.rv)


@pytest.mark.parametrize("lengths,prefixes,partition", [
    ([6000, 1500, 300], [5999, 1499, 299], (6, 1024)),
    ([6000, 1500, 300], [5999, 1499, 299], (40, 256)),  # workgroup-per-row merge
    ([1700, 900], [800, 896], (40, 256)),  # 5424 rows: wavefront-per-row scanned merge
])
def test_token_bounded_fused_step_against_dense_reference(lengths, prefixes, partition):
    # The MI355X split partition of a ragged batch through the fused launches (unwritten
    # split slots above 16 splits) against the dense oracle, and bit for bit against the
    # single-launch order with the same partition.
    c = _case(lengths, prefixes, seed=13)
    n = c.q.shape[0]
    outs = []
    for fused, one in ((True, True), (False, False), (True, False)):
        raw = c.raw.clone()
        k_cache, v_cache = _views(raw, c.layout)
        impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, c.layout.config,
                                             split_policy="mi355x", fused=fused,
                                             one_launch_post=one, layer_step=False)
        impl.set_rotations(c.rk, c.rv)
        impl.partition_for = lambda meta, tokens=None, pt=partition: pt
        c.meta.merged_lse = torch.empty((n, 6), device=DEV)
        out = torch.empty((n, 6 * 256), device=DEV, dtype=torch.bfloat16)
        impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), c.meta, out)
        torch.cuda.synchronize()
        outs.append((out.view(torch.int16).cpu(), c.meta.merged_lse.cpu(), raw.cpu(), out))
    for other in outs[1:]:
        for a, b in zip(outs[0][:3], other[:3]):
            assert torch.equal(a, b)
    check_step_against_cache(outs[0][3], outs[0][1], c.raw, c.layout, c.tables, lengths,
                             prefixes, c.qs, c.ks, c.vs, c.rk, c.rv)
    want, want_lse = [], []
    for qi, ki, vi, p in zip(c.qs, c.ks, c.vs, c.prefixes):
        o, l = O.hybrid_reference(bits(qi), bits(ki), bits(vi), p, bits(c.rk), bits(c.rv),
                                  c.layout.config)
        want.append(o)
        want_lse.append(l)
    want = torch.from_numpy(np.concatenate(want)).reshape(n, -1)
    got = outs[0][3].float().cpu()
    torch.testing.assert_close(got, want, atol=0.035, rtol=0.04)
    assert (got - want).abs().mean().item() <= 2e-3
    torch.testing.assert_close(outs[0][1], torch.from_numpy(np.concatenate(want_lse)), atol=2e-2,
                               rtol=0)


@pytest.mark.parametrize("lengths,prefixes,form", [
    ([900, 517], [896, 516], "fused"),  # MTP: three launches
    ([1300, 700, 2500], [1299, 699, 2499], "layer"),  # decode: the one-launch step
])
def test_fused_step_replays_in_a_graph(lengths, prefixes, form):
    # Reference tests/test_npu_kernels.py:197-245 through the fused step: a captured step
    # replayed with new queries on a reset cache matches the eager step of the same form
    # every time (the three-launch form is also the single-launch step's bits).
    c = _case(lengths, prefixes, seed=21, cfg=OscarConfig(sink_tokens=4, recent_tokens=64))
    n = c.q.shape[0]
    raw_graph, raw_eager = c.raw.clone(), c.raw.clone()
    kg, vg = _views(raw_graph, c.layout)
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, c.layout.config, fused=True,
                                         layer_step=form == "layer")
    impl.set_rotations(c.rk, c.rv)
    impl.partition_for = lambda meta, tokens=None: (8, 0)
    lse = c.meta.merged_lse = torch.empty((n, 6), device=DEV)
    out = torch.empty((n, 6 * 256), device=DEV, dtype=torch.bfloat16)
    impl.forward(None, c.q, c.k, c.v, (kg, vg), c.meta, out)  # warm-up (views, library)
    torch.cuda.synchronize()
    raw_graph.copy_(c.raw)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=stream):
        impl.forward(None, c.q, c.k, c.v, (kg, vg), c.meta, out)
    torch.cuda.synchronize()
    for replay in range(3):
        c.q.normal_()
        raw_graph.copy_(c.raw)
        raw_eager.copy_(c.raw)
        graph.replay()
        torch.cuda.synchronize()
        got = (out.view(torch.int16).cpu(), lse.cpu(), raw_graph.cpu())
        c.meta.merged_lse = lse
        want = _forward(c, "single" if form == "fused" else form, 8, raw=raw_eager)
        for a, b in zip(want, got):
            assert torch.equal(a, b), replay
        _ = (c.q * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("lengths,prefixes,splits", CASES[1:4])
def test_fused_step_against_dense_reference(lengths, prefixes, splits):
    # Reference tests/test_npu_kernels.py:166-194 through the fused launches.
    c = _case(lengths, prefixes, seed=11)
    n = c.q.shape[0]
    k_cache, v_cache = _views(c.raw, c.layout)
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, c.layout.config, fused=True)
    impl.set_rotations(c.rk, c.rv)
    impl.partition_for = lambda meta, tokens=None, s=splits: (s, 0)
    c.meta.merged_lse = torch.empty((n, 6), device=DEV)
    out = torch.empty((n, 6 * 256), device=DEV, dtype=torch.bfloat16)
    before = c.raw.clone()  # the step's window store may overwrite ring slots it read
    impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), c.meta, out)
    torch.cuda.synchronize()
    check_step_against_cache(out, c.meta.merged_lse, before, c.layout, c.tables, lengths,
                             prefixes, c.qs, c.ks, c.vs, c.rk, c.rv)
    want, want_lse = [], []
    for qi, ki, vi, p in zip(c.qs, c.ks, c.vs, c.prefixes):
        o, l = O.hybrid_reference(bits(qi), bits(ki), bits(vi), p, bits(c.rk), bits(c.rv),
                                  c.layout.config)
        want.append(o)
        want_lse.append(l)
    want = torch.from_numpy(np.concatenate(want)).reshape(n, -1)
    got = out.float().cpu()
    torch.testing.assert_close(got, want, atol=0.035, rtol=0.04)
    assert (got - want).abs().mean().item() <= 2e-3
    torch.testing.assert_close(c.meta.merged_lse.cpu(), torch.from_numpy(np.concatenate(want_lse)),
                               atol=2e-2, rtol=0)


def test_pre_attention_matches_single_entry_points():
    c = _case([1804, 2601], [1800, 2600], seed=3)
    meta, layout = c.meta, c.layout
    hist_a, win_a = layout.tensor_views(_views(c.raw.clone(), layout))
    hist_b, win_b = layout.tensor_views(_views(c.raw.clone(), layout))
    rk_t, rv_t = c.rk.T.contiguous(), c.rv.T.contiguous()
    qrot, rp, rl = kernels.pre_attention(c.q, c.k, c.v, hist_a, win_a, meta, layout, 1 / 16,
                                         rk_t, rv_t)
    kernels.store_int2(kernels.rotate(c.k, rk_t.T), kernels.rotate(c.v, rv_t.T), hist_b,
                       meta.slot_mapping, meta.counts, layout)
    q_ref = kernels.rotate(c.q, rk_t.T)
    rp_ref, rl_ref = kernels.attention_partials(c.q, c.k, c.v, hist_b, win_b, meta, layout,
                                                1 / 16, 1, True)
    torch.cuda.synchronize()
    assert torch.equal(qrot.view(torch.int16), q_ref.view(torch.int16))
    assert torch.equal(rp, rp_ref)
    assert torch.equal(rl, rl_ref)
    assert torch.equal(hist_a, hist_b)


@pytest.mark.parametrize("lengths,prefixes,split_tokens", [
    ([1804, 2601], [1803, 2600], 0),  # decode: one query row group per task
    ([69, 263, 1804, 40], [67, 261, 1802, 38], 0),  # two-token MTP (12 rows: > 8, refused)
    ([6000, 300, 4000], [5999, 299, 3999], 512),  # token-bounded splits
    ([6000, 300, 4000], [5999, 299, 3999], -40),  # the device rule, a 40-workgroup budget
])
@pytest.mark.parametrize("q_form", ["launch", "in_history", "roles"])
def test_history_pre_matches_single_entry_points(lengths, prefixes, split_tokens, q_form):
    # in_history: query_rot None, each history workgroup rotates its task's query rows;
    # roles: q rotation role workgroups of the same launch write the rotated rows (q_sync).
    print(f"[history_pre] {lengths} split_tokens {split_tokens} q {q_form}", flush=True)
    c = _case(lengths, prefixes, seed=4)
    meta, layout = c.meta, c.layout
    splits = 8
    hist_a, win_a = layout.tensor_views(_views(c.raw.clone(), layout))
    hist_b, win_b = layout.tensor_views(_views(c.raw.clone(), layout))
    rk_t, rv_t = c.rk.T.contiguous(), c.rv.T.contiguous()
    qrot = kernels.rotate(c.q, rk_t.T)
    if not kernels.history_pre_supported(meta, layout, 6):
        with pytest.raises(ValueError):
            kernels.history_pre(qrot, c.q, c.k, c.v, hist_a, win_a, meta, layout, 1 / 16, splits,
                                rk_t, rv_t)
        return
    q_sync = torch.zeros(4, dtype=torch.int32, device=DEV) if q_form == "roles" else None
    q_arg = {"launch": qrot, "in_history": None, "roles": None}[q_form]
    calls = 2 if q_form == "roles" else 1  # the second call sees the counters the first left
    for _ in range(calls):
        hist_a.copy_(hist_b)
        if q_form == "roles":
            q_arg = torch.full_like(c.q, float("nan"))
        hp, hl, rp, rl = kernels.history_pre(q_arg, c.q, c.k, c.v, hist_a, win_a, meta, layout,
                                             1 / 16, splits, rk_t, rv_t,
                                             split_tokens=split_tokens, q_sync=q_sync)
    if q_form == "roles":
        torch.cuda.synchronize()
        assert q_sync.tolist() == [0, 0, 0, 0]
        assert torch.equal(q_arg.view(torch.int16), qrot.view(torch.int16))
    hp_ref, hl_ref = kernels.attention_partials(qrot, c.k, c.v, hist_b, win_b, meta, layout,
                                                1 / 16, splits, False, split_tokens=split_tokens)
    _, rp_ref, rl_ref = kernels.pre_attention(c.q, c.k, c.v, hist_b, win_b, meta, layout, 1 / 16,
                                              rk_t, rv_t)
    torch.cuda.synchronize()
    live = hl_ref > -float("inf")  # split slots a token-bounded request does not use
    assert torch.equal(hl, hl_ref)
    assert torch.equal(hp[live], hp_ref[live])
    assert torch.equal(rp, rp_ref)
    assert torch.equal(rl, rl_ref)
    assert torch.equal(hist_a, hist_b)


@pytest.mark.parametrize("lengths,prefixes,split_tokens", [
    ([69, 263, 1804, 40], [65, 259, 1800, 36], 512),  # 4-token MTP, token-bounded splits
    ([6000, 300, 4000, 2600], [5996, 296, 3996, 2596], -40),  # the device rule, 40-slot budget
])
def test_history_pre_queue_matches_single_entry_points(lengths, prefixes, split_tokens):
    # 24 rows per task: the history work queue with the BF16 branch and the K/V store as its
    # units, against pre_attention + attention_partials; two calls (the counters the
    # first leaves must be zero for the second).
    print(f"[history_pre queue] {lengths} split_tokens {split_tokens}", flush=True)
    c = _case(lengths, prefixes, seed=6)
    meta, layout = c.meta, c.layout
    n = c.q.shape[0]
    assert kernels.history_rows(meta, layout, 6) == 24
    assert kernels.history_pre_supported(meta, layout, 6, split_tokens, n)
    splits = 8
    hist_a, win_a = layout.tensor_views(_views(c.raw.clone(), layout))
    hist_b, win_b = layout.tensor_views(_views(c.raw.clone(), layout))
    rk_t, rv_t = c.rk.T.contiguous(), c.rv.T.contiguous()
    qrot = kernels.rotate(c.q, rk_t.T)
    for _ in range(2):
        hist_a.copy_(hist_b)
        hp, hl, rp, rl = kernels.history_pre(qrot, c.q, c.k, c.v, hist_a, win_a, meta, layout,
                                             1 / 16, splits, rk_t, rv_t,
                                             split_tokens=split_tokens)
    with pytest.raises(ValueError):  # the queue form takes the rotated query
        kernels.history_pre(None, c.q, c.k, c.v, hist_a, win_a, meta, layout, 1 / 16, splits,
                            rk_t, rv_t, split_tokens=split_tokens)
    hp_ref, hl_ref = kernels.attention_partials(qrot, c.k, c.v, hist_b, win_b, meta, layout,
                                                1 / 16, splits, False, split_tokens=split_tokens)
    _, rp_ref, rl_ref = kernels.pre_attention(c.q, c.k, c.v, hist_b, win_b, meta, layout, 1 / 16,
                                              rk_t, rv_t)
    torch.cuda.synchronize()
    assert kernels.queue_counters(meta, c.q.device)[:2].tolist() == [0, 0]
    live = hl_ref > -float("inf")
    assert torch.equal(hl, hl_ref)
    assert torch.equal(hp[live], hp_ref[live])
    assert torch.equal(rp, rp_ref)
    assert torch.equal(rl, rl_ref)
    assert torch.equal(hist_a, hist_b)


def test_mtp_step_with_queue_roles_is_bitwise_the_single_launch_step():
    # The MTP layer step whose history launch carries the roles (token-bounded splits), and the
    # same step with the roles in a pre-attention launch, against the reference order.
    c = _case([69, 263, 1804, 2600], [65, 259, 1800, 2596], seed=7)
    outs = {}
    for form in ("single", "fused", "fused_serial"):
        n = c.q.shape[0]
        raw = c.raw.clone()
        k_cache, v_cache = _views(raw, c.layout)
        impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, c.layout.config,
                                             fused=form != "single",
                                             overlap=form != "fused_serial")
        impl.set_rotations(c.rk, c.rv)
        impl.partition_for = lambda meta, tokens=None: (8, 512)
        if form == "fused":
            assert impl._queue_roles(c.meta, 512, n)
        c.meta.merged_lse = torch.full((n, 6), 7.0, device=DEV)
        out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
        impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), c.meta, out)
        torch.cuda.synchronize()
        outs[form] = (out.view(torch.int16).cpu(), c.meta.merged_lse.cpu(), raw.cpu())
    for form in ("fused", "fused_serial"):
        for a, b in zip(outs["single"], outs[form]):
            assert torch.equal(a, b), form


def test_post_attention_matches_single_entry_points():
    c = _case([69, 263, 1804], [65, 260, 1800], seed=5)
    meta, layout = c.meta, c.layout
    n = c.q.shape[0]
    splits = 8
    qrot = kernels.rotate(c.q, c.rk.T.contiguous().T)
    hist, win = layout.tensor_views(_views(c.raw, layout))
    hp, hl = kernels.attention_partials(qrot, c.k, c.v, hist, win, meta, layout, 1 / 16, splits,
                                        False)
    rp, rl = kernels.attention_partials(c.q, c.k, c.v, hist, win, meta, layout, 1 / 16, 1, True)
    win_a, win_b = win.clone(), win.clone()
    out_a = torch.empty(n, 6 * 256, device=DEV, dtype=torch.bfloat16)
    lse_a = torch.empty(n, 6, device=DEV)
    kernels.post_attention(hp, hl, rp, rl, c.rv.contiguous(), c.k, c.v, win_a, meta, layout, out_a,
                           lse_a)
    hr, hls = kernels.merge_splits(hp, hl, meta.counts)
    out_b = torch.empty_like(out_a)
    lse_b = torch.empty_like(lse_a)
    kernels.merge_paths(kernels.rotate(hr, c.rv.T), hls, rp, rl, meta.counts, out_b, lse_b)
    kernels.store_windows(c.k, c.v, win_b, meta, layout)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    assert torch.equal(lse_a, lse_b)
    assert torch.equal(win_a.view(torch.int16), win_b.view(torch.int16))


def test_fused_step_masks_padded_tokens_and_dummy_runs():
    # counts = [0, 0] (a dummy / capture run) must leave every cache byte untouched and write
    # zero output rows with -inf LSE, as the single-launch path does.
    c = _case([900, 517], [896, 516], seed=9, cfg=OscarConfig(sink_tokens=4, recent_tokens=64))
    n = c.q.shape[0]
    c.meta.counts.zero_()
    kernels.prepare_tasks(c.meta.query_start_loc, c.meta.counts, c.meta.tasks, c.meta.task_count,
                          c.meta.max_num_reqs, 4)
    before = c.raw.clone()
    k_cache, v_cache = _views(c.raw, c.layout)
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, c.layout.config, fused=True)
    impl.set_rotations(c.rk, c.rv)
    c.meta.merged_lse = torch.empty((n, 6), device=DEV)
    out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), c.meta, out)
    torch.cuda.synchronize()
    assert torch.equal(c.raw, before)
    assert torch.count_nonzero(out).item() == 0
    assert torch.isneginf(c.meta.merged_lse).all()

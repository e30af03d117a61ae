"""The allocation-free entry point ``oscar_history_post_noalloc`` against
``oscar_history_post`` (caller-provided partials, LSEs and counters), through the C ABI.

Two calls in a row on one device, the second with a smaller batch (fewer requests, fewer
query rows, fewer splits), each compared bit for bit with the allocating entry point on the
same inputs: attention output, merged LSE and every byte of the cache (the launch also
stores the windows). The fixed scratch array keeps the previous call's contents, so the
second call also shows that nothing stale leaks into a smaller one. Requests larger than the
array are refused with OSCAR_E_SCRATCH before anything is launched.
"""

import ctypes

import pytest
import torch

from oscar_new_amd import _ext, kernels
from oscar_new_amd.config import attention_programs
from tests.test_gpu_fused import _case, _views

pytestmark = pytest.mark.gpu
DEV = "cuda"
OSCAR_E_SCRATCH = -6


def _noalloc(qrot, hist, meta, layout, splits, rp, rl, rv, k, v, window, out, lse):
    cfg = layout.config
    n, hq, _ = qrot.shape
    table = meta.block_tables
    programs = attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile)
    return _ext.library().oscar_history_post_noalloc(
        qrot.data_ptr(), *qrot.stride(), hist.data_ptr(), hist.numel(),
        meta.query_start_loc.data_ptr(), meta.seq_lens.data_ptr(), table.data_ptr(),
        table.stride(0), table.shape[1], meta.counts.data_ptr(), meta.tasks.data_ptr(),
        meta.task_count.data_ptr(), n, hq, programs, splits, cfg.block_n, cfg.queries_per_tile,
        int(meta.max_query_len), 1 / 16, 0, ctypes.byref(kernels.layout_struct(layout)),
        rp.data_ptr(), rl.data_ptr(), rv.data_ptr(), out.data_ptr(), lse.data_ptr(),
        k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
        window.data_ptr(), window.numel(), meta.max_num_reqs,
        torch.cuda.current_stream().cuda_stream)


def _both(c, splits):
    """(allocating, allocation-free) results of one history + post launch on copies of the
    cache: (output bits, merged LSE, cache bytes)."""
    meta, layout = c.meta, c.layout
    n = c.q.shape[0]
    base = c.raw.clone()
    hist, win = layout.tensor_views(_views(base, layout))
    rk_t, rv_t = c.rk.T.contiguous(), c.rv.T.contiguous()
    rv = c.rv.contiguous()
    qrot, rp, rl = kernels.pre_attention(c.q, c.k, c.v, hist, win, meta, layout, 1 / 16, rk_t,
                                         rv_t)
    results = []
    for free in (False, True):
        raw = base.clone()
        hist, win = layout.tensor_views(_views(raw, layout))
        out = torch.full((n, 6 * 256), 3.0, dtype=torch.bfloat16, device=DEV)
        lse = torch.full((n, 6), 7.0, device=DEV)
        if free:
            status = _noalloc(qrot, hist, meta, layout, splits, rp, rl, rv, c.k, c.v, win, out,
                              lse)
            _ext.check(status, "history_post_noalloc")
        else:
            kernels.history_post(qrot, hist, meta, layout, 1 / 16, splits, rp, rl, rv, c.k, c.v,
                                 win, out, lse)
        torch.cuda.synchronize()
        results.append((out.view(torch.int16).cpu(), lse.cpu(), raw.cpu()))
    return results


def test_noalloc_history_post_matches_the_allocating_entry_point_twice():
    lib = _ext.library()
    big = _case([3000, 1500, 777, 4100], [2999, 1499, 776, 4099], seed=31)
    small = _case([900, 517], [899, 516], seed=32)
    for c, splits in ((big, 16), (small, 8)):
        print(f"[noalloc] {c.meta.num_reqs} requests, {c.q.shape[0]} query rows, {splits} splits",
              flush=True)
        need = lib.oscar_noalloc_scratch_bytes(c.q.shape[0], 6, splits)
        assert 0 < need <= _ext.NOALLOC_SCRATCH_BYTES
        ref, free = _both(c, splits)
        for what, a, b in zip(("output", "merged LSE", "cache bytes"), ref, free):
            assert torch.equal(a, b), what


def test_noalloc_refuses_requests_beyond_its_scratch():
    c = _case([900], [899], seed=33)
    n = 40_000  # 40000 rows x 6 heads x 16 splits x 1028 bytes is far beyond 32 MiB
    assert _ext.library().oscar_noalloc_scratch_bytes(n, 6, 16) > _ext.NOALLOC_SCRATCH_BYTES
    hist, win = c.layout.tensor_views(_views(c.raw, c.layout))
    q = torch.zeros(n, 6, 256, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(n, 1, 256, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(n, 6 * 256, dtype=torch.bfloat16, device=DEV)
    rows = torch.zeros(n, 6, device=DEV)
    before = c.raw.clone()
    status = _noalloc(q, hist, c.meta, c.layout, 16, rows, rows, c.rv, kv, kv, win, out, rows)
    assert status == OSCAR_E_SCRATCH
    with pytest.raises(ValueError, match="fixed scratch"):
        _ext.check(status, "history_post_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(c.raw, before) and torch.count_nonzero(out).item() == 0

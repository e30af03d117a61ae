"""One layer step captured in a HIP graph at a dummy batch's lengths, replayed at BASELINE's
full-size lengths, under the device split rule (the default split policy).

vLLM captures a decode graph per batch size under ``build_for_cudagraph_capture`` (reference
metadata.py:163-170: zero counts mask every access while the launches are recorded) and
replays it for every later step of that size, after ``build`` has refilled the fixed metadata
buffers. The reference keeps that valid by sizing splits from host request counts only
(config.py:84-89). Under the device rule the grid is sized from values fixed at capture and
every history workgroup derives the split length from the lengths in device memory, so the
replay must produce exactly the bits of an eager step at the new lengths:

* a decode graph (1 query token per request, 32 tokens, 32 request slots) replayed at c3
  lengths (32 x 32768) and at c5 lengths (4 x 262144, the other 28 token rows padding);
* an MTP graph (4 query tokens per request, 256 tokens, 64 request slots) replayed at c4
  lengths (64 requests, log-uniform 256..131072, seed 1234, as bench.py draws them).

Each replay is compared bit for bit with an eager step on the same buffers, and against a
step under the reference split rule (config.py:84-89): a different partition of the same
history, so the two agree within rounding (relative L2 <= 5e-3, max-abs <= 2e-3) only if the
device rule's units cover every history token exactly once.
"""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oscar_new_amd import kernels
from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import OscarConfig, task_capacity
from oscar_new_amd.layout import CacheLayout
from tests._state import assert_scaled_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
POOL_PAGES = 1664  # 1.28 M tokens: the largest batch (c4, seed 1234: 1617 pages) fits


def _pool(layout, gen):
    """K/V stripes of POOL_PAGES pages; every history slot holds an INT2 record written by the
    product's rotate + store kernels (random rotated K/V), the windows are zero."""
    bpp = layout.blocks_per_page
    k_cache = torch.zeros(POOL_PAGES * bpp, 128, 1, 256, dtype=torch.bfloat16, device=DEV)
    v_cache = torch.zeros_like(k_cache)
    history, _ = layout.tensor_views((k_cache, v_cache))
    rk = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16().to(DEV)
    rv = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16().to(DEV)
    dgen = torch.Generator(device=DEV).manual_seed(77)
    total = POOL_PAGES * bpp * 128
    for start in range(0, total, 65536):
        t = min(65536, total - start)
        k = torch.randn(t, 1, 256, generator=dgen, device=DEV).bfloat16()
        v = torch.randn(t, 1, 256, generator=dgen, device=DEV).bfloat16()
        slots = torch.arange(start, start + t, device=DEV, dtype=torch.int64)
        counts = torch.tensor([1, t], dtype=torch.int32, device=DEV)
        kernels.store_int2(kernels.rotate(k, rk), kernels.rotate(v, rv), history, slots, counts,
                           layout)
    torch.cuda.synchronize()
    return k_cache, v_cache, rk, rv


class _Buffers:
    """The fixed-pointer metadata buffers of one captured batch size (what the metadata
    builder owns), refilled in place for each step."""

    def __init__(self, layout, max_reqs, tokens, qlen, columns):
        qt = layout.config.queries_per_tile
        self.layout, self.max_reqs, self.tokens, self.qlen = layout, max_reqs, tokens, qlen
        self.qstarts = torch.zeros(max_reqs + 1, dtype=torch.int32, device=DEV)
        self.seqs = torch.zeros(max_reqs, dtype=torch.int32, device=DEV)
        self.table = torch.zeros((max_reqs, columns), dtype=torch.int32, device=DEV)
        self.slots = torch.full((tokens,), -1, dtype=torch.int64, device=DEV)
        self.counts = torch.zeros(2, dtype=torch.int32, device=DEV)
        self.tasks = torch.zeros((task_capacity(tokens, max_reqs, qt), 2), dtype=torch.int32,
                                 device=DEV)
        self.task_count = torch.zeros(1, dtype=torch.int32, device=DEV)
        self.merged_lse = torch.zeros((tokens, 6), dtype=torch.float32, device=DEV)

    def meta(self, num_reqs):
        return SimpleNamespace(
            query_start_loc=self.qstarts, seq_lens=self.seqs, block_tables=self.table,
            slot_mapping=self.slots, counts=self.counts, tasks=self.tasks,
            task_count=self.task_count, merged_lse=self.merged_lse, layout=self.layout,
            num_reqs=num_reqs, num_actual_tokens=self.tokens, max_query_len=self.qlen,
            max_num_reqs=self.max_reqs)

    def dummy(self):
        """The capture build: zero counts mask every access (reference metadata.py:163-170)."""
        self.counts.zero_()
        self.seqs.fill_(self.qlen)
        kernels.prepare_tasks(self.qstarts, self.counts, self.tasks, self.task_count,
                              self.max_reqs, self.layout.config.queries_per_tile, num_reqs=1)
        return self.meta(1)

    def fill(self, lengths, order):
        """A step of len(lengths) requests, each owning fresh pages from `order` (request
        exclusive, first block page-aligned), its last qlen tokens the step's queries."""
        bpp = self.layout.blocks_per_page
        table = torch.zeros_like(self.table, device="cpu")
        qstarts, slots, cursor = [0], [], 0
        for r, length in enumerate(lengths):
            npg = -(-length // self.layout.physical_block_tokens)
            pages, cursor = order[cursor : cursor + npg], cursor + npg
            assert cursor <= len(order)
            blocks = [p * bpp + j for p in pages for j in range(bpp)]
            table[r, : len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
            slots += [blocks[t // 128] * 128 + t % 128 for t in range(length - self.qlen, length)]
            qstarts.append(qstarts[-1] + self.qlen)
        nr, nt = len(lengths), len(slots)
        self.table.copy_(table)
        self.qstarts.zero_()
        self.qstarts[: nr + 1] = torch.tensor(qstarts, dtype=torch.int32)
        self.qstarts[nr + 1 :] = nt
        self.seqs.zero_()
        self.seqs[:nr] = torch.tensor(lengths, dtype=torch.int32)
        self.slots.fill_(-1)
        self.slots[:nt] = torch.tensor(slots, dtype=torch.int64)
        self.counts.copy_(torch.tensor([nr, nt], dtype=torch.int32))
        kernels.prepare_tasks(self.qstarts, self.counts, self.tasks, self.task_count,
                              self.max_reqs, self.layout.config.queries_per_tile, num_reqs=nr)
        return self.meta(nr)


def _c4_lengths():
    """bench.py's c4 draw (seed 1234): 64 lengths log-uniform in [256, 131072]."""
    gen = torch.Generator().manual_seed(1234)
    lo, hi = math.log(256), math.log(131072)
    u = torch.rand(64, generator=gen, dtype=torch.float64)
    return [int(round(math.exp(lo + (hi - lo) * float(x)))) for x in u]


@pytest.mark.parametrize("qlen,max_reqs,tokens,scenarios", [
    (1, 32, 32, {"c3": [32768] * 32, "c5": [262144] * 4}),
    (4, 64, 256, {"c4": None}),
])
def test_graph_captured_at_dummy_lengths_replays_full_size_steps(qlen, max_reqs, tokens,
                                                                 scenarios):
    cfg = OscarConfig(sink_tokens=4, recent_tokens=128, speculative_tokens=3)
    layout = CacheLayout(768, config=cfg)
    gen = torch.Generator().manual_seed(1234)
    print(f"[capture] qlen {qlen}: writing the {POOL_PAGES}-page pool", flush=True)
    k_cache, v_cache, rk, rv = _pool(layout, gen)
    order = (torch.randperm(POOL_PAGES, generator=gen)).tolist()
    columns = POOL_PAGES * layout.blocks_per_page
    buf = _Buffers(layout, max_reqs, tokens, qlen, columns)
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, cfg)
    assert impl.split_policy == "device"
    impl.set_rotations(rk, rv)
    ref = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, cfg, split_policy="reference")
    ref.set_rotations(rk, rv)
    q = torch.randn(tokens, 6, 256, generator=gen).bfloat16().to(DEV)
    k = torch.randn(tokens, 1, 256, generator=gen).bfloat16().to(DEV)
    v = torch.randn(tokens, 1, 256, generator=gen).bfloat16().to(DEV)
    out = torch.zeros(tokens, 6 * 256, dtype=torch.bfloat16, device=DEV)
    cache = (k_cache, v_cache)

    meta = buf.dummy()
    splits, budget = impl.partition_for(meta, tokens)
    print(f"[capture] qlen {qlen}: capturing at dummy lengths (splits {splits}, "
          f"budget {-budget})", flush=True)
    impl.forward(None, q, k, v, cache, meta, out)  # warm-up outside the graph
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        impl.forward(None, q, k, v, cache, meta, out)
    torch.cuda.synchronize()
    # The q rotation as role workgroups of the history launch (opt-in): its own graph.
    qr = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, cfg, q_roles=True)
    qr.set_rotations(rk, rv)
    qr_out = torch.zeros_like(out)
    qr.forward(None, q, k, v, cache, meta, qr_out)
    torch.cuda.synchronize()
    qr_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(qr_graph, stream=stream):
        qr.forward(None, q, k, v, cache, meta, qr_out)
    torch.cuda.synchronize()

    for name, lengths in scenarios.items():
        lengths = lengths or _c4_lengths()
        print(f"[capture] {name}: {len(lengths)} requests, {sum(lengths)} tokens", flush=True)
        meta = buf.fill(lengths, order)
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        got_lse = buf.merged_lse.clone()
        for second in range(2):  # a second replay: nothing left over from the first
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, got) and torch.equal(buf.merged_lse, got_lse), (name, second)
        eager = torch.zeros_like(out)
        impl.forward(None, q, k, v, cache, meta, eager)
        torch.cuda.synchronize()
        assert torch.equal(eager, got), name
        assert torch.equal(buf.merged_lse, got_lse), name
        if kernels.history_pre_supported(meta, meta.layout, 6):
            for _ in range(2):
                qr_out.zero_()
                qr_graph.replay()
                torch.cuda.synchronize()
                qr_got = qr_out.clone()
                qr.forward(None, q, k, v, cache, meta, qr_out)
                torch.cuda.synchronize()
                assert torch.equal(qr_out, qr_got), name
                assert qr.q_sync.tolist() == [0, 0, 0, 0], name
            assert_scaled_close(qr_got[:len(lengths) * qlen].float().cpu().numpy(),
                                got[:len(lengths) * qlen].float().cpu().numpy(),
                                f"{name} q roles", rel=5e-3)
        nt = len(lengths) * qlen
        live = got[:nt].float().view(nt, 6, 256)
        assert torch.isfinite(live).all() and torch.isfinite(got_lse[:nt]).all()
        other = torch.zeros_like(out)
        ref.forward(None, q, k, v, cache, meta, other)
        torch.cuda.synchronize()
        want = other[:nt].float().view(nt, 6, 256).cpu().numpy()
        mine = live.cpu().numpy()
        worst = 0.0
        for r in range(len(lengths)):
            rows = slice(r * qlen, (r + 1) * qlen)
            rel, mx = assert_scaled_close(mine[rows], want[rows], f"{name} request {r}",
                                          rel=5e-3)
            worst = max(worst, rel)
        torch.testing.assert_close(got_lse[:nt], buf.merged_lse[:nt], atol=1e-3, rtol=0)
        print(f"[capture] {name}: replay == eager bits; vs the reference rule worst rel L2 "
              f"{worst:.3g}", flush=True)

"""history_post: the history branch and post-attention of a decode step in ONE launch (no
reference counterpart) against the two launches it replaces, attention_partials(raw=False)
followed by post_attention (the reference order, oscar_ascend/backend.py:205-226).

Bit for bit (output, merged LSE, every byte of the cache after the window store):
  * split counts 1..16 under the reference split rule and under token-bounded splits (the
    split slots a request does not use are neither written nor read);
  * requests with no INT2 history (prefix inside the sink) and padded rows past the token
    count (zero output, LSE -inf, no window write);
  * back-to-back launches with different split counts, and replays of a captured graph: the
    completion counters come back to zero after every launch.
"""

import pytest
import torch

from oscar_new_amd import kernels
from oscar_new_amd.config import OscarConfig, task_capacity
from tests.test_gpu_fused import _case, _views

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pre(c, raw):
    k_cache, v_cache = _views(raw, c.layout)
    hist, win = c.layout.tensor_views((k_cache, v_cache))
    qrot, rp, rl = kernels.pre_attention(c.q, c.k, c.v, hist, win, c.meta, c.layout, 1 / 16,
                                         c.rk.T.contiguous(), c.rv.T.contiguous())
    return hist, win, qrot, rp, rl


def _outputs(n):
    return (torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16),
            torch.full((n, 6), 7.0, device=DEV))


def _step(c, splits, split_tokens, one_launch, raw=None):
    """pre_attention, then the history branch + post-attention in one launch or in two, on a
    copy of the cache; returns (output bits, merged LSE, cache bytes)."""
    n = c.q.shape[0]
    raw = c.raw.clone() if raw is None else raw
    hist, win, qrot, rp, rl = _pre(c, raw)
    out, lse = _outputs(n)
    rv = c.rv.contiguous()
    if one_launch:
        kernels.history_post(qrot, hist, c.meta, c.layout, 1 / 16, splits, rp, rl, rv, c.k, c.v,
                             win, out, lse, split_tokens=split_tokens)
    else:
        hp, hl = kernels.attention_partials(qrot, c.k, c.v, hist, win, c.meta, c.layout, 1 / 16,
                                            splits, False, split_tokens=split_tokens)
        kernels.post_attention(hp, hl, rp, rl, rv, c.k, c.v, win, c.meta, c.layout, out, lse)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu(), lse.cpu(), raw.cpu()


def _same(want, got, label):
    for a, b in zip(want, got):
        assert torch.equal(a, b), label


DECODE = ([3000, 1500, 777], [2999, 1499, 776])


@pytest.mark.parametrize("splits,split_tokens", [(1, 0), (5, 0), (16, 0), (16, 256), (8, 1024)])
def test_one_launch_is_bitwise_the_two_launches(splits, split_tokens):
    c = _case(*DECODE, seed=31)
    print(f"[history_post] splits {splits} split_tokens {split_tokens}", flush=True)
    assert kernels.history_post_supported(c.meta, c.layout, 6, splits)
    _same(_step(c, splits, split_tokens, False), _step(c, splits, split_tokens, True), splits)


def test_no_history_and_padded_rows():
    # Request 0 has no prefix, request 1 a prefix inside the sink (no INT2 history), request 2
    # a long one; three padded rows follow the token count.
    c = _case([1, 65, 2049], [0, 64, 2048], seed=32)
    pad = 3
    c.q = torch.cat([c.q, torch.randn(pad, 6, 256, device=DEV).bfloat16()])
    c.k = torch.cat([c.k, torch.randn(pad, 1, 256, device=DEV).bfloat16()])
    c.v = torch.cat([c.v, torch.randn(pad, 1, 256, device=DEV).bfloat16()])
    n = c.q.shape[0]
    qt = c.layout.config.queries_per_tile
    c.meta.tasks = torch.empty((task_capacity(n, c.meta.max_num_reqs, qt), 2), device=DEV,
                               dtype=torch.int32)  # the grid covers the padded rows too
    kernels.prepare_tasks(c.meta.query_start_loc, c.meta.counts, c.meta.tasks, c.meta.task_count,
                          c.meta.max_num_reqs, qt)
    want = _step(c, 8, 0, False)
    got = _step(c, 8, 0, True)
    _same(want, got, "padded")
    assert torch.count_nonzero(got[0][n - pad:]).item() == 0
    assert torch.isneginf(got[1][n - pad:]).all()


def test_back_to_back_launches_reset_the_counters():
    c = _case(*DECODE, seed=33)
    for splits, split_tokens in ((8, 0), (3, 0), (16, 512), (16, 0), (1, 0)):
        print(f"[history_post] back to back: splits {splits}", flush=True)
        _same(_step(c, splits, split_tokens, False), _step(c, splits, split_tokens, True), splits)


def test_one_launch_replays_in_a_graph():
    # A captured pre_attention + history_post, replayed with new queries on a reset cache,
    # matches the eager two-launch step every time (eager work between the replays).
    c = _case([900, 517, 3000], [899, 516, 2999], seed=34,
              cfg=OscarConfig(sink_tokens=4, recent_tokens=64))
    n = c.q.shape[0]
    raw_graph = c.raw.clone()
    out, lse = _outputs(n)
    rk_t, rv_t, rv = c.rk.T.contiguous(), c.rv.T.contiguous(), c.rv.contiguous()
    k_cache, v_cache = _views(raw_graph, c.layout)
    hist, win = c.layout.tensor_views((k_cache, v_cache))

    def launch():
        qrot, rp, rl = kernels.pre_attention(c.q, c.k, c.v, hist, win, c.meta, c.layout, 1 / 16,
                                             rk_t, rv_t)
        kernels.history_post(qrot, hist, c.meta, c.layout, 1 / 16, 8, rp, rl, rv, c.k, c.v,
                             win, out, lse)

    launch()  # warm-up: library, counters
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=stream):
        launch()
    torch.cuda.synchronize()
    for replay in range(3):
        print(f"[history_post] graph replay {replay}", flush=True)
        c.q.normal_()
        raw_graph.copy_(c.raw)
        graph.replay()
        torch.cuda.synchronize()
        got = (out.view(torch.int16).cpu(), lse.cpu(), raw_graph.cpu())
        _same(_step(c, 8, 0, False), got, replay)
        _ = (c.q * 2).sum().item()  # eager work between replays

"""On-disk layouts beyond the serving default (the reference layout permits them,
oscar_ascend/layout.py:15-28): physical pages of 384 and 1536 tokens and two KV heads (12 query
heads, six per KV head), through every launch of a layer step.

* The fused steps (three launches, and history + post-attention in one where it applies) are
  bit for bit the single-launch order (backend.py:171-226): output, merged LSE and every byte
  of the conv region and both stripes.
* Each KV head's query group against the oracle's dense reference (hybrid_reference: INT2
  history dequantized and inverse-rotated, BF16 sink/recent/current) at the reference test's
  atol 0.035 / rtol 0.04 (tests/test_npu_kernels.py:194), mean-abs <= 2e-3, LSE within 2e-2.
"""

import numpy as np
import pytest
import torch

import oracle as O
from oscar_new_amd import kernels
from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import OscarConfig
from tests._state import (assert_lse_close, assert_scaled_close, bits, make_state, native_views,
                          prepare_prefix)

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, HQ, PAGES = 2, 12, 12
CFG = OscarConfig(sink_tokens=4, recent_tokens=64)  # the window fits a 384-token page


def _qr(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16().to(DEV)


def _case(page, lengths, prefixes, seed):
    torch.manual_seed(seed)
    layout, raw, hist, window, meta, tables = make_state(lengths, prefixes, CFG, pages=PAGES,
                                                         max_reqs=4, page=page, kv_heads=H)
    rk, rv = _qr(seed), _qr(seed + 1)
    ks = [torch.randn(n, H, 256).bfloat16() for n in lengths]
    vs = [torch.randn(n, H, 256).bfloat16() for n in lengths]
    qs = [torch.randn(n - p, HQ, 256).bfloat16() for n, p in zip(lengths, prefixes)]
    prepare_prefix(ks, vs, rk, rv, hist, window, meta, tables, layout, prefixes)
    meta.layout = layout
    meta.num_actual_tokens = sum(q.shape[0] for q in qs)
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, CFG.queries_per_tile)
    cat = lambda xs, ps: torch.cat([x[p:] for x, p in zip(xs, ps)]).to(DEV)  # noqa: E731
    return layout, raw, meta, rk, rv, ks, vs, qs, torch.cat(qs).to(DEV), cat(ks, prefixes), \
        cat(vs, prefixes)


def _step(c, fused, one_launch, splits, layer=False):
    layout, raw0, meta, rk, rv, _, _, _, q, k, v = c
    raw = raw0.clone()
    impl = OscarAttentionImpl.standalone(HQ, 256, 1 / 16, H, CFG, fused=fused,
                                         one_launch_post=one_launch, layer_step=layer)
    impl.set_rotations(rk, rv)
    impl.partition_for = lambda meta, tokens=None: (splits, 0)
    n = q.shape[0]
    meta.merged_lse = torch.full((n, HQ), 7.0, device=DEV)
    out = torch.full((n, HQ * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    impl.forward(None, q, k, v, native_views(raw, layout, PAGES), meta, out)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu(), meta.merged_lse.cpu(), raw.cpu()


@pytest.mark.parametrize("page", [384, 1536])
@pytest.mark.parametrize("lengths,prefixes,splits", [
    ([1300, 700], [1299, 699], 8),  # decode: history + post in one launch on the fused1 form
    ([900, 517], [896, 516], 4),  # MTP, ragged
])
def test_other_pages_and_two_kv_heads(page, lengths, prefixes, splits):
    print(f"[layouts] page {page} lengths {lengths} splits {splits}", flush=True)
    c = _case(page, lengths, prefixes, seed=51)
    want = _step(c, False, False, splits)
    for fused, one in ((True, False), (True, True)):
        got = _step(c, fused, one, splits)
        for a, b in zip(want, got):
            assert torch.equal(a, b), (fused, one)
    # The one-launch step (decode here; MTP with 6 query heads per KV head falls back): same
    # cache bytes, output and LSE within the scale-aware bounds.
    layer = _step(c, True, False, splits, layer=True)
    assert torch.equal(layer[2], want[2])
    assert_scaled_close(layer[0].view(torch.bfloat16).float().numpy(),
                        want[0].view(torch.bfloat16).float().numpy(), "layer step")
    assert_lse_close(layer[1].numpy(), want[1].numpy(), "layer step LSE", atol=1e-3)
    _, _, _, rk, rv, ks, vs, qs, q, _, _ = c
    out = want[0].view(torch.bfloat16).float().numpy().reshape(q.shape[0], HQ, 256)
    lse = want[1].numpy()
    start = 0
    for qi, ki, vi, p in zip(qs, ks, vs, prefixes):
        rows = slice(start, start + qi.shape[0])
        start += qi.shape[0]
        for h in range(H):
            heads = slice(6 * h, 6 * h + 6)
            o, l = O.hybrid_reference(bits(qi[:, heads]), bits(ki[:, h : h + 1]),
                                      bits(vi[:, h : h + 1]), p, bits(rk), bits(rv), CFG)
            got = out[rows, heads]
            np.testing.assert_allclose(got, o, atol=0.035, rtol=0.04)
            assert np.abs(got - o).mean() <= 2e-3
            np.testing.assert_allclose(lse[rows, heads], l, atol=2e-2, rtol=0)

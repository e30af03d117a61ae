"""The metadata builder (reference metadata.py:36-174) on MI355X.

* `OscarMetadataBuilder.build` from a fake vLLM CommonAttentionMetadata (device tensors,
  like vLLM's) fills its fixed buffers and the task table, and drives a fused step to the
  same bits as the hand-built metadata;
* a dummy (graph-padding) build leaves the cache untouched and writes zero rows, as the
  reference's dummy path does.
"""

from types import SimpleNamespace

import pytest
import torch

from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import OscarConfig
from oscar_new_amd.metadata import OscarMetadataBuilder
from tests.test_gpu_fused import _case, _forward, _views

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _common(c, max_seq_len=True):
    """A fake vLLM CommonAttentionMetadata of the case (device tensors, unpadded)."""
    nr = c.meta.num_reqs
    nt = c.q.shape[0]
    return SimpleNamespace(
        num_reqs=nr, num_actual_tokens=nt, max_query_len=c.meta.max_query_len,
        query_start_loc=c.meta.query_start_loc[: nr + 1].clone(),
        seq_lens=c.meta.seq_lens[:nr].clone(),
        seq_lens_cpu=c.meta.seq_lens[:nr].cpu(),
        block_table_tensor=c.meta.block_tables[:nr].clone(),
        slot_mapping=c.meta.slot_mapping[:nt].clone(),
        max_seq_len=int(c.meta.seq_lens.max().item()) if max_seq_len else None,
        causal=True,
    )


def test_builder_metadata_drives_the_same_step():
    c = _case([1804, 2601, 300], [1800, 2600, 299], seed=9)
    want = _forward(c, "fused", 8)
    builder = OscarMetadataBuilder(c.layout, max_num_seqs=7, max_num_batched_tokens=64,
                                   max_model_len=16384, device=DEV)
    meta = builder.build(_common(c))
    torch.cuda.synchronize()
    assert int(meta.task_count.item()) == int(c.meta.task_count.item())
    count = int(meta.task_count.item())
    assert torch.equal(meta.tasks[:count], c.meta.tasks[:count])
    assert meta.total_seq_len == sum([1804, 2601, 300])
    n = c.q.shape[0]
    raw = c.raw.clone()
    k_cache, v_cache = _views(raw, c.layout)
    impl = OscarAttentionImpl(6, 256, 1 / 16, 1, c.layout.config)
    impl.initialize_layer(c.rk, c.rv)
    impl.partition_for = lambda m: (8, 0)
    meta.merged_lse = torch.full((n, 6), 7.0, device=DEV)
    out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), meta, out)
    torch.cuda.synchronize()
    got = (out.view(torch.int16).cpu(), meta.merged_lse.cpu(), raw.cpu())
    for a, b in zip(want, got):
        assert torch.equal(a, b)


def test_builder_dummy_run_touches_nothing():
    c = _case([900, 517], [896, 516], seed=10, cfg=OscarConfig(sink_tokens=4, recent_tokens=64))
    builder = OscarMetadataBuilder(c.layout, max_num_seqs=3, max_num_batched_tokens=16,
                                   max_model_len=16384, device=DEV)
    meta = builder.build(_common(c), dummy=True)
    torch.cuda.synchronize()
    assert int(meta.task_count.item()) == 0
    n = c.q.shape[0]
    before = c.raw.clone()
    k_cache, v_cache = _views(c.raw, c.layout)
    impl = OscarAttentionImpl(6, 256, 1 / 16, 1, c.layout.config)
    impl.initialize_layer(c.rk, c.rv)
    meta.merged_lse = torch.empty((n, 6), device=DEV)
    out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    impl.forward(None, c.q, c.k, c.v, (k_cache, v_cache), meta, out)
    torch.cuda.synchronize()
    assert torch.equal(c.raw, before)
    assert torch.count_nonzero(out).item() == 0
    assert torch.isneginf(meta.merged_lse).all()

"""vLLM's construction path on MI355X (reference metadata.py:36-174, backend.py:67-227,
plugin.py:88-130), on the stand-ins of tests/_vllm_standin.py:

* the Attention layer is built through the hooked layer class (the platform hook routes it
  to OSCAR; the implementation gets vLLM's positional arguments under the engine config),
  its rotations come from artefact files named by the environment at weight-loading time;
* the metadata builder is built with ``(kv_cache_spec, layer_names, vllm_config, device)``
  and fed a fake CommonAttentionMetadata of device tensors with ``build(0, common)``;
* one fused layer step through ``layer.impl.forward`` gives the same bits as the hand-built
  metadata's step; a capture build (``build_for_cudagraph_capture``) touches nothing.
"""

from types import SimpleNamespace

import pytest
import torch

from oscar_new_amd import plugin, rotations
from oscar_new_amd.config import OscarConfig
from oscar_new_amd.metadata import OscarMetadataBuilder
from tests import _vllm_standin as V
from tests.test_gpu_fused import _case, _forward, _views

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAME = "model.layers.3.self_attn.attn"


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
        causal=True, attn_state=SimpleNamespace(name="DecodeOnly"),
    )


def _engine(c, monkeypatch, tmp_path, max_num_seqs=7, max_num_batched_tokens=64):
    """(layer, builder) constructed exactly as vLLM constructs them."""
    cfg = c.layout.config
    for env, value in (("VLLM_OSCAR_SINK_TOKENS", cfg.sink_tokens),
                       ("VLLM_OSCAR_RECENT_TOKENS", cfg.recent_tokens),
                       (plugin.ENV_ENABLED, 1)):
        monkeypatch.setenv(env, str(value))
    for name, r in (("K", c.rk), ("V", c.rv)):
        path = tmp_path / f"{name}.pt"
        rotations.save_rotations(path, {3: r.float().cpu()})
        monkeypatch.setenv(f"VLLM_OSCAR_{name}_ROTATION_PATH", str(path))
    platform = V.make_platform()
    attention = V.make_attention(platform)
    plugin.register(platform, attention)
    config = V.make_vllm_config(num_speculative_tokens=cfg.speculative_tokens,
                                max_num_seqs=max_num_seqs,
                                max_num_batched_tokens=max_num_batched_tokens)
    with V.current_vllm_config(config):
        layer = attention(6, 256, 1 / 16, 1, prefix=NAME).to(DEV)
    config.compilation_config.static_forward_context[NAME] = layer
    layer.process_weights_after_loading(torch.bfloat16)
    builder = OscarMetadataBuilder(V.kv_cache_spec(c.layout.physical_block_tokens), [NAME],
                                   config, DEV)
    got, want = builder.layout, c.layout
    assert (got.physical_block_tokens, got.kv_heads, got.config.sink_tokens,
            got.config.ring_tokens) == (want.physical_block_tokens, want.kv_heads,
                                        want.config.sink_tokens, want.config.ring_tokens)
    return layer, builder


def test_vllm_constructed_step_matches_hand_built_metadata(monkeypatch, tmp_path):
    c = _case([1804, 2601, 300], [1800, 2600, 299], seed=9)
    want = _forward(c, "fused", 8)
    layer, builder = _engine(c, monkeypatch, tmp_path)
    assert torch.equal(layer.impl.rk, c.rk) and torch.equal(layer.impl.rv, c.rv)
    meta = builder.build(0, _common(c))
    torch.cuda.synchronize()
    assert int(meta.task_count.item()) == int(c.meta.task_count.item())
    count = int(meta.task_count.item())
    assert torch.equal(meta.tasks[:count], c.meta.tasks[:count])
    assert meta.total_seq_len == sum([1804, 2601, 300])
    n = c.q.shape[0]
    raw = c.raw.clone()
    kv_cache = _views(raw, c.layout)
    layer.impl.partition_for = lambda m, tokens=None: (8, 0)
    meta.merged_lse = torch.full((n, 6), 7.0, device=DEV)
    out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    layer.impl.forward(layer, c.q.view(n, -1), c.k.view(n, -1), c.v.view(n, -1), kv_cache, meta,
                       out)
    torch.cuda.synchronize()
    got = (out.view(torch.int16).cpu(), meta.merged_lse.cpu(), raw.cpu())
    for a, b in zip(want, got):
        assert torch.equal(a, b)


def test_capture_build_touches_nothing(monkeypatch, tmp_path):
    c = _case([900, 517], [896, 516], seed=10, cfg=OscarConfig(sink_tokens=4, recent_tokens=64))
    layer, builder = _engine(c, monkeypatch, tmp_path, max_num_seqs=3, max_num_batched_tokens=16)
    meta = builder.build_for_cudagraph_capture(_common(c))
    torch.cuda.synchronize()
    assert meta.is_dummy and int(meta.task_count.item()) == 0
    n = c.q.shape[0]
    before = c.raw.clone()
    kv_cache = _views(c.raw, c.layout)
    meta.merged_lse = torch.empty((n, 6), device=DEV)
    out = torch.full((n, 6 * 256), 3.0, device=DEV, dtype=torch.bfloat16)
    layer.impl.forward(layer, c.q, c.k, c.v, kv_cache, meta, out)
    torch.cuda.synchronize()
    assert torch.equal(c.raw, before)
    assert torch.count_nonzero(out).item() == 0
    assert torch.isneginf(meta.merged_lse).all()

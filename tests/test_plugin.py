"""vLLM glue without vLLM (reference tests/test_graph_startup.py:19-168 and plugin.py:13-85):
plugin routing on a stand-in ROCm platform class, the backend class, the vLLM config checks
of backend.py:41-64, and the builder's initial-prefill flag from the scheduler's host state.
"""

from types import SimpleNamespace

import pytest
import torch

from oscar_new_amd import metadata, plugin
from oscar_new_amd.backend import OscarAttentionBackend, OscarAttentionImpl, validate_vllm_config
from oscar_new_amd.layout import CacheLayout


def _selector(**kw):
    base = dict(attn_type="decoder", use_mla=False, use_sparse=False, use_non_causal=False,
                head_size=256)
    base.update(kw)
    return SimpleNamespace(**base)


def _platform():
    class Platform:
        calls = []

        @classmethod
        def get_attn_backend_cls(cls, selected_backend, attn_selector_config, num_heads=None):
            cls.calls.append(selected_backend)
            return "native"

    return Platform


def test_routing_rule_and_draft_layers():
    assert plugin.should_route(_selector())
    for kw in ({"attn_type": "encoder"}, {"use_mla": True}, {"use_sparse": True},
               {"use_non_causal": True}):
        assert not plugin.should_route(_selector(**kw))
    assert plugin.is_draft_layer("model.mtp.layers.0.self_attn")
    assert not plugin.is_draft_layer("model.layers.3.self_attn")


def test_register_is_gated_idempotent_and_routes(monkeypatch):
    platform = _platform()
    monkeypatch.delenv(plugin.ENV_ENABLED, raising=False)
    assert not plugin.register(platform)
    assert platform.get_attn_backend_cls(None, _selector()) == "native"
    monkeypatch.setenv(plugin.ENV_ENABLED, "1")
    assert plugin.register(platform)
    wrapped = platform.get_attn_backend_cls
    assert plugin.register(platform) and platform.get_attn_backend_cls == wrapped  # once
    assert platform.get_attn_backend_cls(None, _selector()) == plugin.BACKEND
    assert platform.get_attn_backend_cls(None, _selector(head_size=0)) == plugin.BACKEND
    assert platform.get_attn_backend_cls("x", _selector(use_mla=True)) == "native"
    assert platform.calls == [None, "x"]  # native before registration, then the MLA layer
    with pytest.raises(ValueError, match="D256"):
        platform.get_attn_backend_cls(None, _selector(head_size=128))
    with pytest.raises(ValueError, match="has_sink"):
        platform.get_attn_backend_cls(None, _selector(has_sink=True))


def test_backend_class_wiring():
    assert OscarAttentionBackend.get_name() == "CUSTOM"
    assert OscarAttentionBackend.get_impl_cls() is OscarAttentionImpl
    assert OscarAttentionBackend.get_builder_cls() is metadata.OscarMetadataBuilder
    assert OscarAttentionBackend.get_kv_cache_shape(10, 768, 1, 256) == (2, 10, 768, 1, 256)
    for op in (OscarAttentionBackend.copy_blocks, OscarAttentionBackend.swap_blocks):
        with pytest.raises(NotImplementedError):
            op()
    assert plugin.BACKEND == (f"{OscarAttentionBackend.__module__}."
                              f"{OscarAttentionBackend.__name__}")


def _config(**over):
    cfg = SimpleNamespace(
        cache_config=SimpleNamespace(enable_prefix_caching=False, cache_dtype="auto"),
        model_config=SimpleNamespace(dtype=torch.bfloat16,
                                     hf_text_config=SimpleNamespace(head_dim=256)),
        kv_transfer_config=None,
        parallel_config=SimpleNamespace(decode_context_parallel_size=1,
                                        prefill_context_parallel_size=1, enable_dbo=False),
    )
    for path, value in over.items():
        obj = cfg
        *head, last = path.split(".")
        for name in head:
            obj = getattr(obj, name)
        setattr(obj, last, value)
    return cfg


@pytest.mark.parametrize("path,value,match", [
    ("cache_config.enable_prefix_caching", True, "prefix-caching"),
    ("cache_config.cache_dtype", "fp8", "kv-cache-dtype"),
    ("model_config.dtype", torch.float16, "BF16"),
    ("kv_transfer_config", object(), "KV transfer"),
    ("parallel_config.decode_context_parallel_size", 2, "PCP=DCP=1"),
    ("parallel_config.enable_dbo", True, "DBO"),
    ("model_config.hf_text_config.head_dim", 128, "D256"),
])
def test_vllm_config_checks(path, value, match):
    validate_vllm_config(_config())
    with pytest.raises(ValueError, match=match):
        validate_vllm_config(_config(**{path: value}))


def test_builder_marks_initial_prefill_from_host_state(monkeypatch):
    # The device task kernel is replaced (no GPU here); every other step of build runs.
    monkeypatch.setattr(metadata.kernels, "prepare_tasks", lambda *a, **k: None)
    builder = metadata.OscarMetadataBuilder(CacheLayout(768), max_num_seqs=3,
                                            max_num_batched_tokens=32, max_model_len=4096,
                                            device="cpu")
    qsl = torch.tensor([0, 5, 12], dtype=torch.int32)
    common = SimpleNamespace(
        num_reqs=2, num_actual_tokens=12, max_query_len=7, query_start_loc=qsl,
        query_start_loc_cpu=qsl.clone(), seq_lens=torch.tensor([5, 7], dtype=torch.int32),
        seq_lens_cpu=torch.tensor([5, 7], dtype=torch.int32),
        block_table_tensor=torch.zeros((2, 8), dtype=torch.int32),
        slot_mapping=torch.arange(12, dtype=torch.int64), max_seq_len=7, causal=True,
        attn_state=SimpleNamespace(name="PrefillNoCache"))
    meta = builder.build(common)
    assert meta.initial_prefill and meta.query_ends == [5, 12] and meta.total_seq_len == 12
    assert not builder.build(common, dummy=True).initial_prefill
    common.attn_state = SimpleNamespace(name="DecodeOnly")
    meta = builder.build(common)
    assert not meta.initial_prefill and meta.query_ends is None
    common.attn_state = SimpleNamespace(name="PrefillNoCache")
    common.query_start_loc_cpu = None
    with pytest.raises(ValueError, match="CPU"):
        builder.build(common)

"""vLLM glue without vLLM (reference tests/test_graph_startup.py:19-168, plugin.py:13-130,
backend.py:13-117, metadata.py:36-174), on stand-ins built as vLLM builds them:

* the platform hook routes full decoder attention (and rejects what it cannot serve);
* Attention layers constructed through the hooked class get an ``OscarAttentionImpl`` built
  with vLLM's positional arguments under the current engine config, except MTP draft layers,
  which keep the native backend; weight loading installs the layer's rotations from the
  artefacts the environment names;
* the metadata builder is constructed with ``(kv_cache_spec, layer_names, vllm_config,
  device)`` and builds with ``(common_prefix_len, common_attn_metadata)``; a capture build is
  a dummy build.
"""

import importlib
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

import oscar_new_amd
from oscar_new_amd import metadata, plugin, rotations
from oscar_new_amd.backend import OscarAttentionBackend, OscarAttentionImpl, validate_vllm_config
from oscar_new_amd.layout import CacheLayout
from tests import _vllm_standin as V


def _selector(**kw):
    base = dict(attn_type="decoder", use_mla=False, use_sparse=False, use_non_causal=False,
                head_size=256)
    base.update(kw)
    return SimpleNamespace(**base)


def test_routing_rule_and_draft_layers():
    assert plugin.should_route(_selector())
    for kw in ({"attn_type": "encoder"}, {"use_mla": True}, {"use_sparse": True},
               {"use_non_causal": True}):
        assert not plugin.should_route(_selector(**kw))
    assert plugin.is_draft_layer("model.mtp.layers.0.self_attn")
    assert not plugin.is_draft_layer("model.layers.3.self_attn")


def test_register_is_gated_idempotent_and_routes(monkeypatch):
    platform = V.make_platform()
    monkeypatch.delenv(plugin.ENV_ENABLED, raising=False)
    assert not plugin.register(platform)
    assert platform.get_attn_backend_cls(None, _selector()) == V.NATIVE_BACKEND
    monkeypatch.setenv(plugin.ENV_ENABLED, "1")
    assert plugin.register(platform)
    wrapped = platform.get_attn_backend_cls
    assert plugin.register(platform) and platform.get_attn_backend_cls == wrapped  # once
    assert platform.get_attn_backend_cls(None, _selector()) == plugin.BACKEND
    assert platform.get_attn_backend_cls(None, _selector(head_size=0)) == plugin.BACKEND
    assert platform.get_attn_backend_cls("x", _selector(use_mla=True)) == V.NATIVE_BACKEND
    # The platform's own selector answers every call (its answer is kept for draft layers):
    # before registration, the two routed layers, then the MLA layer.
    assert platform.calls == [None, None, None, "x"]
    assert plugin.native_backend() is V.NativeBackend
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


@pytest.mark.parametrize("path,value,match", [
    ("cache_config.enable_prefix_caching", True, "prefix-caching"),
    ("cache_config.cache_dtype", "fp8", "kv-cache-dtype"),
    ("model_config.dtype", torch.float16, "bf16"),
    ("kv_transfer_config", object(), "KV transfer"),
    ("parallel_config.decode_context_parallel_size", 2, "PCP=DCP=1"),
    ("parallel_config.enable_dbo", True, "DBO"),
    ("quant_config", SimpleNamespace(enable_c8_quant=True), "C8"),
    ("model_config.hf_text_config.head_dim", 128, "D256"),
])
def test_vllm_config_checks(path, value, match):
    validate_vllm_config(V.make_vllm_config())
    with pytest.raises(ValueError, match=match):
        validate_vllm_config(V.make_vllm_config(**{path: value}))


def test_v2_runner_is_rejected(monkeypatch):
    monkeypatch.setenv("VLLM_USE_V2_MODEL_RUNNER", "1")
    with pytest.raises(ValueError, match="v1 model runner"):
        validate_vllm_config(V.make_vllm_config())


def _impl_args(**over):
    """vLLM's positional implementation arguments (reference backend.py:68-81)."""
    args = dict(num_heads=6, head_size=256, scale=1 / 16, num_kv_heads=1, alibi_slopes=None,
                sliding_window=None, kv_cache_dtype="auto", logits_soft_cap=None,
                attn_type="decoder", kv_sharing_target_layer_name=None)
    args.update(over)
    return list(args.values())


def test_impl_constructed_with_vllm_arguments_under_the_engine_config():
    with V.current_vllm_config(V.make_vllm_config(num_speculative_tokens=2)):
        impl = OscarAttentionImpl(*_impl_args())
    assert impl.cfg.speculative_tokens == 2 and impl.cfg.ring_tokens == impl.cfg.recent_tokens + 3
    with V.current_vllm_config(V.make_vllm_config(num_speculative_tokens=0)):
        impl = OscarAttentionImpl(*_impl_args())
    # No MTP: ring = R + 1 (the reference's 257 with the default R = 256).
    assert impl.cfg.speculative_tokens == 0 and impl.cfg.ring_tokens == impl.cfg.recent_tokens + 1
    with V.current_vllm_config(V.make_vllm_config(**{"cache_config.enable_prefix_caching": True})):
        with pytest.raises(ValueError, match="prefix-caching"):
            OscarAttentionImpl(*_impl_args())


@pytest.mark.parametrize("over,kwargs,match", [
    ({"alibi_slopes": torch.ones(6)}, {}, "ALiBi"),
    ({"sliding_window": 4096}, {}, "sliding-window"),
    ({"logits_soft_cap": 30.0}, {}, "soft-capping"),
    ({"kv_sharing_target_layer_name": "model.layers.1.self_attn.attn"}, {}, "KV sharing"),
    ({}, {"sinks": torch.zeros(6)}, "sinks"),
    ({"attn_type": "encoder"}, {}, "FULL decoder"),
    ({"head_size": 128}, {}, "head size 256"),
    ({"num_heads": 5, "num_kv_heads": 2}, {}, "multiple"),
])
def test_impl_rejects_what_it_cannot_serve(over, kwargs, match):
    with V.current_vllm_config(V.make_vllm_config()):
        with pytest.raises(ValueError, match=match):
            OscarAttentionImpl(*_impl_args(**over), **kwargs)


def test_forward_rejects_fused_output_quantization():
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1)
    out = torch.zeros(2, 6 * 256)
    with pytest.raises(ValueError, match="output quantization"):
        impl.forward(None, out, None, None, None, object(), out, output_scale=torch.ones(1))
    assert impl.forward(None, out, None, None, None, None, out + 1).eq(0).all()


def _rotation_files(tmp_path, layers):
    g = torch.Generator().manual_seed(7)
    paths = []
    for name in ("k", "v"):
        mats = {i: torch.linalg.qr(torch.randn(256, 256, generator=g))[0] for i in layers}
        path = tmp_path / f"{name}.pt"
        rotations.save_rotations(path, mats)
        paths.append((path, mats))
    return paths


def test_attention_hooks_route_target_layers_keep_drafts_native_and_load_rotations(
        monkeypatch, tmp_path):
    (kpath, kmats), (vpath, vmats) = _rotation_files(tmp_path, [0, 3])
    monkeypatch.setenv(plugin.ENV_ENABLED, "1")
    monkeypatch.setenv("VLLM_OSCAR_K_ROTATION_PATH", str(kpath))
    monkeypatch.setenv("VLLM_OSCAR_V_ROTATION_PATH", str(vpath))
    platform = V.make_platform()
    attention = V.make_attention(platform)
    assert plugin.register(platform, attention)
    assert attention._oscar_amd_hooked
    with V.current_vllm_config(V.make_vllm_config()):
        target = attention(6, 256, 1 / 16, 1, prefix="model.layers.3.self_attn.attn")
        draft = attention(6, 256, 1 / 16, 1, prefix="model.mtp.layers.0.self_attn.attn")
        chosen = attention(6, 256, 1 / 16, 1, prefix="model.mtp.layers.1.self_attn.attn",
                           attn_backend=OscarAttentionBackend)
    assert isinstance(target.impl, OscarAttentionImpl)
    assert isinstance(draft.impl, V.NativeImpl) and draft.attn_backend is V.NativeBackend
    assert isinstance(chosen.impl, OscarAttentionImpl)  # an explicit backend is kept
    assert target.impl.rk is None
    target.process_weights_after_loading(torch.bfloat16)
    draft.process_weights_after_loading(torch.bfloat16)
    assert target.loaded and draft.loaded
    assert target.impl.rk.dtype == torch.bfloat16 and target.impl.rk.device.type == "cpu"
    torch.testing.assert_close(target.impl.rk.float(), kmats[3].bfloat16().float())
    torch.testing.assert_close(target.impl.rv.float(), vmats[3].bfloat16().float())
    torch.testing.assert_close(target.impl.rk_t.float(), kmats[3].bfloat16().float().T)
    # A layer whose index the artefact lacks fails at load time, naming the layer.
    with V.current_vllm_config(V.make_vllm_config()):
        other = attention(6, 256, 1 / 16, 1, prefix="model.layers.5.self_attn.attn")
    with pytest.raises(ValueError, match="layer 5"):
        other.process_weights_after_loading(torch.bfloat16)


@pytest.mark.parametrize("draft_first", [False, True])
def test_draft_layers_stay_native_under_a_cached_selector(monkeypatch, draft_first):
    """vLLM caches the selector's answer per argument tuple and draft and target layers ask
    with the same arguments: whichever is built first must not decide the other's backend."""
    monkeypatch.setenv(plugin.ENV_ENABLED, "1")
    monkeypatch.setattr(plugin, "_native_paths", {})
    platform = V.make_platform()
    attention = V.make_attention(platform)
    assert plugin.register(platform, attention)
    layers = {}
    order = ["draft", "target", "draft2"] if draft_first else ["target", "draft", "draft2"]
    prefixes = {"draft": "model.mtp.layers.0.self_attn.attn",
                "draft2": "model.mtp.layers.1.self_attn.attn",
                "target": "model.layers.3.self_attn.attn"}
    with V.current_vllm_config(V.make_vllm_config()):
        for name in order:
            layers[name] = attention(6, 256, 1 / 16, 1, prefix=prefixes[name])
        late_target = attention(6, 256, 1 / 16, 1, prefix="model.layers.7.self_attn.attn")
    for name in ("draft", "draft2"):
        assert layers[name].attn_backend is V.NativeBackend
        assert isinstance(layers[name].impl, V.NativeImpl)
    for layer in (layers["target"], late_target):
        assert layer.attn_backend is OscarAttentionBackend
        assert isinstance(layer.impl, OscarAttentionImpl)


def _builder(config=None, layers=("model.layers.3.self_attn.attn",)):
    config = config or V.make_vllm_config()
    with V.current_vllm_config(config):
        for name in layers:
            config.compilation_config.static_forward_context[name] = SimpleNamespace(
                impl=OscarAttentionImpl(*_impl_args()))
    return metadata.OscarMetadataBuilder(V.kv_cache_spec(), list(layers), config, "cpu")


def _common(**over):
    qsl = torch.tensor([0, 5, 12], dtype=torch.int32)
    base = dict(num_reqs=2, num_actual_tokens=12, max_query_len=7, query_start_loc=qsl,
                query_start_loc_cpu=qsl.clone(), seq_lens=torch.tensor([5, 7], dtype=torch.int32),
                seq_lens_cpu=torch.tensor([5, 7], dtype=torch.int32),
                block_table_tensor=torch.zeros((2, 8), dtype=torch.int32),
                slot_mapping=torch.arange(12, dtype=torch.int64), max_seq_len=7, causal=True,
                attn_state=SimpleNamespace(name="PrefillNoCache"))
    base.update(over)
    return SimpleNamespace(**base)


def test_builder_constructed_as_vllm_does(monkeypatch):
    monkeypatch.setattr(metadata.kernels, "prepare_tasks", lambda *a, **k: None)
    builder = _builder(V.make_vllm_config(num_speculative_tokens=3, max_num_seqs=7,
                                          max_num_batched_tokens=64, max_model_len=16384))
    assert builder.layout == CacheLayout(768, 1, config=builder.layout.config)
    assert builder.layout.config.speculative_tokens == 3
    assert builder.reorder_batch_threshold == 4
    assert builder.max_reqs == 8 and builder.max_tokens == 64 + 7 * 8
    assert builder.table.shape == (8, 16384 // 128 + 6 + 1)
    assert builder.reorder_batch(None, None) is False
    assert str(getattr(builder.get_cudagraph_support(None, None), "name",
                       builder.get_cudagraph_support(None, None))) == "UNIFORM_BATCH"
    config = V.make_vllm_config()
    config.compilation_config.static_forward_context["model.layers.1.self_attn.attn"] = \
        SimpleNamespace(impl=V.NativeImpl())
    with pytest.raises(TypeError, match="model.layers.1"):
        metadata.OscarMetadataBuilder(V.kv_cache_spec(), ["model.layers.1.self_attn.attn"],
                                      config, "cpu")


def test_builder_build_and_capture_build(monkeypatch):
    calls = []
    monkeypatch.setattr(metadata.kernels, "prepare_tasks",
                        lambda *a, **k: calls.append(k["num_reqs"]))
    builder = _builder()
    meta = builder.build(0, _common())
    assert meta.initial_prefill and meta.query_ends == [5, 12] and meta.total_seq_len == 12
    assert meta.attn_state.name == "PrefillNoCache" and meta.causal and not meta.is_dummy
    assert builder.counts.tolist() == [2, 12] and builder.qstarts[:3].tolist() == [0, 5, 12]
    assert builder.slots[:12].tolist() == list(range(12))
    capture = builder.build_for_cudagraph_capture(_common())
    assert capture.is_dummy and not capture.initial_prefill and capture.attn_state == "DecodeOnly"
    assert builder.counts.tolist() == [0, 0] and calls == [2, 1]
    assert not metadata.in_dummy_run()
    meta = builder.build(0, _common(attn_state=SimpleNamespace(name="DecodeOnly")))
    assert not meta.initial_prefill and meta.query_ends is None
    with pytest.raises(ValueError, match="CPU"):
        builder.build(0, _common(query_start_loc_cpu=None))
    with pytest.raises(ValueError, match="prefix"):
        builder.build(16, _common())
    with pytest.raises(ValueError, match="causal"):
        builder.build(0, _common(causal=False))
    with pytest.raises(ValueError, match="exceeds"):
        builder.build(0, _common(num_actual_tokens=10_000))


def test_plugin_entry_point_resolves_to_register():
    """vLLM finds general plugins through the ``vllm.general_plugins`` entry-point group
    (reference pyproject.toml:15-16); the package declares ``register`` there."""
    import tomli

    project = tomli.loads((Path(__file__).resolve().parents[1] / "pyproject.toml").read_text())
    entry = project["project"]["entry-points"]["vllm.general_plugins"]["oscar_new_amd"]
    module, _, attr = entry.partition(":")
    target = getattr(importlib.import_module(module), attr)
    assert target is plugin.register
    assert project["project"]["version"] == oscar_new_amd.__version__

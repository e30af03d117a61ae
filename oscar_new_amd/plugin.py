"""vLLM general plugin for ROCm: routes full decoder attention to the OSCAR backend.

Reference: oscar_ascend/plugin.py:13-130, on vLLM's ROCm platform instead of the NPU one.
Two hooks, both installed once and only when ``OSCAR_AMD_ENABLED=1``:

* the platform's backend selector (``get_attn_backend_cls``) returns the OSCAR backend for
  causal, non-MLA, non-sparse decoder attention (plugin.py:13-85), rejecting the selector
  options the INT2 layout cannot serve;
* vLLM's ``Attention`` layer class: an MTP draft layer keeps the platform's native backend
  (its cache and rotations are separate; plugin.py:106-114), and once a routed layer's
  weights are loaded its implementation loads the layer's rotations (plugin.py:116-125).

vLLM caches backend selection per argument tuple, and draft and target layers ask with the
same arguments, so the selector's answer must not depend on which layer asks. The draft layer
therefore gets its backend class bound explicitly, as the reference binds
``AscendAttentionBackend`` (plugin.py:110-113): the class the platform's own selector chose
for the same arguments. The hooked selector records that native answer on every call; a draft
layer built before any selection asks the platform's unhooked selector directly, through the
selector configuration the layer would have built, without entering vLLM's cache.

The platform and Attention classes are looked up lazily or passed in, so both hooks are
tested against stand-ins without vLLM.
"""

from __future__ import annotations

import functools
import importlib
import inspect
import logging
import os
import sys

LOG = logging.getLogger(__name__)
BACKEND = "oscar_new_amd.backend.OscarAttentionBackend"
ENV_ENABLED = "OSCAR_AMD_ENABLED"
UNSUPPORTED_OPTIONS = ("has_sink", "use_mm_prefix", "use_per_head_quant_scales",
                       "use_kv_connector")
# Where vLLM defines its Attention layer class (newest layout first).
ATTENTION_MODULES = ("vllm.model_executor.layers.attention.attention", "vllm.attention.layer")

_registered_on = set()
# Native backend class path the platform's selector gave, per attention type, and the
# platform's unhooked selector (filled by ``register``).
_native_paths = {}
_native_selector = []


def should_route(selector):
    """Reference plugin.py:13-20: vision/encoder, MLA, sparse and non-causal stay native."""
    return (selector.attn_type == "decoder" and not selector.use_mla
            and not selector.use_sparse and not selector.use_non_causal)


def is_draft_layer(prefix):
    """Reference plugin.py:23-24: an MTP draft layer's module path contains ``mtp``."""
    return "mtp" in prefix.split(".")


def _resolve(path):
    """A backend class from its qualified name (vLLM's ``resolve_obj_by_qualname``)."""
    if not isinstance(path, str):
        return path
    module, _, name = path.rpartition(".")
    return getattr(importlib.import_module(module), name)


def native_backend(attn_type="decoder", selector=None):
    """The platform's native backend class for a draft layer: the answer its own selector
    gave for these arguments (recorded by the hooked selector), or, before any selection,
    the unhooked selector asked directly with ``selector``. None when neither is at hand."""
    path = _native_paths.get(attn_type)
    if path is None and selector is not None and _native_selector:
        platform_cls, original = _native_selector[-1]
        path = original(platform_cls, None, selector)
        _native_paths[attn_type] = path
    return None if path is None else _resolve(path)


def _draft_selector(arguments):
    """The selector configuration a draft layer would ask with, built as vLLM's Attention
    builds it: head size and attention type from the constructor's arguments, dtype, KV cache
    dtype and block size from the engine configuration being built."""
    from types import SimpleNamespace

    model = cache = None
    try:
        from vllm.config import get_current_vllm_config

        config = get_current_vllm_config()
        model = getattr(config, "model_config", None)
        cache = getattr(config, "cache_config", None)
    except Exception:  # vLLM absent or no configuration being built
        pass
    return SimpleNamespace(
        attn_type=arguments.get("attn_type", "decoder") or "decoder",
        head_size=arguments.get("head_size", 0),
        dtype=getattr(model, "dtype", None),
        kv_cache_dtype=getattr(cache, "cache_dtype", "auto"),
        block_size=getattr(cache, "block_size", None),
        use_mla=False, has_sink=False, use_sparse=False, use_non_causal=False,
        use_mm_prefix=False, use_per_head_quant_scales=False, use_kv_connector=False)


def backend_for(selector):
    """The backend class path for a routed selector (plugin.py:63-78 checks)."""
    for name in UNSUPPORTED_OPTIONS:
        if getattr(selector, name, False):
            raise ValueError(f"OSCAR cannot serve a layer with selector option {name}")
    # The runner asks once with head_size 0 before the model exists; layers check D256 again.
    if selector.head_size not in (0, 256):
        raise ValueError("the OSCAR backend serves full D256 attention only")
    return BACKEND


def install_attention_hooks(attention_cls=None):
    """Wrap vLLM's Attention layer class once (reference plugin.py:88-130). Without
    ``attention_cls`` the class is taken from an already imported vLLM module, never
    imported here (vLLM imports it after its platform). Returns True when hooked."""
    if attention_cls is None:
        for name in ATTENTION_MODULES:
            module = sys.modules.get(name)
            if module is None or getattr(getattr(module, "__spec__", None), "_initializing", False):
                continue
            attention_cls = getattr(module, "Attention", None)
            if attention_cls is not None:
                break
        if attention_cls is None:
            return False
    if getattr(attention_cls, "_oscar_amd_hooked", False):
        return True
    init = attention_cls.__init__
    signature = inspect.signature(init)

    @functools.wraps(init)
    def construct(layer, *args, **kwargs):
        bound = signature.bind(layer, *args, **kwargs)
        prefix = bound.arguments.get("prefix", "") or ""
        if is_draft_layer(prefix) and bound.arguments.get("attn_backend") is None:
            # Bind the native class so that vLLM's (cached) selector is not consulted.
            native = native_backend(bound.arguments.get("attn_type", "decoder") or "decoder",
                                    _draft_selector(bound.arguments))
            if native is not None:
                bound.arguments["attn_backend"] = native
        return init(*bound.args, **bound.kwargs)

    after_load = attention_cls.process_weights_after_loading

    @functools.wraps(after_load)
    def process_weights(layer, act_dtype):
        result = after_load(layer, act_dtype)
        from .backend import OscarAttentionImpl

        if isinstance(getattr(layer, "impl", None), OscarAttentionImpl):
            layer.impl.initialize_layer(layer)
        return result

    attention_cls.__init__ = construct
    attention_cls.process_weights_after_loading = process_weights
    attention_cls._oscar_amd_hooked = True
    return True


def register(platform_cls=None, attention_cls=None):
    """Hook the platform's backend selector and the Attention class once (reference
    plugin.py:27-85). A no-op unless ``OSCAR_AMD_ENABLED=1``. Without ``platform_cls`` the ROCm
    platform of an installed vLLM is used. Returns True when the selector hook is in place."""
    if os.getenv(ENV_ENABLED, "0") != "1":
        return False
    if platform_cls is None:
        from vllm.platforms.rocm import RocmPlatform as platform_cls  # noqa: N813
    install_attention_hooks(attention_cls)
    if id(platform_cls) in _registered_on:
        return True
    original = platform_cls.get_attn_backend_cls.__func__

    @classmethod
    @functools.wraps(original)
    def select(cls, selected_backend, attn_selector_config, *args, **kwargs):
        # The Attention module is imported after the platform: hook it on first use.
        install_attention_hooks(attention_cls)
        native = original(cls, selected_backend, attn_selector_config, *args, **kwargs)
        _native_paths[getattr(attn_selector_config, "attn_type", "decoder")] = native
        if should_route(attn_selector_config):
            return backend_for(attn_selector_config)
        return native

    platform_cls.get_attn_backend_cls = select
    _native_selector.append((platform_cls, original))
    _registered_on.add(id(platform_cls))
    LOG.warning("OSCAR INT2 attention serves full decoder layers (prefix caching off; MTP "
                "draft layers stay native)")
    return True

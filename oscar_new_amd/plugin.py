"""vLLM general plugin for ROCm: routes full decoder attention to the OSCAR backend.

Reference: oscar_ascend/plugin.py:13-130, on vLLM's ROCm platform instead of the NPU one.
Two hooks, both installed once and only when ``OSCAR_AMD_ENABLED=1``:

* the platform's backend selector (``get_attn_backend_cls``) returns the OSCAR backend for
  causal, non-MLA, non-sparse decoder attention (plugin.py:13-85), rejecting the selector
  options the INT2 layout cannot serve;
* vLLM's ``Attention`` layer class: an MTP draft layer keeps the platform's native backend
  (its cache and rotations are separate; plugin.py:106-114), and once a routed layer's
  weights are loaded its implementation loads the layer's rotations (plugin.py:116-125).

The platform and Attention classes are looked up lazily or passed in, so both hooks are
tested against stand-ins without vLLM.
"""

from __future__ import annotations

import contextlib
import functools
import inspect
import logging
import os
import sys
import threading

LOG = logging.getLogger(__name__)
BACKEND = "oscar_new_amd.backend.OscarAttentionBackend"
ENV_ENABLED = "OSCAR_AMD_ENABLED"
UNSUPPORTED_OPTIONS = ("has_sink", "use_mm_prefix", "use_per_head_quant_scales",
                       "use_kv_connector")
# Where vLLM defines its Attention layer class (newest layout first).
ATTENTION_MODULES = ("vllm.model_executor.layers.attention.attention", "vllm.attention.layer")

_registered_on = set()
_native = threading.local()  # set while an MTP draft layer is being constructed


def should_route(selector):
    """Reference plugin.py:13-20: vision/encoder, MLA, sparse and non-causal stay native."""
    return (selector.attn_type == "decoder" and not selector.use_mla
            and not selector.use_sparse and not selector.use_non_causal)


def is_draft_layer(prefix):
    """Reference plugin.py:23-24: an MTP draft layer's module path contains ``mtp``."""
    return "mtp" in prefix.split(".")


@contextlib.contextmanager
def _native_selection():
    depth = getattr(_native, "depth", 0)
    _native.depth = depth + 1
    try:
        yield
    finally:
        _native.depth = depth


def _selecting_native():
    return getattr(_native, "depth", 0) > 0


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
            # The backend selector runs inside the constructor: answer it natively.
            with _native_selection():
                return init(*bound.args, **bound.kwargs)
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
        if should_route(attn_selector_config) and not _selecting_native():
            return backend_for(attn_selector_config)
        return original(cls, selected_backend, attn_selector_config, *args, **kwargs)

    platform_cls.get_attn_backend_cls = select
    _registered_on.add(id(platform_cls))
    LOG.warning("OSCAR INT2 attention serves full decoder layers (prefix caching off; MTP "
                "draft layers stay native)")
    return True

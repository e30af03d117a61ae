"""vLLM general plugin for ROCm: routes full decoder attention to the OSCAR backend.

Mirrors ``oscar_ascend/plugin.py:13-85`` (reference) on vLLM's ROCm platform: the same
routing rule (decoder, not MLA, not sparse, causal), the same rejected selector options and
head-size check, the same idempotent, environment-gated registration. The platform class is
looked up lazily (``vllm.platforms.rocm.RocmPlatform``) or passed in, so that the hook can be
tested against a stand-in without vLLM installed.
"""

from __future__ import annotations

import functools
import logging
import os

LOG = logging.getLogger(__name__)
BACKEND = "oscar_new_amd.backend.OscarAttentionBackend"
ENV_ENABLED = "OSCAR_AMD_ENABLED"
UNSUPPORTED_OPTIONS = ("has_sink", "use_mm_prefix", "use_per_head_quant_scales",
                       "use_kv_connector")

_registered_on = set()


def should_route(selector):
    """Reference plugin.py:13-20: vision/encoder, MLA, sparse and non-causal stay native."""
    return (selector.attn_type == "decoder" and not selector.use_mla
            and not selector.use_sparse and not selector.use_non_causal)


def is_draft_layer(prefix):
    """Reference plugin.py:23-24: MTP draft layers keep the native backend."""
    return "mtp" in prefix.split(".")


def backend_for(selector):
    """The backend class path for a routed selector (plugin.py:63-78 checks)."""
    for name in UNSUPPORTED_OPTIONS:
        if getattr(selector, name, False):
            raise ValueError(f"OSCAR does not support selector option {name}")
    # The runner probes with head_size 0 before the model exists; layers check D256 again.
    if selector.head_size not in (0, 256):
        raise ValueError("This OSCAR backend is restricted to full D256 attention")
    return BACKEND


def register(platform_cls=None):
    """Wrap ``platform_cls.get_attn_backend_cls`` once (reference plugin.py:27-85).

    A no-op unless ``OSCAR_AMD_ENABLED=1``. Without ``platform_cls`` the ROCm platform of an
    installed vLLM is used. Returns True when the hook is in place.
    """
    if os.getenv(ENV_ENABLED, "0") != "1":
        return False
    if platform_cls is None:
        from vllm.platforms.rocm import RocmPlatform as platform_cls  # noqa: N813
    if id(platform_cls) in _registered_on:
        return True
    original = platform_cls.get_attn_backend_cls.__func__

    @classmethod
    @functools.wraps(original)
    def select(cls, selected_backend, attn_selector_config, *args, **kwargs):
        if should_route(attn_selector_config):
            return backend_for(attn_selector_config)
        return original(cls, selected_backend, attn_selector_config, *args, **kwargs)

    platform_cls.get_attn_backend_cls = select
    _registered_on.add(id(platform_cls))
    LOG.warning("OSCAR INT2 attention enabled for full decoder layers (prefix caching off, "
                "MTP draft layers native)")
    return True

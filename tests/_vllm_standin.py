"""Stand-ins for the parts of vLLM the OSCAR glue touches (vLLM is not installed here).

Shaped after the reference's fakes (tests/test_graph_startup.py:19-168,
tests/test_integration.py:26-98): a platform class with the backend selector, an Attention
layer class that asks the selector for its backend and constructs the implementation with
vLLM's positional arguments, an engine config, a ``vllm.config`` module with
``get_current_vllm_config`` and the KV cache spec the metadata builder reads.
"""

import functools
import importlib
import sys
import types
from contextlib import contextmanager
from types import SimpleNamespace

import torch

NATIVE_BACKEND = "tests._vllm_standin.NativeBackend"


class NativeImpl:
    def __init__(self, *args, **kwargs):
        self.args = args


class NativeBackend:
    @staticmethod
    def get_impl_cls():
        return NativeImpl


def make_platform():
    class RocmPlatform:
        calls = []

        @classmethod
        def get_attn_backend_cls(cls, selected_backend, attn_selector_config, num_heads=None):
            cls.calls.append(selected_backend)
            return NATIVE_BACKEND

    return RocmPlatform


def _resolve(path):
    if path == NATIVE_BACKEND:
        return NativeBackend
    module, _, name = path.rpartition(".")
    return getattr(importlib.import_module(module), name)


def make_attention(platform):
    """An Attention layer class that selects its backend like vLLM's: through the platform,
    unless one is passed in, and builds the implementation with vLLM's positional order.
    Selection goes through a cache keyed by the selector arguments, as vLLM's
    ``get_attn_backend`` does (``_cached_get_attn_backend``): draft and target layers ask with
    the same arguments and share one answer."""

    @functools.cache
    def cached_backend(attn_type, head_size, num_heads):
        selector = SimpleNamespace(attn_type=attn_type, use_mla=False, use_sparse=False,
                                   use_non_causal=False, head_size=head_size)
        return _resolve(platform.get_attn_backend_cls(None, selector, num_heads))

    class Attention(torch.nn.Module):
        def __init__(self, num_heads, head_size, scale, num_kv_heads=None, alibi_slopes=None,
                     cache_config=None, quant_config=None, logits_soft_cap=None,
                     per_layer_sliding_window=None, prefix="", attn_type="decoder",
                     kv_sharing_target_layer_name=None, attn_backend=None, **extra_impl_args):
            super().__init__()
            num_kv_heads = num_kv_heads or num_heads
            self.layer_name = prefix
            self.register_buffer("_k_scale", torch.ones(()))
            if attn_backend is None:
                attn_backend = cached_backend(attn_type, head_size, num_heads)
            self.attn_backend = attn_backend
            self.impl = attn_backend.get_impl_cls()(
                num_heads, head_size, scale, num_kv_heads, alibi_slopes,
                per_layer_sliding_window, "auto", logits_soft_cap, attn_type,
                kv_sharing_target_layer_name, **extra_impl_args)
            self.loaded = False

        def process_weights_after_loading(self, act_dtype):
            self.loaded = True

    return Attention


def make_vllm_config(num_speculative_tokens=3, max_num_seqs=7, max_num_batched_tokens=64,
                     max_model_len=16384, **over):
    cfg = SimpleNamespace(
        cache_config=SimpleNamespace(enable_prefix_caching=False, cache_dtype="auto"),
        model_config=SimpleNamespace(dtype=torch.bfloat16, max_model_len=max_model_len,
                                     hf_text_config=SimpleNamespace(head_dim=256)),
        kv_transfer_config=None,
        parallel_config=SimpleNamespace(decode_context_parallel_size=1,
                                        prefill_context_parallel_size=1, enable_dbo=False),
        speculative_config=(SimpleNamespace(num_speculative_tokens=num_speculative_tokens)
                            if num_speculative_tokens else None),
        scheduler_config=SimpleNamespace(max_num_seqs=max_num_seqs,
                                         max_num_batched_tokens=max_num_batched_tokens),
        compilation_config=SimpleNamespace(static_forward_context={}),
        quant_config=None,
    )
    for path, value in over.items():
        obj = cfg
        *head, last = path.split(".")
        for name in head:
            obj = getattr(obj, name)
        setattr(obj, last, value)
    return cfg


@contextmanager
def current_vllm_config(config):
    """Install a ``vllm.config`` module whose ``get_current_vllm_config`` returns ``config``
    (vLLM builds layers under such a context)."""
    saved = {name: sys.modules.get(name) for name in ("vllm", "vllm.config")}
    vllm = types.ModuleType("vllm")
    vllm_config = types.ModuleType("vllm.config")
    vllm_config.get_current_vllm_config = lambda: config
    vllm.config = vllm_config
    sys.modules["vllm"], sys.modules["vllm.config"] = vllm, vllm_config
    try:
        yield
    finally:
        for name, module in saved.items():
            if module is None:
                sys.modules.pop(name, None)
            else:
                sys.modules[name] = module


def kv_cache_spec(block_size=768, num_kv_heads=1):
    return SimpleNamespace(block_size=block_size, num_kv_heads=num_kv_heads, head_size=256)

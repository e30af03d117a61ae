"""Per-layer launch order of the OSCAR INT2 attention path.

Reference: oscar_ascend/backend.py:13-227. ``OscarAttentionImpl`` keeps the forward contract:
same arguments, same kernel order, no host reads, the window store last (it must follow both
attention branches because a long current chunk wraps the ring). ``OscarAttentionBackend``
and ``validate_vllm_config`` are the vLLM-facing class and checks (backend.py:13-64), written
against duck-typed vLLM objects so that they import without vLLM. Initial prefill (the
reference's Ascend FIA call, ``meta.initial_prefill``) runs through the INT2 path below with
an empty history: the BF16 branch is the causal attention over the request's own tokens.
"""

from __future__ import annotations

import os

import torch

from . import kernels
from .config import OscarConfig, choose_history_partition, choose_splits


class OscarAttentionBackend:
    """Reference backend.py:13-38: the backend class the plugin routes to."""

    forward_includes_kv_cache_update = True

    @staticmethod
    def get_name():
        return "CUSTOM"

    @staticmethod
    def get_impl_cls():
        return OscarAttentionImpl

    @staticmethod
    def get_builder_cls():
        from .metadata import OscarMetadataBuilder

        return OscarMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, cache_dtype_str="auto"):
        """(K, V) stripes of bf16 [num_blocks, block_size, num_kv_heads, head_size] each: the
        native paged layout whose K stripe holds the INT2 slots and V stripe the windows."""
        return (2, num_blocks, block_size, num_kv_heads, head_size)

    @staticmethod
    def copy_blocks(*args, **kwargs):
        raise NotImplementedError("OSCAR ring ownership does not support shared/copied request pages")

    @staticmethod
    def swap_blocks(*args, **kwargs):
        raise NotImplementedError("OSCAR supports native recompute preemption, not KV swapping")


def validate_vllm_config(config):
    """Reference backend.py:41-64, with the ROCm runner's names: the configurations the INT2
    path does not support are rejected with the reference's reasons."""
    if config.cache_config.enable_prefix_caching:
        raise ValueError("OSCAR requires --no-enable-prefix-caching (BF16 ring owner isolation)")
    if config.cache_config.cache_dtype not in ("auto", "bfloat16"):
        raise ValueError("Use --kv-cache-dtype auto with OSCAR_AMD_ENABLED=1")
    if config.model_config.dtype != torch.bfloat16:
        raise ValueError("OSCAR target model must use BF16 activation/cache dtype")
    if getattr(config, "kv_transfer_config", None) is not None:
        raise ValueError("KV transfer is not supported by this OSCAR layout")
    pc = config.parallel_config
    if (getattr(pc, "decode_context_parallel_size", 1) != 1
            or getattr(pc, "prefill_context_parallel_size", 1) != 1):
        raise ValueError("OSCAR currently requires PCP=DCP=1")
    if getattr(pc, "enable_dbo", False):
        raise ValueError("DBO requires separate metadata buffer sets and is not supported")
    if os.getenv("VLLM_USE_V2_MODEL_RUNNER", "0") == "1":
        raise ValueError("This OSCAR adapter targets the v1 model runner")
    hf = config.model_config.hf_text_config
    if getattr(hf, "head_dim", None) != 256:
        raise ValueError("This implementation targets D256 full attention")


class OscarAttentionImpl:
    """Reference: backend.py:67-227. ``split_policy`` "reference" keeps config.py:84-89,
    "mi355x" fills the 256 CUs (config.choose_splits_mi355x). ``one_launch_post`` runs the
    history branch and post-attention as one launch (``kernels.history_post``) where it applies;
    the result is the same bits either way."""

    def __init__(self, num_heads, head_size, scale, num_kv_heads, cfg=None,
                 split_policy="reference", fused=True, one_launch_post=False):
        if head_size != 256:
            raise ValueError("OSCAR requires FULL decoder attention with D256")
        if num_kv_heads <= 0 or num_heads % num_kv_heads:
            raise ValueError("query heads must be a multiple of kv heads")
        if split_policy not in ("reference", "mi355x"):
            raise ValueError("split_policy must be 'reference' or 'mi355x'")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.cfg = cfg or OscarConfig.from_env()
        self.split_policy = split_policy
        self.fused = fused
        self.one_launch_post = one_launch_post
        self.rk = self.rv = self.rk_cols = self.rv_cols = self.rk_t = self.rv_t = None
        self.history = self.window = None
        self.cache_identity = None

    def initialize_layer(self, rk, rv):
        """Install the layer's calibrated K/V rotations (bf16 [256, 256] on the device)."""
        for r in (rk, rv):
            if tuple(r.shape) != (256, 256):
                raise ValueError("rotations must be 256x256")
        self.rk = rk.to(torch.bfloat16).contiguous()
        self.rv = rv.to(torch.bfloat16).contiguous()
        # x @ R reads R column-wise; a transposed view of R^T stored row-major keeps those
        # reads contiguous (the inverse rotation's R^T view of rv already is).
        self.rk_t = self.rk.T.contiguous()
        self.rv_t = self.rv.T.contiguous()
        self.rk_cols = self.rk_t.T
        self.rv_cols = self.rv_t.T

    def splits_for(self, meta):
        return self.partition_for(meta)[0]

    def partition_for(self, meta):
        """``(splits, split_tokens)`` of the history branch. "reference": config.py:84-89
        with the reference split rule; "mi355x": ``choose_history_partition`` (reads the
        host-side ``meta.max_seq_len`` and, when present, ``meta.total_seq_len``)."""
        if self.split_policy == "reference":
            return choose_splits(meta.num_reqs, self.num_kv_heads, meta.max_query_len), 0
        tasks = -(-meta.num_actual_tokens // self.cfg.queries_per_tile) if meta.max_query_len > 1 \
            else meta.num_reqs
        return choose_history_partition(tasks, self.num_kv_heads, meta.max_query_len,
                                        getattr(meta, "max_seq_len", None),
                                        getattr(meta, "total_seq_len", None))

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None):
        """Reference: backend.py:125-227 (minus the Ascend prefill call).

        ``fused`` (default) runs the step as three launches (``pre_attention``, the history
        kernel, ``post_attention``) that produce the same bits as the reference order of
        single launches below.
        """
        if output is None:
            raise ValueError("an attention output buffer is required")
        if attn_metadata is None:
            return output.zero_()
        if self.rk is None or self.rv is None:
            raise RuntimeError("OSCAR rotations were not initialized for this layer")
        if key is None or value is None:
            raise ValueError("OSCAR requires the current K/V to maintain exact BF16 windows")
        if query.device.type != "cuda":
            raise RuntimeError("OSCAR kernels run on a ROCm GPU")
        meta = attn_metadata
        n = query.shape[0]
        query = query.view(n, self.num_heads, self.head_size)
        key = key.view(key.shape[0], self.num_kv_heads, self.head_size)
        value = value.view(value.shape[0], self.num_kv_heads, self.head_size)
        if key.shape[0] != n or value.shape[0] != n:
            raise ValueError("Q/K/V must have matching current-token dimensions")
        identity = (kv_cache[0].data_ptr(), kv_cache[1].data_ptr(), meta.layout)
        if self.cache_identity != identity:
            self.history, self.window = meta.layout.tensor_views(kv_cache)
            self.cache_identity = identity
        if not output.is_contiguous():
            raise ValueError("Attention output must be contiguous")
        if n == 0:
            return output

        if getattr(meta, "initial_prefill", False):
            # Reference backend.py:171-193 + 225-226: INT2 store, causal attention over each
            # request's own tokens (the fused-infer call), then the window store.
            kernels.rotate_store_int2(key, value, self.rk_t, self.rv_t, self.history,
                                      meta.slot_mapping, meta.counts, meta.layout)
            kernels.prefill_attention(query, key, value, self.window, meta, meta.layout,
                                      self.scale, output.view(n, -1),
                                      getattr(meta, "merged_lse", None))
            kernels.store_windows(key, value, self.window, meta, meta.layout)
            return output

        splits, split_tokens = self.partition_for(meta)
        if self.fused:
            # BF16 branch + rotations + INT2 store; then history, merges + window in two
            # launches, or (one_launch_post, decode-sized tasks, <= 16 splits) in one.
            qrot, rp, rl = kernels.pre_attention(query, key, value, self.history, self.window,
                                                 meta, meta.layout, self.scale, self.rk_t,
                                                 self.rv_t)
            if self.one_launch_post and kernels.history_post_supported(
                    meta, meta.layout, self.num_heads, splits, n):
                kernels.history_post(qrot, self.history, meta, meta.layout, self.scale, splits, rp,
                                     rl, self.rv, key, value, self.window, output.view(n, -1),
                                     getattr(meta, "merged_lse", None), split_tokens=split_tokens)
                return output
            hp, hl = kernels.attention_partials(qrot, key, value, self.history, self.window, meta,
                                                meta.layout, self.scale, splits, raw=False,
                                                split_tokens=split_tokens)
            kernels.post_attention(hp, hl, rp, rl, self.rv, key, value, self.window, meta,
                                   meta.layout, output.view(n, -1), getattr(meta, "merged_lse", None))
            return output

        krot = kernels.rotate(key, self.rk_cols)
        vrot = kernels.rotate(value, self.rv_cols)
        kernels.store_int2(krot, vrot, self.history, meta.slot_mapping, meta.counts, meta.layout)
        qrot = kernels.rotate(query, self.rk_cols)
        hp, hl = kernels.attention_partials(qrot, key, value, self.history, self.window, meta,
                                            meta.layout, self.scale, splits, raw=False,
                                            split_tokens=split_tokens)
        hrot, hlogsum = kernels.merge_splits(hp, hl, meta.counts)
        hout = kernels.rotate(hrot, self.rv.T)
        rp, rl = kernels.attention_partials(query, key, value, self.history, self.window, meta,
                                            meta.layout, self.scale, 1, raw=True)
        kernels.merge_paths(hout, hlogsum, rp, rl, meta.counts, output.view(n, -1),
                            getattr(meta, "merged_lse", None))
        # Must follow BOTH attention branches: long current chunks wrap the ring.
        kernels.store_windows(key, value, self.window, meta, meta.layout)
        return output

"""vLLM attention backend and per-layer launch order of the OSCAR INT2 attention path.

Reference: oscar_ascend/backend.py:13-227. Three parts:

* ``OscarAttentionBackend``: the class the platform hook routes FULL decoder attention to
  (backend.py:13-38): implementation and builder classes, the native two-stripe cache shape,
  no block copies or swaps.
* ``validate_vllm_config``: the engine configurations the INT2 layout cannot serve
  (backend.py:41-64), checked when a layer implementation is built.
* ``OscarAttentionImpl``: constructed by vLLM with its attention-implementation arguments
  (backend.py:67-105), given its calibrated rotations after weight loading
  (``initialize_layer``, backend.py:107-117), and run once per layer step (``forward``,
  backend.py:125-227: no host reads, the window store after both attention branches).

vLLM is not importable in this image; everything here is written against duck-typed vLLM
objects, so it imports and is tested without it. ``OscarAttentionImpl.standalone`` builds a
layer without a vLLM config (benchmarks and tests).
"""

from __future__ import annotations

import os

import torch

from . import kernels
from .config import (OscarConfig, attention_programs, choose_device_partition,
                     choose_history_partition, choose_splits)

SPLIT_POLICIES = ("device", "reference", "mi355x")
ENV_SPLIT_POLICY = "OSCAR_AMD_SPLIT_POLICY"


class OscarAttentionBackend:
    """Routed backend (reference backend.py:13-38)."""

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
        """Two native bf16 stripes [num_blocks, block_size, num_kv_heads, head_size]: the K
        stripe carries the INT2 slots, the V stripe of a request's first page its window."""
        return (2, num_blocks, block_size, num_kv_heads, head_size)

    @staticmethod
    def copy_blocks(*args, **kwargs):
        raise NotImplementedError(
            "OSCAR pages belong to one request (its BF16 window lives in its first page); "
            "pages cannot be copied or shared")

    @staticmethod
    def swap_blocks(*args, **kwargs):
        raise NotImplementedError("OSCAR supports recompute preemption only; KV swapping is "
                                  "not available")


def _config_problems(config):
    """(rejected, reason) for every engine option the INT2 layout cannot serve."""
    cache, model, parallel = config.cache_config, config.model_config, config.parallel_config
    text = getattr(model, "hf_text_config", None)
    return (
        (bool(cache.enable_prefix_caching),
         "OSCAR needs --no-enable-prefix-caching: a request's BF16 ring lives in its own "
         "first page"),
        (cache.cache_dtype not in ("auto", "bfloat16"),
         "OSCAR manages its own KV format; start with --kv-cache-dtype auto"),
        (model.dtype != torch.bfloat16, "the OSCAR target model must run in bf16"),
        (getattr(config, "kv_transfer_config", None) is not None,
         "KV transfer cannot move OSCAR's INT2 pages"),
        (getattr(parallel, "decode_context_parallel_size", 1) != 1
         or getattr(parallel, "prefill_context_parallel_size", 1) != 1,
         "OSCAR runs with PCP=DCP=1 only"),
        (bool(getattr(parallel, "enable_dbo", False)),
         "dual-batch overlap would need two metadata buffer sets; DBO is unsupported"),
        (os.getenv("VLLM_USE_V2_MODEL_RUNNER", "0") == "1",
         "OSCAR plugs into the v1 model runner; unset VLLM_USE_V2_MODEL_RUNNER"),
        (getattr(getattr(config, "quant_config", None), "enable_c8_quant", False),
         "C8 KV quantization replaces the OSCAR layout; W8A8 weights are fine"),
        (getattr(text, "head_dim", None) != 256, "OSCAR covers D256 full attention only"),
    )


def validate_vllm_config(config):
    """Raise ValueError for the first unsupported engine option (reference backend.py:41-64).
    The reference's Qwen3.5 model-type restriction is not kept: any D256 full-attention
    decoder is served."""
    for rejected, reason in _config_problems(config):
        if rejected:
            raise ValueError(reason)


STANDALONE = object()  # ``vllm_config`` value of a layer built outside any vLLM engine


def _current_vllm_config():
    """The engine config vLLM is constructing layers under, or None without vLLM."""
    try:
        from vllm.config import get_current_vllm_config
    except ImportError:
        return None
    return get_current_vllm_config()


class OscarAttentionImpl:
    """One FULL attention layer (reference backend.py:67-227).

    Constructed by vLLM with the standard implementation arguments. Options that are not
    vLLM's are keyword-only: ``vllm_config`` (default: the config vLLM is building under),
    ``oscar_config`` (default: from the environment, with the speculative token count of the
    vLLM config), ``split_policy`` (default: ``OSCAR_AMD_SPLIT_POLICY``, else "device": fill
    the 256 CUs with token-bounded splits whose length the GPU derives from the step's
    lengths, so that a captured graph stays balanced at any context length; "reference":
    config.py:84-89; "mi355x": token-bounded splits sized from the host-side lengths of the
    step, which a captured graph would freeze), ``fused`` (three launches per step instead of the nine single
    launches; same bits), ``layer_step`` (opt-in: the whole step in one launch where it
    applies, the INT2 and window bytes of the other forms and the output within rounding of
    them; slower than three launches on MI355X today, because its latency-bound parts wait
    behind the INT2 stream's memory traffic) and
    ``one_launch_post`` (history branch and post-attention in one launch where it applies and
    the one-launch step does not; same bits as three launches) and ``overlap`` (default on:
    where it applies, the step is the history launch carrying the BF16 branch and the K/V INT2
    store as extra workgroups, and post-attention; same bits). ``rotate_in_history`` (default
    off; with ``overlap``): the history workgroups rotate the query rows themselves; every
    history workgroup then reads all of R_k (57 MB of L2 reads at c3). ``q_roles`` (default
    off; with ``overlap``, unless ``rotate_in_history``): the q rotation runs as role workgroups
    of the history launch, whose history workgroups wait for the rotated rows after their
    first chunk requests; same bits. Under the history stream's load the roles' chain of
    memory round trips (load, write-through, count, poll, copy) ends after the first chunks
    arrive: c5 step 53.0-53.4 against 53.8-54.5 us, c3 55.3-57.2 against 53.7-54.8 us (A/B
    on one box). With neither, the q rotation is a launch of its own ahead of the history
    launch (the default).
    """

    def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes=None,
                 sliding_window=None, kv_cache_dtype="auto", logits_soft_cap=None,
                 attn_type="decoder", kv_sharing_target_layer_name=None, *, vllm_config=None,
                 oscar_config=None, split_policy=None, fused=True, one_launch_post=False,
                 layer_step=False, overlap=True, rotate_in_history=False, q_roles=False,
                 **kwargs):
        unsupported = (
            (alibi_slopes is not None, "ALiBi"),
            (sliding_window is not None, "sliding-window attention"),
            (bool(logits_soft_cap), "logits soft-capping"),
            (kv_sharing_target_layer_name is not None, "cross-layer KV sharing"),
            (kwargs.get("sinks") is not None, "learned attention sinks"),
        )
        for present, feature in unsupported:
            if present:
                raise ValueError(f"OSCAR attention does not implement {feature}")
        if str(getattr(attn_type, "value", attn_type)).lower() != "decoder" or head_size != 256:
            raise ValueError("OSCAR serves FULL decoder attention with head size 256 only")
        if num_kv_heads <= 0 or num_heads % num_kv_heads:
            raise ValueError("the query head count must be a multiple of the KV head count")
        if split_policy is None:
            split_policy = os.getenv(ENV_SPLIT_POLICY, "device")
        if split_policy not in SPLIT_POLICIES:
            raise ValueError(f"split_policy must be one of {', '.join(SPLIT_POLICIES)}")
        if vllm_config is STANDALONE:
            vllm_config = None
        elif vllm_config is None:
            vllm_config = _current_vllm_config()
        self.vllm_config = vllm_config
        if self.vllm_config is not None:
            validate_vllm_config(self.vllm_config)
        if oscar_config is None:
            spec = getattr(self.vllm_config, "speculative_config", None)
            oscar_config = OscarConfig.from_env(spec.num_speculative_tokens if spec else 0)
        self.cfg = oscar_config
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.kv_cache_dtype = kv_cache_dtype
        self.attn_type = attn_type
        self.split_policy = split_policy
        self.fused = fused
        self.one_launch_post = one_launch_post
        self.layer_step = layer_step
        self.overlap = overlap
        self.rotate_in_history = rotate_in_history
        self.q_roles = q_roles
        self.q_sync = None  # int32 [4] of the q rotation roles (zero between launches)
        self.rk = self.rv = self.rk_cols = self.rv_cols = self.rk_t = self.rv_t = None
        self.history = self.window = None
        self.cache_identity = None

    @classmethod
    def standalone(cls, num_heads, head_size, scale, num_kv_heads, cfg=None, **options):
        """A layer outside a vLLM engine (no engine config, no config checks), for benchmarks
        and tests; ``cfg`` defaults to the environment's with no speculative tokens."""
        return cls(num_heads, head_size, scale, num_kv_heads, vllm_config=STANDALONE,
                   oscar_config=cfg, **options)

    def initialize_layer(self, layer):
        """Load this layer's calibrated K/V rotations (reference backend.py:107-117): the
        artefacts named by VLLM_OSCAR_K/V_ROTATION_PATH, matched by ``layer.layer_name``'s
        decoder index, validated on the CPU and copied to the current device as bf16."""
        from .rotations import get_rotation

        # The layer's own scale buffer sits on its device; otherwise the current GPU.
        scale = getattr(layer, "_k_scale", None)
        device = scale.device if torch.is_tensor(scale) else torch.device(
            "cuda", torch.cuda.current_device())
        name = layer.layer_name
        self.set_rotations(get_rotation(self.cfg.k_rotation_path, name, device),
                           get_rotation(self.cfg.v_rotation_path, name, device))

    def set_rotations(self, rk, rv):
        """Install K/V rotations directly (bf16 [256, 256] on the device)."""
        for r in (rk, rv):
            if tuple(r.shape) != (256, 256):
                raise ValueError("rotations must be 256x256")
        self.rk = rk.to(torch.bfloat16).contiguous()
        self.rv = rv.to(torch.bfloat16).contiguous()
        # x @ R reads R column-wise; R^T stored row-major keeps those reads contiguous. The
        # inverse rotation's R^T view of rv already is.
        self.rk_t = self.rk.T.contiguous()
        self.rv_t = self.rv.T.contiguous()
        self.rk_cols = self.rk_t.T
        self.rv_cols = self.rv_t.T
        # Allocated here, outside any graph capture; the launches keep it zero.
        self.q_sync = torch.zeros(4, dtype=torch.int32, device=self.rk.device)

    def splits_for(self, meta):
        return self.partition_for(meta)[0]

    def _q_roles(self):
        """Whether the q rotation runs as role workgroups of the history launch."""
        return self.q_roles and not self.rotate_in_history

    def _roles_share_history_launch(self, meta):
        """Whether the step's history launch carries the pre-attention role workgroups."""
        layout = getattr(meta, "layout", None)
        return (self.fused and self.overlap and not self.one_launch_post and not self.layer_step
                and layout is not None
                and kernels.history_pre_supported(meta, layout, self.num_heads))

    def _queue_roles(self, meta, split_tokens, tokens):
        """Whether the step's history launch is the 17-32-row work queue carrying the BF16
        branch and the K/V store as units of its own (MTP steps with token-bounded splits; the
        q rotation stays a launch of its own)."""
        layout = getattr(meta, "layout", None)
        return (self.fused and self.overlap and not self.one_launch_post and not self.layer_step
                and layout is not None and not self.rotate_in_history and not self.q_roles
                and kernels.history_rows(meta, layout, self.num_heads) > 8
                and kernels.history_pre_supported(meta, layout, self.num_heads, split_tokens,
                                                  tokens))

    def partition_for(self, meta, tokens=None):
        """``(splits, split_tokens)`` of the history branch for a step of ``tokens`` query
        tokens (default ``meta.num_actual_tokens``). "device": ``choose_device_partition``
        from values fixed when a graph is captured (grid capacity, token count, launch form);
        the GPU derives the split length from the step's lengths. "reference": config.py:84-89
        with the reference split rule. "mi355x": ``choose_history_partition`` (host-side
        ``meta.max_seq_len`` and, when present, ``meta.total_seq_len``). Both token-bounded
        policies leave the slots of the pre-attention role workgroups free when those share the
        history launch. The one-launch forms (``one_launch_post``, ``layer_step``) count a grid
        of split slots and take the "mi355x" partition under "device"."""
        if self.split_policy == "reference":
            return choose_splits(meta.num_reqs, self.num_kv_heads, meta.max_query_len), 0
        roles = self._roles_share_history_launch(meta)
        if self.split_policy == "device" and not (self.one_launch_post or self.layer_step):
            n = int(meta.num_actual_tokens if tokens is None else tokens)
            programs = attention_programs(n, meta.max_num_reqs, self.cfg.queries_per_tile)
            # BF16 branch: one workgroup per (task, kv head); K/V store: 8 per 16 rows.
            reserved = (programs * self.num_kv_heads + 8 * -(-n * self.num_kv_heads // 16)
                        + (-(-n * self.num_heads // 16) if self._q_roles() else 0)
                        if roles else 0)
            return choose_device_partition(programs, self.num_kv_heads, meta.max_query_len, n,
                                           self.num_heads, self.cfg.queries_per_tile,
                                           reserved=reserved)
        tasks = meta.num_reqs if meta.max_query_len <= 1 else \
            -(-meta.num_actual_tokens // self.cfg.queries_per_tile)
        rows = min(meta.max_query_len, self.cfg.queries_per_tile) * (
            self.num_heads // self.num_kv_heads)
        reserved = 0
        if roles:
            kv_rows = meta.num_actual_tokens * self.num_kv_heads
            reserved = tasks * self.num_kv_heads + 8 * -(-kv_rows // 16)
            if self._q_roles():
                reserved += -(-meta.num_actual_tokens * self.num_heads // 16)
        return choose_history_partition(tasks, self.num_kv_heads, meta.max_query_len,
                                        getattr(meta, "max_seq_len", None),
                                        getattr(meta, "total_seq_len", None), rows=rows,
                                        reserved=reserved)

    def _bind_cache(self, kv_cache, layout):
        identity = (kv_cache[0].data_ptr(), kv_cache[1].data_ptr(), layout)
        if self.cache_identity != identity:
            self.history, self.window = layout.tensor_views(kv_cache)
            self.cache_identity = identity

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        """One layer step (reference backend.py:125-227); returns ``output``."""
        if output is None:
            raise ValueError("OSCAR writes into a caller-provided attention output buffer")
        if output_scale is not None or output_block_scale is not None:
            raise ValueError("OSCAR does not fuse output quantization")
        if attn_metadata is None:  # profiling run: nothing scheduled
            return output.zero_()
        if self.rk is None or self.rv is None:
            raise RuntimeError("this OSCAR layer has no rotations: initialize_layer runs after "
                               "weight loading")
        if key is None or value is None:
            raise ValueError("OSCAR needs the current K/V: the BF16 window is exact")
        if query.device.type != "cuda":
            raise RuntimeError("OSCAR kernels run on a ROCm GPU")
        meta = attn_metadata
        n = query.shape[0]
        q = query.view(n, self.num_heads, self.head_size)
        k = key.view(key.shape[0], self.num_kv_heads, self.head_size)
        v = value.view(value.shape[0], self.num_kv_heads, self.head_size)
        if k.shape[0] != n or v.shape[0] != n:
            raise ValueError("query, key and value must cover the same tokens")
        self._bind_cache(kv_cache, meta.layout)
        if not output.is_contiguous():
            raise ValueError("the attention output must be contiguous")
        if n == 0:
            return output
        rows = output.view(n, -1)
        lse = getattr(meta, "merged_lse", None)
        layout = meta.layout
        if getattr(meta, "initial_prefill", False):
            # Every request starts here: INT2 store of all tokens, causal attention over each
            # request's own tokens (the reference's fused-infer call), then the windows.
            kernels.rotate_store_int2(k, v, self.rk_t, self.rv_t, self.history,
                                      meta.slot_mapping, meta.counts, layout)
            kernels.prefill_attention(q, k, v, self.window, meta, layout, self.scale, rows, lse)
            kernels.store_windows(k, v, self.window, meta, layout)
            return output
        splits, split_tokens = self.partition_for(meta, n)
        if self.fused:
            self._fused_step(q, k, v, meta, splits, split_tokens, rows, lse)
        else:
            self._single_launch_step(q, k, v, meta, splits, split_tokens, rows, lse)
        return output

    def _fused_step(self, q, k, v, meta, splits, split_tokens, rows, lse):
        """The whole step in one launch (``layer_step``, where it applies); else, with
        ``overlap``, the history launch carrying the pre-attention work (BF16 branch, K/V INT2
        store and, with ``rotate_in_history``, the q rotation) -> post (split merge, inverse V
        rotation, path merge, windows); else pre-attention -> history -> post, the last two in
        one launch with ``one_launch_post``."""
        layout = meta.layout
        if self.layer_step and kernels.layer_step_supported(meta, layout, self.num_heads, splits,
                                                            q.shape[0]):
            kernels.layer_step(q, k, v, self.history, self.window, meta, layout, self.scale,
                               splits, self.rk_t, self.rv_t, self.rv, rows, lse,
                               split_tokens=split_tokens)
            return
        queue = self._queue_roles(meta, split_tokens, q.shape[0])
        if queue or (self.overlap and not self.one_launch_post
                     and kernels.history_pre_supported(meta, layout, self.num_heads)):
            # One launch holding the history branch (its workgroups rotate the query rows, or a
            # q rotation launch goes first) and, dispatched ahead of it, the BF16 branch and
            # the INT2 store (the history branch never reads the slots the store writes), then
            # post-attention.
            q_sync = None
            if self._q_roles() and not queue:
                qrot = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
                q_sync = self.q_sync
            else:
                qrot = (None if self.rotate_in_history and not queue
                        else kernels.rotate(q, self.rk_cols))
            hp, hl, rp, rl = kernels.history_pre(qrot, q, k, v, self.history, self.window, meta,
                                                 layout, self.scale, splits, self.rk_t,
                                                 self.rv_t, split_tokens=split_tokens,
                                                 q_sync=q_sync)
            kernels.post_attention(hp, hl, rp, rl, self.rv, k, v, self.window, meta, layout,
                                   rows, lse)
            return
        # A long chunk's BF16 branch runs as the chunk flash launch (same bits).
        qrot, rp, rl = kernels.pre_attention(q, k, v, self.history, self.window, meta, layout,
                                             self.scale, self.rk_t, self.rv_t,
                                             raw=not kernels.chunk_raw_preferred(meta))
        if self.one_launch_post and kernels.history_post_supported(
                meta, layout, self.num_heads, splits, q.shape[0]):
            kernels.history_post(qrot, self.history, meta, layout, self.scale, splits, rp, rl,
                                 self.rv, k, v, self.window, rows, lse, split_tokens=split_tokens)
            return
        hp, hl = kernels.attention_partials(qrot, k, v, self.history, self.window, meta, layout,
                                            self.scale, splits, raw=False,
                                            split_tokens=split_tokens)
        kernels.post_attention(hp, hl, rp, rl, self.rv, k, v, self.window, meta, layout, rows,
                               lse)

    def _single_launch_step(self, q, k, v, meta, splits, split_tokens, rows, lse):
        """The reference's order of single launches (backend.py:171-226)."""
        layout = meta.layout
        kernels.store_int2(kernels.rotate(k, self.rk_cols), kernels.rotate(v, self.rv_cols),
                           self.history, meta.slot_mapping, meta.counts, layout)
        hp, hl = kernels.attention_partials(kernels.rotate(q, self.rk_cols), k, v, self.history,
                                            self.window, meta, layout, self.scale, splits,
                                            raw=False, split_tokens=split_tokens)
        merged, merged_lse = kernels.merge_splits(hp, hl, meta.counts)
        hout = kernels.rotate(merged, self.rv.T)
        rp, rl = kernels.attention_partials(q, k, v, self.history, self.window, meta, layout,
                                            self.scale, 1, raw=True)
        kernels.merge_paths(hout, merged_lse, rp, rl, meta.counts, rows, lse)
        # Last: a chunk longer than the ring overwrites window slots both branches read.
        kernels.store_windows(k, v, self.window, meta, layout)

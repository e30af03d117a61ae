"""Per-step attention metadata in fixed device buffers (graph capture and replay).

Reference: oscar_ascend/metadata.py:15-174. The builder is constructed by vLLM with
``(kv_cache_spec, layer_names, vllm_config, device)``, allocates its buffers once, and
``build`` copies each step's scheduler metadata into them with asynchronous device copies
(no host reads), then launches the task-table kernel, so a captured HIP graph replays with
new lengths, pages and request counts. A capture (dummy) build clears ``counts``, which masks
every cache access on the device. vLLM is not importable here: the builder is written against
duck-typed vLLM objects, and ``OscarMetadataBuilder.standalone`` makes one without an engine.
"""

from __future__ import annotations

import contextlib
import math
import threading
from dataclasses import dataclass

import torch

from . import kernels
from .config import OscarConfig, task_capacity
from .layout import CacheLayout


@dataclass
class OscarMetadata:
    """Reference metadata.py:15-33, plus host-side bounds the MI355X split policy reads."""

    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    block_tables: torch.Tensor
    slot_mapping: torch.Tensor
    counts: torch.Tensor
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_num_reqs: int
    layout: CacheLayout
    attn_state: object = None
    initial_prefill: bool = False
    actual_seq_lengths_q: list | None = None  # cumulative query ends (host), initial prefill
    causal: bool = True
    is_dummy: bool = False
    tasks: torch.Tensor | None = None
    task_count: torch.Tensor | None = None
    max_seq_len: int | None = None  # host upper bound on seq_lens
    total_seq_len: int | None = None  # host sum of seq_lens
    merged_lse: torch.Tensor | None = None  # optional [n, hq] output of the merged LSE
    finish_counters: torch.Tensor | None = None  # zeroed int32 slots of one-launch post
    queue_counters: torch.Tensor | None = None  # two zeroed int32 work-queue counters

    @property
    def query_ends(self):
        return self.actual_seq_lengths_q


# ---------------------------------------------------------------- dummy (capture) runs

_scope = threading.local()


@contextlib.contextmanager
def dummy_run_scope(capturing=True):
    """Builds inside this scope are dummy builds: they own no KV pages, so they clear
    ``counts`` and every kernel of the step masks all of its cache accesses."""
    previous = getattr(_scope, "dummy", False)
    _scope.dummy = bool(capturing)
    try:
        yield
    finally:
        _scope.dummy = previous


def in_dummy_run():
    return getattr(_scope, "dummy", False)


def _state_name(state):
    return getattr(state, "name", state)


def _graph_support_uniform_batch():
    try:
        from vllm.v1.attention.backend import AttentionCGSupport
    except ImportError:
        return "UNIFORM_BATCH"
    return AttentionCGSupport.UNIFORM_BATCH


class OscarMetadataBuilder:
    """Reference metadata.py:36-174."""

    supports_update_block_table = False

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        from .backend import OscarAttentionImpl

        context = vllm_config.compilation_config.static_forward_context
        for name in layer_names:
            if not isinstance(context[name].impl, OscarAttentionImpl):
                raise TypeError(f"layer {name} is no longer served by OSCAR attention (its "
                                "implementation was replaced after routing)")
        spec = vllm_config.speculative_config
        cfg = OscarConfig.from_env(spec.num_speculative_tokens if spec else 0)
        layout = CacheLayout(kv_cache_spec.block_size, kv_cache_spec.num_kv_heads, config=cfg)
        sched = vllm_config.scheduler_config
        self.kv_cache_spec, self.layer_names, self.vllm_config = kv_cache_spec, layer_names, vllm_config
        self._allocate(layout, sched.max_num_seqs, sched.max_num_batched_tokens,
                       vllm_config.model_config.max_model_len, device)

    @classmethod
    def standalone(cls, layout, max_num_seqs, max_num_batched_tokens, max_model_len, device):
        """A builder outside a vLLM engine (benchmarks and tests)."""
        self = cls.__new__(cls)
        self.kv_cache_spec = self.layer_names = self.vllm_config = None
        self._allocate(layout, max_num_seqs, max_num_batched_tokens, max_model_len, device)
        return self

    def _allocate(self, layout, max_num_seqs, max_num_batched_tokens, max_model_len, device):
        cfg = layout.config
        self.layout = layout
        self.device = torch.device(device)
        self.query_tile = cfg.queries_per_tile
        # vLLM treats requests with up to spec + 1 query tokens as decodes.
        self.reorder_batch_threshold = cfg.speculative_tokens + 1
        self.max_reqs = max_num_seqs + 1  # graph padding may add one dummy request row
        # Padding slots and the MTP tail the native block table allows.
        self.max_tokens = max_num_batched_tokens + (cfg.speculative_tokens + 4) * self.max_reqs
        columns = math.ceil(max_model_len / layout.kernel_block_tokens) + layout.blocks_per_page + 1
        i32 = dict(dtype=torch.int32, device=device)
        self.qstarts = torch.zeros(self.max_reqs + 1, **i32)
        self.seqs = torch.zeros(self.max_reqs, **i32)
        self.table = torch.zeros((self.max_reqs, columns), **i32)
        self.slots = torch.full((self.max_tokens,), -1, dtype=torch.int64, device=device)
        self.counts = torch.zeros(2, **i32)
        self.tasks = torch.zeros(
            (task_capacity(self.max_tokens, self.max_reqs, self.query_tile), 2), **i32)
        self.task_count = torch.zeros(1, **i32)
        # Completion counters of the one-launch history + post form: one per (task, kv head)
        # of the largest grid, allocated once (graphs keep the address), left zero by every
        # launch.
        self.finish_counters = torch.zeros(self.tasks.shape[0] * layout.kv_heads, **i32)
        # Work-queue counters of the 17-32-row history launch (token-bounded splits), zero at
        # rest like the completion counters.
        self.queue_counters = torch.zeros(2, **i32)

    @classmethod
    def get_cudagraph_support(cls, vllm_config=None, kv_cache_spec=None):
        """Graphs of uniform decode batches (what vLLM dispatches to the graph path)."""
        return _graph_support_uniform_batch()

    def reorder_batch(self, input_batch, scheduler_output):
        return False

    def _check(self, cm, common_prefix_len):
        if common_prefix_len:
            raise ValueError("OSCAR cannot share a prefix between requests: each request's "
                             "BF16 ring lives in its own first page")
        if not getattr(cm, "causal", True):
            raise ValueError("OSCAR serves causal decoder attention only")
        if cm.num_reqs > self.max_reqs or cm.num_actual_tokens > self.max_tokens:
            raise ValueError(f"step of {cm.num_reqs} requests / {cm.num_actual_tokens} tokens "
                             f"exceeds the OSCAR buffers ({self.max_reqs} / {self.max_tokens})")
        if cm.block_table_tensor.shape[1] > self.table.shape[1]:
            raise ValueError("the block table is wider than the OSCAR table buffer")
        for name in ("query_start_loc", "seq_lens", "block_table_tensor", "slot_mapping"):
            if getattr(cm, name).device.type != self.device.type:
                raise ValueError(f"{name} must be on the {self.device.type} device (no host "
                                 "round trips)")

    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        """Reference metadata.py:82-161: fill the fixed buffers for one step."""
        cm = common_attn_metadata
        self._check(cm, common_prefix_len)
        nr, nt = cm.num_reqs, cm.num_actual_tokens
        columns = cm.block_table_tensor.shape[1]
        dummy = in_dummy_run()
        max_seq_len = getattr(cm, "max_seq_len", None)
        copy_columns = 0
        if dummy:
            # A capture run owns no pages, and vLLM invalidates its slot mapping after this
            # build: zero counts mask every cache access while every launch is recorded.
            self.counts.zero_()
        else:
            self.qstarts[: nr + 1].copy_(cm.query_start_loc[: nr + 1], non_blocking=True)
            self.seqs[:nr].copy_(cm.seq_lens[:nr], non_blocking=True)
            self.slots[:nt].copy_(cm.slot_mapping[:nt], non_blocking=True)
            self.counts[0].fill_(nr)
            self.counts[1].fill_(nt)
            # Only the columns the longest request can reach (host-side bound) are copied.
            copy_columns = columns
            if isinstance(max_seq_len, int):
                block = self.layout.kernel_block_tokens
                copy_columns = min(columns, max(1, -(-max_seq_len // block)))
        # An initial prefill is recognized from the scheduler's host state only, never from a
        # read of device lengths; its query ends come from the host copy of the query starts.
        state = getattr(cm, "attn_state", None)
        initial = not dummy and _state_name(state) == "PrefillNoCache"
        query_ends = None
        if initial:
            host = getattr(cm, "query_start_loc_cpu", None)
            if host is None or getattr(host, "device", None) is None or host.device.type != "cpu":
                raise ValueError("query_start_loc_cpu must really be on CPU")
            query_ends = host[1 : nr + 1].tolist()
        kernels.prepare_tasks(self.qstarts, self.counts, self.tasks, self.task_count,
                              self.max_reqs, self.query_tile, num_reqs=1 if dummy else nr,
                              source_table=cm.block_table_tensor, table=self.table,
                              copy_columns=copy_columns)
        seq_cpu = getattr(cm, "seq_lens_cpu", None)
        return OscarMetadata(
            self.qstarts, self.seqs, self.table, self.slots, self.counts, nr, nt,
            cm.max_query_len, self.max_reqs, self.layout, attn_state=state,
            initial_prefill=initial, actual_seq_lengths_q=query_ends,
            causal=getattr(cm, "causal", True), is_dummy=dummy, tasks=self.tasks,
            task_count=self.task_count, max_seq_len=max_seq_len,
            finish_counters=self.finish_counters, queue_counters=self.queue_counters,
            total_seq_len=None if dummy or seq_cpu is None else int(seq_cpu[:nr].sum()),
        )

    def build_for_cudagraph_capture(self, common_attn_metadata, attn_state="DecodeOnly"):
        """Reference metadata.py:163-170: a dummy build, marked as a decode step."""
        with dummy_run_scope(capturing=True):
            meta = self.build(0, common_attn_metadata)
        meta.initial_prefill = False
        meta.actual_seq_lengths_q = None
        meta.attn_state = attn_state
        return meta

    build_for_graph_capture = build_for_cudagraph_capture

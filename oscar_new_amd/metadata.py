"""Fixed-pointer device metadata for graph capture (vLLM-free builder).

Reference: oscar_ascend/metadata.py:15-174. Buffers are allocated once; ``build`` copies the
scheduler's per-step metadata into them in place (asynchronous device copies, no host
reads), so a captured HIP graph replays with new lengths, pages and request counts. A dummy
(capture) build zeroes ``counts``, which masks every KV access on device.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .config import OscarConfig, task_capacity
from .layout import CacheLayout
from . import kernels


@dataclass
class OscarMetadata:
    """Reference: metadata.py:15-33 (plus ``max_seq_len``, a host upper bound)."""

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
    is_dummy: bool = False
    tasks: torch.Tensor | None = None
    task_count: torch.Tensor | None = None
    max_seq_len: int | None = None
    merged_lse: torch.Tensor | None = None
    total_seq_len: int | None = None  # host-side sum of seq_lens (MI355X split partition)
    initial_prefill: bool = False  # every request starts here (host scheduler state)
    query_ends: list | None = None  # cumulative query ends (host), for initial prefill


class OscarMetadataBuilder:
    """Reference: metadata.py:36-174 without the vLLM base class.

    ``common`` passed to ``build`` is duck-typed like vLLM's CommonAttentionMetadata:
    ``num_reqs``, ``num_actual_tokens``, ``max_query_len``, ``query_start_loc``,
    ``seq_lens``, ``block_table_tensor``, ``slot_mapping`` (device tensors) and optionally
    ``max_seq_len`` (host int), ``seq_lens_cpu`` (host tensor, for the batch's total history)
    and ``causal``.
    """

    def __init__(self, layout: CacheLayout, max_num_seqs: int, max_num_batched_tokens: int,
                 max_model_len: int, device, cfg: OscarConfig | None = None):
        cfg = cfg or layout.config
        self.layout = layout
        self.query_tile = cfg.queries_per_tile
        self.max_reqs = max_num_seqs + 1  # graph padding may add one dummy request row
        self.max_tokens = max_num_batched_tokens + (cfg.speculative_tokens + 4) * self.max_reqs
        columns = math.ceil(max_model_len / layout.kernel_block_tokens) + layout.blocks_per_page + 1
        i32 = dict(dtype=torch.int32, device=device)
        self.qstarts = torch.zeros(self.max_reqs + 1, **i32)
        self.seqs = torch.zeros(self.max_reqs, **i32)
        self.table = torch.zeros((self.max_reqs, columns), **i32)
        self.slots = torch.full((self.max_tokens,), -1, dtype=torch.int64, device=device)
        self.counts = torch.zeros(2, **i32)
        self.tasks = torch.zeros((task_capacity(self.max_tokens, self.max_reqs, self.query_tile), 2),
                                 **i32)
        self.task_count = torch.zeros(1, **i32)

    def build(self, common, dummy: bool = False) -> OscarMetadata:
        """Reference: metadata.py:82-161."""
        if not getattr(common, "causal", True):
            raise ValueError("OSCAR supports causal decoder attention only")
        nr, nt = common.num_reqs, common.num_actual_tokens
        if nr > self.max_reqs or nt > self.max_tokens:
            raise ValueError("OSCAR metadata capacity exceeded")
        columns = common.block_table_tensor.shape[1]
        if columns > self.table.shape[1]:
            raise ValueError("block table exceeds the configured OSCAR buffer")
        copy_columns = 0
        if dummy:
            self.counts.zero_()
        else:
            self.qstarts[: nr + 1].copy_(common.query_start_loc[: nr + 1], non_blocking=True)
            self.seqs[:nr].copy_(common.seq_lens[:nr], non_blocking=True)
            copy_columns = columns
            max_seq_len = getattr(common, "max_seq_len", None)
            if isinstance(max_seq_len, int):
                block = self.layout.kernel_block_tokens
                copy_columns = min(columns, max(1, -(-max_seq_len // block)))
            self.slots[:nt].copy_(common.slot_mapping[:nt], non_blocking=True)
            self.counts[0].fill_(nr)
            self.counts[1].fill_(nt)
        kernels.prepare_tasks(self.qstarts, self.counts, self.tasks, self.task_count,
                              self.max_reqs, self.query_tile, num_reqs=1 if dummy else nr,
                              source_table=common.block_table_tensor, table=self.table,
                              copy_columns=copy_columns)
        seq_cpu = getattr(common, "seq_lens_cpu", None)
        # Reference metadata.py:120-128: only the scheduler's host state marks an initial
        # prefill (no device read); its query ends come from the host copy of qstarts.
        state = getattr(common, "attn_state", None)
        initial = not dummy and getattr(state, "name", state) == "PrefillNoCache"
        query_ends = None
        if initial:
            qcpu = getattr(common, "query_start_loc_cpu", None)
            if qcpu is None or getattr(qcpu, "device", None) is None or qcpu.device.type != "cpu":
                raise ValueError("query_start_loc_cpu must really be on CPU")
            query_ends = qcpu[1 : nr + 1].tolist()
        return OscarMetadata(
            self.qstarts, self.seqs, self.table, self.slots, self.counts, nr, nt,
            common.max_query_len, self.max_reqs, self.layout, is_dummy=dummy, tasks=self.tasks,
            task_count=self.task_count, max_seq_len=getattr(common, "max_seq_len", None),
            total_seq_len=None if dummy or seq_cpu is None else int(seq_cpu[:nr].sum()),
            initial_prefill=initial, query_ends=query_ends,
        )

"""OSCAR INT2 KV-cache kernels for MI355X, behind the reference's Python entry points.

Same names, signatures, return values and error behaviour as ``oscar_ascend/kernels.py``
(reference), so the backend glue and tests can import either module. Every function
launches hand-written gfx950 HIP kernels through the C ABI of ``liboscar_hip.so`` on the
current HIP stream; there is no CPU execution path, no host read-back and no
synchronization. Output tensors are allocated with ``torch.empty`` on the input's device,
as in the reference.
"""

from __future__ import annotations

import torch

from . import _ext
from .config import CLIP_MODES, attention_programs

__all__ = [
    "rotate",
    "store_int2",
    "prepare_tasks",
    "attention_partials",
    "merge_splits",
    "merge_paths",
    "store_windows",
    "dequant_inverse_rotate",
    "pre_attention",
    "post_attention",
    "history_post",
    "layer_step",
    "history_pre",
    "history_pre_supported",
    "layout_struct",
    "clip_struct",
]


# --------------------------------------------------------------------------- helpers


def _device_check(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("OSCAR kernels run on a ROCm GPU; got a tensor on " + str(t.device))


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _bf16(t):
    """The reference kernels cast their inputs to bf16 on load; do the same up front."""
    return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)


def _rows_contiguous(t):
    """bf16 [n, h, d] view with unit last stride and 16-byte aligned rows, copying if needed."""
    t = _bf16(t)
    s0, s1, s2 = t.stride()
    if s2 != 1 or s0 % 8 or s1 % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def layout_struct(layout):
    """``CacheLayout`` -> C ``oscar_layout``."""
    cfg = layout.config
    return _ext.OscarLayout(
        cfg.head_dim,
        layout.kv_heads,
        layout.physical_block_tokens,
        layout.kernel_block_tokens,
        cfg.slot_bytes,
        cfg.vector_bytes,
        cfg.sink_tokens,
        cfg.recent_tokens,
        cfg.ring_tokens,
        0,
        layout.stripe_page_bytes,
    )


def clip_struct(cfg):
    """``OscarConfig`` -> C ``oscar_clip``."""
    return _ext.OscarClip(
        CLIP_MODES[cfg.clip_mode],
        cfg.k_clip_ratio,
        cfg.v_clip_ratio,
        cfg.k_clip_factor,
        cfg.v_clip_factor,
    )


def _int32(t, name):
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    return t


# --------------------------------------------------------------------------- entry points


def rotate(x, rotation):
    """``x @ rotation`` per (token, head) row, bf16 out (reference kernels.py:51-66).

    x: [n, h, 256] any strides; rotation: [256, 256] (a transposed view is fine).
    """
    _device_check(x, rotation)
    n, h, d = x.shape
    out = torch.empty((n, h, d), device=x.device, dtype=torch.bfloat16)
    if n:
        x = _bf16(x)
        rotation = _bf16(rotation)
        _ext.check(
            _ext.library().oscar_rotate(
                _ptr(x), n, h, d, *x.stride(), _ptr(rotation), *rotation.stride(), _ptr(out),
                _stream(x),
            ),
            "rotate",
        )
    return out


def store_int2(key_rot, value_rot, history, slots, counts, layout):
    """Clip + INT2 pack rotated K/V into 160-byte slots (reference kernels.py:175-202)."""
    _device_check(key_rot, value_rot, history, slots, counts)
    n = key_rot.shape[0]
    key_rot = _bf16(key_rot).contiguous()
    value_rot = _bf16(value_rot).contiguous()
    if slots.dtype != torch.int64:
        raise ValueError("slot mapping must be int64")
    _int32(counts, "counts")
    lay = layout_struct(layout)
    clip = clip_struct(layout.config)
    _ext.check(
        _ext.library().oscar_store_int2(
            _ptr(key_rot), _ptr(value_rot), n, _ptr(history), history.numel() * history.element_size(),
            _ptr(slots), _ptr(counts), lay, clip, _stream(key_rot),
        ),
        "store_int2",
    )


def rotate_store_int2(key, value, rk_t, rv_t, history, slots, counts, layout):
    """``store_int2(rotate(key, Rk), rotate(value, Rv), ...)`` as one launch (the same
    cache bytes; the rotated rows stay on chip). ``rk_t``/``rv_t`` are R^T as contiguous
    bf16 [256, 256]; ``key``/``value`` are bf16 [n, kv_heads, 256] with contiguous rows.
    Reference: backend.py:171-173 (kernels.py:51-66, 175-202)."""
    _device_check(key, value, rk_t, rv_t, history, slots, counts)
    n = key.shape[0]
    if value.shape[0] != n:
        raise ValueError("key and value must have the same token count")
    for r in (rk_t, rv_t):
        if r.dtype != torch.bfloat16 or not r.is_contiguous() or tuple(r.shape) != (256, 256):
            raise ValueError("rk_t / rv_t must be contiguous bf16 [256, 256] (R transposed)")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    if slots.dtype != torch.int64:
        raise ValueError("slot mapping must be int64")
    _int32(counts, "counts")
    _ext.check(
        _ext.library().oscar_rotate_store_int2(
            _ptr(key), k0, k1, _ptr(value), v0, v1, n, _ptr(rk_t), _ptr(rv_t), _ptr(history),
            history.numel() * history.element_size(), _ptr(slots), _ptr(counts),
            layout_struct(layout), clip_struct(layout.config), _stream(key),
        ),
        "rotate_store_int2",
    )


def prepare_tasks(qstarts, counts, tasks, task_count, max_reqs, query_tile, num_reqs=None,
                  source_table=None, table=None, copy_columns=0):
    """Compact (request, query offset) task table on device (reference kernels.py:262-287)."""
    _device_check(qstarts, counts, tasks, task_count, source_table, table)
    _int32(qstarts, "qstarts")
    _int32(counts, "counts")
    _int32(tasks, "tasks")
    _int32(task_count, "task_count")
    programs = max(1, max_reqs if num_reqs is None else num_reqs)
    src_stride = table_stride = 0
    if source_table is not None:
        if table is None:
            raise ValueError("prepare_tasks: source_table given without a destination table")
        source_table = _int32(source_table.as_subclass(torch.Tensor), "source_table")
        _int32(table, "table")
        src_stride = source_table.stride(0)
        table_stride = table.stride(0)
    _ext.check(
        _ext.library().oscar_prepare_tasks(
            _ptr(qstarts), _ptr(counts), _ptr(tasks), _ptr(task_count), tasks.shape[0],
            max_reqs, query_tile, programs, _ptr(source_table), src_stride,
            _ptr(table) if source_table is not None else None, table_stride,
            int(copy_columns) if source_table is not None else 0, _stream(qstarts),
        ),
        "prepare_tasks",
    )


def attention_partials(query, key, value, history, window, meta, layout, scale, splits, raw,
                       split_tokens=0, use_queue=True):
    """Per-split partial attention and LSE of one branch (reference kernels.py:439-482).

    raw=False: INT2 history (``query`` must be the rotated query). raw=True: BF16 sink /
    recent window plus causal current tokens (unrotated query/key/value).
    Returns ``(partials float32 [n, hq, splits, 256], lse float32 [n, hq, splits])``.
    ``meta.max_query_len``, when present, lets decode steps skip query-tile padding rows.
    ``split_tokens`` (history branch; no reference counterpart, 0 keeps kernels.py:368-370):
    a request with L history tokens uses min(splits, ceil(L / split_tokens)) splits and its
    remaining split slots get LSE -inf with no partial row, which the split merges skip.
    A negative value is the device rule (``config.DEVICE_RULE``): the same token-bounded
    splits with the split length derived on the GPU from the step's lengths for a budget of
    ``-split_tokens`` workgroups, so that a captured launch stays balanced at any lengths.
    ``use_queue`` (no reference counterpart): tasks of 17-32 rows with token-bounded splits
    run as a work queue over the units in use (``queue_counters``); the same bits as the
    grid form (``use_queue=False``).
    """
    if raw and split_tokens:
        raise ValueError("split_tokens applies to the history branch only")
    _device_check(query, key, value, history, window)
    n, hq, d = query.shape
    cfg = layout.config
    partials = torch.empty((n, hq, splits, d), dtype=torch.float32, device=query.device)
    lse = torch.empty((n, hq, splits), dtype=torch.float32, device=query.device)
    if n == 0:
        return partials, lse
    programs = attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile)
    if meta.tasks.shape[0] < programs:
        raise ValueError(f"task table holds {meta.tasks.shape[0]} rows; the grid needs {programs}")
    query = _rows_contiguous(query)
    if raw:
        key = _rows_contiguous(key)
        value = _rows_contiguous(value)
    table = _int32(meta.block_tables, "block_tables")
    max_query_len = getattr(meta, "max_query_len", None)
    max_query_len = int(max_query_len) if isinstance(max_query_len, int) else 0
    kq = key if raw else None
    vq = value if raw else None
    _ext.check(
        _ext.library().oscar_attention_partials(
            _ptr(query), *query.stride(),
            _ptr(kq), *(kq.stride() if raw else (0, 0, 1)),
            _ptr(vq), *(vq.stride() if raw else (0, 0, 1)),
            _ptr(history), history.numel() * history.element_size(),
            _ptr(window), window.numel(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")),
            _ptr(table), table.stride(0), table.shape[1],
            _ptr(_int32(meta.counts, "counts")), _ptr(_int32(meta.tasks, "tasks")),
            _ptr(_int32(meta.task_count, "task_count")),
            n, hq, programs, splits, cfg.block_n, cfg.queries_per_tile, max_query_len,
            float(scale), 1 if raw else 0, int(split_tokens), layout_struct(layout),
            _ptr(partials), _ptr(lse),
            _ptr(queue_counters(meta, query.device))
            if use_queue and not raw and split_tokens else None,
            _stream(query),
        ),
        "attention_partials",
    )
    return partials, lse


def merge_splits(partials, lse, counts):
    """LSE merge of split partials (reference kernels.py:506-511) -> (bf16 out, logsum)."""
    _device_check(partials, lse, counts)
    n, hq, splits, d = partials.shape
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=partials.device)
    logsum = torch.empty((n, hq), dtype=torch.float32, device=partials.device)
    if n:
        partials = partials.contiguous()
        lse = lse.contiguous()
        _ext.check(
            _ext.library().oscar_merge_splits(
                _ptr(partials), _ptr(lse), _ptr(_int32(counts, "counts")), n, hq, splits, d,
                _ptr(out), _ptr(logsum), _stream(partials),
            ),
            "merge_splits",
        )
    return out, logsum


def merge_paths(history_out, history_lse, raw_partials, raw_lse, counts, output, merged_lse=None):
    """History/raw LSE merge into ``output`` (reference kernels.py:530-541).

    ``merged_lse`` (optional float32 [n, hq]) additionally receives the merged LSE, which
    the reference does not produce.
    """
    _device_check(history_out, history_lse, raw_partials, raw_lse, counts, output, merged_lse)
    n, hq, d = history_out.shape
    if not output.is_contiguous():
        raise ValueError("Attention output must be contiguous")
    if n == 0:
        return
    history_out = _bf16(history_out).contiguous()
    raw_partials = raw_partials.contiguous()
    _ext.check(
        _ext.library().oscar_merge_paths(
            _ptr(history_out), _ptr(history_lse.contiguous()), _ptr(raw_partials),
            _ptr(raw_lse.contiguous()), _ptr(_int32(counts, "counts")), n, hq, d, _ptr(output),
            _ptr(merged_lse), _stream(history_out),
        ),
        "merge_paths",
    )


def store_windows(key, value, window, meta, layout):
    """Write current BF16 K/V into sink/ring windows (reference kernels.py:598-620)."""
    _device_check(key, value, window)
    n = key.shape[0]
    key = _bf16(key)
    value = _bf16(value)
    table = _int32(meta.block_tables, "block_tables")
    _ext.check(
        _ext.library().oscar_store_windows(
            _ptr(key), *key.stride(), _ptr(value), *value.stride(), n, _ptr(window),
            window.numel(), _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(table), table.stride(0),
            _ptr(_int32(meta.counts, "counts")), meta.max_num_reqs, layout_struct(layout),
            _stream(key),
        ),
        "store_windows",
    )


def dequant_inverse_rotate(history, slots, rk, rv, layout):
    """Diagnostic unpack + inverse rotation of <= 4096 slots (reference kernels.py:651-672)."""
    _device_check(history, slots, rk, rv)
    n, h, d = slots.numel(), layout.kv_heads, layout.config.head_dim
    if n > 4096:
        raise ValueError("Diagnostic dequant is limited to 4096 tokens; use fused attention")
    k = torch.empty((n, h, d), device=history.device, dtype=torch.bfloat16)
    v = torch.empty_like(k)
    if n:
        slots = slots.to(torch.int64).contiguous()
        _ext.check(
            _ext.library().oscar_unpack(
                _ptr(history), history.numel() * history.element_size(), _ptr(slots), n,
                layout_struct(layout), _ptr(k), _ptr(v), _stream(history),
            ),
            "dequant_inverse_rotate",
        )
    return rotate(k, rk.T), rotate(v, rv.T)


# --------------------------------------------------------------------------- fused launches
#
# Not reference entry points: the backend's layer step uses these two launches around the
# history kernel instead of the nine single launches above (same bits, fewer launches).


def _row_strides(t, name):
    t = _bf16(t)
    s0, s1, s2 = t.stride()
    if s2 != 1 or s0 % 8 or s1 % 8 or t.data_ptr() % 16:
        raise ValueError(f"{name} rows must be contiguous and 16-byte aligned")
    return t, s0, s1


def pre_attention(query, key, value, history, window, meta, layout, scale, rk_t, rv_t,
                  raw=True):
    """BF16-branch partials, q rotation and the K/V INT2 store of one step, in one launch.

    Replaces ``rotate(key, Rk)``, ``rotate(value, Rv)``, ``store_int2``, ``rotate(query, Rk)``
    and ``attention_partials(..., 1, raw=True)`` of the reference layer step
    (backend.py:171-173, 195, 211-222). ``rk_t``/``rv_t`` are R^T as contiguous bf16 [256, 256].
    Returns ``(qrot bf16 [n, hq, 256], raw_partials fp32 [n, hq, 1, 256], raw_lse [n, hq, 1])``.
    ``raw=False``: the launch leaves the BF16 branch out and the partials come from
    ``chunk_raw_attention`` (a launch of its own, for long chunks), with the same bits. From
    SPLIT_PRE_ROWS query rows on, the q rotation and the K/V store run as ``rotate`` (the
    tiled form: R staged once per workgroup) and ``rotate_store_int2`` (32-row workgroups)
    instead of role workgroups that each read R from L2 for one 16-row tile: the same bits.
    """
    _device_check(query, key, value, history, window, rk_t, rv_t)
    n, hq, d = query.shape
    cfg = layout.config
    if not raw and n * hq >= SPLIT_PRE_ROWS and n > 0:
        qrot = rotate(query, rk_t.t())
        rotate_store_int2(key, value, rk_t, rv_t, history, meta.slot_mapping, meta.counts,
                          layout)
        partials, lse = chunk_raw_attention(query, key, value, window, meta, layout, scale)
        return qrot, partials, lse
    qrot = torch.empty((n, hq, d), dtype=torch.bfloat16, device=query.device)
    partials = torch.empty((n, hq, 1, d), dtype=torch.float32, device=query.device)
    lse = torch.empty((n, hq, 1), dtype=torch.float32, device=query.device)
    if n == 0:
        return qrot, partials, lse
    programs = attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile)
    if meta.tasks.shape[0] < programs:
        raise ValueError(f"task table holds {meta.tasks.shape[0]} rows; the grid needs {programs}")
    for r in (rk_t, rv_t):
        if r.dtype != torch.bfloat16 or not r.is_contiguous() or tuple(r.shape) != (d, d):
            raise ValueError("rk_t / rv_t must be contiguous bf16 [256, 256] (R transposed)")
    query, q0, q1 = _row_strides(query, "query")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    if meta.slot_mapping.dtype != torch.int64:
        raise ValueError("slot mapping must be int64")
    table = _int32(meta.block_tables, "block_tables")
    max_query_len = getattr(meta, "max_query_len", None)
    max_query_len = int(max_query_len) if isinstance(max_query_len, int) else 0
    _ext.check(
        _ext.library().oscar_pre_attention(
            _ptr(query), q0, q1, _ptr(key), k0, k1, _ptr(value), v0, v1,
            _ptr(window), window.numel(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(table), table.stride(0), table.shape[1],
            _ptr(_int32(meta.counts, "counts")), _ptr(_int32(meta.tasks, "tasks")),
            _ptr(_int32(meta.task_count, "task_count")),
            n, hq, programs, cfg.block_n, cfg.queries_per_tile, max_query_len, float(scale),
            _ptr(rk_t), _ptr(rv_t), _ptr(history), history.numel() * history.element_size(),
            _ptr(meta.slot_mapping), clip_struct(cfg), layout_struct(layout),
            _ptr(partials) if raw else None, _ptr(lse) if raw else None, _ptr(qrot),
            _stream(query),
        ),
        "pre_attention",
    )
    if not raw:
        chunk_raw_attention(query, key, value, window, meta, layout, scale, partials, lse)
    return qrot, partials, lse


# Query tokens per request from which a step's BF16 branch runs as the chunk flash launch
# (chunk_raw_attention) instead of decode-shaped roles of the pre-attention launch.
CHUNK_RAW_FROM = 64


# Query rows from which a long chunk's q rotation and K/V store leave the pre-attention launch
# for the tiled rotation and the fused rotate + store (pre_attention(raw=False)).
SPLIT_PRE_ROWS = 4096


def chunk_raw_preferred(meta):
    """Whether a step's BF16 branch runs as ``chunk_raw_attention``: a host bound of at least
    CHUNK_RAW_FROM query tokens per request (a continuation chunk)."""
    mql = getattr(meta, "max_query_len", None)
    return isinstance(mql, int) and mql >= CHUNK_RAW_FROM


def chunk_raw_attention(query, key, value, window, meta, layout, scale, partials=None, lse=None):
    """The BF16 branch (reference kernels.py:439-482: ``attention_partials(..., 1, raw=True)``,
    sink + recent window rows, then the chunk's current tokens causally) as a flash launch in
    which the rows of 32 consecutive query tokens share each 32-key block; the bits of
    ``attention_partials(..., 1, raw=True)``. Returns ``(partials fp32 [n, hq, 1, 256], lse
    fp32 [n, hq, 1])`` (into the given buffers when passed); rows of tokens at or past
    ``counts[1]`` are not written."""
    _device_check(query, key, value, window, partials, lse)
    n, hq, d = query.shape
    if partials is None:
        partials = torch.empty((n, hq, 1, d), dtype=torch.float32, device=query.device)
    if lse is None:
        lse = torch.empty((n, hq, 1), dtype=torch.float32, device=query.device)
    if (partials.dtype != torch.float32 or not partials.is_contiguous()
            or tuple(partials.shape) != (n, hq, 1, d)):
        raise ValueError("partials must be contiguous fp32 [n, hq, 1, 256]")
    if lse.dtype != torch.float32 or not lse.is_contiguous() or lse.numel() != n * hq:
        raise ValueError("lse must be contiguous fp32 [n, hq, 1]")
    if n == 0:
        return partials, lse
    query, q0, q1 = _row_strides(query, "query")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    table = _int32(meta.block_tables, "block_tables")
    max_query_len = getattr(meta, "max_query_len", None)
    max_query_len = int(max_query_len) if isinstance(max_query_len, int) else 0
    _ext.check(
        _ext.library().oscar_chunk_raw_attention(
            _ptr(query), q0, q1, _ptr(key), k0, k1, _ptr(value), v0, v1,
            _ptr(window), window.numel(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(table), table.stride(0), table.shape[1],
            _ptr(_int32(meta.counts, "counts")),
            n, hq, int(meta.max_num_reqs), max_query_len, float(scale), layout_struct(layout),
            _ptr(partials), _ptr(lse), _stream(query),
        ),
        "chunk_raw_attention",
    )
    return partials, lse


def prefill_attention(query, key, value, window, meta, layout, scale, output, merged_lse=None):
    """Initial prefill (every request's history empty): causal attention of each request over
    its own current tokens, written to ``output`` (contiguous bf16 [n, hq * 256]); rows past
    the token count are zeroed. Replaces the reference's fused-infer call
    (backend.py:175-193) with a flash kernel whose rows have the bits the INT2 path's BF16
    branch gives when the history is empty. ``window`` is not read (kept for the call's
    shape); requests with cached tokens get NaN rows."""
    _device_check(query, key, value, window, output, merged_lse)
    n, hq, d = query.shape
    if not output.is_contiguous():
        raise ValueError("Attention output must be contiguous")
    if n == 0:
        return output
    query, q0, q1 = _row_strides(query, "query")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    max_query_len = getattr(meta, "max_query_len", None)
    max_query_len = int(max_query_len) if isinstance(max_query_len, int) else 0
    _ext.check(
        _ext.library().oscar_prefill_attention(
            _ptr(query), q0, q1, _ptr(key), k0, k1, _ptr(value), v0, v1,
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(_int32(meta.counts, "counts")),
            n, hq, int(meta.max_num_reqs), max_query_len, float(scale), layout_struct(layout),
            _ptr(output), _ptr(merged_lse), _stream(query),
        ),
        "prefill_attention",
    )
    return output


_COUNTERS = {}
_QUEUE_COUNTERS = {}
DEFAULT_COUNTER_SLOTS = 1 << 16


def finish_counters(meta, device, slots):
    """The int32 completion counters a ``history_post`` launch uses: the metadata's own
    (``meta.finish_counters``, sized by the builder from its task capacity) or else one
    per-device buffer of ``DEFAULT_COUNTER_SLOTS``. Both are allocated once, zeroed, and never
    replaced (a captured graph keeps their address); every launch leaves them zero. A launch
    needing more slots than they hold is refused. Launches that overlap on one device (two
    streams at once) must not share counters."""
    buf = getattr(meta, "finish_counters", None)
    if buf is None:
        buf = _COUNTERS.get(device)
        if buf is None:
            buf = torch.zeros(DEFAULT_COUNTER_SLOTS, dtype=torch.int32, device=device)
            _COUNTERS[device] = buf
    if buf.numel() < slots:
        raise ValueError(f"history_post needs {slots} completion counters; the buffer holds "
                         f"{buf.numel()}")
    return buf


def queue_counters(meta, device):
    """The two int32 work-queue counters of a history launch: the metadata's own
    (``meta.queue_counters``, allocated by the builder) or else one per-device buffer. Both
    are zero at rest: every launch leaves them zero, and a captured graph keeps their address.
    Launches that overlap on one device (two streams at once) must not share them."""
    buf = getattr(meta, "queue_counters", None)
    if buf is None:
        buf = _QUEUE_COUNTERS.get(device)
        if buf is None:
            buf = torch.zeros(2, dtype=torch.int32, device=device)
            _QUEUE_COUNTERS[device] = buf
    if buf.numel() < 2 or buf.dtype != torch.int32:
        raise ValueError("queue counters must be at least two int32 values")
    return buf


def history_rows(meta, layout, hq):
    """Query rows per history task: query tokens per task (``meta.max_query_len`` when it is
    below the tile) times the query heads of one KV head."""
    mql = getattr(meta, "max_query_len", None)
    qt = layout.config.queries_per_tile
    return (mql if isinstance(mql, int) and 0 < mql < qt else qt) * (hq // layout.kv_heads)


def history_kernel_name(meta, layout, hq, tokens=0, split_tokens=0, use_queue=True):
    """The history-branch kernel ``attention_partials`` launches for ``tokens`` query rows:
    the paired kernel up to 8 rows per task, the one-tile kernel up to 16, then the
    two-row-group kernel (four wavefronts per workgroup up to 512 task rows, eight above), as
    a work queue with token-bounded splits (``use_queue``, a grid of at most 2048 task
    rows)."""
    rows = history_rows(meta, layout, hq)
    if rows <= 8:
        return "history_pair_kernel"
    if rows <= 16:
        return "history_kernel<1>"
    programs = attention_programs(tokens, meta.max_num_reqs, layout.config.queries_per_tile)
    if use_queue and split_tokens and programs <= 2048:
        return "history_queue_kernel"
    return "history_w8_kernel"


def history_post_supported(meta, layout, hq, splits, tokens=None):
    """Whether ``history_post`` covers this launch: <= 8 query rows per task, <= 16 splits,
    split rows below 4 GiB (``tokens``: the launch's query rows n, when known)."""
    small = tokens is None or tokens * hq * splits * layout.config.head_dim * 4 < 1 << 32
    return history_rows(meta, layout, hq) <= 8 and 1 <= splits <= 16 and small


# Task rows of the four-wavefront history work queue (the MTP step's history launch).
QUEUE_PRE_TASKS = 512


def history_pre_supported(meta, layout, hq, split_tokens=None, tokens=None):
    """Whether ``history_pre`` covers this batch: <= 8 query rows per task (the paired history
    kernel and a one-tile BF16 branch), or, given the launch's ``split_tokens`` and query
    ``tokens``, 17-32 rows per task with token-bounded splits and at most QUEUE_PRE_TASKS task
    rows (the work queue with the roles as units of its own)."""
    rows = history_rows(meta, layout, hq)
    if rows <= 8:
        return True
    if not 16 < rows <= 32 or not split_tokens or tokens is None:
        return False
    return attention_programs(int(tokens), meta.max_num_reqs,
                              layout.config.queries_per_tile) <= QUEUE_PRE_TASKS


def history_pre(query_rot, query, key, value, history, window, meta, layout, scale, splits,
                rk_t, rv_t, split_tokens=0, q_sync=None):
    """The history branch and the pre-attention work other than the q rotation (BF16 branch,
    K/V INT2 store) in one launch, the latter as workgroups dispatched ahead of the history
    splits (no reference counterpart as one call; it replaces ``attention_partials(qrot, ...,
    raw=False)`` plus ``pre_attention`` without its q rotation, with their bits).

    ``query_rot``: the rotated query, or None: then the history workgroups rotate the query
    rows by R_k themselves (the bits of ``rotate(query, R_k)``; no launch of its own).
    ``q_sync`` (int32 [4] on the device, zero before the first call, left zero by every call):
    the q rotation runs as role workgroups of the same launch and ``query_rot`` is its output
    buffer (bf16 [n, hq, 256], contiguous), which the history workgroups read once the roles
    are done; ``q_sync[2]`` is non-zero after a launch in which a workgroup gave up waiting.
    ``query``/``key``/``value``: the step's unrotated rows. Returns ``(partials [n, hq, splits,
    256], lse [n, hq, splits], raw_partials [n, hq, 1, 256], raw_lse [n, hq, 1])``, all fp32.
    17-32 query rows per task (MTP) run as the history work queue with the BF16 branch and
    the K/V store as units of the queue (``query_rot`` given, token-bounded ``split_tokens``,
    ``meta``'s queue counters as for ``attention_partials``).
    """
    _device_check(query_rot, query, key, value, history, window, rk_t, rv_t)
    n, hq, d = query.shape
    cfg = layout.config
    if not history_pre_supported(meta, layout, hq, split_tokens, n):
        raise ValueError("history_pre covers <= 8 query rows per task, or 17-32 with "
                         "token-bounded splits and at most 512 task rows")
    queue = history_rows(meta, layout, hq) > 8
    if queue and (query_rot is None or q_sync is not None):
        raise ValueError("history_pre with 17-32 rows per task takes the rotated query")
    dev = query.device
    partials = torch.empty((n, hq, splits, d), dtype=torch.float32, device=dev)
    lse = torch.empty((n, hq, splits), dtype=torch.float32, device=dev)
    raw_partials = torch.empty((n, hq, 1, d), dtype=torch.float32, device=dev)
    raw_lse = torch.empty((n, hq, 1), dtype=torch.float32, device=dev)
    if n == 0:
        return partials, lse, raw_partials, raw_lse
    programs = attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile)
    if meta.tasks.shape[0] < programs:
        raise ValueError(f"task table holds {meta.tasks.shape[0]} rows; the grid needs {programs}")
    for r in (rk_t, rv_t):
        if r.dtype != torch.bfloat16 or not r.is_contiguous() or tuple(r.shape) != (d, d):
            raise ValueError("rk_t / rv_t must be contiguous bf16 [256, 256] (R transposed)")
    if q_sync is not None:
        if (query_rot is None or query_rot.dtype != torch.bfloat16 or not query_rot.is_contiguous()
                or tuple(query_rot.shape) != (n, hq, d)):
            raise ValueError("with q_sync, query_rot must be a contiguous bf16 [n, hq, 256] buffer")
        if q_sync.dtype != torch.int32 or q_sync.numel() < 4 or q_sync.device != dev:
            raise ValueError("q_sync must be an int32 device tensor of at least 4 elements")
    else:
        query_rot = _rows_contiguous(query_rot) if query_rot is not None else None
    rot_strides = query_rot.stride() if query_rot is not None else (0, 0, 1)
    query, q0, q1 = _row_strides(query, "query")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    if meta.slot_mapping.dtype != torch.int64:
        raise ValueError("slot mapping must be int64")
    table = _int32(meta.block_tables, "block_tables")
    max_query_len = getattr(meta, "max_query_len", None)
    max_query_len = int(max_query_len) if isinstance(max_query_len, int) else 0
    tail = ()
    if q_sync is not None:
        entry, lead = _ext.library().oscar_history_pre_q, (_ptr(query_rot), _ptr(q_sync))
    elif queue:
        entry, lead = _ext.library().oscar_history_pre_queue, (_ptr(query_rot), *rot_strides)
        tail = (_ptr(queue_counters(meta, dev)),)
    else:
        entry, lead = _ext.library().oscar_history_pre, (_ptr(query_rot), *rot_strides)
    _ext.check(
        entry(
            *lead, _ptr(query), q0, q1, _ptr(key), k0, k1,
            _ptr(value), v0, v1, _ptr(history), history.numel() * history.element_size(),
            _ptr(window), window.numel(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(table), table.stride(0), table.shape[1],
            _ptr(_int32(meta.counts, "counts")), _ptr(_int32(meta.tasks, "tasks")),
            _ptr(_int32(meta.task_count, "task_count")),
            n, hq, programs, splits, cfg.block_n, cfg.queries_per_tile, max_query_len,
            float(scale), int(split_tokens), _ptr(rk_t), _ptr(rv_t), _ptr(meta.slot_mapping),
            clip_struct(cfg), layout_struct(layout), _ptr(partials), _ptr(lse),
            _ptr(raw_partials), _ptr(raw_lse), *tail, _stream(query),
        ),
        "history_pre",
    )
    return partials, lse, raw_partials, raw_lse


def history_post(query, history, meta, layout, scale, splits, raw_partials, raw_lse, rv, key,
                 value, window, output, merged_lse=None, split_tokens=0):
    """History branch + post-attention of one step in ONE launch (no reference counterpart).

    Same output / merged LSE bits as ``attention_partials(raw=False)`` followed by
    ``post_attention`` (backend.py:205-226 order); the split workgroup that completes a
    (task, kv head) merges that task's rows. ``query`` is the rotated query [n, hq, 256].
    Requires ``history_post_supported``.
    """
    _device_check(query, history, raw_partials, raw_lse, rv, key, value, window, output,
                  merged_lse)
    n, hq, d = query.shape
    if not output.is_contiguous():
        raise ValueError("Attention output must be contiguous")
    if n == 0:
        return
    if not history_post_supported(meta, layout, hq, splits, n):
        raise ValueError("history_post covers <= 8 query rows per task, <= 16 splits and "
                         "split rows below 4 GiB")
    if split_tokens < 0:
        raise ValueError("history_post counts a grid of split slots: the device split rule "
                         "(split_tokens < 0) is not available")
    if rv.dtype != torch.bfloat16 or not rv.is_contiguous():
        raise ValueError("rv must be contiguous bf16 [256, 256]")
    cfg = layout.config
    programs = attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile)
    if meta.tasks.shape[0] < programs:
        raise ValueError(f"task table holds {meta.tasks.shape[0]} rows; the grid needs {programs}")
    query = _rows_contiguous(query)
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    partials = torch.empty((n, hq, splits, d), dtype=torch.float32, device=query.device)
    lse = torch.empty((n, hq, splits), dtype=torch.float32, device=query.device)
    stream = _stream(query)
    counters = finish_counters(meta, query.device, programs * layout.kv_heads)
    table = _int32(meta.block_tables, "block_tables")
    max_query_len = getattr(meta, "max_query_len", None)
    max_query_len = int(max_query_len) if isinstance(max_query_len, int) else 0
    _ext.check(
        _ext.library().oscar_history_post(
            _ptr(query), *query.stride(),
            _ptr(history), history.numel() * history.element_size(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")),
            _ptr(table), table.stride(0), table.shape[1],
            _ptr(_int32(meta.counts, "counts")), _ptr(_int32(meta.tasks, "tasks")),
            _ptr(_int32(meta.task_count, "task_count")),
            n, hq, programs, splits, cfg.block_n, cfg.queries_per_tile, max_query_len,
            float(scale), int(split_tokens), layout_struct(layout), _ptr(partials), _ptr(lse),
            _ptr(counters), counters.numel(),
            _ptr(raw_partials.contiguous()), _ptr(raw_lse.contiguous()), _ptr(rv), _ptr(output),
            _ptr(merged_lse), _ptr(key), k0, k1, _ptr(value), v0, v1, _ptr(window),
            window.numel(), meta.max_num_reqs, stream,
        ),
        "history_post",
    )


RAW_SPLITS = 4  # BF16-branch partials per row in layer_step


def layer_step_supported(meta, layout, hq, splits, tokens=None):
    """Whether ``layer_step`` covers this step: one task per request (1 <= max_query_len <=
    query_tile <= 4), <= 8 query rows per task, <= 16 splits, split rows below 4 GiB."""
    cfg = layout.config
    mql = getattr(meta, "max_query_len", None)
    qt = cfg.queries_per_tile
    if not isinstance(mql, int) or not 1 <= mql <= qt or qt > 4:
        return False
    rows = mql * (hq // layout.kv_heads)
    small = tokens is None or tokens * hq * splits * cfg.head_dim * 4 < 1 << 32
    return rows <= 8 and 1 <= splits <= 16 and small


def layer_step(query, key, value, history, window, meta, layout, scale, splits, rk_t, rv_t, rv,
               output, merged_lse=None, split_tokens=0):
    """One layer step in ONE launch (no reference counterpart): the work of backend.py:171-226
    (rotations, INT2 store, both attention branches, merges, inverse V rotation, window store)
    with the INT2 and window bytes of the single entry points and the output within rounding
    of them. ``query``/``key``/``value`` are the unrotated rows; ``rk_t``/``rv_t`` are R^T and
    ``rv`` is R_v, contiguous bf16 [256, 256]. Requires ``layer_step_supported``."""
    _device_check(query, key, value, history, window, rk_t, rv_t, rv, output, merged_lse)
    n, hq, d = query.shape
    if not output.is_contiguous():
        raise ValueError("Attention output must be contiguous")
    if split_tokens < 0:
        raise ValueError("layer_step counts a grid of split slots: the device split rule "
                         "(split_tokens < 0) is not available")
    if n == 0:
        return
    if not layer_step_supported(meta, layout, hq, splits, n):
        raise ValueError("layer_step covers one task per request, <= 8 query rows per task and "
                         "<= 16 splits")
    for r in (rk_t, rv_t, rv):
        if r.dtype != torch.bfloat16 or not r.is_contiguous() or tuple(r.shape) != (d, d):
            raise ValueError("rk_t / rv_t / rv must be contiguous bf16 [256, 256]")
    cfg = layout.config
    programs = attention_programs(n, meta.max_num_reqs, cfg.queries_per_tile)
    if meta.tasks.shape[0] < programs:
        raise ValueError(f"task table holds {meta.tasks.shape[0]} rows; the grid needs {programs}")
    if meta.slot_mapping.dtype != torch.int64:
        raise ValueError("slot mapping must be int64")
    query, q0, q1 = _row_strides(query, "query")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    dev = query.device
    partials = torch.empty((n, hq, splits, d), dtype=torch.float32, device=dev)
    lse = torch.empty((n, hq, splits), dtype=torch.float32, device=dev)
    raw_partials = torch.empty((n, hq, RAW_SPLITS, d), dtype=torch.float32, device=dev)
    raw_lse = torch.empty((n, hq, RAW_SPLITS), dtype=torch.float32, device=dev)
    counters = finish_counters(meta, dev, programs * layout.kv_heads)
    table = _int32(meta.block_tables, "block_tables")
    _ext.check(
        _ext.library().oscar_layer_step(
            _ptr(query), q0, q1, _ptr(key), k0, k1, _ptr(value), v0, v1,
            _ptr(history), history.numel() * history.element_size(), _ptr(window), window.numel(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(table), table.stride(0), table.shape[1],
            _ptr(_int32(meta.counts, "counts")), _ptr(_int32(meta.tasks, "tasks")),
            _ptr(_int32(meta.task_count, "task_count")), _ptr(meta.slot_mapping),
            n, hq, programs, splits, cfg.block_n, cfg.queries_per_tile, int(meta.max_query_len),
            float(scale), int(split_tokens), _ptr(rk_t), _ptr(rv_t), _ptr(rv), clip_struct(cfg),
            layout_struct(layout), _ptr(partials), _ptr(lse), _ptr(raw_partials), _ptr(raw_lse),
            _ptr(counters), counters.numel(), _ptr(output), _ptr(merged_lse), meta.max_num_reqs,
            _stream(query),
        ),
        "layer_step",
    )


def post_attention(history_partials, history_lse, raw_partials, raw_lse, rv, key, value, window,
                   meta, layout, output, merged_lse=None):
    """Split merge, inverse V rotation, path merge and window store of one step, in one launch.

    Replaces ``merge_splits``, ``rotate(hrot, Rv.T)``, ``merge_paths`` and ``store_windows``
    (backend.py:209-210, 223-226). ``rv`` is R_v as contiguous bf16 [256, 256]; ``output`` is
    the contiguous bf16 [n, hq * 256] attention output.
    """
    _device_check(history_partials, history_lse, raw_partials, raw_lse, rv, key, value, window,
                  output, merged_lse)
    n, hq, splits, d = history_partials.shape
    if not output.is_contiguous():
        raise ValueError("Attention output must be contiguous")
    if n == 0:
        return
    if rv.dtype != torch.bfloat16 or not rv.is_contiguous():
        raise ValueError("rv must be contiguous bf16 [256, 256]")
    key, k0, k1 = _row_strides(key, "key")
    value, v0, v1 = _row_strides(value, "value")
    table = _int32(meta.block_tables, "block_tables")
    _ext.check(
        _ext.library().oscar_post_attention(
            _ptr(history_partials.contiguous()), _ptr(history_lse.contiguous()), splits,
            _ptr(raw_partials.contiguous()), _ptr(raw_lse.contiguous()),
            _ptr(_int32(meta.counts, "counts")), _ptr(rv), n, hq, _ptr(output), _ptr(merged_lse),
            _ptr(key), k0, k1, _ptr(value), v0, v1, _ptr(window), window.numel(),
            _ptr(_int32(meta.query_start_loc, "query_start_loc")),
            _ptr(_int32(meta.seq_lens, "seq_lens")), _ptr(table), table.stride(0),
            meta.max_num_reqs, layout_struct(layout), _stream(history_partials),
        ),
        "post_attention",
    )

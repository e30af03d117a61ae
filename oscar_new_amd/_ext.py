"""ctypes binding of ``liboscar_hip.so`` (the C ABI declared in ``include/oscar_hip.h``).

The library is loaded from this package directory only. There is no fallback: if the
library is missing or a call fails, a Python exception is raised.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_int64, c_void_p
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "liboscar_hip.so"

# Entry points exported by the library: name -> (argtypes). All return int.
_P = c_void_p
_I64 = c_int64
_I32 = c_int32
_F = c_float


class OscarLayout(ctypes.Structure):
    """Mirror of ``struct oscar_layout``."""

    _fields_ = [
        ("head_dim", c_int32),
        ("kv_heads", c_int32),
        ("physical_block_tokens", c_int32),
        ("kernel_block_tokens", c_int32),
        ("slot_bytes", c_int32),
        ("vector_bytes", c_int32),
        ("sink_tokens", c_int32),
        ("recent_tokens", c_int32),
        ("ring_tokens", c_int32),
        ("reserved", c_int32),
        ("stripe_page_bytes", c_int64),
    ]


class OscarClip(ctypes.Structure):
    """Mirror of ``struct oscar_clip``."""

    _fields_ = [
        ("mode", c_int32),
        ("k_ratio", c_float),
        ("v_ratio", c_float),
        ("k_factor", c_float),
        ("v_factor", c_float),
    ]


SIGNATURES = {
    "oscar_abi_version": [],
    "oscar_rotate": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _P],
    "oscar_store_int2": [_P, _P, _I64, _P, _I64, _P, _P, POINTER(OscarLayout),
                         POINTER(OscarClip), _P],
    "oscar_rotate_store_int2": [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P,
                                POINTER(OscarLayout), POINTER(OscarClip), _P],
    "oscar_prepare_tasks": [_P, _P, _P, _P, _I64, _I64, _I32, _I64, _P, _I64, _P, _I64, _I64,
                            _P],
    "oscar_attention_partials": [
        _P, _I64, _I64, _I64,  # query
        _P, _I64, _I64, _I64,  # key
        _P, _I64, _I64, _I64,  # value
        _P, _I64, _P, _I64,  # history, window
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale raw
        _I32,  # split_tokens
        POINTER(OscarLayout), _P, _P, _P, _P,  # layout, partials, lse, queue counters, stream
    ],
    "oscar_merge_splits": [_P, _P, _P, _I64, _I64, _I32, _I32, _P, _P, _P],
    "oscar_merge_paths": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _P, _P, _P],
    "oscar_store_windows": [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P,
                            _P, _I64, _P, _I64, POINTER(OscarLayout), _P],
    "oscar_unpack": [_P, _I64, _P, _I64, POINTER(OscarLayout), _P, _P, _P],
    "oscar_pre_attention": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _I64,  # window
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _F,  # n hq programs bn qt mql scale
        _P, _P,  # rk_t, rv_t
        _P, _I64, _P, POINTER(OscarClip),  # history, bytes, slots, clip
        POINTER(OscarLayout), _P, _P, _P, _P,  # layout, raw partials, raw lse, qrot, stream
    ],
    "oscar_post_attention": [
        _P, _P, _I32, _P, _P, _P, _P,  # hp, hl, splits, rp, rl, counts, rv
        _I64, _I64, _P, _P,  # n, hq, output, merged_lse
        _P, _I64, _I64, _P, _I64, _I64,  # key, value (+ row strides)
        _P, _I64, _P, _P, _P, _I64, _I64,  # window, elems, qstarts, seq_lens, table, stride, max_reqs
        POINTER(OscarLayout), _P,
    ],
    "oscar_prefill_attention": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _P, _P,  # qstarts, seq_lens, counts
        _I64, _I64, _I64, _I32, _F,  # n, hq, max_reqs, max_query_len, scale
        POINTER(OscarLayout), _P, _P, _P,  # layout, output, merged_lse, stream
    ],
    "oscar_chunk_raw_attention": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _I64,  # window, elements
        _P, _P, _P, _I64, _I64, _P,  # qstarts, seq_lens, block_tables, stride, columns, counts
        _I64, _I64, _I64, _I32, _F,  # n, hq, max_reqs, max_query_len, scale
        POINTER(OscarLayout), _P, _P, _P,  # layout, raw_partials, raw_lse, stream
    ],
    "oscar_history_post": [
        _P, _I64, _I64, _I64,  # query (rotated)
        _P, _I64,  # history, bytes
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale st
        POINTER(OscarLayout), _P, _P,  # layout, partials, lse
        _P, _I64,  # counters, slots
        _P, _P, _P, _P, _P,  # raw partials, raw lse, rv, output, merged_lse
        _P, _I64, _I64, _P, _I64, _I64,  # key, value (+ row strides)
        _P, _I64, _I64, _P,  # window, elems, max_reqs, stream
    ],
    "oscar_layer_step": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _I64, _P, _I64,  # history, bytes, window, elems
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P, _P,  # counts, tasks, task_count, slots
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale st
        _P, _P, _P, POINTER(OscarClip), POINTER(OscarLayout),  # rk_t, rv_t, rv, clip, layout
        _P, _P, _P, _P, _P, _I64,  # partials, lse, raw partials, raw lse, counters, slots
        _P, _P, _I64, _P,  # output, merged_lse, max_reqs, stream
    ],
    "oscar_history_post_noalloc": [
        _P, _I64, _I64, _I64,  # query (rotated)
        _P, _I64,  # history, bytes
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale st
        POINTER(OscarLayout),  # layout
        _P, _P, _P, _P, _P,  # raw partials, raw lse, rv, output, merged_lse
        _P, _I64, _I64, _P, _I64, _I64,  # key, value (+ row strides)
        _P, _I64, _I64, _P,  # window, elems, max_reqs, stream
    ],
    "oscar_history_pre": [
        _P, _I64, _I64, _I64,  # query (rotated)
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _I64, _P, _I64,  # history, bytes, window, elems
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale st
        _P, _P, _P, POINTER(OscarClip), POINTER(OscarLayout),  # rk_t, rv_t, slots, clip, layout
        _P, _P, _P, _P, _P,  # partials, lse, raw partials, raw lse, stream
    ],
    "oscar_history_pre_queue": [
        _P, _I64, _I64, _I64,  # query (rotated)
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _I64, _P, _I64,  # history, bytes, window, elems
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale st
        _P, _P, _P, POINTER(OscarClip), POINTER(OscarLayout),  # rk_t, rv_t, slots, clip, layout
        _P, _P, _P, _P, _P, _P,  # partials, lse, raw partials, raw lse, queue counters, stream
    ],
    "oscar_history_pre_q": [
        _P, _P,  # qrot (out), qsync
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # query, key, value (+ row strides)
        _P, _I64, _P, _I64,  # history, bytes, window, elems
        _P, _P, _P, _I64, _I64,  # qstarts, seq_lens, block_tables, stride, columns
        _P, _P, _P,  # counts, tasks, task_count
        _I64, _I64, _I64, _I32, _I32, _I32, _I32, _F, _I32,  # n hq programs splits bn qt mql scale st
        _P, _P, _P, POINTER(OscarClip), POINTER(OscarLayout),  # rk_t, rv_t, slots, clip, layout
        _P, _P, _P, _P, _P,  # partials, lse, raw partials, raw lse, stream
    ],
    "oscar_noalloc_scratch_bytes": [_I64, _I64, _I32],
    # calibration (startup): gram, attention weights, normalize, eigensolver + U H Pbr
    "oscar_accumulate_gram": [_P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P],
    "oscar_sst_weights": [_P, _I32, _I64, _I64, _I64, _I64, _P, _P, _P, _P],
    "oscar_normalize": [_P, _I64, _P, _F, _P, _P],
    "oscar_calibration_workspace_bytes": [_I32, _I32],
    "oscar_calibrated_rotations": [_P, _I32, _I32, _I32, _F, _P, _I64, _P, _P, _P, _P],
}
RESTYPES = {"oscar_noalloc_scratch_bytes": c_int64, "oscar_calibration_workspace_bytes": c_int64}
NOALLOC_SCRATCH_BYTES = 32 << 20  # OSCAR_NOALLOC_SCRATCH_BYTES

_lib = None


def library():
    """Load (once) and return the HIP library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"{LIBRARY_PATH.name} is not built; run `python -m oscar_new_amd.build` "
            "(OSCAR has no CPU execution path)"
        )
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, c_int32)
    lib.oscar_status_string.argtypes = [c_int32]
    lib.oscar_status_string.restype = ctypes.c_char_p
    _lib = lib
    return lib


def exported_symbols():
    """Names of every C entry point this binding expects (for load checks)."""
    return sorted([*SIGNATURES, "oscar_status_string"])


def check(status: int, what: str) -> None:
    """Raise on a non-zero status: ValueError for argument errors, RuntimeError for HIP."""
    if status == 0:
        return
    message = library().oscar_status_string(status).decode()
    if status < 0:
        raise ValueError(f"{what}: {message} (status {status})")
    raise RuntimeError(f"{what}: HIP error {status}: {message}")

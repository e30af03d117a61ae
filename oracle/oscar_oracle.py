"""numpy restatement of OSCAR's INT2 KV-cache path (TEST INFRASTRUCTURE, never product).

Every function cites the reference file:line it restates (paths are relative to the
``jpl123123/Oscar_new`` tree, package ``oscar_ascend``). Byte and integer work is exact;
floating point follows the rounding points of ``tests/oracle.py`` (fp32 arithmetic,
IEEE fp16/bf16 round-to-nearest-even).

bf16 values are carried as ``uint16`` bit patterns because numpy has no bfloat16.

Pinning (what checks each function independently of its own formula):
  * geometry (``Geometry``): the known-answer constants of tests/test_layout.py:11-19 and the
    sentinel/ring tests of tests/test_layout.py:28-75.
  * ``quantile_threshold``: torch.quantile (a library routine) on random rows, ties and
    constants; brute force on sorted values.
  * ``quantize``/``packed_slots``: hand answers (constant rows, zero/0.5/1e-12 rows, the
    2**-14 scale floor), an independent torch restatement built on torch.quantile, and
    decode-error bounds.
  * ``load_vec``: the constructed known answer of tests/test_packed_load.py:13-93.
  * ``prepare_tasks``: the closed-form task list of tests/test_tasks.py:101-108.
  * attention (``attention_partials``/``merge_*``/``dense_attention``): split invariance,
    logsumexp identities, softmax of a single key, float64 brute force on tiny inputs.
  * ``fma_f32``: exact rational arithmetic (fractions.Fraction) on random triples.
  * ``search`` clip mode: BASELINE extension with no reference counterpart; pinned by a
    brute-force argmin over the 8 factors computed with Python floats.
  * ``cached_decode_variants``: "exact" against ``dense_attention`` on the float64 dequant
    (and against "oracle" within bf16 dequant rounding); "reference_kernel" against the
    blocked online softmax reducing to the dense softmax when no rounding is applied, and
    the split merge's invariance to the split count.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

__all__ = [
    "Geometry",
    "bf16_to_f32",
    "f32_to_bf16",
    "fma_f32",
    "quantile_threshold",
    "search_factors",
    "quantize",
    "packed_slots",
    "rotate",
    "load_vec",
    "prepare_tasks",
    "store_int2",
    "store_windows",
    "attention_partials",
    "merge_splits",
    "merge_paths",
    "dense_attention",
    "hybrid_reference",
    "unpack",
    "dequant_rows",
    "cached_decode_reference",
    "cached_decode_variants",
]

NEG_INF = np.float32(-np.inf)


# --------------------------------------------------------------------------- number formats


def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even, quiet NaN (torch .bfloat16())."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        sign = ((u >> np.uint64(16)) & np.uint64(0x8000)).astype(np.uint16)
        out = np.where(nan, sign | np.uint16(0x7FC0), out)
    return out


def fma_f32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 fused multiply-add ``a*b + c`` (one rounding).

    The float64 product of two float32 values is exact. The float64 sum can round once
    more; a second rounding to float32 only errs when that sum lands exactly on a float32
    midpoint, which is detected with the exact TwoSum error and resolved toward it.
    """
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b
    s = p + c
    bb = s - p
    err = (p - (s - bb)) + (c - bb)
    r = s.astype(np.float32)
    r64 = r.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        toward = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
        neighbour = np.nextafter(r, toward).astype(np.float64)
        mid = (r64 + neighbour) * 0.5
        tie = (s != r64) & (s == mid) & (err != 0) & np.isfinite(s)
        # True value lies beyond the midpoint toward err's sign.
        beyond = np.where(err > 0, neighbour > r64, neighbour < r64)
        fixed = np.where(tie & beyond, neighbour.astype(np.float32), r)
    return fixed.astype(np.float32)


# --------------------------------------------------------------------------- geometry


@dataclass(frozen=True)
class Geometry:
    """Byte geometry of one KV stripe (oscar_ascend/layout.py:30-73, config.py:45-63)."""

    physical_block_tokens: int = 768
    kv_heads: int = 1
    kernel_block_tokens: int = 128
    head_dim: int = 256
    sink_tokens: int = 64
    recent_tokens: int = 256
    speculative_tokens: int = 3

    @property
    def data_bytes(self):  # config.py:45-47
        return self.head_dim // 4

    @property
    def vector_bytes(self):  # config.py:49-51
        return self.data_bytes + 4

    @property
    def slot_bytes(self):  # config.py:53-55: two vectors rounded up to 32 bytes
        return ((2 * self.vector_bytes + 31) // 32) * 32

    @property
    def ring_tokens(self):  # config.py:57-59
        return self.recent_tokens + self.speculative_tokens + 1

    @property
    def window_tokens(self):  # config.py:61-63
        return self.sink_tokens + self.ring_tokens

    @property
    def stripe_page_bytes(self):  # layout.py:30-32
        return self.physical_block_tokens * self.kv_heads * self.head_dim * 2

    @property
    def blocks_per_page(self):  # layout.py:42-44
        return self.physical_block_tokens // self.kernel_block_tokens

    def slot_offset(self, slot, head=0):  # layout.py:46-53
        page, position = divmod(int(slot), self.physical_block_tokens)
        return page * self.stripe_page_bytes + (position * self.kv_heads + head) * self.slot_bytes

    def logical_slot(self, table_row, position):  # layout.py:55-57
        block, token = divmod(int(position), self.kernel_block_tokens)
        return int(table_row[block]) * self.kernel_block_tokens + token

    def window_index(self, position):  # layout.py:65-69
        s = self.sink_tokens
        return position if position < s else s + position % self.ring_tokens

    def window_element(self, first_block, position, kv=0, head=0):
        """Window address in bf16 ELEMENTS (layout.py:59-73 divided by 2)."""
        owner = int(first_block) // self.blocks_per_page
        index = self.window_index(int(position))
        return owner * (self.stripe_page_bytes // 2) + (
            (index * 2 + kv) * self.kv_heads + head
        ) * self.head_dim


# --------------------------------------------------------------------------- quantizer


def quantile_threshold(absolute, ratio) -> np.ndarray:
    """torch.quantile(|x|, ratio, dim=-1) as used by tests/oracle.py:13.

    rank = f32(ratio) * 255 in float32; a, b = ascending order statistics floor/ceil(rank);
    threshold = fma(rank - floor(rank), b - a, a) with one rounding.
    """
    absolute = np.asarray(absolute, np.float32)
    n = absolute.shape[-1]
    rank = np.float32(ratio) * np.float32(n - 1)
    lo = int(math.floor(float(rank)))
    hi = int(math.ceil(float(rank)))
    weight = np.float32(rank - np.float32(lo))
    ordered = np.sort(absolute, axis=-1)
    a = ordered[..., lo]
    b = ordered[..., hi]
    return fma_f32(weight, (b - a).astype(np.float32), a)


def search_factors() -> np.ndarray:
    """The 8 clip factors of the BASELINE ``search`` mode: f32(0.6 + 0.4*i/7), i=0..7."""
    return np.array([0.6 + 0.4 * i / 7.0 for i in range(8)], dtype=np.float64).astype(np.float32)


def _tree_sum(values: np.ndarray) -> np.ndarray:
    """Pairwise float32 sum over the last axis: level by level, (2j, 2j+1) pairs."""
    v = np.asarray(values, np.float32)
    while v.shape[-1] > 1:
        v = (v[..., 0::2] + v[..., 1::2]).astype(np.float32)
    return v[..., 0]


def _quantize_clipped(x: np.ndarray):
    """Codes/scale/zero of already clipped float32 rows (tests/oracle.py:15-17)."""
    lo = x.min(-1, keepdims=True)
    hi = x.max(-1, keepdims=True)
    zero = lo.astype(np.float16)
    spread = ((hi - lo) / np.float32(3)).astype(np.float32)
    scale = np.maximum(spread, np.float32(2.0**-14)).astype(np.float16)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        q = ((x - zero.astype(np.float32)) / scale.astype(np.float32) + np.float32(0.5)).astype(
            np.float32
        )
        code = np.clip(np.trunc(q), 0, 3).astype(np.int32)
    return code, scale, zero


def _clip(x, threshold):
    return np.minimum(np.maximum(x, -threshold), threshold).astype(np.float32)


def quantize(x, ratio=0.0, mode="percentile", factor=1.0):
    """INT2 quantizer of tests/oracle.py:6-21 (+ the BASELINE ``search`` clip mode).

    Returns ``(packed uint8[..., D/4], scale float16[..., 1], zero float16[..., 1],
    decoded bf16-bits uint16[..., D])``.
    """
    x = np.asarray(x, np.float32)
    if mode == "factor":
        threshold = (np.abs(x).max(-1, keepdims=True) * np.float32(factor)).astype(np.float32)
        xc = _clip(x, threshold)
    elif mode == "search":
        maxabs = np.abs(x).max(-1, keepdims=True)
        best = None
        best_err = None
        for f in search_factors():
            xc_i = _clip(x, (maxabs * f).astype(np.float32))
            code, scale, zero = _quantize_clipped(xc_i)
            decoded = (code.astype(np.float32) * scale.astype(np.float32) + zero.astype(np.float32))
            err = (x - decoded.astype(np.float32)).astype(np.float32)
            mse = _tree_sum((err * err).astype(np.float32))
            if best is None:
                best, best_err = xc_i, mse
            else:
                better = mse < best_err
                best = np.where(better[..., None], xc_i, best)
                best_err = np.where(better, mse, best_err)
        xc = best
    elif mode == "percentile":
        if ratio:
            threshold = quantile_threshold(np.abs(x), ratio)[..., None]
            xc = _clip(x, threshold)
        else:
            xc = x
    else:
        raise ValueError(f"unknown clip mode {mode}")
    code, scale, zero = _quantize_clipped(xc)
    c = code.reshape(*code.shape[:-1], -1, 4)
    packed = (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)
    decoded = f32_to_bf16(
        (code.astype(np.float32) * scale.astype(np.float32)).astype(np.float32)
        + zero.astype(np.float32)
    )
    return packed, scale, zero, decoded


def _cfg_get(cfg, name, default):
    return getattr(cfg, name, default) if not isinstance(cfg, dict) else cfg.get(name, default)


def packed_slots(k_bits, v_bits, cfg):
    """160-byte slot images of rotated bf16 K/V rows (tests/oracle.py:24-39).

    ``cfg`` provides clip_mode, k/v_clip_ratio, k/v_clip_factor, head_dim.
    Bytes 136..159 stay zero (the reference oracle allocates zeros).
    """
    k = bf16_to_f32(k_bits)
    v = bf16_to_f32(v_bits)
    d = k.shape[-1]
    data = d // 4
    vector = data + 4
    slot = ((2 * vector + 31) // 32) * 32
    out = np.zeros((*k.shape[:-1], slot), np.uint8)
    mode = _cfg_get(cfg, "clip_mode", "percentile")
    for x, offset, ratio, factor in (
        (k, 0, _cfg_get(cfg, "k_clip_ratio", 0.96), _cfg_get(cfg, "k_clip_factor", 1.0)),
        (v, vector, _cfg_get(cfg, "v_clip_ratio", 0.92), _cfg_get(cfg, "v_clip_factor", 1.0)),
    ):
        codes, scale, zero, _ = quantize(x, ratio, mode, factor)
        out[..., offset : offset + data] = codes
        out[..., offset + data : offset + data + 2] = np.ascontiguousarray(scale).view(np.uint8)
        out[..., offset + data + 2 : offset + data + 4] = np.ascontiguousarray(zero).view(
            np.uint8
        )
    return out


# --------------------------------------------------------------------------- rotation


def rotate(x_bits, r_bits) -> np.ndarray:
    """``(x.float() @ R.float()).bfloat16()`` (tests/oracle.py:58; kernels.py:14-66).

    x: bf16 bits [..., D]; R: bf16 bits [D, D] (any view). Accumulates in float64, rounds
    once to float32 and then to bf16.
    """
    x = bf16_to_f32(x_bits).astype(np.float64)
    r = bf16_to_f32(r_bits).astype(np.float64)
    return f32_to_bf16((x @ r).astype(np.float32))


# --------------------------------------------------------------------------- byte kernels


def load_vec(history: np.ndarray, address: int, d: int = 256) -> np.ndarray:
    """Dequantize one packed vector to bf16 bits (kernels.py:205-219).

    code = (byte[i/4] >> 2(i%4)) & 3; value = bf16(code * f32(scale) + f32(zero)).
    """
    data = history[address : address + d // 4].astype(np.int32)
    codes = (data[:, None] >> (2 * np.arange(4))[None, :]) & 3
    codes = codes.reshape(-1)
    scale = np.frombuffer(history[address + d // 4 : address + d // 4 + 2].tobytes(), np.float16)
    zero = np.frombuffer(history[address + d // 4 + 2 : address + d // 4 + 4].tobytes(), np.float16)
    value = (codes.astype(np.float32) * scale.astype(np.float32)[0]).astype(np.float32) + zero.astype(
        np.float32
    )[0]
    return f32_to_bf16(value.astype(np.float32))


def unpack(history, slots, geometry: Geometry, active=None):
    """Diagnostic dequant of ``slots`` rows (kernels.py:623-648): bf16 bits [n, H, D] x2.

    Rows whose slot is negative decode to zeros, as the masked loads do.
    """
    n = len(slots)
    h, d = geometry.kv_heads, geometry.head_dim
    k = np.zeros((n, h, d), np.uint16)
    v = np.zeros((n, h, d), np.uint16)
    for t, slot in enumerate(slots):
        if slot < 0:
            continue
        for head in range(h):
            base = geometry.slot_offset(slot, head)
            k[t, head] = load_vec(history, base, d)
            v[t, head] = load_vec(history, base + geometry.vector_bytes, d)
    return k, v


def prepare_tasks(qstarts, counts, max_reqs, query_tile, num_reqs=None, source_table=None,
                  table=None, copy_columns=0):
    """Compact task table (kernels.py:222-287).

    Returns ``(tasks list[(req, q_offset)], task_count)``; copies table columns in place.
    """
    qstarts = np.asarray(qstarts, np.int64)
    nr, active = int(counts[0]), int(counts[1])
    lanes = 1 << (int(max_reqs) - 1).bit_length() if max_reqs > 1 else 1
    programs = max(1, max_reqs if num_reqs is None else num_reqs)
    if source_table is not None and table is not None:
        for req in range(programs):
            if req < nr:
                cols = int(copy_columns)
                table[req, :cols] = source_table[req, :cols]
    tiles = []
    for req in range(lanes):
        if req < nr:
            start = min(int(qstarts[req]), active)
            end = min(int(qstarts[req + 1]), active)
            tiles.append(-(-max(end - start, 0) // query_tile))
        else:
            tiles.append(0)
    tasks = []
    for req in range(programs):
        count = tiles[req] if req < lanes else 0
        for j in range(count):
            tasks.append((req, j * query_tile))
    return tasks, int(sum(tiles))


def store_int2(history, k_bits, v_bits, slots, counts, geometry: Geometry, cfg):
    """Write packed slots of rotated rows into a byte image (kernels.py:140-172).

    Rows with ``token >= counts[1]`` or ``slot < 0`` are skipped; bytes 136..159 untouched.
    """
    active = int(counts[1])
    images = packed_slots(k_bits, v_bits, cfg)
    used = 2 * geometry.vector_bytes
    for t in range(k_bits.shape[0]):
        if t >= active:
            continue
        slot = int(slots[t])
        if slot < 0:
            continue
        for head in range(geometry.kv_heads):
            base = geometry.slot_offset(slot, head)
            history[base : base + used] = images[t, head, :used]
    return history


def store_windows(window, k_bits, v_bits, qstarts, seq_lens, table, counts, geometry, max_reqs):
    """BF16 sink/ring window writes of the current tokens (kernels.py:544-620).

    ``window`` is the bf16-bit (uint16) flat V stripe. Index i < S holds position i; ring
    index i >= S holds the latest position pos < seq with pos = i - S (mod C).
    """
    nr, active = int(counts[0]), int(counts[1])
    s_tok, ring = geometry.sink_tokens, geometry.ring_tokens
    h, d = geometry.kv_heads, geometry.head_dim
    programs = min(k_bits.shape[0], max_reqs)
    for req in range(programs):
        if req >= nr:
            continue
        qstart = int(qstarts[req])
        qend = min(int(qstarts[req + 1]), active)
        seq = int(seq_lens[req])
        prefix = seq - (qend - qstart)
        owner = int(table[req, 0]) // geometry.blocks_per_page
        for index in range(s_tok + ring):
            if index < s_tok:
                pos = index
            else:
                residue = index - s_tok
                if seq - 1 - residue < 0:
                    continue
                pos = seq - 1 - (seq - 1 - residue) % ring
                if pos < s_tok:
                    continue
            if not (prefix <= pos < seq and qend > qstart):
                continue
            current = qstart + pos - prefix
            for head in range(h):
                base = owner * (geometry.stripe_page_bytes // 2) + (index * 2 * h + head) * d
                window[base : base + d] = k_bits[current, head]
                window[base + h * d : base + h * d + d] = v_bits[current, head]
    return window


# --------------------------------------------------------------------------- attention


def _row_softmax(scores: np.ndarray, values: np.ndarray):
    """Masked (-inf) float64 softmax-weighted sum and natural-log LSE of one score row."""
    finite = np.isfinite(scores)
    if not finite.any():
        return np.zeros(values.shape[-1]), -np.inf
    m = scores[finite].max()
    p = np.where(finite, np.exp(np.where(finite, scores, m) - m), 0.0)
    den = p.sum()
    return (p @ values) / den, m + math.log(den)


def _chunk_cut(h, lo, length, chunk=64):
    """History index of a token-bounded split boundary: history index h (position lo + h)
    moved down to the chunk grid of absolute positions, the ends kept (this build's rule,
    csrc/attention.h history_positions)."""
    if h <= 0:
        return 0
    if h >= length:
        return length
    return max(lo, (lo + h) // chunk * chunk) - lo


def attention_partials(q_bits, k_bits, v_bits, history, window, qstarts, seq_lens, table,
                       counts, tasks, task_count, geometry: Geometry, scale, splits, raw,
                       block_n=32, query_tile=4, programs=None, split_tokens=0):
    """Split-exact partials and LSE of one attention branch (kernels.py:290-482).

    History (raw=False): INT2 positions [min(S, prefix), max(sink_len, prefix - R)) through the
    block table, dequantized to bf16 (``load_vec``) and dotted with the (rotated) query.
    Raw (raw=True): BF16 sink + recent window positions plus the causal current tokens.
    Rows not written by a live task stay NaN. Split ranges follow kernels.py:368-370.
    ``split_tokens`` > 0 (history only; this build's token-bounded rule, no reference
    counterpart): a request of ``length`` history tokens uses
    ``min(splits, max(1, ceil(length / split_tokens)))`` splits with the same range rule,
    except that every inner boundary moves down to the 64-token grid of absolute positions
    (``_chunk_cut``); the split slots above that get LSE -inf and keep NaN partials (never
    written).
    """
    n, hq, d = q_bits.shape
    h = geometry.kv_heads
    g = hq // h
    bk = geometry.kernel_block_tokens
    s_tok, recent = geometry.sink_tokens, geometry.recent_tokens
    q = bf16_to_f32(q_bits).astype(np.float64)
    kc = bf16_to_f32(k_bits).astype(np.float64)
    vc = bf16_to_f32(v_bits).astype(np.float64)
    partials = np.full((n, hq, splits, d), np.nan, np.float32)
    lse = np.full((n, hq, splits), np.nan, np.float32)
    active = int(counts[1])
    total = int(task_count)
    programs = len(tasks) if programs is None else programs
    for task in range(programs):
        if task >= total:
            continue
        req, qoff = tasks[task]
        qstart = int(qstarts[req])
        qend = min(int(qstarts[req + 1]), active)
        qlen = qend - qstart
        seq = int(seq_lens[req])
        prefix = seq - qlen
        sink_len = min(s_tok, prefix)
        recent_begin = max(sink_len, prefix - recent)
        if raw:
            length = sink_len + prefix - recent_begin + qlen
            lo = 0
            owner_block = int(table[req, 0])
        else:
            lo = sink_len
            length = recent_begin - lo
        nsplit = splits
        if split_tokens and not raw:
            nsplit = min(splits, max(1, -(-max(length, 0) // split_tokens)))
        tps = -(-(-(-length // block_n)) // nsplit)
        for head in range(h):
            # Gather this task's keys/values once, in position order.
            keys, values, positions = [], [], []
            for ns in range(max(length, 0)):
                if raw:
                    high = sink_len + prefix - recent_begin
                    if ns < sink_len:
                        pos = ns
                    elif ns < high:
                        pos = recent_begin + ns - sink_len
                    else:
                        pos = prefix + ns - high
                    if pos >= prefix:
                        ci = qstart + pos - prefix
                        keys.append(kc[ci, head])
                        values.append(vc[ci, head])
                    else:
                        kb = geometry.window_element(owner_block, pos, 0, head)
                        vb = geometry.window_element(owner_block, pos, 1, head)
                        keys.append(bf16_to_f32(window[kb : kb + d]).astype(np.float64))
                        values.append(bf16_to_f32(window[vb : vb + d]).astype(np.float64))
                else:
                    pos = lo + ns
                    slot = int(table[req, pos // bk]) * bk + pos % bk
                    base = geometry.slot_offset(slot, head)
                    keys.append(bf16_to_f32(load_vec(history, base, d)).astype(np.float64))
                    values.append(
                        bf16_to_f32(load_vec(history, base + geometry.vector_bytes, d)).astype(
                            np.float64
                        )
                    )
                positions.append(pos)
            keys = np.array(keys).reshape(-1, d)
            values = np.array(values).reshape(-1, d)
            positions = np.array(positions, np.int64)
            for row in range(query_tile * g):
                qi = qoff + row // g
                if qi >= qlen:
                    continue
                qhead = head * g + row % g
                token = qstart + qi
                for split in range(splits):
                    if split >= nsplit:
                        lse[token, qhead, split] = -np.inf
                        continue
                    begin = split * tps * block_n
                    end = min((split + 1) * tps * block_n, length)
                    if split_tokens and not raw:
                        begin = _chunk_cut(begin, lo, length)
                        end = _chunk_cut(end, lo, length)
                    sel = slice(begin, max(begin, end))
                    sc = keys[sel] @ q[token, qhead] * float(np.float32(scale))
                    mask = positions[sel] <= prefix + qi
                    sc = np.where(mask, sc, -np.inf)
                    out, l = _row_softmax(sc, values[sel])
                    partials[token, qhead, split] = out
                    lse[token, qhead, split] = l
    return partials, lse


def merge_splits(partials, lse, counts):
    """LSE-weighted merge of splits (kernels.py:485-511): bf16-bits out, float32 logsum.

    Rows with token >= counts[1] become 0 / -inf. Splits with -inf LSE get zero weight.
    """
    n, hq, splits, d = partials.shape
    out = np.zeros((n, hq, d), np.float32)
    logsum = np.full((n, hq), -np.inf, np.float32)
    active = int(counts[1])
    for t in range(min(n, active)):
        for head in range(hq):
            ls = lse[t, head].astype(np.float64)
            m = ls.max()
            safe = 0.0 if m == -np.inf else m
            w = np.exp(ls - safe)
            den = w.sum()
            keep = w > 0
            acc = (w[keep, None] * partials[t, head, keep].astype(np.float64)).sum(0)
            out[t, head] = acc / max(den, 1e-30)
            logsum[t, head] = m + math.log(max(den, 1e-30)) if den > 0 else -np.inf
    return f32_to_bf16(out), logsum


def merge_paths(a_bits, la, b, lb, counts):
    """LSE merge of history and raw branches (kernels.py:514-541).

    Returns ``(output bf16-bits [n, hq*D], merged_lse float32 [n, hq])``. The merged LSE is
    an addition of this build (the reference stores no merged LSE).
    """
    n, hq, d = a_bits.shape
    a = bf16_to_f32(a_bits).astype(np.float64)
    b = np.asarray(b, np.float64).reshape(n, hq, d)
    out = np.zeros((n, hq, d), np.float32)
    lse = np.full((n, hq), -np.inf, np.float32)
    active = int(counts[1])
    for t in range(min(n, active)):
        for head in range(hq):
            x, y = float(la[t, head]), float(lb[t, head])
            m = max(x, y)
            m = 0.0 if m == -np.inf else m
            wa, wb = math.exp(x - m), math.exp(y - m)
            out[t, head] = (wa * a[t, head] + wb * b[t, head]) / max(wa + wb, 1e-30)
            lse[t, head] = m + math.log(wa + wb) if wa + wb > 0 else -np.inf
    return f32_to_bf16(out).reshape(n, hq * d), lse


def dense_attention(q, k, v, prefix):
    """Dense causal attention (tests/oracle.py:42-52) in float64, plus natural-log LSE.

    q: float [T, Hq, D]; k, v: float [K, Hk, D]; query i sees keys j <= prefix + i.
    Returns ``(out float32 [T, Hq, D], lse float32 [T, Hq])``.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    t, hq, d = q.shape
    hk = k.shape[1]
    keys = np.repeat(k, hq // hk, axis=1)
    values = np.repeat(v, hq // hk, axis=1)
    scores = np.einsum("qhd,khd->hqk", q, keys) / math.sqrt(d)
    qi = np.arange(t)[:, None] + prefix
    ki = np.arange(k.shape[0])[None, :]
    scores = np.where((ki > qi)[None], -np.inf, scores)
    m = scores.max(-1, keepdims=True)
    p = np.exp(scores - m)
    den = p.sum(-1, keepdims=True)
    out = np.einsum("hqk,khd->qhd", p / den, values)
    lse = (m + np.log(den))[..., 0].T
    return out.astype(np.float32), lse.astype(np.float32)


def hybrid_reference(q_bits, k_bits, v_bits, prefix, rk_bits, rv_bits, cfg):
    """Quantized-history reference of tests/oracle.py:55-65 (+ LSE).

    Keys/values [S, end) with end = max(min(S, prefix), prefix - R) are rotated, quantized,
    dequantized (bf16) and inverse-rotated; sink, recent and current stay BF16.
    """
    s_tok = _cfg_get(cfg, "sink_tokens", 64)
    recent = _cfg_get(cfg, "recent_tokens", 256)
    end = max(min(s_tok, prefix), prefix - recent)
    rk = bf16_to_f32(rk_bits).astype(np.float64)
    rv = bf16_to_f32(rv_bits).astype(np.float64)
    kr = rotate(k_bits, rk_bits)
    vr = rotate(v_bits, rv_bits)
    mode = _cfg_get(cfg, "clip_mode", "percentile")
    _, _, _, kd = quantize(
        bf16_to_f32(kr), _cfg_get(cfg, "k_clip_ratio", 0.96), mode, _cfg_get(cfg, "k_clip_factor", 1.0)
    )
    _, _, _, vd = quantize(
        bf16_to_f32(vr), _cfg_get(cfg, "v_clip_ratio", 0.92), mode, _cfg_get(cfg, "v_clip_factor", 1.0)
    )
    keys = bf16_to_f32(k_bits).astype(np.float64).copy()
    values = bf16_to_f32(v_bits).astype(np.float64).copy()
    if end > s_tok:
        keys[s_tok:end] = bf16_to_f32(kd[s_tok:end]).astype(np.float64) @ rk.T
        values[s_tok:end] = bf16_to_f32(vd[s_tok:end]).astype(np.float64) @ rv.T
    return dense_attention(bf16_to_f32(q_bits), keys, values, prefix)


# --------------------------------------------------------------------------- bulk decode


def dequant_rows(history, offsets, d=256):
    """Vectorized ``load_vec`` (kernels.py:205-219) of many vectors: bf16 bits [N, d]."""
    offsets = np.asarray(offsets, np.int64)
    data = history[offsets[:, None] + np.arange(d // 4)[None, :]].astype(np.int32)
    codes = ((data[:, :, None] >> (2 * np.arange(4))[None, None, :]) & 3).reshape(len(offsets), d)
    sz = history[offsets[:, None] + d // 4 + np.arange(4)[None, :]]
    scale = np.ascontiguousarray(sz[:, :2]).view(np.float16)[:, 0].astype(np.float32)
    zero = np.ascontiguousarray(sz[:, 2:]).view(np.float16)[:, 0].astype(np.float32)
    value = (codes.astype(np.float32) * scale[:, None]).astype(np.float32) + zero[:, None]
    return f32_to_bf16(value.astype(np.float32))


def cached_decode_reference(history, window, table_row, seq, q_bits, k_bits, v_bits, rk_bits,
                            rv_bits, geometry: Geometry, scale=None, head=0):
    """Hybrid attention of tests/oracle.py:55-65, read back from a quantized paged cache.

    Positions [0, sink_len) and [recent_begin, prefix) come from the BF16 window, history
    positions [sink_len, recent_begin) are dequantized from their INT2 slots and
    inverse-rotated (``kd @ R.T``), current positions [prefix, seq) come from k/v.
    One request, one kv head. Returns ``(out float32 [T, Hq, D], lse float32 [T, Hq])``.
    """
    t, hq, d = q_bits.shape
    prefix = seq - t
    s_tok, recent = geometry.sink_tokens, geometry.recent_tokens
    sink_len = min(s_tok, prefix)
    recent_begin = max(sink_len, prefix - recent)
    bk = geometry.kernel_block_tokens
    pos = np.arange(sink_len, recent_begin)
    slots = np.asarray(table_row, np.int64)[pos // bk] * bk + pos % bk
    pages, within = np.divmod(slots, geometry.physical_block_tokens)
    offs = pages * geometry.stripe_page_bytes + (within * geometry.kv_heads + head) * geometry.slot_bytes
    rk = bf16_to_f32(rk_bits)
    rv = bf16_to_f32(rv_bits)
    keys = np.empty((seq, d), np.float32)
    values = np.empty((seq, d), np.float32)
    keys[sink_len:recent_begin] = bf16_to_f32(dequant_rows(history, offs, d)) @ rk.T
    values[sink_len:recent_begin] = bf16_to_f32(dequant_rows(history, offs + geometry.vector_bytes, d)) @ rv.T
    first = int(table_row[0])
    for p in list(range(0, sink_len)) + list(range(recent_begin, prefix)):
        kb = geometry.window_element(first, p, 0, head)
        vb = geometry.window_element(first, p, 1, head)
        keys[p] = bf16_to_f32(window[kb : kb + d])
        values[p] = bf16_to_f32(window[vb : vb + d])
    keys[prefix:] = bf16_to_f32(k_bits[:, head])
    values[prefix:] = bf16_to_f32(v_bits[:, head])
    q = bf16_to_f32(q_bits).astype(np.float64).reshape(t * hq, d)
    sc = (q @ keys.astype(np.float64).T) * (d ** -0.5 if scale is None else float(scale))
    qi = np.repeat(np.arange(t), hq)[:, None] + prefix
    sc = np.where(np.arange(seq)[None, :] > qi, -np.inf, sc)
    m = sc.max(-1, keepdims=True)
    p = np.exp(sc - m)
    den = p.sum(-1, keepdims=True)
    out = (p / den) @ values.astype(np.float64)
    lse = (m + np.log(den))[:, 0]
    return out.reshape(t, hq, d).astype(np.float32), lse.reshape(t, hq).astype(np.float32)


def _dequant_exact(history, offsets, d=256):
    """Dequantized vectors without the bf16 rounding of ``load_vec``: code * scale + zero in
    float64 (fp16 scale and zero are exact in float64), [N, d]."""
    offsets = np.asarray(offsets, np.int64)
    data = history[offsets[:, None] + np.arange(d // 4)[None, :]].astype(np.int32)
    codes = ((data[:, :, None] >> (2 * np.arange(4))[None, None, :]) & 3).reshape(len(offsets), d)
    sz = history[offsets[:, None] + d // 4 + np.arange(4)[None, :]]
    scale = np.ascontiguousarray(sz[:, :2]).view(np.float16)[:, 0].astype(np.float64)
    zero = np.ascontiguousarray(sz[:, 2:]).view(np.float16)[:, 0].astype(np.float64)
    return codes.astype(np.float64) * scale[:, None] + zero[:, None]


def _blocked_softmax(q, keys, values, pos, limit, scale, block_n, round_p):
    """One split of the reference kernel's online softmax (kernels.py:421-436) for rows q
    [R, D] over keys/values [L, D] (float64 holding bf16 values) in blocks of ``block_n``:
    fp32 scores, running max with the -inf guard, ``p.to(bf16)`` in the P V product
    (``round_p``), fp32 state. ``limit`` [R]: a row sees positions <= limit. Returns
    (normalized [R, D] float32, lse [R] float32); an empty split gives 0 / -inf."""
    r = q.shape[0]
    f32 = np.float32
    m = np.full(r, -np.inf, f32)
    den = np.zeros(r, f32)
    acc = np.zeros((r, q.shape[1]), f32)
    for b0 in range(0, max(len(pos), 1), block_n):
        sl = slice(b0, b0 + block_n)
        if b0 >= len(pos):
            break
        score = ((q @ keys[sl].T).astype(f32) * f32(scale)).astype(f32)
        score = np.where(pos[sl][None, :] <= limit[:, None], score, -np.inf).astype(f32)
        new_m = np.maximum(m, score.max(1))
        safe = np.where(new_m == -np.inf, f32(0), new_m).astype(f32)
        alpha = np.exp((m - safe).astype(np.float64)).astype(f32)
        pr = np.exp((score - safe[:, None]).astype(np.float64)).astype(f32)
        pv = bf16_to_f32(f32_to_bf16(pr)) if round_p else pr
        acc = (acc * alpha[:, None] + (pv.astype(np.float64) @ values[sl]).astype(f32)).astype(f32)
        den = (den * alpha + pr.sum(1, dtype=np.float64).astype(f32)).astype(f32)
        m = new_m
    out = (acc / np.maximum(den, f32(1e-30))[:, None]).astype(f32)
    lse = np.where(den > 0, m + np.log(np.maximum(den, f32(1e-30))), -np.inf).astype(f32)
    return out, lse


def cached_decode_variants(history, window, table_row, seq, q_bits, k_bits, v_bits, rk_bits,
                           rv_bits, geometry: Geometry, scale=None, head=0, splits=16,
                           block_n=32):
    """Three references for one request's decode step, read back from one quantized cache.

    * "oracle": ``cached_decode_reference`` (tests/oracle.py:55-65: the dequantized history
      rounded to bf16, inverse-rotated in float, dense attention).
    * "exact": the same attention with the history dequantized exactly (code * scale + zero,
      no bf16 rounding), inverse-rotated and attended in float64: the value every
      implementation of this cache format approximates.
    * "reference_kernel": the rounding points of the reference's own kernels in
      backend.py:195-226 order: q rotated by R_k and rounded to bf16 (rotate); history keys
      and values dequantized to bf16 (_load_vec, kernels.py:205-219); each of ``splits``
      splits (kernels.py:368-370) a blocked online softmax with fp32 state and ``p.to(bf16)``
      (kernels.py:421-431); the LSE merge of the splits rounded to bf16 (merge_splits); the
      inverse V rotation rounded to bf16 (rotate(hrot, Rv.T)); the BF16 branch the same
      blocked softmax over the window and current rows (one split); the path merge to bf16.

    Returns {name: (out float32 [T, Hq, D], lse float32 [T, Hq])}; "reference_kernel" holds
    bf16 values and the merged LSE of merge_paths.
    """
    t, hq, d = q_bits.shape
    scale = d ** -0.5 if scale is None else float(scale)
    prefix = seq - t
    s_tok, recent = geometry.sink_tokens, geometry.recent_tokens
    sink_len = min(s_tok, prefix)
    recent_begin = max(sink_len, prefix - recent)
    bk = geometry.kernel_block_tokens
    pos = np.arange(sink_len, recent_begin)
    slots = np.asarray(table_row, np.int64)[pos // bk] * bk + pos % bk
    pages, within = np.divmod(slots, geometry.physical_block_tokens)
    offs = pages * geometry.stripe_page_bytes + (within * geometry.kv_heads + head) * geometry.slot_bytes
    rk = bf16_to_f32(rk_bits).astype(np.float64)
    rv = bf16_to_f32(rv_bits).astype(np.float64)
    first = int(table_row[0])
    window_pos = list(range(0, sink_len)) + list(range(recent_begin, prefix))
    wk = np.array([bf16_to_f32(window[geometry.window_element(first, p, 0, head):][:d])
                   for p in window_pos], np.float64).reshape(-1, d)
    wv = np.array([bf16_to_f32(window[geometry.window_element(first, p, 1, head):][:d])
                   for p in window_pos], np.float64).reshape(-1, d)
    ck = bf16_to_f32(k_bits[:, head]).astype(np.float64)
    cv = bf16_to_f32(v_bits[:, head]).astype(np.float64)
    q = bf16_to_f32(q_bits).astype(np.float64).reshape(t * hq, d)
    qi = np.repeat(np.arange(t), hq) + prefix  # position limit of each row

    def dense(keys, values):
        sc = (q @ keys.T) * scale
        sc = np.where(np.arange(seq)[None, :] > qi[:, None], -np.inf, sc)
        m = sc.max(-1, keepdims=True)
        p = np.exp(sc - m)
        den = p.sum(-1, keepdims=True)
        out = (p / den) @ values
        lse = (m + np.log(den))[:, 0]
        return out.reshape(t, hq, d).astype(np.float32), lse.reshape(t, hq).astype(np.float32)

    def assemble(hk, hv):
        keys = np.empty((seq, d), np.float64)
        values = np.empty((seq, d), np.float64)
        keys[sink_len:recent_begin], values[sink_len:recent_begin] = hk, hv
        keys[window_pos], values[window_pos] = wk, wv
        keys[prefix:], values[prefix:] = ck, cv
        return keys, values

    out = {"oracle": cached_decode_reference(history, window, table_row, seq, q_bits, k_bits,
                                             v_bits, rk_bits, rv_bits, geometry, scale, head)}
    out["exact"] = dense(*assemble(_dequant_exact(history, offs, d) @ rk.T,
                                   _dequant_exact(history, offs + geometry.vector_bytes, d) @ rv.T))

    # The reference kernels' rounding points, in the rotated space for the history branch.
    q_rot = bf16_to_f32(rotate(q_bits.reshape(t * hq, d), rk_bits)).astype(np.float64)
    hk = bf16_to_f32(dequant_rows(history, offs, d)).astype(np.float64)
    hv = bf16_to_f32(dequant_rows(history, offs + geometry.vector_bytes, d)).astype(np.float64)
    length = recent_begin - sink_len
    tps = -(-(-(-length // block_n)) // splits)
    parts = np.zeros((t * hq, splits, d), np.float32)
    lses = np.full((t * hq, splits), -np.inf, np.float32)
    for split in range(splits):
        b, e = split * tps * block_n, min((split + 1) * tps * block_n, length)
        if e > b:
            parts[:, split], lses[:, split] = _blocked_softmax(
                q_rot, hk[b:e], hv[b:e], pos[b:e], qi, scale, block_n, True)
        else:
            parts[:, split] = 0.0
    counts = np.array([1, t * hq])
    hrot, hl = merge_splits(parts[:, None], lses[:, None], counts)
    hout = rotate(hrot[:, 0], rv_bits.T)
    raw_pos = np.array(window_pos + list(range(prefix, seq)), np.int64)
    raw_k = np.concatenate([wk, ck])
    raw_v = np.concatenate([wv, cv])
    rp, rl = _blocked_softmax(q, raw_k, raw_v, raw_pos, qi, scale, block_n, True)
    merged, mlse = merge_paths(hout.reshape(t * hq, 1, d), hl.reshape(t * hq, 1), rp,
                               rl.reshape(t * hq, 1), np.array([1, t * hq]))
    out["reference_kernel"] = (bf16_to_f32(merged).reshape(t, hq, d), mlse.reshape(t, hq))
    return out

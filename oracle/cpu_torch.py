"""torch float32 CPU restatement of the decode step and of quantize+pack (TEST INFRASTRUCTURE,
never product): the CPU baseline that ``bench.py`` times beside the GPU numbers.

It computes what ``oscar_oracle`` computes, vectorized in torch on the host cores:

  * ``decode_step``: one request's hybrid attention read back from a quantized paged cache
    (reference tests/oracle.py:55-65 semantics, the cache addressing of layout.py:46-73 and
    the unpacking of kernels.py:205-219): the INT2 history is dequantized and inverse-rotated
    (``kd @ R.T``), sink and recent rows come from the BF16 window, current rows from k/v,
    and the softmax is dense float32.
  * ``quantize_pack``: rotate (``x @ R`` rounded to bf16, kernels.py:14-66), clip and INT2 pack
    into 160-byte slot images (tests/oracle.py:6-39, plus the 8-factor ``search`` clip mode).

Pinned against ``oscar_oracle`` in tests/test_cpu_torch.py: dequantized rows and slot images
are bit-exact, rotations within one bf16 step, attention within float32 rounding of the
float64 oracle.
"""

from __future__ import annotations

import numpy as np
import torch

from .oscar_oracle import Geometry, fma_f32, search_factors

__all__ = ["dequant", "decode_step", "rotate", "quantize", "quantize_pack"]

_SHIFTS = torch.tensor([0, 2, 4, 6], dtype=torch.int32)


def dequant(history: torch.Tensor, offsets: torch.Tensor, d: int = 256) -> torch.Tensor:
    """float32 values of the bf16 rows decoded from the INT2 vectors at byte ``offsets``
    (kernels.py:205-219): code * scale rounded to float32, + zero, rounded to bf16."""
    n = offsets.numel()
    raw = history[offsets[:, None] + torch.arange(d // 4 + 4)]
    codes = ((raw[:, : d // 4].to(torch.int32)[:, :, None] >> _SHIFTS) & 3).reshape(n, d)
    scale = raw[:, d // 4 : d // 4 + 2].contiguous().view(torch.float16).float()
    zero = raw[:, d // 4 + 2 : d // 4 + 4].contiguous().view(torch.float16).float()
    return (codes.float() * scale + zero).bfloat16().float()


def decode_step(history, window, table_row, seq, q, k, v, rk, rv, geometry: Geometry,
                scale=None, head=0):
    """Hybrid attention of one request and one KV head from a quantized paged cache.

    ``history``: uint8 [bytes] (the KV stripe); ``window``: bf16 [elements] (the V stripe);
    ``q``: bf16 [t, hq, d]; ``k``/``v``: bf16 [t, kv_heads, d]; ``rk``/``rv``: bf16 [d, d].
    Returns ``(out float32 [t, hq, d], lse float32 [t, hq])``.
    """
    t, hq, d = q.shape
    prefix = seq - t
    sink_len = min(geometry.sink_tokens, prefix)
    recent_begin = max(sink_len, prefix - geometry.recent_tokens)
    bk = geometry.kernel_block_tokens
    table_row = torch.as_tensor(np.asarray(table_row), dtype=torch.int64)
    pos = torch.arange(sink_len, recent_begin, dtype=torch.int64)
    slots = table_row[pos // bk] * bk + pos % bk
    pages = slots // geometry.physical_block_tokens
    within = slots % geometry.physical_block_tokens
    offs = pages * geometry.stripe_page_bytes + (within * geometry.kv_heads + head) * geometry.slot_bytes
    keys = torch.empty(seq, d, dtype=torch.float32)
    values = torch.empty(seq, d, dtype=torch.float32)
    keys[sink_len:recent_begin] = dequant(history, offs, d) @ rk.float().T
    values[sink_len:recent_begin] = dequant(history, offs + geometry.vector_bytes, d) @ rv.float().T
    first = int(table_row[0])
    win_pos = list(range(sink_len)) + list(range(recent_begin, prefix))
    if win_pos:
        base = torch.tensor([geometry.window_element(first, p, 0, head) for p in win_pos])
        vbase = torch.tensor([geometry.window_element(first, p, 1, head) for p in win_pos])
        rows = torch.arange(d)
        idx = torch.tensor(win_pos)
        keys[idx] = window[base[:, None] + rows].float()
        values[idx] = window[vbase[:, None] + rows].float()
    keys[prefix:] = k[:, head].float()
    values[prefix:] = v[:, head].float()
    sc = (q.float().reshape(t * hq, d) @ keys.T) * (d ** -0.5 if scale is None else float(scale))
    qi = torch.arange(t).repeat_interleave(hq)[:, None] + prefix
    sc = sc.masked_fill(torch.arange(seq)[None, :] > qi, float("-inf"))
    m = sc.amax(-1, keepdim=True)
    p = torch.exp(sc - m)
    den = p.sum(-1, keepdim=True)
    out = (p / den) @ values
    lse = (m + torch.log(den))[:, 0]
    return out.reshape(t, hq, d), lse.reshape(t, hq)


def rotate(x: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
    """``(x.float() @ R.float()).bfloat16()`` (tests/oracle.py:58)."""
    return (x.float() @ r.float()).bfloat16()


def _tree_sum(v: torch.Tensor) -> torch.Tensor:
    """Pairwise float32 sum over the last axis, level by level on (2j, 2j+1) pairs."""
    while v.shape[-1] > 1:
        v = v[..., 0::2] + v[..., 1::2]
    return v[..., 0]


def _quantize_clipped(x: torch.Tensor):
    """Codes, fp16 scale and fp16 zero of clipped float32 rows (tests/oracle.py:15-17)."""
    lo = x.amin(-1, keepdim=True)
    hi = x.amax(-1, keepdim=True)
    zero = lo.half()
    scale = torch.clamp_min((hi - lo) / 3.0, 2.0 ** -14).half()
    q = (x - zero.float()) / scale.float() + 0.5
    return torch.clamp(torch.trunc(q), 0, 3).to(torch.int32), scale, zero


def quantize(x: torch.Tensor, ratio=0.0, mode="percentile", factor=1.0):
    """INT2 codes, scale and zero of float32 rows [..., D] under one clip mode."""
    if mode == "factor":
        t = x.abs().amax(-1, keepdim=True) * float(np.float32(factor))
        xc = torch.minimum(torch.maximum(x, -t), t)
    elif mode == "search":
        maxabs = x.abs().amax(-1, keepdim=True)
        best, best_err = None, None
        for f in search_factors():
            t = maxabs * float(f)
            xc_i = torch.minimum(torch.maximum(x, -t), t)
            code, s, z = _quantize_clipped(xc_i)
            err = x - (code.float() * s.float() + z.float())
            mse = _tree_sum(err * err)
            if best is None:
                best, best_err = xc_i, mse
            else:
                better = mse < best_err
                best = torch.where(better[..., None], xc_i, best)
                best_err = torch.where(better, mse, best_err)
        xc = best
    elif mode == "percentile":
        xc = x
        if ratio:
            # torch.quantile's rank interpolation with a single rounding (fma), per row.
            n = x.shape[-1]
            rank = np.float32(ratio) * np.float32(n - 1)
            lo, hi = int(np.floor(rank)), int(np.ceil(rank))
            ordered = x.abs().sort(-1).values
            a, b = ordered[..., lo].numpy(), ordered[..., hi].numpy()
            thr = torch.from_numpy(fma_f32(np.float32(rank - np.float32(lo)), b - a, a))[..., None]
            xc = torch.minimum(torch.maximum(x, -thr), thr)
    else:
        raise ValueError(f"unknown clip mode {mode}")
    return _quantize_clipped(xc)


def quantize_pack(k_rot: torch.Tensor, v_rot: torch.Tensor, mode="percentile", k_ratio=0.96,
                  v_ratio=0.92, k_factor=1.0, v_factor=1.0) -> torch.Tensor:
    """160-byte slot images (uint8 [..., 160]) of rotated bf16 K/V rows (tests/oracle.py:24-39);
    bytes 136..159 stay zero."""
    d = k_rot.shape[-1]
    data, vector = d // 4, d // 4 + 4
    slot = ((2 * vector + 31) // 32) * 32
    out = torch.zeros(*k_rot.shape[:-1], slot, dtype=torch.uint8)
    for x, off, ratio, factor in ((k_rot, 0, k_ratio, k_factor), (v_rot, vector, v_ratio, v_factor)):
        code, s, z = quantize(x.float(), ratio, mode, factor)
        c = code.reshape(*code.shape[:-1], data, 4)
        out[..., off : off + data] = (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4)
                                      | (c[..., 3] << 6)).to(torch.uint8)
        out[..., off + data : off + data + 2] = s.view(torch.uint8)
        out[..., off + data + 2 : off + vector] = z.view(torch.uint8)
    return out

"""Long continuation chunks: the chunk flash form of the BF16 branch (chunk_raw_attention)
against the decode form (attention_partials raw, one split; reference kernels.py:439-482),
bit for bit, and the step that uses it against the reference order of single launches.

The chunk form runs the decode form's row arithmetic (same MFMA operands and k order, same
lazy max and normalization) over the same 32-key blocks of the raw index sequence (sink rows,
recent rows, then the chunk's tokens), so every written row and LSE must carry the same bits.
"""

from types import SimpleNamespace

import pytest
import torch

from oscar_new_amd import kernels
from tests._state import make_state, prepare_prefix

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qr(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16().to(DEV)


def _case(lengths, prefixes, seed, kv_heads=1, hq=6):
    torch.manual_seed(seed)
    layout, raw, hist, window, meta, tables = make_state(lengths, prefixes, kv_heads=kv_heads)
    rk, rv = _qr(seed), _qr(seed + 1)
    ks = [torch.randn(n, kv_heads, 256).bfloat16() for n in lengths]
    vs = [torch.randn(n, kv_heads, 256).bfloat16() for n in lengths]
    qs = [torch.randn(n - p, hq, 256).bfloat16() for n, p in zip(lengths, prefixes)]
    prepare_prefix(ks, vs, rk, rv, hist, window, meta, tables, layout, prefixes)
    q = torch.cat(qs).to(DEV)
    k = torch.cat([x[p:] for x, p in zip(ks, prefixes)]).to(DEV)
    v = torch.cat([x[p:] for x, p in zip(vs, prefixes)]).to(DEV)
    meta.layout = layout
    meta.num_actual_tokens = q.shape[0]
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, layout.config.queries_per_tile)
    return SimpleNamespace(layout=layout, raw=raw, hist=hist, window=window, meta=meta, q=q,
                           k=k, v=v)


def _decode_form(c):
    p, l = kernels.attention_partials(c.q, c.k, c.v, c.hist, c.window, c.meta, c.layout, 1 / 16,
                                      1, raw=True)
    return p, l


def _chunk_form(c):
    n, hq, _ = c.q.shape
    p = torch.full((n, hq, 1, 256), 5.0, device=DEV)
    l = torch.full((n, hq, 1), 5.0, device=DEV)
    kernels.chunk_raw_attention(c.q, c.k, c.v, c.window, c.meta, c.layout, 1 / 16, p, l)
    return p, l


CASES = [
    ([2052], [4], 1),  # prefix = sink: no recent rows
    ([300], [2], 1),  # prefix below the sink
    ([500], [60], 1),  # recent rows fewer than the ring
    ([1700], [800], 1),  # the ring wrapped several times, 900-token chunk
    ([100, 1200, 77], [0, 1000, 40], 1),  # a batch with an initial prefill in it
    ([2048 + 1000], [1000], 1),  # a 2048-token chunk (the p2 shape at a smaller prefix)
    ([1000, 333], [700, 0], 2),  # two KV heads (GQA 3:1)
]


@pytest.mark.parametrize("lengths,prefixes,kv_heads", CASES)
def test_chunk_form_is_bitwise_the_decode_form(lengths, prefixes, kv_heads):
    c = _case(lengths, prefixes, seed=21, kv_heads=kv_heads)
    print(f"[chunk] {lengths} {prefixes} H{kv_heads}", flush=True)
    want_p, want_l = _decode_form(c)
    got_p, got_l = _chunk_form(c)
    torch.cuda.synchronize()
    assert torch.isfinite(got_p).all() and torch.isfinite(got_l).all()
    assert torch.equal(got_p.view(torch.int32), want_p.view(torch.int32))
    assert torch.equal(got_l.view(torch.int32), want_l.view(torch.int32))


def test_rows_past_the_token_count_are_not_written():
    c = _case([1300, 900], [1000, 100], seed=22)
    n = c.q.shape[0]
    live = n - 37
    c.meta.counts[1] = live  # the last request's chunk is cut short
    want_p, want_l = _decode_form(c)
    got_p, got_l = _chunk_form(c)
    torch.cuda.synchronize()
    assert torch.equal(got_p[:live].view(torch.int32), want_p[:live].view(torch.int32))
    assert torch.equal(got_l[:live].view(torch.int32), want_l[:live].view(torch.int32))
    assert got_p[live:].eq(5.0).all() and got_l[live:].eq(5.0).all()


def test_rows_past_the_host_bound_are_nan():
    # A request with more query tokens than the caller's max_query_len: the rows past the
    # launch's spans are NaN, never silently wrong.
    c = _case([900], [100], seed=23)
    c.meta.max_query_len = 64  # the chunk has 800 tokens
    got_p, got_l = _chunk_form(c)
    torch.cuda.synchronize()
    rows = got_p.view(-1, 256)
    covered = 64 * 6  # spans of 192, 96 or 48 rows: 384 rows either way
    assert torch.isnan(rows[covered:]).all()
    assert torch.isnan(got_l.view(-1)[covered:]).all()
    c.meta.max_query_len = 800
    want_p, _ = _decode_form(c)
    assert torch.equal(rows[:covered].view(torch.int32),
                       want_p.view(-1, 256)[:covered].view(torch.int32))


def _views(raw, layout, pages=20):
    """Native (K, V) cache views of a make_state byte buffer (conv | K | V)."""
    stripe = pages * layout.stripe_page_bytes
    conv = raw.numel() - 2 * stripe
    k = raw[conv : conv + stripe].view(torch.bfloat16).view(-1, 128, 1, 256)
    v = raw[conv + stripe :].view(torch.bfloat16).view(-1, 128, 1, 256)
    return k, v


def test_pre_attention_without_the_bf16_role_keeps_every_other_output():
    # raw=False: the pre-attention launch without its BF16 role, then the chunk launch. The
    # q rotation, the INT2 store (every cache byte) and the partials match the one launch.
    c = _case([1700, 260], [800, 200], seed=24)
    rk_t = _qr(5).T.contiguous()
    rv_t = _qr(6).T.contiguous()
    outs = []
    for raw in (True, False):
        cache = c.raw.clone()
        hist, window = c.layout.tensor_views(_views(cache, c.layout))
        qrot, rp, rl = kernels.pre_attention(c.q, c.k, c.v, hist, window, c.meta, c.layout,
                                             1 / 16, rk_t, rv_t, raw=raw)
        torch.cuda.synchronize()
        outs.append((qrot.view(torch.int16).cpu(), rp.view(torch.int32).cpu(),
                     rl.view(torch.int32).cpu(), cache.cpu()))
    for a, b in zip(*outs):
        assert a.shape == b.shape and torch.equal(a, b)

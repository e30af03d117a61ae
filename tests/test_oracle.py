"""Pins of the CPU oracle against library routines, known answers and invariants.

Every check compares the oracle with something that does not share its code: torch library
routines (quantile, softmax, logsumexp, fp16/bf16 casts), exact rational arithmetic, the
known-answer tests of the reference (tests/test_layout.py, tests/test_packed_load.py,
tests/test_tasks.py, tests/test_npu_kernels.py) and mathematical invariants.
"""

import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle as O
from oracle import oscar_oracle as OO

# ------------------------------------------------------------------ number formats


def test_bf16_roundtrip_matches_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.cat([torch.randn(20000, generator=g) * 10 ** torch.randint(-30, 30, (20000,),
                                                                          generator=g).float(),
                   torch.tensor([0.0, -0.0, 1e-40, -1e-40, 3.4e38, float("inf"), -float("inf")])])
    want = x.bfloat16().view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16(x.numpy())
    assert np.array_equal(got, want)
    back = O.bf16_to_f32(got)
    assert np.array_equal(back, x.bfloat16().float().numpy())


def _fma_exact(a, b, c):
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    return np.float32(_round_fraction_to_f32(exact))


def _round_fraction_to_f32(q: Fraction) -> float:
    """Round a rational to the nearest float32 (ties to even) by bracketing."""
    f = np.float32(float(q))  # float(q) is correctly rounded to double; then adjust to f32
    lo = np.nextafter(f, np.float32(-np.inf), dtype=np.float32)
    hi = np.nextafter(f, np.float32(np.inf), dtype=np.float32)
    best = min((lo, f, hi), key=lambda v: (abs(Fraction(float(v)) - q),
                                            int(np.array(v).view(np.uint32)) & 1))
    return float(best)


def test_fma_is_correctly_rounded():
    rng = random.Random(5)
    a_list, b_list, c_list = [], [], []
    for _ in range(3000):
        a_list.append(np.float32(rng.uniform(0, 1)))
        b_list.append(np.float32(rng.uniform(-1, 1) * 10 ** rng.randint(-8, 2)))
        c_list.append(np.float32(rng.uniform(0, 4)))
    # Constructed double-rounding cases: a*b tiny relative to c around a float midpoint.
    for _ in range(500):
        c = np.float32(rng.uniform(1, 2))
        half_ulp = float(np.spacing(c)) / 2
        a_list.append(np.float32(0.5))
        b_list.append(np.float32(half_ulp * 2 * (1 + 2.0**-20) * rng.choice([1, -1])))
        c_list.append(c)
    a, b, c = (np.array(v, np.float32) for v in (a_list, b_list, c_list))
    got = O.fma_f32(a, b, c)
    want = np.array([_fma_exact(x, y, z) for x, y, z in zip(a, b, c)], np.float32)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ quantile threshold


@pytest.mark.parametrize("ratio", [0.875, 0.9, 0.92, 0.93, 0.95, 0.96, 0.99, 1.0])
def test_quantile_threshold_matches_torch_quantile_bitwise(ratio):
    g = torch.Generator().manual_seed(9)
    x = torch.cat(
        (
            torch.randn(3000, 256, generator=g),
            torch.zeros(1, 256),
            torch.ones(1, 256),
            torch.randint(0, 4, (200, 256), generator=g).float(),  # heavy ties
            (torch.arange(256).float().remainder(11) - 5)[None],
            torch.randn(100, 256, generator=g).bfloat16().float(),
        )
    ).abs()
    want = torch.quantile(x, ratio, dim=-1).numpy()
    got = O.quantile_threshold(x.numpy(), ratio)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quantile_brute_force_order_statistics():
    rng = np.random.default_rng(3)
    x = np.abs(rng.standard_normal((50, 256)).astype(np.float32))
    for ratio in (0.875, 0.96, 1.0):
        rank = float(np.float32(ratio) * np.float32(255))
        lo, hi = math.floor(rank), math.ceil(rank)
        for row in x:
            s = sorted(row.tolist())
            a, b = s[lo], s[hi]
            thr = O.quantile_threshold(row[None], ratio)[0]
            assert min(a, b) <= thr <= max(a, b)


# ------------------------------------------------------------------ quantizer


@pytest.mark.parametrize("value", [0.0, 1e-20, 0.5, -3.0])
def test_constant_rows_decode_exactly(value):
    # Reference tests/test_layout.py:103-110.
    _, scale, _, decoded = O.quantize(np.full((2, 1, 256), value, np.float32))
    assert np.isfinite(O.bf16_to_f32(decoded)).all()
    assert (scale.astype(np.float32) > 0).all()
    assert np.allclose(O.bf16_to_f32(decoded), value, atol=1e-7, rtol=0)


def test_special_rows_known_answers():
    # Rows of reference tests/test_npu_kernels.py:77-80: zero, 0.5, 1e-12 constants.
    for value in (0.0, 0.5, 1e-12):
        packed, scale, zero, _ = O.quantize(np.full((1, 256), value, np.float32), 0.96)
        assert np.all(packed == 0)
        assert scale.view(np.uint16)[0, 0] == 0x0400  # the 2**-14 floor, fp16 bits
        assert zero[0, 0] == np.float16(value)


def test_quantizer_error_bound_and_code_range():
    rng = np.random.default_rng(11)
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((2000, 256)).astype(np.float32)))
    for ratio in (0.0, 0.92, 0.96, 1.0):
        packed, scale, zero, decoded = O.quantize(x, ratio)
        codes = (packed[..., :, None] >> (2 * np.arange(4))) & 3
        codes = codes.reshape(x.shape)
        thr = (O.quantile_threshold(np.abs(x), ratio)[:, None] if ratio
               else np.full((len(x), 1), np.inf, np.float32))
        xc = np.clip(x, -thr, thr)
        sf = scale.astype(np.float32)
        dq = codes * sf + zero.astype(np.float32)
        # Rounding to the nearest of 4 levels: error at most half a step (+ fp16 slack).
        slack = 0.5 * sf + np.abs(xc.min(-1, keepdims=True) - zero.astype(np.float32)) + 1e-6
        assert (np.abs(dq - xc) <= slack + 1e-3 * sf).all()
        # Extremes land on the end codes.
        assert (codes[np.arange(len(x)), xc.argmin(-1)] == 0).all()
        assert (codes[np.arange(len(x)), xc.argmax(-1)] == 3).all()
        assert np.array_equal(decoded, O.f32_to_bf16(dq.astype(np.float32)))


def test_quantizer_matches_torch_library_restatement():
    """Independent torch evaluation (torch.quantile, clamp, half casts, int cast)."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(512, 1, 256, generator=g).bfloat16().float()
    x[3] = 0
    x[4] = 0.5
    for ratio in (0.0, 0.92, 0.96, 1.0):
        xt = x.clone()
        if ratio:
            thr = torch.quantile(xt.abs(), ratio, dim=-1, keepdim=True)
            xt = xt.clamp(-thr, thr)
        zero = xt.amin(-1, keepdim=True).half()
        scale = ((xt.amax(-1, keepdim=True) - xt.amin(-1, keepdim=True)) / 3).clamp_min(2**-14).half()
        code = ((xt - zero.float()) / scale.float() + 0.5).to(torch.int32).clamp(0, 3)
        c = code.reshape(*code.shape[:-1], -1, 4)
        packed = (c[..., 0] | c[..., 1] << 2 | c[..., 2] << 4 | c[..., 3] << 6).byte()
        p, s, z, _ = O.quantize(x.numpy(), ratio)
        assert np.array_equal(p, packed.numpy())
        assert np.array_equal(s.view(np.uint16), scale.numpy().view(np.uint16))
        assert np.array_equal(z.view(np.uint16), zero.numpy().view(np.uint16))


def test_factor_mode_threshold():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    for factor in (0.5, 0.8, 1.0):
        _, scale, zero, _ = O.quantize(x, 0.0, "factor", factor)
        thr = np.abs(x).max(-1) * np.float32(factor)
        lo = np.maximum(x.min(-1), -thr)
        hi = np.minimum(x.max(-1), thr)
        assert np.array_equal(zero[:, 0], lo.astype(np.float16))
        spread = ((hi - lo) / np.float32(3)).astype(np.float32)
        assert np.array_equal(scale[:, 0], np.maximum(spread, np.float32(2**-14)).astype(np.float16))


def test_search_mode_brute_force_argmin():
    """BASELINE 8-factor MSE search: pinned by a scalar Python re-evaluation per factor."""
    rng = np.random.default_rng(8)
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((40, 256)).astype(np.float32)))
    x[:, 7] *= 10
    packed, scale, zero, _ = O.quantize(x, 0.0, "search")
    factors = [np.float32(0.6 + 0.4 * i / 7.0) for i in range(8)]
    for r, row in enumerate(x):
        errs = []
        for f in factors:
            p, s, z, _ = O.quantize(row[None], 0.0, "factor", float(f))
            codes = ((p[0][:, None] >> (2 * np.arange(4))) & 3).reshape(-1)
            dec = [np.float32(np.float32(c) * np.float32(s[0, 0]) + np.float32(z[0, 0]))
                   for c in codes]
            errs.append(sum(float(np.float32(xv - d)) ** 2 for xv, d in zip(row, dec)))
        # Choose by the float64 MSE; accept any factor whose MSE ties within fp32 noise.
        best = min(errs)
        chosen = [i for i, f in enumerate(factors)
                  if np.array_equal(O.quantize(row[None], 0.0, "factor", float(f))[0][0], packed[r])
                  and np.array_equal(O.quantize(row[None], 0.0, "factor", float(f))[1], scale[r:r + 1])]
        assert chosen, "search result is not one of the 8 factor quantizations"
        assert min(errs[i] for i in chosen) <= best * (1 + 1e-5) + 1e-12


def test_packed_slot_byte_layout():
    rng = np.random.default_rng(6)
    k = O.f32_to_bf16(rng.standard_normal((5, 1, 256)).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal((5, 1, 256)).astype(np.float32))
    cfg = {"k_clip_ratio": 0.96, "v_clip_ratio": 0.92}
    slots = O.packed_slots(k, v, cfg)
    assert slots.shape == (5, 1, 160)
    kp, ks, kz, _ = O.quantize(O.bf16_to_f32(k), 0.96)
    vp, vs, vz, _ = O.quantize(O.bf16_to_f32(v), 0.92)
    assert np.array_equal(slots[..., :64], kp)
    assert np.array_equal(slots[..., 64:66].view(np.float16), ks)
    assert np.array_equal(slots[..., 66:68].view(np.float16), kz)
    assert np.array_equal(slots[..., 68:132], vp)
    assert np.array_equal(slots[..., 132:134].view(np.float16), vs)
    assert np.array_equal(slots[..., 134:136].view(np.float16), vz)
    assert not slots[..., 136:].any()


# ------------------------------------------------------------------ unpack known answer


@pytest.mark.parametrize("rows", [4, 16, 32])
def test_load_vec_known_answer(rows):
    # Constructed bytes of reference tests/test_packed_load.py:13-93.
    cache = np.zeros(rows * 160 + 8, np.uint8)
    for row in range(rows):
        codes = (np.arange(256) + row) % 4
        packed = (codes.reshape(64, 4) << (np.arange(4) * 2)).sum(1).astype(np.uint8)
        start = row * 160 + 7
        cache[start : start + 64] = packed
        cache[start + 64 : start + 66] = np.array([0.125 * (row + 1)], np.float16).view(np.uint8)
        cache[start + 66 : start + 68] = np.array([-0.25 * row], np.float16).view(np.uint8)
        expected = torch.tensor(codes * 0.125 * (row + 1) - 0.25 * row, dtype=torch.float32)
        want = expected.bfloat16().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(O.load_vec(cache, start), want)


# ------------------------------------------------------------------ geometry


def test_geometry_known_constants():
    # Reference tests/test_layout.py:11-19.
    geo = O.Geometry(768)
    assert geo.vector_bytes == 68 and geo.slot_bytes == 160
    assert geo.stripe_page_bytes == 393216
    assert 768 * geo.slot_bytes == 122880
    assert geo.window_tokens * 2 * 256 * 2 == 331776
    assert geo.blocks_per_page == 6
    assert 15360 + geo.stripe_page_bytes * 2 == 801792


def test_ring_rollback_invariant():
    # Reference tests/test_layout.py:61-75 on the oracle's window indexing.
    geo = O.Geometry(768)
    memory, end = {}, 0
    for chunk, rejected in ((1024, 0), (4, 3), (4, 2), (4, 0), (300, 0), (4, 3)):
        prefix = end
        for t in range(max(geo.sink_tokens, prefix - geo.recent_tokens), prefix):
            assert memory[geo.window_element(12, t)] == t
        for t in range(min(prefix, geo.sink_tokens)):
            assert memory[geo.window_element(12, t)] == t
        for t in range(prefix, prefix + chunk):
            memory[geo.window_element(12, t)] = t
        end = prefix + chunk - rejected


def test_store_windows_latest_writer_only():
    """Closed-form latest-writer window store == sequential simulation of every write."""
    geo = O.Geometry(768, sink_tokens=4, recent_tokens=8, speculative_tokens=3)
    n = 40  # one chunk wraps the 12-entry ring three times
    k = np.arange(n * 256, dtype=np.uint16).reshape(n, 1, 256)
    v = (k + 7).astype(np.uint16)
    table = np.array([[6, 7, 8, 9, 10, 11]], np.int32)
    window = np.zeros(2 * geo.stripe_page_bytes // 2, np.uint16)
    O.store_windows(window, k, v, [0, n], [n], table, [1, n], geo, 4)
    simulated = np.zeros_like(window)
    for t in range(n):  # in order: the last write to an entry wins
        kb = geo.window_element(6, t, 0)
        vb = geo.window_element(6, t, 1)
        simulated[kb : kb + 256] = k[t, 0]
        simulated[vb : vb + 256] = v[t, 0]
    assert np.array_equal(window, simulated)


# ------------------------------------------------------------------ task table


@pytest.mark.parametrize("query_tile", [1, 2, 4])
@pytest.mark.parametrize(
    "lengths,active",
    [([], 0), ([0, 0], 0), ([4] * 128, 512), ([7, 0, 1, 11], 19), ([7, 0, 1, 11], 10)],
)
def test_task_table_closed_form(query_tile, lengths, active):
    # Reference tests/test_tasks.py:82-108.
    max_reqs = 129
    starts = [0]
    for size in lengths:
        starts.append(starts[-1] + size)
    qstarts = np.zeros(max_reqs + 1, np.int32)
    qstarts[: len(starts)] = starts
    tasks, count = O.prepare_tasks(qstarts, [len(lengths), active], max_reqs, query_tile,
                                   num_reqs=max(1, len(lengths)))
    expected = [
        (req, off)
        for req in range(len(lengths))
        for off in range(0, min(starts[req + 1], active) - min(starts[req], active), query_tile)
    ]
    assert count == len(expected)
    assert tasks == expected


# ------------------------------------------------------------------ attention


def test_dense_attention_matches_torch_softmax():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(3, 6, 256, generator=g)
    k = torch.randn(9, 1, 256, generator=g)
    v = torch.randn(9, 1, 256, generator=g)
    out, lse = O.dense_attention(q.numpy(), k.numpy(), v.numpy(), prefix=6)
    scores = torch.einsum("qhd,khd->hqk", q.double(), k.double().expand(9, 6, 256)) / 16
    mask = torch.arange(9)[None, :] > (torch.arange(3)[:, None] + 6)
    scores = scores.masked_fill(mask[None], -float("inf"))
    want = torch.einsum("hqk,khd->qhd", scores.softmax(-1), v.double().expand(9, 6, 256))
    np.testing.assert_allclose(out, want.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, scores.logsumexp(-1).T.numpy(), rtol=1e-6, atol=1e-6)


def test_single_key_attention_returns_value():
    q = np.random.default_rng(0).standard_normal((1, 2, 256)).astype(np.float32)
    v = np.random.default_rng(1).standard_normal((1, 1, 256)).astype(np.float32)
    out, _ = O.dense_attention(q, np.ones((1, 1, 256), np.float32), v, prefix=0)
    np.testing.assert_allclose(out[0, 0], v[0, 0], rtol=1e-6)
    np.testing.assert_allclose(out[0, 1], v[0, 0], rtol=1e-6)


def _paged_state(lengths, prefixes, geo, seed=0):
    """Oracle-only paged cache: history via oracle store_int2, window via store_windows."""
    rng = np.random.default_rng(seed)
    pages = 12
    history = np.full(pages * geo.stripe_page_bytes, 0x5A, np.uint8)
    window = np.full(pages * geo.stripe_page_bytes // 2, 0x5A5A, np.uint16)
    table = np.zeros((len(lengths), 6 * pages), np.int32)
    avail = list(range(1, pages))
    ks, vs = [], []
    rk = O.f32_to_bf16(np.linalg.qr(rng.standard_normal((256, 256)))[0].astype(np.float32))
    rv = O.f32_to_bf16(np.linalg.qr(rng.standard_normal((256, 256)))[0].astype(np.float32))
    cfg = {"sink_tokens": geo.sink_tokens, "recent_tokens": geo.recent_tokens}
    for i, (length, prefix) in enumerate(zip(lengths, prefixes)):
        need = -(-length // geo.physical_block_tokens)
        owned, avail = avail[:need], avail[need:]
        blocks = [p * geo.blocks_per_page + j for p in owned for j in range(geo.blocks_per_page)]
        table[i, : len(blocks)] = blocks
        k = O.f32_to_bf16(rng.standard_normal((length, 1, 256)).astype(np.float32))
        v = O.f32_to_bf16(rng.standard_normal((length, 1, 256)).astype(np.float32))
        ks.append(k)
        vs.append(v)
        if prefix:
            slots = [geo.logical_slot(table[i], t) for t in range(prefix)]
            O.store_int2(history, O.rotate(k[:prefix], rk), O.rotate(v[:prefix], rv), slots,
                         [1, prefix], geo, cfg)
            O.store_windows(window, k[:prefix], v[:prefix], [0, prefix], [prefix], table[i:i + 1],
                            [1, prefix], geo, 1)
    return history, window, table, ks, vs, rk, rv


@pytest.mark.parametrize("splits,split_tokens", [(1, 0), (3, 0), (8, 0), (8, 64), (40, 32)])
def test_history_partials_merge_to_split_invariant_result(splits, split_tokens):
    geo = O.Geometry(768, sink_tokens=4, recent_tokens=16, speculative_tokens=3)
    lengths, prefixes = [300, 130], [299, 128]
    history, window, table, ks, vs, rk, rv = _paged_state(lengths, prefixes, geo)
    rng = np.random.default_rng(3)
    qlens = [l - p for l, p in zip(lengths, prefixes)]
    q = O.f32_to_bf16(rng.standard_normal((sum(qlens), 6, 256)).astype(np.float32))
    qstarts = np.array([0, qlens[0], sum(qlens)], np.int32)
    counts = [2, sum(qlens)]
    tasks, count = O.prepare_tasks(qstarts, counts, 2, 4)
    qrot = O.rotate(q, rk)
    kc = np.concatenate([k[p:] for k, p in zip(ks, prefixes)])
    vc = np.concatenate([v[p:] for v, p in zip(vs, prefixes)])
    ref_p, ref_l = O.attention_partials(qrot, kc, vc, history, window, qstarts, lengths, table,
                                        counts, tasks, count, geo, 1 / 16, 1, False)
    p, l = O.attention_partials(qrot, kc, vc, history, window, qstarts, lengths, table, counts,
                                tasks, count, geo, 1 / 16, splits, False,
                                split_tokens=split_tokens)
    if split_tokens:
        # Token-bounded rule: request r (history length L_r) leaves splits - min(splits,
        # ceil(L_r / split_tokens)) slots unwritten (NaN partials, LSE -inf).
        for r, (seq, qlen) in enumerate(zip(lengths, qlens)):
            prefix = seq - qlen
            sink = min(4, prefix)
            hist_len = max(sink, prefix - 16) - sink
            used = min(splits, max(1, -(-hist_len // split_tokens)))
            rows = slice(int(qstarts[r]), int(qstarts[r + 1]))
            assert np.isnan(p[rows, :, used:]).all() and np.isneginf(l[rows, :, used:]).all()
            assert not np.isnan(p[rows, :, :used]).any()
    out1, lse1 = O.merge_splits(ref_p, ref_l, counts)
    outk, lsek = O.merge_splits(p, l, counts)
    np.testing.assert_allclose(O.bf16_to_f32(outk), O.bf16_to_f32(out1), atol=1e-2)
    np.testing.assert_allclose(lsek, lse1, atol=1e-5)
    # Per-split LSEs are logsumexps of disjoint score sets: logsumexp(l_s) == LSE(1 split).
    both = np.logaddexp.reduce(l.astype(np.float64), axis=-1)
    np.testing.assert_allclose(both, ref_l[..., 0], atol=1e-5)


def test_full_oracle_path_matches_hybrid_reference():
    """attention_partials + merges of the oracle equal the dense hybrid reference."""
    geo = O.Geometry(768, sink_tokens=4, recent_tokens=16, speculative_tokens=3)
    lengths, prefixes = [300, 69], [296, 65]
    history, window, table, ks, vs, rk, rv = _paged_state(lengths, prefixes, geo, seed=7)
    rng = np.random.default_rng(4)
    qlens = [l - p for l, p in zip(lengths, prefixes)]
    qs = [O.f32_to_bf16(rng.standard_normal((n, 6, 256)).astype(np.float32)) for n in qlens]
    q = np.concatenate(qs)
    qstarts = np.array([0, qlens[0], sum(qlens)], np.int32)
    counts = [2, sum(qlens)]
    tasks, count = O.prepare_tasks(qstarts, counts, 2, 4)
    kc = np.concatenate([k[p:] for k, p in zip(ks, prefixes)])
    vc = np.concatenate([v[p:] for v, p in zip(vs, prefixes)])
    hp, hl = O.attention_partials(O.rotate(q, rk), kc, vc, history, window, qstarts, lengths,
                                  table, counts, tasks, count, geo, 1 / 16, 4, False)
    hrot, hlse = O.merge_splits(hp, hl, counts)
    hout = O.rotate(hrot, rv.T.copy())
    rp, rl = O.attention_partials(q, kc, vc, history, window, qstarts, lengths, table, counts,
                                  tasks, count, geo, 1 / 16, 1, True)
    out, lse = O.merge_paths(hout, hlse, rp, rl[..., 0], counts)
    cfg = {"sink_tokens": 4, "recent_tokens": 16}
    want = np.concatenate([O.hybrid_reference(qi, k, v, p, rk, rv, cfg)[0]
                           for qi, k, v, p in zip(qs, ks, vs, prefixes)])
    want_lse = np.concatenate([O.hybrid_reference(qi, k, v, p, rk, rv, cfg)[1]
                               for qi, k, v, p in zip(qs, ks, vs, prefixes)])
    got = O.bf16_to_f32(out).reshape(want.shape)
    np.testing.assert_allclose(got, want, atol=0.035, rtol=0.04)
    np.testing.assert_allclose(lse, want_lse, atol=2e-2)


def test_raw_branch_is_causal_dense_softmax():
    # Reference tests/test_attention_empty_tasks.py:197-204 on the oracle.
    geo = O.Geometry(768, sink_tokens=64, recent_tokens=256)
    rng = np.random.default_rng(15)
    n = 4
    q = O.f32_to_bf16(rng.standard_normal((n, 6, 256)).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal((n, 1, 256)).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal((n, 1, 256)).astype(np.float32))
    table = np.full((1, 6), 6, np.int32)
    tasks, count = O.prepare_tasks(np.array([0, n], np.int32), [1, n], 1, 4)
    p, l = O.attention_partials(q, k, v, np.zeros(1, np.uint8), np.zeros(1, np.uint16),
                                [0, n], [n], table, [1, n], tasks, count, geo, 1 / 16, 1, True)
    qt, kt, vt = (torch.from_numpy(O.bf16_to_f32(x)).double() for x in (q, k, v))
    scores = torch.einsum("thd,sd->hts", qt, kt[:, 0]) / 16
    scores.masked_fill_(torch.ones(n, n, dtype=torch.bool).triu(1), -float("inf"))
    want = torch.einsum("hts,sd->thd", scores.softmax(-1), vt[:, 0])
    np.testing.assert_allclose(p[:, :, 0], want.numpy(), atol=1e-5)
    np.testing.assert_allclose(l[:, :, 0], scores.logsumexp(-1).T.numpy(), atol=1e-5)


def test_empty_history_split_gives_zero_and_neg_inf():
    # Reference tests/test_attention_empty_tasks.py:190-194.
    geo = O.Geometry(768)
    rng = np.random.default_rng(2)
    q = O.f32_to_bf16(rng.standard_normal((4, 6, 256)).astype(np.float32))
    tasks, count = O.prepare_tasks(np.array([0, 4], np.int32), [1, 4], 8, 4)
    p, l = O.attention_partials(q, q[:, :1], q[:, :1], np.zeros(1, np.uint8),
                                np.zeros(1, np.uint16), [0, 4], [4],
                                np.full((1, 6), 2**30, np.int32), [1, 4], tasks, count, geo,
                                1 / 16, 2, False)
    assert (p == 0).all() and np.isneginf(l).all()


def test_inactive_programs_write_nothing():
    geo = O.Geometry(768)
    q = np.zeros((4, 6, 256), np.uint16)
    p, l = O.attention_partials(q, q[:, :1], q[:, :1], np.zeros(1, np.uint8),
                                np.zeros(1, np.uint16), [0, 0], [0], np.zeros((1, 6), np.int32),
                                [0, 0], [(0, 0)] * 4, 0, geo, 1 / 16, 1, False, programs=4)
    assert np.isnan(p).all() and np.isnan(l).all()


def test_merge_paths_limits():
    a = O.f32_to_bf16(np.full((1, 2, 256), 2.0, np.float32))
    b = np.full((1, 2, 1, 256), -1.0, np.float32)
    la = np.array([[-np.inf, 0.0]], np.float32)
    lb = np.array([[0.0, -np.inf]], np.float32)
    out, lse = O.merge_paths(a, la, b, lb, [1, 1])
    out = O.bf16_to_f32(out).reshape(1, 2, 256)
    assert (out[0, 0] == -1).all() and (out[0, 1] == 2).all()
    assert (lse == 0).all()
    out, lse = O.merge_paths(a, np.log([[1.0, 3.0]]).astype(np.float32), b,
                             np.log([[1.0, 1.0]]).astype(np.float32), [1, 1])
    out = O.bf16_to_f32(out).reshape(1, 2, 256)
    np.testing.assert_allclose(out[0, 0], 0.5, rtol=1e-2)
    np.testing.assert_allclose(out[0, 1], (3 * 2 - 1) / 4, rtol=1e-2)
    np.testing.assert_allclose(lse[0], [math.log(2), math.log(4)], rtol=1e-6)


def test_cached_decode_reference_equals_hybrid_reference():
    """The cache read-back restatement equals the dense hybrid reference on one request."""
    geo = O.Geometry(768, sink_tokens=4, recent_tokens=16, speculative_tokens=3)
    lengths, prefixes = [300], [299]
    history, window, table, ks, vs, rk, rv = _paged_state(lengths, prefixes, geo, seed=9)
    q = O.f32_to_bf16(np.random.default_rng(1).standard_normal((1, 6, 256)).astype(np.float32))
    got, lse = O.cached_decode_reference(history, window, table[0], 300, q, ks[0][299:],
                                         vs[0][299:], rk, rv, geo)
    want, want_lse = O.hybrid_reference(q, ks[0], vs[0], 299, rk, rv,
                                        {"sink_tokens": 4, "recent_tokens": 16})
    np.testing.assert_allclose(got, want, atol=2e-3)
    np.testing.assert_allclose(lse, want_lse, atol=2e-4)
    rows = O.dequant_rows(history, [geo.slot_offset(geo.logical_slot(table[0], 50))])
    assert np.array_equal(rows[0], O.load_vec(history, geo.slot_offset(geo.logical_slot(table[0], 50))))


@pytest.mark.parametrize("lo,length,nsplit,block_n", [(4, 32635, 16, 32), (4, 2000, 7, 32),
                                                      (0, 1000, 5, 128), (3, 130, 40, 32),
                                                      (4, 64, 3, 32)])
def test_token_bounded_boundaries_sit_on_the_absolute_chunk_grid(lo, length, nsplit, block_n):
    # The token-bounded split rule: the reference ranges (kernels.py:368-370) with each inner
    # boundary moved down to a multiple of 64 in absolute positions (lo + history index).
    tps = -(-(-(-length // block_n)) // nsplit)
    cuts = []
    for split in range(nsplit):
        begin = split * tps * block_n
        end = min((split + 1) * tps * block_n, length)
        b, e = O.oscar_oracle._chunk_cut(begin, lo, length), O.oscar_oracle._chunk_cut(end, lo, length)
        cuts.append((b, max(b, e)))
        if 0 < begin < length:
            assert (lo + b) % 64 == 0 or b == 0, (split, b)
            assert 0 <= begin - b < 64
    covered = [t for b, e in cuts for t in range(b, e)]
    assert covered == list(range(length))  # contiguous, in order, each token once


def test_blocked_online_softmax_reduces_to_the_dense_softmax():
    # The reference kernel's blocked online softmax (kernels.py:421-436) without the bf16
    # rounding of p is the dense softmax up to fp32 state; with it, each p carries one bf16
    # rounding (relative 2^-8 at most), so the output moves by at most that fraction of the
    # values' magnitude. Masked positions (pos > limit) take no weight.
    rng = np.random.default_rng(21)
    q = rng.standard_normal((6, 256))
    keys = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((300, 256)).astype(np.float32)))
    values = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((300, 256)).astype(np.float32)))
    pos = np.arange(300)
    limit = np.array([299, 299, 150, 150, 37, 0])
    keys64, values64 = keys.astype(np.float64), values.astype(np.float64)
    for r in range(6):
        sc = (keys64[: limit[r] + 1] @ q[r]) / 16
        want, want_l = OO._row_softmax(sc, values64[: limit[r] + 1])
        out, lse = OO._blocked_softmax(q[r:r + 1], keys64, values64, pos, limit[r:r + 1], 1 / 16,
                                      32, False)
        np.testing.assert_allclose(out[0], want, atol=2e-6)
        np.testing.assert_allclose(lse[0], want_l, atol=2e-6)
        rounded, _ = OO._blocked_softmax(q[r:r + 1], keys64, values64, pos, limit[r:r + 1],
                                        1 / 16, 32, True)
        assert np.abs(rounded[0] - want).max() <= 2.0 ** -8 * np.abs(values).max()
    out, lse = OO._blocked_softmax(q[:1], keys64[:0], values64[:0], pos[:0], limit[:1], 1 / 16,
                                  32, True)
    assert not out.any() and np.isneginf(lse).all()


def test_decode_variants_agree_within_their_rounding():
    # One cache, three references: "exact" (float64 dequant) is dense attention over the
    # exactly dequantized history; "oracle" rounds the dequantized values to bf16 and
    # "reference_kernel" adds the reference kernels' bf16 roundings (q_rot, p, merged
    # history, inverse rotation, output), so both stay within a few bf16 steps of "exact"
    # in relative L2 (a bf16 rounding is 2^-9 relative at most). The reference kernel's
    # result does not depend on its split count beyond rounding.
    geo = O.Geometry(768, sink_tokens=4, recent_tokens=16, speculative_tokens=3)
    history, window, table, ks, vs, rk, rv = _paged_state([700], [696], geo, seed=11)
    q = O.f32_to_bf16(np.random.default_rng(2).standard_normal((4, 6, 256)).astype(np.float32))
    args = (history, window, table[0], 700, q, ks[0][696:], vs[0][696:], rk, rv, geo)
    v = O.cached_decode_variants(*args, scale=1 / 16, splits=4)
    exact, exact_l = v["exact"]

    def rel(a):
        return np.linalg.norm(a - exact) / np.linalg.norm(exact)

    assert rel(v["oracle"][0]) < 1e-2 and rel(v["reference_kernel"][0]) < 1.5e-2
    np.testing.assert_allclose(v["oracle"][1], exact_l, atol=2e-3)
    np.testing.assert_allclose(v["reference_kernel"][1], exact_l, atol=2e-2)
    # "exact" is dense attention over the float64 dequantized history (recomputed here).
    d = 256
    bk = geo.kernel_block_tokens
    pos = np.arange(4, 696 - 16)
    slots = table[0][pos // bk].astype(np.int64) * bk + pos % bk
    offs = np.array([geo.slot_offset(s) for s in slots])
    keys = np.zeros((700, d))
    values = np.zeros((700, d))
    rkf, rvf = O.bf16_to_f32(rk).astype(np.float64), O.bf16_to_f32(rv).astype(np.float64)
    keys[4:680] = OO._dequant_exact(history, offs) @ rkf.T
    values[4:680] = OO._dequant_exact(history, offs + geo.vector_bytes) @ rvf.T
    for p in list(range(4)) + list(range(680, 696)):
        keys[p] = O.bf16_to_f32(window[geo.window_element(table[0][0], p, 0):][:d])
        values[p] = O.bf16_to_f32(window[geo.window_element(table[0][0], p, 1):][:d])
    keys[696:] = O.bf16_to_f32(ks[0][696:, 0])
    values[696:] = O.bf16_to_f32(vs[0][696:, 0])
    want, want_l = O.dense_attention(O.bf16_to_f32(q), keys[:, None], values[:, None], 696)
    np.testing.assert_allclose(exact, want, atol=1e-6)
    np.testing.assert_allclose(exact_l, want_l, atol=1e-5)
    # The exact dequant differs from load_vec's only by the bf16 rounding.
    diff = OO._dequant_exact(history, offs[:8]) - O.bf16_to_f32(O.dequant_rows(history, offs[:8]))
    assert np.abs(diff).max() <= 2.0 ** -8 * np.abs(OO._dequant_exact(history, offs[:8])).max()
    one = O.cached_decode_variants(*args, scale=1 / 16, splits=1)["reference_kernel"][0]
    assert np.linalg.norm(one - v["reference_kernel"][0]) <= 1e-2 * np.linalg.norm(exact)

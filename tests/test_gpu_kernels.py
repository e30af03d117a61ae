"""Device parity of every entry point against the CPU oracle (runs on an MI355X).

Bars: INT2 codes, packed bytes and task tables bit-exact; rotation within the reference's
tolerance (tests/test_npu_kernels.py:99-109: atol 0.03125, rtol 0.015); attention partials
within bf16 tolerances stated per test.
"""

import numpy as np
import pytest
import torch
from dataclasses import replace

import oracle as O
from oscar_new_amd import kernels
from oscar_new_amd.config import OscarConfig, task_capacity
from tests._state import bits, from_bits, make_state, oracle_geometry

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qr_bf16(seed, device=DEV):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16().to(device)


def test_library_loaded_from_tree():
    from oscar_new_amd import _ext

    lib = _ext.library()
    assert lib.oscar_abi_version() == 1
    assert str(_ext.LIBRARY_PATH).endswith("oscar_new_amd/liboscar_hip.so")


# ------------------------------------------------------------------ rotate


def test_rotation_strides_match_oracle():
    # Reference tests/test_npu_kernels.py:99-109.
    torch.manual_seed(7)
    x = torch.randn(23, 12, 256, device=DEV, dtype=torch.bfloat16)[:, ::2]
    r = _qr_bf16(0).T
    out = kernels.rotate(x, r)
    want = O.rotate(bits(x), bits(r.contiguous()))
    got = bits(out)
    torch.testing.assert_close(torch.from_numpy(O.bf16_to_f32(got)),
                               torch.from_numpy(O.bf16_to_f32(want)), atol=0.03125, rtol=0.015)
    # fp32 accumulation in a different order moves a result by at most one bf16 step.
    g32, w32 = O.bf16_to_f32(got), O.bf16_to_f32(want)
    assert np.all(np.abs(g32 - w32) <= 2.0**-7 * np.abs(w32) + 1e-4)
    assert (g32 != w32).mean() < 0.02


@pytest.mark.parametrize("rows", [1, 7, 64, 65, 4096])
def test_rotation_sizes_contiguous(rows):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 1, 256, generator=g).bfloat16().to(DEV)
    r = _qr_bf16(3)
    got = O.bf16_to_f32(bits(kernels.rotate(x, r)))
    want = O.bf16_to_f32(O.rotate(bits(x), bits(r)))
    # A different fp32 summation order may move a result across one bf16 rounding boundary.
    assert np.all(np.abs(got - want) <= 2.0**-7 * np.abs(want) + 1e-4)
    assert (got != want).mean() < 0.02


@pytest.mark.parametrize("tokens,heads,layout", [
    (4096, 1, "rows"),  # the store benchmark's shape, R row-major
    (1029, 2, "cols"),  # ragged row count, two heads, R column-contiguous
    (8200, 1, "rows"),  # more 16-row blocks than workgroups: each workgroup loops
    (700, 3, "strided"),  # strided x (every other head of a [700, 6, 256] buffer)
])
def test_rotation_tiled_is_bitwise_the_small_kernel(tokens, heads, layout):
    # From 1024 rows on, rotate stages R in LDS (rotate_tiled_kernel); slices below that
    # size take the per-tile kernel. Same operands and k order: the same bits.
    g = torch.Generator().manual_seed(tokens)
    r = _qr_bf16(5)
    if layout == "cols":
        r = r.T.contiguous().T  # column-contiguous view of the same matrix
    if layout == "strided":
        x = torch.randn(tokens, 2 * heads, 256, generator=g).bfloat16().to(DEV)[:, ::2]
    else:
        x = torch.randn(tokens, heads, 256, generator=g).bfloat16().to(DEV)
    assert x.shape[0] * x.shape[1] >= 1024
    got = kernels.rotate(x, r)
    step = 1000 // heads
    want = torch.cat([kernels.rotate(x[i : i + step], r) for i in range(0, tokens, step)])
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


# ------------------------------------------------------------------ store_int2 / unpack


def _check_slots(history_cpu, slots, expected, layout):
    for index, slot in enumerate(slots):
        off = layout.slot_offset(int(slot))
        assert np.array_equal(history_cpu[off : off + 136], expected[index, 0, :136]), index
        assert (history_cpu[off + 136 : off + 160] == 0x5A).all()


@pytest.mark.parametrize(
    "mode,ratio",
    [("percentile", 0), ("percentile", 0.92), ("percentile", 0.96), ("percentile", 1.0),
     ("factor", 0), ("search", 0)],
)
def test_store_bytes_bit_exact_and_sentinels(mode, ratio):
    # Reference tests/test_npu_kernels.py:71-96.
    kw = dict(k_clip_ratio=ratio, v_clip_ratio=ratio, clip_mode=mode)
    if mode == "factor":
        kw.update(k_clip_factor=0.7, v_clip_factor=0.9)
    cfg = replace(OscarConfig(), **kw)
    layout, raw, history, _, meta, _ = make_state([800], [760], cfg)
    torch.manual_seed(3)
    k = torch.randn(40, 1, 256).bfloat16()
    v = torch.randn_like(k)
    k[0].zero_()
    k[1].fill_(0.5)
    k[2].fill_(1e-12)
    # Values on half- and quarter-step grids put (x - zero) / scale + 0.5 exactly on 1, 2
    # and 3 for many clip thresholds: the quotients the fast path must hand to IEEE division.
    idx = torch.arange(256)
    g = torch.Generator().manual_seed(5)
    for row, (mod, step, off) in enumerate([(7, 0.5, 3), (13, 0.25, 6), (4, 1.0, 0),
                                            (9, 0.5, 4), (25, 0.125, 12)], start=3):
        vals = ((idx % mod) - off).float() * step
        k[row, 0] = vals[torch.randperm(256, generator=g)].bfloat16()
        v[row, 0] = (-vals).bfloat16()
    kernels.store_int2(k.to(DEV), v.to(DEV), history, meta.slot_mapping, meta.counts, layout)
    expected = O.packed_slots(bits(k), bits(v), cfg)
    history_cpu = history.cpu().numpy()
    _check_slots(history_cpu, meta.slot_mapping.cpu().tolist(), expected, layout)
    assert (raw[: 20 * 15360].cpu() == 0x5A).all()
    assert (history_cpu[: layout.stripe_page_bytes] == 0x5A).all()
    # Diagnostic dequant: the unpack is exact, identity rotation keeps it exact.
    eye = torch.eye(256, device=DEV, dtype=torch.bfloat16)
    kd, vd = kernels.dequant_inverse_rotate(history, meta.slot_mapping, eye, eye, layout)
    geo = oracle_geometry(layout)
    ko, vo = O.unpack(history_cpu, meta.slot_mapping.cpu().numpy(), geo)
    assert np.array_equal(bits(kd), ko) and np.array_equal(bits(vd), vo)


@pytest.mark.parametrize("tokens,heads,mode,active", [
    (4096, 1, "search", 4096),  # the store benchmark's shape
    (37, 2, "percentile", 30),  # ragged block, two heads, padded tokens past the count
    (300, 1, "factor", 300),
])
def test_rotate_store_is_bitwise_rotate_then_store(tokens, heads, mode, active):
    # One launch against oscar_rotate (K, V) + oscar_store_int2: every cache byte.
    g = torch.Generator().manual_seed(tokens + heads)
    cfg = replace(OscarConfig(), clip_mode=mode, k_clip_ratio=0.96, v_clip_ratio=0.92,
                  k_clip_factor=0.7, v_clip_factor=0.9)
    from oscar_new_amd.layout import CacheLayout

    layout = CacheLayout(768, kv_heads=heads, config=cfg)
    pages = max(2, -(-tokens // 768) + 1)
    base = torch.full((pages * layout.stripe_page_bytes,), 0x5A, dtype=torch.uint8, device=DEV)
    k = torch.randn(tokens, 2 * heads, 256, generator=g).bfloat16().to(DEV)[:, ::2]  # strided
    v = torch.randn(tokens, heads, 256, generator=g).bfloat16().to(DEV)
    perm = torch.randperm((pages - 1) * 768, generator=g)[:tokens] + 768
    slots = perm.to(torch.int64).to(DEV)
    slots[3] = -1  # a masked row
    counts = torch.tensor([1, active], dtype=torch.int32, device=DEV)
    rk, rv = _qr_bf16(11), _qr_bf16(12)
    want = base.clone()
    kernels.store_int2(kernels.rotate(k, rk), kernels.rotate(v, rv), want, slots, counts, layout)
    got = base.clone()
    kernels.rotate_store_int2(k, v, rk.T.contiguous(), rv.T.contiguous(), got, slots, counts,
                              layout)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want.cpu())
    assert not torch.equal(got.cpu(), base.cpu())


def test_store_skips_masked_rows():
    layout, raw, history, _, meta, _ = make_state([800], [760])
    before = history.clone()
    k = torch.randn(40, 1, 256, device=DEV, dtype=torch.bfloat16)
    slots = meta.slot_mapping.clone()
    slots[5] = -1
    counts = torch.tensor([1, 30], device=DEV, dtype=torch.int32)
    kernels.store_int2(k, k, history, slots, counts, layout)
    changed = (history != before).nonzero().flatten().cpu().numpy()
    touched = set()
    for t, s in enumerate(slots.cpu().tolist()):
        if t < 30 and s >= 0:
            off = layout.slot_offset(s)
            touched.update(range(off, off + 136))
    assert set(changed.tolist()) <= touched
    off5 = layout.slot_offset(int(meta.slot_mapping[5]))
    assert (history[off5 : off5 + 160] == 0x5A).all()


def test_store_c2_scale_rotated_outliers_permuted_pages():
    """4096 tokens, 2% outlier channels x10, permuted page slots."""
    g = torch.Generator().manual_seed(2)
    n = 4096
    cfg = OscarConfig(sink_tokens=4, recent_tokens=128)
    layout = __import__("oscar_new_amd.layout", fromlist=["CacheLayout"]).CacheLayout(768, config=cfg)
    pages = 12
    history = torch.full((pages * layout.stripe_page_bytes,), 0x5A, dtype=torch.uint8, device=DEV)
    blocks = torch.randperm(pages * 6, generator=g)[: n // 128]
    slots = (blocks[:, None] * 128 + torch.arange(128)[None]).reshape(-1).to(torch.int64)
    k = torch.randn(n, 1, 256, generator=g)
    v = torch.randn(n, 1, 256, generator=g)
    chans = torch.randperm(256, generator=g)[:5]
    k[..., chans] *= 10
    v[..., chans] *= 10
    r_k, r_v = _qr_bf16(11), _qr_bf16(12)
    kr = kernels.rotate(k.bfloat16().to(DEV), r_k)
    vr = kernels.rotate(v.bfloat16().to(DEV), r_v)
    counts = torch.tensor([1, n], dtype=torch.int32, device=DEV)
    for mode in ("percentile", "search"):
        history.fill_(0x5A)
        cfg_m = replace(cfg, clip_mode=mode)
        lay = replace(layout, config=cfg_m)
        kernels.store_int2(kr, vr, history, slots.to(DEV), counts, lay)
        expected = O.packed_slots(bits(kr), bits(vr), cfg_m)
        _check_slots(history.cpu().numpy(), slots.tolist(), expected, lay)


def test_store_search_degenerate_ranges_bit_exact():
    """Search clip mode on vectors whose clipped range spans under three steps (spreads below
    3 * 2^-14, large offsets against small spreads): the fast candidate pass does not apply
    and the exact pass decides; bytes as the oracle's."""
    g = torch.Generator().manual_seed(31)
    n = 2048
    cfg = OscarConfig(sink_tokens=4, recent_tokens=128, clip_mode="search")
    layout = __import__("oscar_new_amd.layout", fromlist=["CacheLayout"]).CacheLayout(768, config=cfg)
    pages = 6
    history = torch.full((pages * layout.stripe_page_bytes,), 0x5A, dtype=torch.uint8, device=DEV)
    blocks = torch.randperm(pages * 6, generator=g)[: n // 128]
    slots = (blocks[:, None] * 128 + torch.arange(128)[None]).reshape(-1).to(torch.int64)
    parts = [1e-5 * torch.randn(512, 1, 256, generator=g),
             3e-5 * torch.randn(512, 1, 256, generator=g),
             100 + 0.02 * torch.randn(256, 1, 256, generator=g),
             37 + 0.05 * torch.randn(256, 1, 256, generator=g),
             -50 + torch.rand(256, 1, 256, generator=g),
             torch.full((256, 1, 256), 3.25)]
    k = torch.cat(parts).bfloat16()
    v = torch.cat(parts[::-1]).bfloat16()
    counts = torch.tensor([1, n], dtype=torch.int32, device=DEV)
    kernels.store_int2(k.to(DEV), v.to(DEV), history, slots.to(DEV), counts, layout)
    expected = O.packed_slots(bits(k), bits(v), cfg)
    _check_slots(history.cpu().numpy(), slots.tolist(), expected, layout)


# ------------------------------------------------------------------ prepare_tasks


@pytest.mark.parametrize("query_tile", [1, 2, 4])
@pytest.mark.parametrize(
    "lengths,active",
    [([], 0), ([0, 0], 0), ([4] * 128, 512), ([7, 0, 1, 11], 19), ([7, 0, 1, 11], 10)],
)
def test_prepare_tasks_bit_exact(query_tile, lengths, active):
    # Reference tests/test_tasks.py:82-108 (closed form) on device.
    max_reqs = 129
    starts = [0]
    for size in lengths:
        starts.append(starts[-1] + size)
    qstarts = torch.zeros(max_reqs + 1, dtype=torch.int32)
    qstarts[: len(starts)] = torch.tensor(starts, dtype=torch.int32)
    counts = torch.tensor([len(lengths), active], dtype=torch.int32)
    capacity = task_capacity(max(active, 1), max_reqs, query_tile)
    tasks = torch.full((capacity, 2), -99, dtype=torch.int32, device=DEV)
    total = torch.full((1,), -99, dtype=torch.int32, device=DEV)
    kernels.prepare_tasks(qstarts.to(DEV), counts.to(DEV), tasks, total, max_reqs, query_tile,
                          num_reqs=max(1, len(lengths)))
    want, count = O.prepare_tasks(qstarts.numpy(), counts.numpy(), max_reqs, query_tile,
                                  num_reqs=max(1, len(lengths)))
    assert total.item() == count
    assert [tuple(r) for r in tasks[:count].tolist()] == want
    assert tasks[count:].eq(-99).all()


def test_prepare_tasks_copies_reachable_columns():
    max_reqs, cols = 5, 700
    src = torch.arange(max_reqs * 800, dtype=torch.int32, device=DEV).view(max_reqs, 800)
    table = torch.full((max_reqs, 900), -1, dtype=torch.int32, device=DEV)
    qstarts = torch.tensor([0, 1, 2, 3, 0, 0], dtype=torch.int32, device=DEV)
    counts = torch.tensor([3, 3], dtype=torch.int32, device=DEV)
    tasks = torch.zeros((8, 2), dtype=torch.int32, device=DEV)
    total = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.prepare_tasks(qstarts, counts, tasks, total, max_reqs, 4, num_reqs=3,
                          source_table=src, table=table, copy_columns=cols)
    assert torch.equal(table[:3, :cols], src[:3, :cols])
    assert table[:3, cols:].eq(-1).all() and table[3:].eq(-1).all()

"""Host mirror of config.py / layout.py against the reference's known answers."""

from dataclasses import replace

import numpy as np
import pytest
import torch

from oscar_new_amd.config import (
    OscarConfig,
    attention_programs,
    choose_splits,
    choose_device_partition,
    choose_history_partition,
    choose_splits_mi355x,
    device_split_tokens,
    percentile_selection,
    task_capacity,
)
from oscar_new_amd.layout import CacheLayout


def test_exact_target_geometry():
    # Reference tests/test_layout.py:11-19.
    layout = CacheLayout(768)
    assert layout.config.vector_bytes == 68
    assert layout.config.slot_bytes == 160
    assert layout.stripe_page_bytes == 393216
    assert layout.history_page_bytes == 122880
    assert layout.window_page_bytes == 331776
    assert layout.blocks_per_page == 6
    assert 15360 + layout.stripe_page_bytes * 2 == 801792


@pytest.mark.parametrize("bad", [0, 128, 256, 384, 512, 640, 769])
def test_reject_small_or_nondivisible_page(bad):
    # Reference tests/test_layout.py:22-25.
    with pytest.raises(ValueError):
        CacheLayout(bad)


def test_bench_geometry_fits_and_small_windows():
    cfg = OscarConfig(sink_tokens=4, recent_tokens=128)
    layout = CacheLayout(768, config=cfg)
    assert cfg.ring_tokens == 132 and cfg.window_tokens == 136
    assert layout.window_page_bytes <= layout.stripe_page_bytes
    CacheLayout(384, config=OscarConfig(sink_tokens=4, recent_tokens=64))


def test_virtual_blocks_resolve_to_physical_page_and_do_not_overlap():
    # Reference tests/test_layout.py:28-58.
    layout = CacheLayout(768)
    pages = 9
    conv_bytes = 15360 * pages
    stripe_bytes = layout.stripe_page_bytes * pages
    raw = torch.full((conv_bytes + 2 * stripe_bytes,), 0x5A, dtype=torch.uint8)
    k = raw[conv_bytes : conv_bytes + stripe_bytes].view(torch.bfloat16).view(-1, 128, 1, 256)
    v = raw[conv_bytes + stripe_bytes :].view(torch.bfloat16).view(-1, 128, 1, 256)
    hist, ring = layout.tensor_views((k, v))
    assert hist.data_ptr() == k.data_ptr() and ring.data_ptr() == v.data_ptr()
    table = [p * 6 + j for p in (5, 2, 7) for j in range(6)]
    for t in range(2304):
        begin = layout.slot_offset(layout.logical_slot(table, t))
        hist[begin : begin + 136] = 7
        offset = layout.window_offset(table[0], t)
        raw[conv_bytes + stripe_bytes + offset : conv_bytes + stripe_bytes + offset + 1024] = 3
    for p in (0, 1, 3, 4, 6, 8):
        assert (hist[p * layout.stripe_page_bytes : (p + 1) * layout.stripe_page_bytes] == 0x5A).all()
    assert (raw[:conv_bytes] == 0x5A).all()
    vbytes = v.view(torch.uint8).view(-1)
    for p in range(pages):
        if p != 5:
            assert (vbytes[p * layout.stripe_page_bytes : (p + 1) * layout.stripe_page_bytes] == 0x5A).all()


def test_ring_preserves_rejection_rollback_and_sink():
    # Reference tests/test_layout.py:61-75.
    cfg = OscarConfig()
    layout = CacheLayout(768, config=cfg)
    memory, end = {}, 0
    for chunk, rejected in ((1024, 0), (4, 3), (4, 2), (4, 0), (300, 0), (4, 3)):
        prefix = end
        for t in range(max(cfg.sink_tokens, prefix - cfg.recent_tokens), prefix):
            assert memory[layout.window_offset(12, t)] == t
        for t in range(min(prefix, cfg.sink_tokens)):
            assert memory[layout.window_offset(12, t)] == t
        for t in range(prefix, prefix + chunk):
            memory[layout.window_offset(12, t)] = t
        end = prefix + chunk - rejected


def test_reorder_and_reuse_do_not_use_batch_indices():
    # Reference tests/test_layout.py:78-85.
    layout = CacheLayout(768)
    owners = {"a": 12, "b": 30}
    before = {r: layout.window_offset(o, 810) for r, o in owners.items()}
    after = {r: layout.window_offset(owners[r], 810) for r in reversed(owners)}
    assert before == after and before["a"] != before["b"]
    with pytest.raises(ValueError):
        layout.window_offset(13, 0)


def test_tensor_views_reject_bad_caches():
    layout = CacheLayout(768)
    good = torch.zeros(6, 128, 1, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        layout.tensor_views(good)
    with pytest.raises(ValueError):
        layout.tensor_views((good.float(), good.float()))
    with pytest.raises(ValueError):
        layout.tensor_views((torch.zeros(5, 128, 1, 256, dtype=torch.bfloat16),) * 2)


def test_split_policy_bounds_current_scratch():
    # Reference tests/test_layout.py:113-115.
    assert [choose_splits(b, 1, 4) for b in (1, 16, 128)] == [32, 16, 8]
    assert choose_splits(1, 1, 16384) == 1


def test_mi355x_split_policy_fills_the_chip():
    assert choose_splits_mi355x(32, 1, 1, 32768) == 16  # 512 workgroups
    assert choose_splits_mi355x(4, 1, 1, 262144) == 128
    assert choose_splits_mi355x(64, 1, 4, 131072) == 8
    assert choose_splits_mi355x(4, 1, 1, 2048) == 2  # never below 1024 tokens per split
    assert choose_splits_mi355x(1, 1, 17) == 1


def test_history_partition_mi355x():
    # Uniform batches: the same splits as choose_splits_mi355x, split_tokens = the even share.
    assert choose_history_partition(32, 1, 1, 32768, 32 * 32768) == (16, 2048)
    assert choose_history_partition(4, 1, 1, 262144, 4 * 262144) == (128, 2048)
    # Ragged batch: the longest request takes ceil(131072 / 2368) splits of the even share.
    assert choose_history_partition(64, 1, 4, 131072, 1212000) == (56, 2368)
    # Small batches keep at least 1024 tokens per split; unknown bounds fall back.
    assert choose_history_partition(1, 1, 1, 4096, 4096) == (4, 1024)
    assert choose_history_partition(4, 1, 1, None) == (choose_splits_mi355x(4, 1, 1), 0)
    assert choose_history_partition(2, 1, 17, 8192, 9000) == (1, 0)


def test_history_partition_leaves_the_role_slots_free():
    # c3 (32 x 32635 history tokens) beside 48 role workgroups: at most 512 - 48 - 32 full
    # shares, so 14 splits of 2432 tokens (448 history workgroups); c5 beside 12: 121 x 2176.
    assert choose_history_partition(32, 1, 1, 32768, 32 * 32635, reserved=48) == (14, 2432)
    assert choose_history_partition(4, 1, 1, 262144, 4 * 262011, reserved=12) == (121, 2176)
    # For any lengths with that total, the splits in use fit the slots left.
    rng = __import__("random").Random(5)
    for _ in range(200):
        tasks = rng.randint(1, 64)
        lengths = [rng.randint(1, 70000) for _ in range(tasks)]
        reserved = rng.randint(1, 200)
        splits, tokens = choose_history_partition(tasks, 1, 1, max(lengths), sum(lengths),
                                                  reserved=reserved, max_splits=10**6)
        used = sum(-(-n // tokens) for n in lengths)
        assert used <= max(512 - reserved, tasks) or tokens == 1024, (lengths, reserved)


def test_bad_config_rejected():
    # Reference tests/test_layout.py:118-127.
    for kwargs in ({"group_size": 128}, {"head_dim": 128}, {"k_clip_ratio": 0.5},
                   {"k_clip_factor": float("nan")}, {"sink_tokens": -1},
                   {"speculative_tokens": 16}, {"clip_mode": "median"}, {"block_n": 64},
                   {"queries_per_tile": 3}):
        with pytest.raises(ValueError):
            replace(OscarConfig(), **kwargs)
    replace(OscarConfig(), clip_mode="search")


def test_percentile_selection_and_grid_known_values():
    # Reference docs/design.md: 12 (K, r=0.96) and 22 (V, r=0.92) selection rounds; tests/test_tasks.py:123-124.
    assert percentile_selection(0.96)[:2] == (11, 10)
    assert percentile_selection(0.92)[:2] == (21, 20)
    assert abs(percentile_selection(0.96)[2] - 0.8) < 1e-9
    assert attention_programs(512, 129, 4) * 8 == 2048
    assert attention_programs(512, 129, 4) == 256
    assert task_capacity(32, 33, 4) == 32


def test_from_env(monkeypatch):
    monkeypatch.setenv("VLLM_OSCAR_SINK_TOKENS", "4")
    monkeypatch.setenv("VLLM_OSCAR_RECENT_TOKENS", "128")
    monkeypatch.setenv("OSCAR_ASCEND_CLIP_MODE", "factor")
    cfg = OscarConfig.from_env(speculative_tokens=0)
    assert (cfg.sink_tokens, cfg.recent_tokens, cfg.ring_tokens, cfg.clip_mode) == (4, 128, 129, "factor")


def test_device_partition_is_sized_from_capture_stable_values():
    # Decode (6 rows per task, paired kernel): 512 slots less the roles of the launch (one
    # BF16-branch workgroup per task, 8 K/V store workgroups per 16 rows); splits bound a
    # request at twice the even share of a 32-request batch, never below 16.
    assert choose_device_partition(32, 1, 1, 32, 6, reserved=32 + 16) == (16, -464)
    assert choose_device_partition(4, 1, 1, 4, 6, reserved=4 + 8) == (128, -500)
    assert choose_device_partition(8, 1, 1, 8, 6) == (64, -512)
    assert choose_device_partition(512, 1, 1, 512, 6)[0] == 16
    # MTP (24 rows per task, work queue): 448 slots, splits bounded by 128 MiB of scratch.
    assert choose_device_partition(127, 1, 4, 256, 6) == (85, -448)
    assert choose_device_partition(2048, 1, 4, 8192, 6) == (16, -448)
    # Long prefill chunks keep one split (config.py:86-87).
    assert choose_device_partition(4, 1, 17, 4096, 6) == (1, 0)


def test_device_split_tokens_matches_the_host_partition_on_baseline_batches():
    # c3: 32 x 32635 history tokens, budget 464 -> 2432-token splits, 14 per request, 448
    # units (the measured host partition); c5: 4 x 262011, budget 500 -> 2176, 121 each.
    t = device_split_tokens(32 * 32635, 32, 1, 464)
    assert t == 2432 and -(-32635 // t) == 14
    t = device_split_tokens(4 * 262011, 4, 1, 500)
    assert t == 2176 and -(-262011 // t) == 121
    # Never below 1024 tokens; one split per task once the budget is spent on tasks.
    assert device_split_tokens(10, 2, 1, 512) == 1024
    assert device_split_tokens(10 ** 6, 600, 1, 512) == 10 ** 6
    # The work queue (no grid to fit): about `budget` units; c4 (seed 1234: 1,207,677 history
    # tokens over 64 requests) -> 2752-token splits, 475 units, the host partition's.
    assert device_split_tokens(1207677, 64, 1, 448, fit_grid=False) == 2752


@pytest.mark.parametrize("seed", range(20))
def test_device_rule_units_fit_the_budget(seed):
    # Sum over tasks of ceil(L / T) stays within max(B / H, tasks + 1): the grid the host
    # sizes (device_unit_slices) holds every unit of any batch.
    rng = np.random.default_rng(seed)
    tasks = int(rng.integers(1, 300))
    heads = int(rng.integers(1, 3))
    budget = int(rng.integers(16, 520))
    lengths = rng.integers(0, 300000, tasks) * (rng.random(tasks) < 0.9)
    t = device_split_tokens(int(lengths.sum()), tasks, heads, budget)
    units = sum(max(1, -(-int(l) // t)) for l in lengths)
    assert units <= max(-(-budget // heads), tasks + 1)

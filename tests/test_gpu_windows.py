"""BF16 window bytes on the device against the oracle's ``store_windows`` (reference
kernels.py:544-620; ring rules of tests/test_layout.py:61-75 and the device rollback test
tests/test_npu_kernels.py:248-290).

Two requests, two KV heads (4 query heads), S = 4 sink tokens and a 68-token ring (R 64 +
3 speculative + 1), run through a sequence of steps that covers sink writes (a request's
first 3 tokens), a first chunk of 100 tokens that wraps the ring, a 70-token chunk that
overwrites the whole ring, and MTP verification steps of 4 tokens with 3, 2, 0, 3 and 1
rejected drafts (the next step rewrites the rejected positions). After every step the
whole V stripe (every window of every page, and the 0x5A sentinel bytes around them) must
equal, byte for byte, the oracle's window store applied to the stripe before the step, for
each of the three device paths that store windows:

* ``kernels.store_windows`` (the single entry point);
* the fused layer step (``post_attention``'s window workgroups);
* the two-launch history + post step (the window slice of its grid);
* the one-launch layer step (the workgroup that completes a task stores its window).

The single entry point must also leave the K stripe untouched.
"""

import numpy as np
import pytest
import torch

import oracle as O
from oscar_new_amd import kernels
from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import OscarConfig
from tests._state import bits, make_state, native_views, oracle_geometry

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, HQ = 2, 4
# (prefix, chunk, rejected) per request and step.
STEPS = [
    ((0, 3, 0), (0, 100, 0)),
    ((3, 4, 3), (100, 1, 0)),
    ((4, 4, 2), (101, 4, 0)),
    ((6, 4, 0), (105, 70, 0)),
    ((10, 4, 3), (175, 4, 1)),
    ((11, 4, 1), (178, 1, 0)),
    ((14, 1, 0), (179, 1, 0)),
]


def _set_step(meta, tables, layout, step):
    qstarts, seqs, slots = [0], [], []
    for r, (prefix, chunk, _) in enumerate(step):
        qstarts.append(qstarts[-1] + chunk)
        seqs.append(prefix + chunk)
        slots += [int(tables[r, t // 128]) * 128 + t % 128 for t in range(prefix, prefix + chunk)]
    n = qstarts[-1]
    meta.query_start_loc[: len(qstarts)].copy_(torch.tensor(qstarts, dtype=torch.int32))
    meta.seq_lens[: len(seqs)].copy_(torch.tensor(seqs, dtype=torch.int32))
    meta.counts.copy_(torch.tensor([len(step), n], dtype=torch.int32))
    meta.slot_mapping = torch.tensor(slots, dtype=torch.int64, device=DEV)
    meta.num_reqs, meta.num_actual_tokens = len(step), n
    meta.max_query_len = max(chunk for _, chunk, _ in step)
    meta.layout = layout
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count,
                          meta.max_num_reqs, layout.config.queries_per_tile)
    return n


def test_window_bytes_match_oracle_through_ring_wraps_and_rollbacks():
    cfg = OscarConfig(sink_tokens=4, recent_tokens=64)
    assert cfg.ring_tokens == 68
    layout, raw, _, _, meta, tables = make_state([768, 768], [0, 0], cfg, kv_heads=H, max_reqs=4)
    # Room for the longest step's tasks.
    meta.tasks = torch.zeros((256, 2), dtype=torch.int32, device=DEV)
    geo = oracle_geometry(layout)
    eye = torch.eye(256, dtype=torch.bfloat16, device=DEV)
    g = torch.Generator().manual_seed(17)
    for index, step in enumerate(STEPS):
        n = _set_step(meta, tables, layout, step)
        print(f"[windows] step {index}: {step}", flush=True)
        q = torch.randn(n, HQ, 256, generator=g).bfloat16().to(DEV)
        k = torch.randn(n, H, 256, generator=g).bfloat16().to(DEV)
        v = torch.randn(n, H, 256, generator=g).bfloat16().to(DEV)
        before_k, before_v = native_views(raw, layout)
        want = O.store_windows(bits(before_v).reshape(-1), bits(k), bits(v),
                               meta.query_start_loc.cpu().numpy(), meta.seq_lens.cpu().numpy(),
                               tables.numpy(), meta.counts.cpu().numpy(), geo, meta.max_num_reqs)
        k_stripe = before_k.view(torch.int16).clone()  # bit patterns: INT2 bytes hold NaNs

        single = raw.clone()
        _, window = layout.tensor_views(native_views(single, layout))
        kernels.store_windows(k, v, window, meta, layout)
        torch.cuda.synchronize()
        got_k, got_v = native_views(single, layout)
        assert np.array_equal(bits(got_v).reshape(-1), want), f"store_windows, step {index}"
        assert torch.equal(got_k.view(torch.int16), k_stripe), \
            f"store_windows wrote the K stripe, step {index}"

        for one_launch, layer in ((False, False), (True, False), (False, True)):
            fused = raw.clone()
            impl = OscarAttentionImpl.standalone(HQ, 256, 1 / 16, H, cfg,
                                                 one_launch_post=one_launch, layer_step=layer)
            impl.set_rotations(eye, eye)
            out = torch.empty(n, HQ * 256, dtype=torch.bfloat16, device=DEV)
            impl.forward(None, q, k, v, native_views(fused, layout), meta, out)
            torch.cuda.synchronize()
            got_v = native_views(fused, layout)[1]
            assert np.array_equal(bits(got_v).reshape(-1), want), \
                f"fused step (one-launch post {one_launch}, layer step {layer}), step {index}"
        raw = fused  # the next step sees this step's INT2 slots and windows

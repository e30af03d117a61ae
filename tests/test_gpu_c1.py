"""BASELINE config c1 on the GPU: one decode step, batch 1, GQA 2:1 (Hq 2 / Hkv 1), D256.

Context 512 tokens (511 cached + the current one); S = 4 BF16 sink tokens, a 64-token BF16
recent window, the rest INT2 history; K/V ~ N(0, 1) with 4 outlier channels scaled x8;
rotations are QR factors of seeded Gaussians (fp32, then bf16). "Page size 128" is the
128-token kernel block of the block table: the reference layout needs a physical page of
at least 2 x window = 144 tokens for the BF16 window (layout.py:15-28), so the physical page
stays 768 tokens as in every other config.

The step runs four ways: the reference order of single launches (backend.py:171-226), the
fused three-launch layer step and the two-launch history + post form, which must give the
same bits, and the one-launch layer step, which must write the same cache bytes and an
output within the bounds below of theirs. They are checked against

* ``O.cached_decode_reference`` (the device cache read back: INT2 history dequantized and
  inverse-rotated, BF16 window, current K/V; dense fp64 attention) with scale-aware bounds:
  relative L2 error <= 1e-2, max-abs <= max(2e-3, 2 % of max |want|), LSE within 1e-2;
* ``O.hybrid_reference`` (tests/oracle.py:55-65: quantization redone on the CPU) at the
  reference test's tolerance, atol 0.035 / rtol 0.04 (tests/test_npu_kernels.py:194), plus
  mean-abs <= 2e-3.

Negative controls show that the scale-aware check rejects an all-zero output and the output
of a cache in which the V row of a single recent-window token (the one with the largest
attention weight) has its sign flipped.
"""

import numpy as np
import pytest
import torch

import oracle as O
from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import OscarConfig, choose_splits
from tests._state import (assert_lse_close, assert_scaled_close, bits, make_state, native_views,
                          oracle_geometry, prepare_prefix, run_attention, scaled_close)

pytestmark = pytest.mark.gpu
DEV = "cuda"
CTX, HQ = 512, 2


def _c1_inputs(seed=2024):
    g = torch.Generator().manual_seed(seed)
    rk = torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16()
    rv = torch.linalg.qr(torch.randn(256, 256, generator=g))[0].bfloat16()
    k = torch.randn(CTX, 1, 256, generator=g)
    v = torch.randn(CTX, 1, 256, generator=g)
    for x in (k, v):
        x[..., torch.randperm(256, generator=g)[:4]] *= 8
    q = torch.randn(1, HQ, 256, generator=g).bfloat16()
    return q, k.bfloat16(), v.bfloat16(), rk, rv


def test_c1_decode_step_matches_oracle():
    cfg = OscarConfig(sink_tokens=4, recent_tokens=64)
    assert (cfg.ring_tokens, cfg.window_tokens) == (68, 72)
    q, ks, vs, rk, rv = _c1_inputs()
    print(f"[c1] B1 Hq{HQ}/Hkv1 ctx {CTX}", flush=True)
    layout, raw, hist, window, meta, tables = make_state([CTX], [CTX - 1], cfg)
    meta.layout, meta.num_actual_tokens = layout, 1
    rk_d, rv_d = rk.to(DEV), rv.to(DEV)
    prepare_prefix([ks], [vs], rk_d, rv_d, hist, window, meta, tables, layout, [CTX - 1])
    qd, kd, vd = q.to(DEV), ks[CTX - 1 :].to(DEV), vs[CTX - 1 :].to(DEV)
    splits = choose_splits(1, 1, 1)
    assert splits == 32

    merged = torch.empty(1, HQ, device=DEV)
    single = run_attention(qd, kd, vd, rk_d, rv_d, hist, window, meta, layout, splits, merged)
    cache = raw.clone()
    forms = {}
    for one_launch, layer in ((False, False), (True, False), (False, True)):
        # The reference split rule: the fused forms carry the single launches' bits under the
        # same partition.
        impl = OscarAttentionImpl.standalone(HQ, 256, 1 / 16, 1, cfg, one_launch_post=one_launch,
                                             layer_step=layer, split_policy="reference")
        impl.set_rotations(rk_d, rv_d)
        meta.merged_lse = torch.empty(1, HQ, device=DEV)
        out = torch.empty(1, HQ * 256, dtype=torch.bfloat16, device=DEV)
        step_cache = cache.clone()
        impl.forward(None, qd, kd, vd, native_views(step_cache, layout), meta, out)
        forms[(one_launch, layer)] = (out, meta.merged_lse, step_cache)
    torch.cuda.synchronize()
    for (one_launch, layer), (out, lse, step_cache) in forms.items():
        assert torch.equal(step_cache, cache), "the step rewrote different cache bytes"
        if layer:
            assert_scaled_close(out.view(1, HQ, 256).float().cpu().numpy(),
                                single.float().cpu().numpy(), "one-launch step")
            assert_lse_close(lse.cpu().numpy(), merged.cpu().numpy(), "one-launch LSE", atol=1e-3)
        else:
            assert torch.equal(out.view(1, HQ, 256), single), "fused forms differ"
            assert torch.equal(lse, merged)

    got = single.float().cpu().numpy()
    got_lse = merged.cpu().numpy()
    geo = oracle_geometry(layout)
    history = hist.cpu().numpy()
    win = bits(window).reshape(-1)
    args = (tables[0].numpy(), CTX, bits(q), bits(ks[CTX - 1 :]), bits(vs[CTX - 1 :]), bits(rk),
            bits(rv), geo)
    want, want_lse = O.cached_decode_reference(history, win, *args, scale=1 / 16)
    rel, mx = assert_scaled_close(got, want, "c1 vs cached_decode_reference")
    assert_lse_close(got_lse, want_lse, "c1 merged LSE")
    print(f"[c1] rel L2 {rel:.3g}, max-abs {mx:.3g}", flush=True)

    dense, dense_lse = O.hybrid_reference(bits(q), bits(ks), bits(vs), CTX - 1, bits(rk), bits(rv),
                                          cfg)
    np.testing.assert_allclose(got, dense, atol=0.035, rtol=0.04)
    assert np.abs(got - dense).mean() <= 2e-3
    np.testing.assert_allclose(got_lse, dense_lse, atol=2e-2, rtol=0)

    # Negative controls: the check rejects a zero output and a single wrong window token.
    assert not scaled_close(np.zeros_like(want), want)
    first = int(tables[0, 0])
    recent = range(CTX - 1 - cfg.recent_tokens, CTX - 1)
    qf = O.bf16_to_f32(bits(q)).astype(np.float64)
    keys = [O.bf16_to_f32(win[e : e + 256]) for e in
            (geo.window_element(first, t, 0, 0) for t in recent)]
    top = recent[int(np.argmax(np.abs(qf @ np.array(keys, np.float64).T).max(0)))]
    bad = win.copy()
    element = geo.window_element(first, top, 1, 0)
    bad[element : element + 256] ^= np.uint16(0x8000)
    perturbed, _ = O.cached_decode_reference(history, bad, *args, scale=1 / 16)
    assert not scaled_close(perturbed, want), "one wrong window token went unnoticed"

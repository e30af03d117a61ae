"""Parity at BASELINE.json's full sizes: one fused layer step of configs c3, c4 and c5.

Each workload is built by bench.py's builder (every request's whole prefix written through
the product's rotate / INT2 store / window kernels), then one layer step runs through
`OscarAttentionImpl` with the config's split policy (c4, c5: the MI355X partition with
token-bounded splits). Whole requests are then checked against the oracle's
`cached_decode_reference`, which reads the same paged cache back (INT2 history dequantized
and inverse-rotated, BF16 window, current K/V) and computes dense fp64 attention:

* the shortest and the longest request of the batch (c4: ragged 256..131072 tokens, four
  MTP query tokens each; c5: 262144 tokens);
* tolerance: the reference test's atol 0.035 / rtol 0.04 (tests/test_npu_kernels.py:194),
  mean-abs <= 2e-3 and merged LSE within 2e-2.

Size-independent properties checked on the whole batch: every output row and merged LSE
is finite, and the INT2 slots the step wrote for its own tokens decode (oracle unpack of
the device bytes) to the bytes the oracle quantizer gives for the rotated K/V rows.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import bench
import oracle as O
from oscar_new_amd import kernels
from oscar_new_amd.backend import OscarAttentionImpl

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("config", ["c3", "c4", "c5"])
def test_full_size_layer_step_matches_oracle(config):
    cfg = bench.CONFIGS[config]
    print(f"[fullsize] {config}: building workload", flush=True)
    w = bench.build_workload(SimpleNamespace(seed=1234), cfg, "cuda")
    impl = OscarAttentionImpl(6, 256, 1 / 16, 1, w.cfg, split_policy=cfg["splits"])
    impl.initialize_layer(w.rk, w.rv)
    splits, split_tokens = impl.partition_for(w.meta)
    n = w.q.shape[0]
    out = torch.empty((n, 6 * 256), dtype=torch.bfloat16, device="cuda")
    print(f"[fullsize] {config}: step, splits {splits}, split_tokens {split_tokens}", flush=True)
    impl.forward(None, w.q, w.k, w.v, (w.k_cache, w.v_cache), w.meta, out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(n, 6, 256)
    got_lse = w.meta.merged_lse.cpu().numpy()
    assert np.isfinite(got).all() and np.isfinite(got_lse).all()

    geo = O.Geometry(w.layout.physical_block_tokens, 1, 128, 256, w.cfg.sink_tokens,
                     w.cfg.recent_tokens, w.cfg.speculative_tokens)
    history = w.k_cache.view(torch.uint8).view(-1).cpu().numpy()
    window = w.v_cache.view(torch.int16).view(-1).cpu().numpy().view(np.uint16)
    rk, rv = _bits(w.rk), _bits(w.rv)
    order = np.argsort(w.seqs)
    for r in sorted({int(order[0]), int(order[-1])}):
        rows = slice(r * w.qlen, (r + 1) * w.qlen)
        want, want_lse = O.cached_decode_reference(history, window, w.table[r].numpy(),
                                                   w.seqs[r], _bits(w.q[rows]), _bits(w.k[rows]),
                                                   _bits(w.v[rows]), rk, rv, geo, scale=1 / 16)
        err = np.abs(got[rows] - want)
        print(f"[fullsize] {config}: request {r} ({w.seqs[r]} tokens) max {err.max():.3g} "
              f"mean {err.mean():.3g}", flush=True)
        np.testing.assert_allclose(got[rows], want, atol=0.035, rtol=0.04)
        assert err.mean() <= 2e-3
        np.testing.assert_allclose(got_lse[rows], want_lse, atol=2e-2, rtol=0)

    # The step's own INT2 slots: device bytes == oracle quantizer bytes of the device's
    # rotated rows (bit-exact codes, scale and zero).
    kr = kernels.rotate(w.k, w.rk)
    vr = kernels.rotate(w.v, w.rv)
    slots = w.meta.slot_mapping.cpu().numpy()
    want_bytes = O.packed_slots(_bits(kr), _bits(vr), w.cfg)
    for i, slot in enumerate(slots[: min(len(slots), 64)]):
        base = geo.slot_offset(int(slot), 0)
        assert np.array_equal(history[base : base + 136], want_bytes[i, 0, :136]), i

"""Parity at BASELINE.json's full sizes: one fused layer step of configs c3, c4 and c5.

Each workload is built by bench.py's builder (every request's whole prefix written through
the product's rotate / INT2 store / window kernels; c5's pages scattered over a 300k-block
pool), then one layer step runs through `OscarAttentionImpl` with the config's split policy
(c4, c5: the MI355X partition with token-bounded splits). Requests are checked against the
oracle's `cached_decode_reference`, which reads the same paged cache back (INT2 history
dequantized and inverse-rotated, BF16 window, current K/V) and computes dense fp64
attention:

* c3 and c5: every request; c4: a seeded sample of 8 requests plus the shortest and the
  longest (ragged 256..131072 tokens, four MTP query tokens each);
* scale-aware bounds per request: max-abs <= 2e-3 (the output RMS is about 0.009 at 32k
  context and 0.003 at 262k, so an elementwise atol of 0.035 would accept a zero output; the
  largest measured error at 32k and beyond is about 3e-4), relative L2 error <= 2e-2 and
  merged LSE within 1e-2; a zero output fails the same check (asserted). The relative
  error grows with context (about 0.5 % at 1k tokens, 0.6 % at 40k, 1.0 % at 262k): the
  history output is the small difference of two terms of size ~1.7, sum_t p_t s_t c_t and
  sum_t p_t z_t, so an error of a few 1e-5 in either, constant in context, is a growing
  fraction of an output that shrinks like 1 / sqrt(context).

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
from tests._state import assert_lse_close, assert_scaled_close, scaled_close

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _request_cache(w, r, geo):
    """The pages request r owns, copied to the host as a compact cache: (K stripe bytes,
    V stripe bf16 bits, block-table row renumbered onto the compact pages)."""
    bpp = geo.blocks_per_page
    ncols = -(-w.seqs[r] // 128)
    row = w.table[r, :ncols].numpy().astype(np.int64)
    pages = list(dict.fromkeys((row // bpp).tolist()))
    index = {p: j for j, p in enumerate(pages)}
    sel = torch.tensor(pages, device=w.k_cache.device)
    stripe = geo.stripe_page_bytes
    k = w.k_cache.view(torch.uint8).view(-1, stripe).index_select(0, sel)
    v = w.v_cache.view(torch.uint8).view(-1, stripe).index_select(0, sel)
    history = k.cpu().numpy().reshape(-1)
    window = v.cpu().numpy().reshape(-1).view(np.uint16)
    compact = np.array([index[b // bpp] * bpp + b % bpp for b in row], np.int64)
    return history, window, compact


@pytest.mark.parametrize("config", ["c3", "c4", "c5"])
def test_full_size_layer_step_matches_oracle(config):
    cfg = bench.CONFIGS[config]
    print(f"[fullsize] {config}: building workload", flush=True)
    w = bench.build_workload(SimpleNamespace(seed=1234), cfg, "cuda")
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, w.cfg, split_policy=cfg["splits"])
    impl.set_rotations(w.rk, w.rv)
    splits, split_tokens = impl.partition_for(w.meta)
    n = w.q.shape[0]
    out = torch.empty((n, 6 * 256), dtype=torch.bfloat16, device="cuda")
    print(f"[fullsize] {config}: step, splits {splits}, split_tokens {split_tokens}, pool "
          f"{w.k_cache.shape[0]} blocks", flush=True)
    impl.forward(None, w.q, w.k, w.v, (w.k_cache, w.v_cache), w.meta, out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(n, 6, 256)
    got_lse = w.meta.merged_lse.cpu().numpy()
    assert np.isfinite(got).all() and np.isfinite(got_lse).all()

    geo = O.Geometry(w.layout.physical_block_tokens, 1, 128, 256, w.cfg.sink_tokens,
                     w.cfg.recent_tokens, w.cfg.speculative_tokens)
    rk, rv = _bits(w.rk), _bits(w.rv)
    order = np.argsort(w.seqs)
    requests = set(range(len(w.seqs)))
    if config == "c4":
        rng = np.random.default_rng(1234)
        requests = {int(order[0]), int(order[-1])} | set(
            rng.choice(len(w.seqs), 8, replace=False).tolist())
    worst = 0.0
    for r in sorted(requests):
        rows = slice(r * w.qlen, (r + 1) * w.qlen)
        history, window, table = _request_cache(w, r, geo)
        want, want_lse = O.cached_decode_reference(history, window, table, w.seqs[r],
                                                   _bits(w.q[rows]), _bits(w.k[rows]),
                                                   _bits(w.v[rows]), rk, rv, geo, scale=1 / 16)
        rel, mx = assert_scaled_close(got[rows], want, f"{config} request {r}", rel=2e-2)
        assert_lse_close(got_lse[rows], want_lse, f"{config} request {r}")
        assert not scaled_close(np.zeros_like(want), want)
        worst = max(worst, mx)
        print(f"[fullsize] {config}: request {r} ({w.seqs[r]} tokens) rel L2 {rel:.3g} "
              f"max-abs {mx:.3g}", flush=True)
    print(f"[fullsize] {config}: {len(requests)} requests, worst max-abs {worst:.3g}", flush=True)

    # The step's own INT2 slots: device bytes == oracle quantizer bytes of the device's
    # rotated rows (bit-exact codes, scale and zero).
    kr = kernels.rotate(w.k, w.rk)
    vr = kernels.rotate(w.v, w.rv)
    slots = w.meta.slot_mapping.cpu().numpy()[:64]
    want_bytes = O.packed_slots(_bits(kr[:64]), _bits(vr[:64]), w.cfg)
    stripe = geo.stripe_page_bytes
    flat = w.k_cache.view(torch.uint8).view(-1)
    for i, slot in enumerate(slots):
        base = geo.slot_offset(int(slot), 0)
        got_bytes = flat[base : base + 136].cpu().numpy()
        assert np.array_equal(got_bytes, want_bytes[i, 0, :136]), i
    assert stripe == w.layout.stripe_page_bytes

"""Precision of the fused decode step at BASELINE's full sizes against three references read
back from the same INT2 cache (oracle ``cached_decode_variants``):

* "exact": the attention value of the stored cache (history dequantized exactly as
  code * scale + zero, inverse-rotated and attended in float64);
* "oracle": the reference test oracle's semantics (tests/oracle.py:55-65: dequantized history
  rounded to bf16);
* "reference_kernel": the reference kernels' own rounding points (bf16 rotated q, bf16
  ``_load_vec``, ``p.to(bf16)``, bf16 merged history, bf16 inverse rotation, bf16 output;
  kernels.py:205-219, 421-431, 506-541, backend.py:195-226), with the reference split rule.

The step under test runs the default configuration (device split rule, fused launches).
The kernel's bound against "exact" comes from an error model (ERROR MODEL below), not from
the observed maximum; the kernel must also be closer to "exact" than the reference kernel's
arithmetic on every request and than the reference test oracle on the batch's worst request,
and a one-token perturbation of the c5 history must break the bound.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import bench
import oracle as O
from oscar_new_amd.backend import OscarAttentionImpl
from oscar_new_amd.config import choose_splits
from tests.test_gpu_fullsize import _bits, _request_cache

pytestmark = pytest.mark.gpu

# ERROR MODEL. A bf16 rounding of a value x errs by at most 2^-9 |x|; an attention output
# averages such independent per-term errors without amplifying them, so one rounding stage
# adds about U = 2^-9 relative L2 to the output (rms over the rows of a request), and
# independent stages add in quadrature. The kernel has four: the merged history rounded to
# bf16, the inverse V rotation's bf16 output, the path merge's bf16 output, and its FP4 x
# two-term FP8 products (about 2^-8 relative per product, averaged like a bf16 stage); the
# history is dequantized exactly (scale and zero folded out of the products). So
# kernel vs exact <= 2 sqrt(4) U, the factor 2 for the worst request of a batch.
# The references round the dequantized history to bf16 (tests/oracle.py:18,
# kernels.py:219). That stage does not behave like one independent rounding: measured
# against "exact" it grows with context (0.55 % at 32k, 1.0 % at 262k on this data), so it
# is not bounded here; instead the kernel must be closer to "exact" than the references.
U = 2.0 ** -9
KERNEL_BOUND = 2.0 * 2.0 * U  # 2 sqrt(4) U = 0.78 %


def _rel(a, b):
    """Relative L2 distance of a from b."""
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("config", ["c3", "c4", "c5"])
def test_step_precision_against_exact_and_reference_rounding(config):
    cfg = bench.CONFIGS[config]
    print(f"[precision] {config}: building workload", flush=True)
    w = bench.build_workload(SimpleNamespace(seed=1234), cfg, "cuda")
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, w.cfg)
    impl.set_rotations(w.rk, w.rv)
    n = w.q.shape[0]
    out = torch.empty((n, 6 * 256), dtype=torch.bfloat16, device="cuda")
    impl.forward(None, w.q, w.k, w.v, (w.k_cache, w.v_cache), w.meta, out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(n, 6, 256)
    geo = O.Geometry(w.layout.physical_block_tokens, 1, 128, 256, w.cfg.sink_tokens,
                     w.cfg.recent_tokens, w.cfg.speculative_tokens)
    rk, rv = _bits(w.rk), _bits(w.rv)
    ref_splits = choose_splits(len(w.seqs), 1, w.qlen)
    requests = range(len(w.seqs))
    if config == "c4":
        order = np.argsort(w.seqs)
        rng = np.random.default_rng(1234)
        requests = sorted({int(order[0]), int(order[-1])} |
                          set(rng.choice(len(w.seqs), 6, replace=False).tolist()))
    worst = {}
    kept = None
    for r in requests:
        rows = slice(r * w.qlen, (r + 1) * w.qlen)
        history, window, table = _request_cache(w, r, geo)
        qb, kb, vb = _bits(w.q[rows]), _bits(w.k[rows]), _bits(w.v[rows])
        var = O.cached_decode_variants(history, window, table, w.seqs[r], qb, kb, vb, rk, rv,
                                       geo, scale=1 / 16, splits=ref_splits)
        outs = {"kernel": got[rows], **{k: v[0] for k, v in var.items()}}
        err = {name: _rel(outs[name], outs["exact"])
               for name in ("kernel", "oracle", "reference_kernel")}
        err["kernel/oracle"] = _rel(outs["kernel"], outs["oracle"])
        for key, e in err.items():
            worst[key] = max(worst.get(key, 0.0), e)
        print(f"[precision] {config} request {r} ({w.seqs[r]} tokens) vs exact: kernel "
              f"{err['kernel']:.3g}, oracle {err['oracle']:.3g}, reference kernel "
              f"{err['reference_kernel']:.3g}; kernel vs oracle {err['kernel/oracle']:.3g}",
              flush=True)
        assert err["kernel"] <= KERNEL_BOUND, (config, r, err)
        assert err["kernel"] < err["reference_kernel"], (config, r, err)
        if kept is None:
            kept = (r, history, window, table, qb, kb, vb)
    print(f"[precision] {config} worst vs exact: " + ", ".join(
        f"{k} {e:.3g}" for k, e in worst.items()) + f" (kernel bound {KERNEL_BOUND:.3g})",
        flush=True)
    # At short contexts the oracle's two bf16 dequant stages and the kernel's four stages are
    # at the same floor (a 304-token c4 request: 0.351 % against 0.359 %); over a batch the
    # kernel's worst request is closer to "exact" than the oracle's.
    assert worst["kernel"] < worst["oracle"], worst

    if config == "c5":
        # A one-token change of the history breaks the kernel-vs-exact bound: the token the
        # query rows weigh most (exact scores), its value codes mirrored (c -> 3 - c).
        r, history, window, table, qb, kb, vb = kept
        rows = slice(r * w.qlen, (r + 1) * w.qlen)
        seq = w.seqs[r]
        prefix = seq - w.qlen
        sink = min(geo.sink_tokens, prefix)
        recent_begin = max(sink, prefix - geo.recent_tokens)
        pos = np.arange(sink, recent_begin)
        bk = geo.kernel_block_tokens
        slots = table[pos // bk].astype(np.int64) * bk + pos % bk
        offs = np.array([geo.slot_offset(s) for s in slots])
        keys = O.bf16_to_f32(O.dequant_rows(history, offs)).astype(np.float64) @ \
            O.bf16_to_f32(rk).astype(np.float64).T
        scores = O.bf16_to_f32(qb).reshape(-1, 256).astype(np.float64) @ keys.T
        top = int(np.argmax(scores.max(0)))
        bad = history.copy()
        base = offs[top] + geo.vector_bytes
        bad[base:base + 64] = ~bad[base:base + 64]  # every 2-bit code c -> 3 - c
        var = O.cached_decode_variants(bad, window, table, seq, qb, kb, vb, rk, rv, geo,
                                       scale=1 / 16, splits=ref_splits)
        e = _rel(got[rows], var["exact"][0])
        print(f"[precision] c5 request {r}: history token {int(pos[top])} of {seq} perturbed: "
              f"kernel vs exact {e:.3g} (bound {KERNEL_BOUND:.3g})", flush=True)
        assert e > KERNEL_BOUND

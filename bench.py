#!/usr/bin/env python3
"""OSCAR INT2 decode-attention benchmark on one MI355X.

One step = one FULL-attention layer forward of a decode batch (BASELINE config 3 by
default): rotate K/V/q, INT2 store of the current token, split-KV history attention,
split merge, inverse V rotation, BF16 sink/recent/current attention, LSE path merge,
window store. The steps of ``--layers`` consecutive layers, each with its own KV cache
(> 1 GB each, so the 256 MB Infinity Cache cannot serve a step from the previous step's
reads), are captured back to back in one HIP graph, as a model's decode graph holds them.

Printed JSON (one line): ``value`` is the whole step's algorithmic HBM GB/s; also the
per-layer-step microseconds, the dominant (history) kernel's roofline from HIP events, the
store throughput, the CPU oracle baseline and a full-size parity sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "INT2 decode-attn µs/layer-step + achieved HBM GB/s at 32k ctx; store tokens/s"
PEAK_HBM_GBPS = 8000.0

CONFIGS = {
    "c3": dict(batch=32, context=32768, qlen=1, ragged=False, splits="device",
               desc="one TP rank of a Qwen3.5-27B-class layer: B32 x 32768 ctx, GQA 6:1, D256, "
                    "INT2 history + 4 sink + 128 recent BF16, device split rule"),
    "c4": dict(batch=64, context=131072, qlen=4, ragged=True, splits="device",
               desc="ragged MTP: B64, ctx log-uniform [256, 131072], 4 query tokens each"),
    "c5": dict(batch=4, context=262144, qlen=1, ragged=False, splits="device",
               pool_blocks=300_000,
               desc="long context: B4 x 262144 ctx, adaptive splits, 128-token blocks scattered "
                    "over a 300k-block (50k-page, 39 GB) pool"),
    # --mode prefill only (initial prefill, no cached tokens): every token is a query token.
    "p1": dict(batch=4, context=4096, qlen=4096, ragged=False, splits="reference",
               desc="initial prefill: B4 x 4096 tokens, GQA 6:1, D256, causal"),
    # --mode prefill: a continuation chunk over a cached prefix (one history split, the long
    # chunk rule of config.py:86-87); the history branch is MFMA-bound.
    "p2": dict(batch=1, context=32768 + 2048, qlen=2048, ragged=False, splits="device",
               desc="continuation chunk: 2048 query tokens over 32768 cached tokens, GQA 6:1, "
                    "D256, one history split"),
}


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    p.add_argument("--layers", type=int, default=None,
                   help="independent KV caches cycled per step (default 4; 2 when one cache "
                        "exceeds 16 GB)")
    p.add_argument("--seed", type=int, default=1234)
    p.add_argument("--cpu-sample", type=int, default=0,
                   help="requests timed on the CPU baseline (0: a seeded sample of about "
                        "2**18 context tokens)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="eager launches instead of HIP graphs")
    p.add_argument("--one-launch-post", action="store_true",
                   help="history branch and post-attention in one launch (kernels.history_post)")
    p.add_argument("--no-overlap", action="store_true",
                   help="pre-attention (q rotation, BF16 branch, INT2 store) as its own "
                        "launch instead of q rotation + history launch carrying the rest")
    p.add_argument("--layer-step", action="store_true",
                   help="the one-launch layer step (kernels.layer_step) instead of three launches")
    p.add_argument("--rotate-in-history", action="store_true",
                   help="the history workgroups rotate their query rows (default: the q "
                        "rotation is a launch of its own ahead of the history launch)")
    p.add_argument("--q-roles", action="store_true",
                   help="the q rotation as role workgroups of the history launch instead of a "
                        "launch of its own")
    p.add_argument("--mode", default="step",
                   choices=("step", "history", "copy", "prefill", "store"),
                   help="step: full benchmark; history: only the history-attention launches "
                        "(for rocprofv3 counters); copy: a plain device copy of --copy-mib MiB "
                        "(counter calibration); prefill: the initial-prefill launch (--config "
                        "p1) or the continuation-chunk step (--config p2); store: the c2 store "
                        "forms, plain "
                        "launches (for rocprofv3 counters)")
    p.add_argument("--copy-mib", type=int, default=1024)
    p.add_argument("--split-policy", default=None, choices=("device", "reference", "mi355x"),
                   help="history split policy (default: the config's, the device rule)")
    p.add_argument("--branch", action="store_true",
                   help="--mode history: the history branch alone instead of the step's "
                        "history launch")
    p.add_argument("--no-sub-configs", action="store_true",
                   help="c3: skip the c4 / c5 / p1 / p2 sub-records")
    return p.parse_args(argv)


def copy_calibration(args, device):
    """A plain copy of known size, to scale FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = args.copy_mib << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_per_copy": n, "copies": args.steps}))
    return 0


# ------------------------------------------------------------------ workload


def context_lengths(cfg, gen):
    import torch

    b, ctx = cfg["batch"], cfg["context"]
    if not cfg["ragged"]:
        return [ctx] * b
    lo, hi = math.log(256), math.log(ctx)
    u = torch.rand(b, generator=gen, dtype=torch.float64)
    return [int(round(math.exp(lo + (hi - lo) * float(x)))) for x in u]


def build_workload(args, cfg, device):
    """Paged INT2 cache of every request written through the product kernels."""
    import torch

    from oscar_new_amd import kernels
    from oscar_new_amd.config import OscarConfig, task_capacity
    from oscar_new_amd.layout import CacheLayout

    ocfg = OscarConfig(sink_tokens=4, recent_tokens=128, speculative_tokens=3)
    layout = CacheLayout(768, config=ocfg)
    gen = torch.Generator().manual_seed(args.seed)
    seqs = context_lengths(cfg, gen)
    qlen = cfg["qlen"]
    b = len(seqs)
    bpp = layout.blocks_per_page
    pages_per_req = [-(-s // layout.physical_block_tokens) for s in seqs]
    # Pages are drawn at random from the pool (page 0 never owned): the owned pages of a
    # request scatter over the whole pool, as after a long serving run.
    pool = max(sum(pages_per_req) + 1, -(-cfg.get("pool_blocks", 0) // bpp))
    order = (torch.randperm(pool - 1, generator=gen) + 1).tolist()
    columns = max(pages_per_req) * bpp
    table = torch.zeros((b, columns), dtype=torch.int32)
    cursor = 0
    for r, npg in enumerate(pages_per_req):
        pages = order[cursor : cursor + npg]
        cursor += npg
        table[r, : npg * bpp] = torch.tensor([p * bpp + j for p in pages for j in range(bpp)],
                                             dtype=torch.int32)
    table_d = table.to(device)
    rk = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16().to(device)
    rv = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16().to(device)

    k_cache = torch.zeros(pool * bpp, 128, 1, 256, dtype=torch.bfloat16, device=device)
    v_cache = torch.zeros_like(k_cache)
    history, window = layout.tensor_views((k_cache, v_cache))
    dgen = torch.Generator(device=device).manual_seed(args.seed + 1)
    prefixes = [s - qlen for s in seqs]
    chunk = 65536
    for r, prefix in enumerate(prefixes):  # earlier steps, written by the real kernels
        for start in range(0, prefix, chunk):
            stop = min(prefix, start + chunk)
            t = stop - start
            k = torch.randn(t, 1, 256, generator=dgen, device=device).bfloat16()
            v = torch.randn(t, 1, 256, generator=dgen, device=device).bfloat16()
            pos = torch.arange(start, stop, device=device)
            slots = (table_d[r, pos // 128].to(torch.int64) * 128 + pos % 128)
            counts = torch.tensor([1, t], dtype=torch.int32, device=device)
            kernels.store_int2(kernels.rotate(k, rk), kernels.rotate(v, rv), history, slots,
                               counts, layout)
            # Window: sink positions and, per ring slot, the latest position (later chunks
            # overwrite earlier ones, exactly as successive decode steps would).
            meta = SimpleNamespace(
                query_start_loc=torch.tensor([0, t], dtype=torch.int32, device=device),
                seq_lens=torch.tensor([stop], dtype=torch.int32, device=device),
                block_tables=table_d[r : r + 1], counts=counts, max_num_reqs=1)
            kernels.store_windows(k, v, window, meta, layout)
    torch.cuda.synchronize()

    ntok = sum(qlen for _ in seqs)
    q = torch.randn(ntok, 6, 256, generator=dgen, device=device).bfloat16()
    kc = torch.randn(ntok, 1, 256, generator=dgen, device=device).bfloat16()
    vc = torch.randn(ntok, 1, 256, generator=dgen, device=device).bfloat16()
    slot_list = []
    for r, s in enumerate(seqs):
        for p in range(s - qlen, s):
            slot_list.append(int(table[r, p // 128]) * 128 + p % 128)
    meta = SimpleNamespace(
        query_start_loc=torch.arange(0, ntok + 1, qlen, dtype=torch.int32, device=device),
        seq_lens=torch.tensor(seqs, dtype=torch.int32, device=device),
        block_tables=table_d,
        slot_mapping=torch.tensor(slot_list, dtype=torch.int64, device=device),
        counts=torch.tensor([b, ntok], dtype=torch.int32, device=device),
        num_reqs=b, num_actual_tokens=ntok, max_query_len=qlen, max_num_reqs=b,
        max_seq_len=max(seqs), total_seq_len=sum(seqs), layout=layout,
        tasks=torch.zeros((task_capacity(ntok, b, ocfg.queries_per_tile), 2), dtype=torch.int32,
                          device=device),
        task_count=torch.zeros(1, dtype=torch.int32, device=device),
        merged_lse=torch.empty(ntok, 6, dtype=torch.float32, device=device),
    )
    kernels.prepare_tasks(meta.query_start_loc, meta.counts, meta.tasks, meta.task_count, b,
                          ocfg.queries_per_tile)
    return SimpleNamespace(layout=layout, cfg=ocfg, seqs=seqs, prefixes=prefixes, qlen=qlen,
                           table=table, k_cache=k_cache, v_cache=v_cache, rk=rk, rv=rv, q=q,
                           k=kc, v=vc, meta=meta)


def algorithmic_bytes(w):
    """Bytes a step must move: 136 B per INT2 history token-head, 1024 B per BF16
    sink/recent/current token-head, q + output + used block-table entries."""
    cfg = w.cfg
    hist = bf16 = cols = 0
    for s, prefix in zip(w.seqs, w.prefixes):
        sink = min(cfg.sink_tokens, prefix)
        recent_begin = max(sink, prefix - cfg.recent_tokens)
        hist += recent_begin - sink
        bf16 += sink + (prefix - recent_begin) + w.qlen
        cols += -(-s // 128)
    ntok = w.q.shape[0]
    q_out = 2 * ntok * 6 * 256 * 2
    return SimpleNamespace(history_tokens=hist, int2=136 * hist, bf16=1024 * bf16,
                           q_out=q_out, table=4 * cols, total=136 * hist + 1024 * bf16 + q_out + 4 * cols)


def history_lengths(w):
    """History tokens of each request (positions [sink_len, recent_begin))."""
    cfg = w.cfg
    out = []
    for prefix in w.prefixes:
        sink = min(cfg.sink_tokens, prefix)
        out.append(max(sink, prefix - cfg.recent_tokens) - sink)
    return out


def effective_split_tokens(w, split_tokens):
    """The split length the kernels use: split_tokens, or under the device rule (negative)
    the length the GPU derives from the step's lengths (config.device_split_tokens; one task
    per request at these configs; a grid of unit slots up to 8 query rows per task)."""
    from oscar_new_amd import config

    if split_tokens >= 0:
        return split_tokens
    return config.device_split_tokens(sum(history_lengths(w)), len(w.seqs), 1, -split_tokens,
                                      fit_grid=w.qlen * 6 <= 8)


def split_partial_bytes(w, splits, split_tokens):
    """Bytes the history launch writes: a 1024-byte partial row + 4-byte LSE per live split
    of each query row; only the LSE for the split slots a request does not use."""
    st = effective_split_tokens(w, split_tokens)
    total = 0
    for hist in history_lengths(w):
        used = splits if not st else min(splits, max(1, -(-hist // st)))
        total += w.qlen * 6 * (used * (256 * 4 + 4) + (splits - used) * 4)
    return total


# ------------------------------------------------------------------ measurements


def time_store(device, args, steps, eager=False):
    """rotate + clip-search + INT2 pack of 4096 tokens into permuted pages
    (device time per call from HIP-graph replays). ``eager``: only run each form ``steps``
    times with plain launches (for rocprofv3 counters) and return None."""
    import torch

    from oscar_new_amd import kernels
    from oscar_new_amd.config import OscarConfig
    from oscar_new_amd.layout import CacheLayout

    n = 4096
    cfg = OscarConfig(sink_tokens=4, recent_tokens=128, clip_mode="search")
    layout = CacheLayout(768, config=cfg)
    gen = torch.Generator().manual_seed(args.seed + 2)
    k = torch.randn(n, 1, 256, generator=gen)
    v = torch.randn(n, 1, 256, generator=gen)
    chans = torch.randperm(256, generator=gen)[:5]
    k[..., chans] *= 10
    v[..., chans] *= 10
    k, v = k.bfloat16().to(device), v.bfloat16().to(device)
    rk = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16().to(device)
    rv = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16().to(device)
    pages = 64
    history = torch.zeros(pages * layout.stripe_page_bytes, dtype=torch.uint8, device=device)
    blocks = torch.randperm(pages * 6, generator=gen)[: n // 128]
    slots = (blocks[:, None] * 128 + torch.arange(128)[None]).reshape(-1).to(torch.int64).to(device)
    counts = torch.tensor([1, n], dtype=torch.int32, device=device)

    rk_t, rv_t = rk.T.contiguous(), rv.T.contiguous()

    def once():  # the product's path: rotation and store in one launch
        kernels.rotate_store_int2(k, v, rk_t, rv_t, history, slots, counts, layout)

    def unfused():  # the reference's sequence: rotate K, rotate V, store_int2
        kernels.store_int2(kernels.rotate(k, rk), kernels.rotate(v, rv), history, slots, counts,
                           layout)

    for _ in range(5):
        once()
    kr, vr = kernels.rotate(k, rk), kernels.rotate(v, rv)
    torch.cuda.synchronize()
    if eager:
        for _ in range(steps):
            once()
        for _ in range(steps):
            unfused()
        torch.cuda.synchronize()
        return None

    # Device time without host submission gaps: each form is captured `reps` times in one
    # HIP graph, and the graph's replays are timed with events on the capture stream.
    reps = 10
    stream = torch.cuda.Stream()

    def timed(fn):
        graph = torch.cuda.CUDAGraph()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(reps):
                fn()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
            times = []
            for _ in range(max(1, steps // reps)):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                graph.replay()
                b.record(stream)
                times.append((a, b))
        torch.cuda.synchronize()
        return statistics.median(a.elapsed_time(b) for a, b in times) * 1e3 / reps

    t_full = timed(once)
    t_unfused = timed(unfused)
    t_store = timed(lambda: kernels.store_int2(kr, vr, history, slots, counts, layout))
    alg = n * (2 * 512) + 2 * 256 * 256 * 2 + n * 136 + n * 8
    return {
        "workload": "c2: 4096 tokens x 1 kv head, D256, 2% outlier channels x10, seeded QR "
                    "rotation, 8-factor MSE clip search, 128-token pages on permuted slots",
        "tokens_per_s": n / (t_full * 1e-6),
        "us_per_call": t_full,
        "path": "rotate_store_int2 (one launch)",
        "unfused_us_per_call": t_unfused,
        "unfused_tokens_per_s": n / (t_unfused * 1e-6),
        "store_kernel_us": t_store,
        "store_kernel_tokens_per_s": n / (t_store * 1e-6),
        "algorithmic_bytes": alg,
        "store_kernel_GBps": alg / (t_store * 1e-6) / 1e9,
    }


CPU_RUNS, CPU_WARMUP = 5, 1
CPU_SAMPLE_TOKENS = 1 << 18  # context tokens of the sampled requests per timed run


def cpu_threads():
    """Host threads for the CPU baseline: the job's share (OMP_NUM_THREADS) or every core."""
    import torch

    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS") or 0) or os.cpu_count() or 1)
    return torch.get_num_threads()


def median_run(fn, runs=CPU_RUNS, warmup=CPU_WARMUP):
    """Median wall seconds of ``runs`` timed calls after ``warmup`` untimed ones."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_c1_decode(seed):
    """c1 (B1, Hq 2 / Hkv 1, ctx 512, 4 sink + 64 recent) decode step on the torch float32
    restatement, over a cache of slot images packed by that restatement: (us, description)."""
    import torch

    import oracle as O
    from oracle import cpu_torch as T

    gen = torch.Generator().manual_seed(seed)
    geo = O.Geometry(768, 1, 128, 256, 4, 64, 3)
    seq, pages = 512, 2
    history = torch.zeros(pages * geo.stripe_page_bytes, dtype=torch.uint8)
    window = torch.randn(pages * geo.stripe_page_bytes // 2, generator=gen).bfloat16()
    k = torch.randn(seq, 1, 256, generator=gen)
    v = torch.randn(seq, 1, 256, generator=gen)
    k[..., :4] *= 8.0  # 4 outlier channels x8
    rk = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16()
    rv = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16()
    images = T.quantize_pack(T.rotate(k.bfloat16(), rk), T.rotate(v.bfloat16(), rv))
    table = list(range(geo.blocks_per_page, 2 * geo.blocks_per_page))
    history.view(pages, -1)[1, : seq * 160] = images.reshape(-1)
    q = torch.randn(1, 2, 256, generator=gen).bfloat16()
    cur_k, cur_v = k[-1:].bfloat16(), v[-1:].bfloat16()
    sec = median_run(lambda: T.decode_step(history, window, table, seq, q, cur_k, cur_v, rk, rv,
                                           geo, scale=1 / 16), runs=21, warmup=3)
    return sec * 1e6, "c1: B1 x 512 ctx, Hq 2 / Hkv 1, 4 sink + 64 recent, median of 21 after 3"


def cpu_c2_store(seed):
    """c2 quantize+pack of 4096 tokens (rotate K and V, 8-factor MSE clip search, INT2 pack
    into 160-byte slot images) on the torch float32 restatement: tokens/s."""
    import torch

    from oracle import cpu_torch as T

    gen = torch.Generator().manual_seed(seed)
    n = 4096
    k = torch.randn(n, 1, 256, generator=gen)
    v = torch.randn(n, 1, 256, generator=gen)
    hot = torch.randperm(256, generator=gen)[:5]  # 2 % outlier channels x10
    k[..., hot] *= 10.0
    rk = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16()
    rv = torch.linalg.qr(torch.randn(256, 256, generator=gen))[0].bfloat16()
    kb, vb = k.bfloat16(), v.bfloat16()
    sec = median_run(lambda: T.quantize_pack(T.rotate(kb, rk), T.rotate(vb, rv), "search"))
    return n / sec


def cpu_baseline(w, args, outputs):
    """CPU baseline on the host cores: the torch float32 restatement of the decode step
    (oracle/cpu_torch.py: INT2 history dequantized and inverse-rotated, BF16 window and current
    rows, dense float32 softmax) over a seeded sample of the workload's requests read back
    from the device cache, median of 5 timed runs after 1 warm-up, scaled to the whole batch
    by context tokens; beside it c1's decode step and c2's quantize+pack tokens/s. Also the
    sample's parity against the GPU output."""
    import numpy as np
    import torch

    import oracle as O
    from oracle import cpu_torch as T

    cores = cpu_threads()
    geo = O.Geometry(w.layout.physical_block_tokens, 1, 128, 256, w.cfg.sink_tokens,
                     w.cfg.recent_tokens, w.cfg.speculative_tokens)
    rk, rv = w.rk.cpu(), w.rv.cpu()
    q, k, v = w.q.cpu(), w.k.cpu(), w.v.cpu()
    order = torch.randperm(len(w.seqs), generator=torch.Generator().manual_seed(args.seed))
    sample, tokens = [], 0
    for r in order.tolist():
        if args.cpu_sample and len(sample) >= args.cpu_sample:
            break
        if not args.cpu_sample and sample and tokens >= CPU_SAMPLE_TOKENS:
            break
        sample.append(r)
        tokens += w.seqs[r]
    # Host copy of the sample's own pages only (the pool can be tens of GB), blocks renumbered.
    bpp = geo.blocks_per_page
    rows = {r: w.table[r, : -(-w.seqs[r] // 128)].tolist() for r in sample}
    pages = sorted({b // bpp for row in rows.values() for b in row})
    renumber = {p: i for i, p in enumerate(pages)}
    tables = {r: np.array([renumber[b // bpp] * bpp + b % bpp for b in row], np.int64)
              for r, row in rows.items()}
    idx = torch.tensor(pages, device=w.k_cache.device)
    npool = w.k_cache.shape[0] // bpp
    history = w.k_cache.view(torch.uint8).reshape(npool, -1).index_select(0, idx).reshape(-1).cpu()
    window = w.v_cache.reshape(npool, -1).index_select(0, idx).reshape(-1).cpu()
    got = outputs.float().cpu().reshape(-1, 6, 256)
    got_lse = w.meta.merged_lse.cpu()
    results = {}

    def run():
        for r in sample:
            rows = slice(r * w.qlen, (r + 1) * w.qlen)
            results[r] = T.decode_step(history, window, tables[r], w.seqs[r], q[rows],
                                       k[rows], v[rows], rk, rv, geo, scale=1 / 16)

    sec = median_run(run)
    scale = sum(w.seqs) / tokens
    num = den = max_abs = lse_err = 0.0
    for r in sample:
        rows = slice(r * w.qlen, (r + 1) * w.qlen)
        want, want_lse = results[r]
        diff = got[rows] - want
        num += float((diff * diff).sum())
        den += float((want * want).sum())
        max_abs = max(max_abs, float(diff.abs().max()))
        lse_err = max(lse_err, float((got_lse[rows] - want_lse).abs().max()))
    c1_us, c1_desc = cpu_c1_decode(args.seed)
    cpu = {
        "value": sec * scale * 1e6,
        "unit": "us/layer-step",
        "cores": int(cores),
        "kind": "port",
        "sample": f"{len(sample)} of {len(w.seqs)} requests ({tokens} of {sum(w.seqs)} context "
                  f"tokens) of layer 0, torch float32 restatement (oracle/cpu_torch.py: INT2 "
                  f"dequant + inverse rotation + dense float32 attention), median of "
                  f"{CPU_RUNS} runs after {CPU_WARMUP} warm-up, scaled x{scale:.3g} by tokens",
        "c1_us_per_step": c1_us,
        "c1_sample": c1_desc,
        "c2_store_tokens_per_s": cpu_c2_store(args.seed),
        "c2_sample": "c2: 4096 tokens x 1 kv head, rotate K and V + 8-factor MSE clip search + "
                     f"INT2 pack, median of {CPU_RUNS} runs after {CPU_WARMUP} warm-up",
    }
    parity = {"requests": len(sample), "rel_l2": math.sqrt(num / max(den, 1e-30)),
              "max_abs": max_abs, "lse_max_abs": lse_err}
    return cpu, parity


HIST_LAUNCHES = 20  # history launches per timed batch of the dominant-kernel measurement
TRAFFIC_PROFILES = {  # rocprof PMC summaries (FETCH_SIZE / WRITE_SIZE runs) per (kernel, config)
    ("history_pre_kernel", "c3"): "history_pre_kernel_c3_traffic.txt",
    ("history_pre_kernel", "c5"): "history_pre_kernel_c5_traffic.txt",
    ("history_pair_kernel", "c3"): "history_kernel_c3_traffic.txt",
    ("history_pair_kernel", "c5"): "history_kernel_c5_traffic.txt",
    ("history_queue_kernel", "c4"): "history_queue_kernel_c4_traffic.txt",
    ("history_queue_pre_kernel", "c4"): "history_queue_pre_kernel_c4_traffic.txt",
}


def read_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprof PMC summary, if any."""
    name = TRAFFIC_PROFILES.get((kernel, config))
    path = ROOT / "profiles" / name if name else None
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def prefill_measurement(args, w, device):
    """Initial-prefill launch alone (HIP events): useful causal FLOPs (QK and PV over each
    request's own tokens, 4 flop per query-key pair and dim) against the bf16 MFMA peak."""
    import torch

    from oscar_new_amd import kernels

    ntok = w.q.shape[0]
    if any(p != 0 for p in w.prefixes):
        print(json.dumps(continuation_measurement(args, w, device, args.config, args.steps)))
        return 0
    w.meta.initial_prefill = True
    _, win = w.layout.tensor_views((w.k_cache, w.v_cache))
    out = torch.empty(ntok, 6 * 256, dtype=torch.bfloat16, device=device)
    run = lambda: kernels.prefill_attention(w.q, w.k, w.v, win, w.meta, w.layout, 1 / 16, out)
    for _ in range(max(1, args.warmup)):
        run()
    torch.cuda.synchronize()
    evs = []
    for _ in range(args.steps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        run()
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    us = statistics.mean(a.elapsed_time(b) for a, b in evs) * 1e3
    pairs = sum(s * (s + 1) // 2 for s in w.seqs)
    flops = 4.0 * pairs * 6 * 256
    print(json.dumps({"mode": "prefill", "config": args.config, "tokens": ntok,
                      "us": us, "tflops": flops / (us * 1e-6) / 1e12,
                      "mfma_bf16_peak_tflops": 2500.0,
                      "frac": flops / (us * 1e-6) / 1e12 / 2500.0}))
    return 0


def continuation_flops(w):
    """MFMA work of a continuation step: per request, the history branch (every query row
    against the request's INT2 history tokens) and the BF16 branch (the sink and recent
    window, then the chunk's own tokens causally). Useful flops count 4 per (query row, key,
    dim): QK and PV products. The history kernel issues 6: its QK runs the query as two FP8
    terms (hi + lo) against the FP4 codes."""
    cfg = w.cfg
    hist_pairs = bf16_pairs = 0
    for prefix, hist in zip(w.prefixes, history_lengths(w)):
        sink = min(cfg.sink_tokens, prefix)
        window = sink + (prefix - max(sink, prefix - cfg.recent_tokens))
        hist_pairs += w.qlen * hist
        bf16_pairs += w.qlen * window + w.qlen * (w.qlen + 1) // 2
    per_pair = 6 * 256  # query heads x head dim
    return SimpleNamespace(history_useful=4.0 * hist_pairs * per_pair,
                           history_issued=6.0 * hist_pairs * per_pair,
                           bf16=4.0 * bf16_pairs * per_pair)


def continuation_measurement(args, w, device, name, steps):
    """A continuation chunk (config p2): the layer step as ``impl.forward`` runs it (eager
    launches: a 2048-token step is far above launch overheads), and its history branch alone,
    timed with HIP events. The history branch is MFMA-bound: its issued FP8 x FP4 work over
    the launch time against the FP8 dense peak (5.0 PFLOP/s, the rate of
    v_mfma_scale_f32_16x16x128_f8f6f4 with an FP8 operand)."""
    import torch

    from oscar_new_amd.backend import OscarAttentionImpl

    cfg = CONFIGS[name]
    impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, w.cfg,
                                         split_policy=args.split_policy or cfg["splits"])
    impl.set_rotations(w.rk, w.rv)
    ntok = w.q.shape[0]
    layers = [(w.k_cache, w.v_cache)]
    out = torch.empty(ntok, 6 * 256, dtype=torch.bfloat16, device=device)
    splits, split_tokens = impl.partition_for(w.meta, ntok)
    step_us = time_launch(lambda i: impl.forward(None, w.q, w.k, w.v, layers[0], w.meta, out),
                          1, steps, False)
    bname, _, bfn = branch_launch(impl, w, layers, splits, split_tokens)
    b_us = time_launch(bfn, 1, steps, False)
    fl = continuation_flops(w)
    hist_tf = fl.history_issued / (b_us * 1e-6) / 1e12
    return {"mode": "prefill", "config": name, "workload": f"{name}: {cfg['desc']}",
            "tokens": ntok, "cached_tokens": sum(w.prefixes), "splits": splits,
            "split_tokens": split_tokens, "us_per_layer_step": step_us,
            "step_useful_tflops": (fl.history_useful + fl.bf16) / (step_us * 1e-6) / 1e12,
            "history_branch": {
                "kernel": bname, "us": b_us, "issued_flops": fl.history_issued,
                "useful_flops": fl.history_useful, "tflops_issued": hist_tf,
                "tflops_useful": fl.history_useful / (b_us * 1e-6) / 1e12,
                "peak_tflops": 5000.0, "frac": hist_tf / 5000.0, "bound": "mfma (fp8 x fp4)"},
            "bf16_branch_flops": fl.bf16}


def in_step_launch(impl, w, layers, splits, split_tokens):
    """The launch the layer step makes for its history branch, as ``impl.forward`` makes it:
    ``(kernel name, algorithmic bytes, fn(i))``, fn(i) launching it on layer i's cache.

    With the pre-attention roles in the history launch (up to 8 query rows per task, or the
    17-32-row work queue with token-bounded splits) that is ``history_pre`` (its workgroups
    run the BF16 branch and the K/V INT2 store beside the INT2 stream); otherwise the step
    runs the pre-attention launch first and this is the history branch alone
    (``attention_partials``)."""
    from oscar_new_amd import kernels

    views = [w.layout.tensor_views(c) for c in layers]
    meta, layout = w.meta, w.layout
    ntok = w.q.shape[0]
    alg = algorithmic_bytes(w)
    hist = alg.int2 + ntok * 6 * 256 * 2 + alg.table + split_partial_bytes(w, splits,
                                                                         split_tokens)
    queue = impl._queue_roles(meta, split_tokens, ntok)
    if impl._roles_share_history_launch(meta) or queue:
        rows = ntok * 6
        # + the BF16 branch (window and current K/V rows, its partial rows), the step's INT2
        # slots and R_k / R_v.
        extra = alg.bf16 + rows * 1028 + ntok * 136 + 2 * 256 * 256 * 2
        q_sync = None
        if queue:
            # The 17-32-row work queue with the roles as units of its own.
            name, qrot = "history_queue_pre_kernel", kernels.rotate(w.q, impl.rk_cols)
        elif impl._q_roles():
            # + the rotation roles' rotated rows (written, then read by the history rows).
            name = "history_pre_q_kernel"
            extra += ntok * 6 * 256 * 2
            qrot = w.q.new_empty(w.q.shape)
            q_sync = impl.q_sync
        elif impl.rotate_in_history:
            name, qrot = "history_pre_rot_kernel", None
        else:
            name, qrot = "history_pre_kernel", kernels.rotate(w.q, impl.rk_cols)

        def fn(i):
            h, win = views[i % len(views)]
            kernels.history_pre(qrot, w.q, w.k, w.v, h, win, meta, layout, 1 / 16, splits,
                                impl.rk_t, impl.rv_t, split_tokens=split_tokens,
                                q_sync=q_sync)

        return name, hist + extra, fn
    qrot = kernels.rotate(w.q, impl.rk_cols)

    def fn(i):
        h, win = views[i % len(views)]
        kernels.attention_partials(qrot, w.k, w.v, h, win, meta, layout, 1 / 16, splits, False,
                                   split_tokens=split_tokens)

    return kernels.history_kernel_name(meta, layout, 6, ntok, split_tokens), hist, fn


def branch_launch(impl, w, layers, splits, split_tokens):
    """The history branch alone (``attention_partials`` on a pre-rotated query, no role
    workgroups), with the step's partition: ``(kernel name, algorithmic bytes, fn(i))``."""
    from oscar_new_amd import kernels

    from oscar_new_amd import config

    views = [w.layout.tensor_views(c) for c in layers]
    ntok = w.q.shape[0]
    alg = algorithmic_bytes(w)
    qrot = kernels.rotate(w.q, impl.rk_cols)
    if split_tokens < 0:  # the branch alone has no role workgroups: the whole launch budget
        split_tokens = -(config.HISTORY_SLOTS if kernels.history_rows(w.meta, w.layout, 6) <= 16
                         else config.QUEUE_SLOTS)
    hist = alg.int2 + ntok * 6 * 256 * 2 + alg.table + split_partial_bytes(w, splits,
                                                                         split_tokens)

    def fn(i):
        h, win = views[i % len(views)]
        kernels.attention_partials(qrot, w.k, w.v, h, win, w.meta, w.layout, 1 / 16, splits,
                                   False, split_tokens=split_tokens)

    return kernels.history_kernel_name(w.meta, w.layout, 6, ntok, split_tokens), hist, fn


def time_launch(fn, nlayers, steps, use_graph, stream=None, pool=None):
    """Mean device time of fn(i) per launch: HIST_LAUNCHES back-to-back launches (cycling the
    layers' caches) captured in one graph, replays timed with HIP events on the launching
    stream (torch's current stream when graphs are off)."""
    import torch

    for i in range(nlayers):
        fn(i)
    torch.cuda.synchronize()
    reps = max(1, -(-steps // HIST_LAUNCHES))
    if use_graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, pool=pool):
            for i in range(HIST_LAUNCHES):
                fn(i)
        torch.cuda.synchronize()
        g.replay()
        run = g.replay
    else:
        def run():
            for i in range(HIST_LAUNCHES):
                fn(i)
    torch.cuda.synchronize()
    h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h0.record()
    for _ in range(reps):
        run()
    h1.record()
    torch.cuda.synchronize()
    return h0.elapsed_time(h1) * 1e3 / (reps * HIST_LAUNCHES)


def measure_step(args, name, device, steps, warmup):
    """Build config `name`, time `steps` layer steps (graph replays cycling the layers), the
    step's history launch and the history branch alone. Returns a dict of figures and the
    workload (for the CPU baseline)."""
    import torch

    from oscar_new_amd import kernels
    from oscar_new_amd.backend import OscarAttentionImpl

    cfg = CONFIGS[name]
    print(f"[bench] building {name} workload", file=sys.stderr, flush=True)
    w = build_workload(args, cfg, device)
    nlayers = args.layers or (2 if w.k_cache.numel() * 2 > 16 << 30 else 4)
    layers = [(w.k_cache, w.v_cache)]
    for _ in range(nlayers - 1):
        layers.append((w.k_cache.clone(), w.v_cache.clone()))
    impls = []
    for _ in layers:
        impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, w.cfg,
                                             split_policy=args.split_policy or cfg["splits"],
                                             one_launch_post=args.one_launch_post,
                                             overlap=not args.no_overlap,
                                             layer_step=args.layer_step,
                                             rotate_in_history=args.rotate_in_history,
                                             q_roles=args.q_roles)
        impl.set_rotations(w.rk, w.rv)
        impls.append(impl)
    ntok = w.q.shape[0]
    outputs = [torch.empty(ntok, 6 * 256, dtype=torch.bfloat16, device=device) for _ in layers]
    splits, split_tokens = impls[0].partition_for(w.meta, ntok)

    def step(i):
        impls[i].forward(None, w.q, w.k, w.v, layers[i], w.meta, outputs[i])

    for i in range(len(layers)):  # eager warm-up (also builds the tensor views)
        step(i)
    torch.cuda.synchronize()
    # The layer steps of consecutive layers are captured back to back in one HIP graph, as a
    # model's decode graph holds them; a step is one layer's forward. `full` replays all
    # layers once, `tail` covers a remainder so that exactly `steps` steps are timed. Under the
    # device split rule the graph is captured at a dummy batch's lengths (zero counts, as
    # vLLM's capture build leaves them) and replayed at the workload's.
    nl = len(layers)
    graphs = stream = pool = None
    dummy_capture = not args.no_graph and split_tokens < 0
    if not args.no_graph:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graphs = {}
        counts = w.meta.counts.clone()
        if dummy_capture:
            w.meta.counts.zero_()
            kernels.prepare_tasks(w.meta.query_start_loc, w.meta.counts, w.meta.tasks,
                                  w.meta.task_count, w.meta.max_num_reqs,
                                  w.cfg.queries_per_tile)
            torch.cuda.synchronize()
        for count in sorted({nl, steps % nl, warmup % nl} - {0}):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream, pool=pool):
                for i in range(count):
                    step(i)
            pool = g.pool()
            graphs[count] = g
        torch.cuda.synchronize()
        if dummy_capture:
            w.meta.counts.copy_(counts)
            kernels.prepare_tasks(w.meta.query_start_loc, w.meta.counts, w.meta.tasks,
                                  w.meta.task_count, w.meta.max_num_reqs,
                                  w.cfg.queries_per_tile)
            torch.cuda.synchronize()

    def run_steps(count):
        """`count` layer steps, cycling layers 0, 1, ..., nl - 1, 0, ..."""
        if graphs is None:
            for i in range(count):
                step(i % nl)
            return
        for _ in range(count // nl):
            graphs[nl].replay()
        if count % nl:
            graphs[count % nl].replay()

    print(f"[bench] {name}: warmup {warmup}, timed {steps}", file=sys.stderr, flush=True)
    run_steps(warmup)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    run_steps(steps)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    us_step = wall / steps * 1e6
    alg = algorithmic_bytes(w)

    use_graph = graphs is not None
    kname, kbytes, kfn = in_step_launch(impls[0], w, layers, splits, split_tokens)
    k_us = time_launch(kfn, nl, steps, use_graph, stream, pool)
    bname, bbytes, bfn = branch_launch(impls[0], w, layers, splits, split_tokens)
    b_us = time_launch(bfn, nl, steps, use_graph, stream, pool)
    print(f"[bench] {name}: step {us_step:.1f} us, {kname} {k_us:.1f} us, history branch alone "
          f"({bname}) {b_us:.1f} us", file=sys.stderr, flush=True)
    t_dev = effective_split_tokens(w, split_tokens)
    figures = {
        "workload": f"{name}: {cfg['desc']}",
        "us_per_layer_step": us_step,
        "gpu_us_per_layer_step": gpu_ms / steps * 1e3,
        "algorithmic_bytes_per_step": alg.total,
        "GBps": alg.total / (us_step * 1e-6) / 1e9,
        "splits": splits,
        "split_tokens": t_dev,
        "split_rule": ("device (budget %d workgroups)" % -split_tokens if split_tokens < 0
                       else "token-bounded" if split_tokens else "reference"),
        "graph_captured_at": ("dummy lengths" if dummy_capture else
                              "workload lengths" if use_graph else None),
        "dominant": {
            "kernel": kname, "us": k_us, "algorithmic_bytes": kbytes,
            "GBps": kbytes / (k_us * 1e-6) / 1e9,
            "frac": kbytes / (k_us * 1e-6) / 1e9 / PEAK_HBM_GBPS,
            "traffic": read_traffic(kname, name),
        },
        "history_branch": {
            "kernel": bname, "us": b_us, "algorithmic_bytes": bbytes,
            "history_tokens": alg.history_tokens,
            "GBps": bbytes / (b_us * 1e-6) / 1e9,
            "int2_GBps": alg.int2 / (b_us * 1e-6) / 1e9,
            "frac": bbytes / (b_us * 1e-6) / 1e9 / PEAK_HBM_GBPS,
            "traffic": read_traffic(bname, name),
        },
        "layers_cycled": nl,
        "hip_graph": use_graph,
    }
    return figures, SimpleNamespace(w=w, layers=layers, outputs=outputs, step=step)


def prefill_record(args, device, steps, warmup):
    """Sub-record of the initial-prefill launch (config p1)."""
    import torch

    from oscar_new_amd import kernels

    w = build_workload(args, CONFIGS["p1"], device)
    ntok = w.q.shape[0]
    w.meta.initial_prefill = True
    _, win = w.layout.tensor_views((w.k_cache, w.v_cache))
    out = torch.empty(ntok, 6 * 256, dtype=torch.bfloat16, device=device)
    us = time_launch(lambda i: kernels.prefill_attention(w.q, w.k, w.v, win, w.meta, w.layout,
                                                         1 / 16, out), 1, steps, False)
    pairs = sum(s * (s + 1) // 2 for s in w.seqs)
    tflops = 4.0 * pairs * 6 * 256 / (us * 1e-6) / 1e12
    return {"workload": f"p1: {CONFIGS['p1']['desc']}", "kernel": "prefill_flash_kernel",
            "us": us, "tflops": tflops, "peak_tflops": 2500.0, "frac": tflops / 2500.0,
            "bound": "mfma (bf16)"}


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one MI355X; --gpus {args.gpus} is not supported "
              "(no multi-GPU path exists; run with --gpus 1)", file=sys.stderr)
        return 2
    import torch

    from oscar_new_amd import kernels

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.mode == "copy":
        return copy_calibration(args, device)
    if args.mode == "store":
        time_store(device, args, args.steps, eager=True)
        print(json.dumps({"mode": "store", "calls_per_form": args.steps}))
        return 0
    if args.mode == "prefill":
        cfg = CONFIGS[args.config]
        print(f"[bench] building {args.config} workload", file=sys.stderr, flush=True)
        return prefill_measurement(args, build_workload(args, cfg, device), device)
    if args.mode == "history":
        from oscar_new_amd.backend import OscarAttentionImpl

        cfg = CONFIGS[args.config]
        w = build_workload(args, cfg, device)
        impl = OscarAttentionImpl.standalone(6, 256, 1 / 16, 1, w.cfg,
                                             split_policy=args.split_policy or cfg["splits"])
        impl.set_rotations(w.rk, w.rv)
        splits, split_tokens = impl.partition_for(w.meta, w.q.shape[0])
        kname, _, fn = (branch_launch if args.branch else in_step_launch)(
            impl, w, [(w.k_cache, w.v_cache)], splits, split_tokens)
        for i in range(args.warmup + args.steps):
            fn(i)
        torch.cuda.synchronize()
        alg = algorithmic_bytes(w)
        print(json.dumps({"mode": "history", "kernel": kname,
                          "launches": args.warmup + args.steps, "splits": splits,
                          "split_tokens": split_tokens, "history_tokens": alg.history_tokens,
                          "int2_bytes": alg.int2,
                          "physical_record_bytes": 160 * alg.history_tokens}))
        return 0

    fig, run = measure_step(args, args.config, device, args.steps, args.warmup)
    w = run.w
    store = time_store(device, args, max(20, args.steps // 2))
    cfg = CONFIGS[args.config]
    dom = fig["dominant"]
    result = {
        "metric": METRIC,
        "value": fig["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": fig["us_per_layer_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": fig["workload"],
            "batch": len(w.seqs),
            "context": cfg["context"],
            "query_tokens_per_request": w.qlen,
            "q_heads": 6, "kv_heads": 1, "head_dim": 256,
            "page_tokens": 768, "kernel_block_tokens": 128,
            "splits": fig["splits"], "split_tokens": fig["split_tokens"],
            "split_rule": fig["split_rule"], "graph_captured_at": fig["graph_captured_at"],
            "layers_cycled": fig["layers_cycled"],
            "hip_graph": fig["hip_graph"], "seed": args.seed,
            "one_launch_post": bool(args.one_launch_post),
            "overlap": not args.no_overlap,
            "layer_step": bool(args.layer_step),
            "rotate_in_history": bool(args.rotate_in_history),
            "q_roles": bool(args.q_roles),
        },
        "us_per_layer_step": fig["us_per_layer_step"],
        "gpu_us_per_layer_step": fig["gpu_us_per_layer_step"],
        "algorithmic_bytes_per_step": fig["algorithmic_bytes_per_step"],
        "dominant_kernel": dom,
        "history_kernel": fig["history_branch"],
        "store": store,
        "roofline": {
            "bound": "hbm",
            "kernel": dom["kernel"],
            "achieved": dom["GBps"],
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": dom["frac"],
            "traffic": dom["traffic"],
        },
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU oracle baseline", file=sys.stderr, flush=True)
        run.step(0)
        torch.cuda.synchronize()
        cpu, parity = cpu_baseline(SimpleNamespace(**{**vars(w), "k_cache": run.layers[0][0],
                                                      "v_cache": run.layers[0][1]}),
                                   args, run.outputs[0])
        result["cpu_baseline"] = cpu
        result["parity_sample"] = parity
    if args.config == "c3" and not args.no_sub_configs:
        # The other BASELINE decode configs and the initial prefill, each on its own workload
        # (built after the previous one is freed): step, dominant launch and its roofline.
        del run, w
        torch.cuda.empty_cache()
        subs = {}
        for name in ("c4", "c5"):
            sub, srun = measure_step(args, name, device, max(10, args.steps), args.warmup)
            subs[name] = sub
            del srun
            torch.cuda.empty_cache()
        print("[bench] p1 prefill", file=sys.stderr, flush=True)
        subs["p1"] = prefill_record(args, device, max(10, args.steps), args.warmup)
        torch.cuda.empty_cache()
        print("[bench] p2 continuation chunk", file=sys.stderr, flush=True)
        w2 = build_workload(args, CONFIGS["p2"], device)
        subs["p2"] = continuation_measurement(args, w2, device, "p2", min(max(10, args.steps), 50))
        del w2
        torch.cuda.empty_cache()
        result["configs"] = subs
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())

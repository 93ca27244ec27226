#!/usr/bin/env python3
"""Benchmark of the paged KV-cache decode path on one MI355X.

Workload (the metric's configuration): Qwen2.5-0.5B attention shape (14 query / 2 KV heads,
head_dim 64), bf16, batch 256, contexts log-uniform in [128, 4096], block size 16, the pool
fragmented by a seeded 5,000-event alloc/free churn trace, 24 layers. One step = for each
of the 24 layers: KV append of the step's 256 new tokens + paged decode attention, one
fused call (mip_paged_decode_append, as PagedDecodeContext.attend issues it). Inputs are
resident in HBM before the timed region; the pool holds N(0, 1) data.

Reported (one JSON line on stdout):
  value         algorithmic bytes of the step (append + attention, 24 layers) / step time, GB/s
  roofline      one append + decode-attention call (the stream kernel paged_decode_stream, which
                also appends the new rows, plus its partition merge paged_decode_stream_merge,
                launched back to back on the caller's stream): algorithmic bytes per call
                (attention + append) / average call duration (HIP events around a timed loop of
                the calls), against the 8 TB/s HBM peak; traffic = measured HBM bytes per call
                when a counter summary exists under profiles/
  decode_tok_s  B / full decode-step time of a random-init Qwen2.5-0.5B (embedding, 24 layers
                with GEMMs, RoPE, KV append + attention, MLP, final norm, logits) through the
                model's unchanged call protocol (engine/model.py:249-250: apply_rope in torch,
                then ctx.attend, which appends and attends in one mip_paged_decode_append),
                the step replayed as one captured HIP graph (engine/cuda_graphs.py);
                decode_tok_s_eager: the same step launched eagerly;
                decode_tok_s_fused_rope / decode_tok_s_eager_fused_rope: the same two with the
                opt-in attend_rope protocol (RoPE fused into the append, mip_rope_kv_append)
  prefill       packed prefill attention over a cached prefix (64 forks of a 520-token prefix,
                suffixes U[32, 512], fp16): time per layer and TFLOP/s against the fp16 MFMA peak
  long_context  the same append + attention step at 28 query / 4 KV heads, head_dim 128, bf16,
                B=128, contexts log-uniform in [512, 8192], block 32: time per layer and GB/s,
                and the read probe over the same bytes as 8 KiB chunks (hbm_ceiling)
  cpu_baseline  the reference's torch CPU path (index_put_ append + table gather + SDPA,
                the oracle's restatement) timed on this host's cores for one layer, fp32

Algorithmic bytes per layer (e = element bytes, L_b = context + 1):
  attention = sum_b 2*Hkv*L_b*D*e  +  2*B*Hq*D*e (q, out)  +  sum_b ceil(L_b/BS)*4 (table)  +  4*B (lens)
  append    = 2 * (2*B*Hkv*D*e)  +  8*B (slot mapping)
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

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "mini-inference_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0
METRIC = "paged decode-attn HBM GB/s (% of peak) + decode tok/s, Qwen2.5-0.5B b256"
TRAFFIC_FILE = ROOT / "profiles" / "paged_decode_stream_bf16_b256_ctx128-4096_traffic.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def attention_bytes(lens: list[int], shape) -> int:
    e = shape.dtype.itemsize
    kv = sum(2 * shape.num_kv_heads * n * shape.head_dim * e for n in lens)
    qo = 2 * shape.batch * shape.num_heads * shape.head_dim * e
    tables = sum(-(-n // shape.block_size) * 4 for n in lens)
    return kv + qo + tables + 4 * shape.batch


def append_bytes(shape) -> int:
    e = shape.dtype.itemsize
    return 2 * (2 * shape.batch * shape.num_kv_heads * shape.head_dim * e) + 8 * shape.batch


def time_loop(fn, iters: int) -> float:
    """Seconds per iteration of ``fn`` on the current stream, by HIP events around ``iters`` calls."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / iters


def cpu_baseline(batch, layer_q, layer_k, layer_v, budget_s: float) -> dict:
    """The reference CPU torch path (oracle restatement) on one layer, fp32, this host's cores."""
    import torch

    from oracle import paged_ref as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cache = batch.cache
    tables = [list(cache.block_tables[s]) for s in batch.slots]
    inputs = ref.decode_inputs(batch.ctx, tables, cache.block_size)
    # Only the blocks the batch owns matter to the per-step work; copy those into a compact fp32 pool.
    used = sorted({b for t in tables for b in t})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, device=cache.k.device)
    k_cpu = cache.k[0].index_select(0, idx).float().cpu()
    v_cpu = cache.v[0].index_select(0, idx).float().cpu()
    compact = [[remap[b] for b in t] for t in tables]
    inputs = ref.decode_inputs(batch.ctx, compact, cache.block_size)
    q, k, v = layer_q.float().cpu(), layer_k.float().cpu(), layer_v.float().cpu()
    times = []
    t_start = time.perf_counter()
    warm = 2
    while True:
        t0 = time.perf_counter()
        ref.paged_decode_torch(q, k_cpu, v_cpu, k, v, inputs)
        times.append(time.perf_counter() - t0)
        runs = len(times) - warm
        if runs >= 5 or (runs >= 1 and time.perf_counter() - t_start > budget_s):
            break
    timed = times[warm:] if len(times) > warm else times
    per_layer = statistics.median(timed)
    try:
        model = next(line.split(":", 1)[1].strip() for line in open("/proc/cpuinfo") if line.startswith("model name"))
    except (OSError, StopIteration):
        model = "unknown"
    return {"per_layer_s": per_layer, "runs": len(timed), "warmup": min(warm, len(times)), "cores": cores,
            "cpu_model": model}


def decode_step(batch, dev, calls_per_step: int | None = None):
    """One decode step over every layer of ``batch``'s cache, as PagedDecodeContext.attend
    issues it: the step's work plan once, then per layer one fused append + attention call
    (``mip_paged_decode_append``) with distinct per-layer q/k/v. With ``calls_per_step`` the
    step makes that many calls, cycling over the cache's layers. Returns the step and the
    per-layer (q, k, v) lists."""
    import torch

    from engine import paged_ops, workloads

    shape, cache = batch.shape, batch.cache
    layers = shape.num_layers
    qs, ks, vs = [], [], []
    for layer in range(layers):
        q, k, v = workloads.step_inputs(batch, seed=100 + layer)
        qs.append(q)
        ks.append(k)
        vs.append(v)
    ctx = cache.decode_context(batch.slots)
    outs = [torch.empty(shape.batch, shape.num_heads, shape.head_dim, dtype=shape.dtype, device=dev)
            for _ in range(layers)]
    plan_call, plan = paged_ops.prepare_decode_plan(ctx.context_lens, ctx.block_tables, shape.num_heads,
                                                    shape.num_kv_heads, shape.head_dim, shape.block_size, shape.dtype,
                                                    max_blocks=ctx.num_blocks)
    calls = [paged_ops.prepare_paged_decode(qs[i][:, :, 0], cache.k[i], cache.v[i], ctx.block_tables,
                                            ctx.context_lens, ctx.scale, out=outs[i], max_blocks=ctx.num_blocks,
                                            append=(ks[i][:, :, 0], vs[i][:, :, 0], ctx.slot_mapping), plan=plan)[0]
             for i in range(layers)]

    n_calls = layers if calls_per_step is None else calls_per_step

    def hot_step():
        if plan_call is not None:
            plan_call()  # once per step: the work split every layer shares
        for i in range(n_calls):
            calls[i % layers]()

    return hot_step, (qs, ks, vs)


def long_context_measure(dev, steps: int = 10) -> dict:
    """Append + decode attention at the long-context shape as configured: 28 query / 4 KV heads,
    head_dim 128, bf16, 28 layers, batch 128, contexts log-uniform in [512, 8192], block size
    32, block tables randomly permuted over a pool of about 60 % of the 288 GB HBM (every
    layer's K and V). A step is the plan plus one fused call per layer, each on its own layer
    of the pool. HIP events; the figure is the step time over 28."""
    import torch

    from engine import workloads

    shape = workloads.SHAPES[5]
    batch = workloads.build_decode_batch(shape, dev, seed=0)
    pool_gb = 2 * batch.cache.k.numel() * batch.cache.k.element_size() / 1e9
    n_calls = shape.num_layers
    step, _ = decode_step(batch, dev)
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t = time_loop(step, steps) / n_calls
    lens = [n + 1 for n in batch.ctx]
    nbytes = attention_bytes(lens, shape) + append_bytes(shape)
    gbps = nbytes / t / 1e9
    num_blocks = batch.cache.num_blocks
    del batch, step
    torch.cuda.empty_cache()
    return {
        "workload": "paged decode step (KV append + paged attention), 28q/4kv heads d128, bf16, B=128, ctx "
                    f"log-uniform[512,8192], block 32, tables randomly permuted over a {num_blocks}-block pool "
                    f"({pool_gb:.1f} GB of K/V over 28 layers); plan + 28 calls per step, one per layer",
        "kernel": "paged_decode_stream_tiles<bf16, D=128, QR=8, NS=3> (planned, with the fused append) + "
                  "paged_decode_stream_merge<bf16, D=128>",
        "us_per_layer": round(t * 1e6, 2),
        "bound": "hbm",
        "achieved": round(gbps, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(gbps / HBM_PEAK_GBPS, 4),
        "bytes_per_layer": nbytes,
        "mean_ctx": round(statistics.mean(lens) - 1, 1),
    }


def decode_tok_s(batch, steps: int, warmup: int) -> dict:
    """Full random-init Qwen2.5-0.5B decode step at this batch: eager, and replayed as one HIP graph.

    A step = host tables + H2D, embedding, 24 layers (GEMMs, RoPE, KV append, paged attention,
    MLP), final norm and logits, synchronised. Each is timed twice: with the RoPE fused into
    the append (the contexts' default ``fuse_rope``), and through the reference's own call
    protocol (the model applies ``apply_rope`` and calls ``ctx.attend(layer_idx, q, k, v)``,
    engine/model.py:249-250), which a drop-in caller runs unchanged. Sequence lengths are
    restored after every step, so each step appends at the same positions and attends the
    same contexts.
    """
    import torch

    from engine.cuda_graphs import GraphedDecoder
    from engine.model import Qwen2Config, Qwen2ForCausalLM, random_init_

    cfg = Qwen2Config.qwen2_5_0_5b()
    cache = batch.cache
    dev = cache.k.device
    with torch.device(dev):
        model = Qwen2ForCausalLM(cfg)
    model = random_init_(model.to(dev, batch.shape.dtype), seed=0)
    tokens = torch.randint(0, cfg.vocab_size, (len(batch.slots),), generator=torch.Generator().manual_seed(5))
    ids = tokens.to(dev).unsqueeze(1)
    lengths = {s: cache.lengths[s] for s in batch.slots}
    token_list = tokens.tolist()

    def eager(fuse_rope: bool):
        @torch.inference_mode()
        def step():
            ctx = cache.decode_context(batch.slots)  # host tables + H2D, as the runner does each step
            ctx.fuse_rope = fuse_rope
            hidden = model(ids, ctx.positions.unsqueeze(1), ctx)
            return model.compute_logits(hidden[:, -1]).float()
        return step

    def graphed(fuse_rope: bool):
        dec = GraphedDecoder(model, cache, max_batch=len(batch.slots), fuse_rope=fuse_rope)
        dec.capture(batches=[len(batch.slots)])

        @torch.inference_mode()
        def step():
            out = dec.decode(batch.slots, token_list)
            cache.lengths.update(lengths)
            return out
        return step

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(steps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        return statistics.median(times)

    t_eager = timed(eager(True))
    t_graph = timed(graphed(True))
    t_eager_attend = timed(eager(False))
    t_graph_attend = timed(graphed(False))
    n = len(batch.slots)
    return {"tok_s": n / t_graph, "ms_per_step": t_graph * 1e3, "eager_tok_s": n / t_eager,
            "eager_ms_per_step": t_eager * 1e3, "attend_tok_s": n / t_graph_attend,
            "attend_ms_per_step": t_graph_attend * 1e3, "eager_attend_tok_s": n / t_eager_attend,
            "eager_attend_ms_per_step": t_eager_attend * 1e3, "steps": steps}


def prefill_measure(dev, iters: int = 30, dtype: str = "float16") -> dict:
    """Packed prefill attention of the shared-prefix workload (64 forks of a 520-token cached
    prefix, suffixes U[32, 512], fp16 or bf16, 14q/2kv heads d64, block 16), one layer, HIP
    events.

    The new tokens attend their sequence's cached prefix and their own earlier tokens through
    the paged prefill kernel (``mip_paged_prefill``); flops = 4 * D * Hq * sum(position + 1).
    """
    import torch

    from engine import paged_ops, workloads

    dt = getattr(torch, dtype)
    short = {"float16": "fp16", "bfloat16": "bf16"}[dtype]
    pb = workloads.build_prefix_batch(dev, seed=0, num_layers=1, dtype=dt)
    ctx = pb.cache.packed_prefill_context(pb.children, pb.suffix_lens)  # appends nothing; CoW of the shared block
    hq, d = 14, 64
    n = sum(pb.suffix_lens)
    gen = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(n, hq, d, generator=gen, device=dev).to(dt)
    out = torch.empty_like(q)
    k_layer, v_layer = pb.cache.k[0], pb.cache.v[0]

    call = paged_ops.prepare_paged_prefill(q, k_layer, v_layer, ctx.block_tables, ctx.cu_q, ctx.ctx_start,
                                           ctx.max_q_len, out=out)[0]

    for _ in range(3):
        call()
    torch.cuda.synchronize()
    t_cold = time_loop(call, iters)
    # The GPU raises its clocks over some tens of milliseconds of sustained MFMA work (from a
    # pause the kernel starts near 95 us and settles about 15 % lower), so the sustained figure
    # is taken after 0.1 s of back-to-back calls; the figure right after the other legs is
    # kept as us_per_layer_cold.
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.1:
        for _ in range(50):
            call()
        torch.cuda.synchronize()
    t = time_loop(call, iters)
    keys = sum(sum(a + i + 1 for i in range(m)) for a, m in zip(ctx.starts, pb.suffix_lens))
    tflops = 4 * d * hq * keys / t / 1e12
    return {
        "workload": f"packed prefill attention over a cached prefix: {len(pb.children)} forks of a "
                    f"{pb.prefix_len}-token prefix + suffixes U[32,512] ({n} new tokens), {short}, 14q/2kv heads d64, "
                    "block 16, one layer",
        "kernel": f"paged_prefill_kernel<{'f16' if short == 'fp16' else 'bf16'}, D=64, NC=4> (query rows packed as "
                  "(token, head) pairs, 36 tokens per workgroup" + ("; V staged as fp16)" if short == "bf16" else ")"),
        "us_per_layer": round(t * 1e6, 1),
        "us_per_layer_cold": round(t_cold * 1e6, 1),
        "timing": "HIP events over 30 calls after 0.1 s of back-to-back calls (sustained clocks); "
                  "us_per_layer_cold: 30 calls right after 3 warm-up calls",
        "bound": "mfma",
        "achieved": round(tflops, 1),
        "peak": 2500.0,
        "unit": "TFLOP/s",
        "frac": round(tflops / 2500.0, 4),
        "frac_cold": round(4 * d * hq * keys / t_cold / 1e12 / 2500.0, 4),
        "keys_attended": keys,
    }


def append_measure(dev, iters: int = 40) -> dict:
    """Packed prefill append of the shared-prefix workload: every fork's new suffix tokens
    (U[32, 512] each, 64 forks) scattered into the pool of one layer through the context's
    slot mapping (``mip_kv_append`` with N tokens), fp16, 2 kv heads d64, block 16. The k/v
    rows are the model's [1, Hkv, N, D] projections viewed token-major, as the reference
    scatters them (engine/kv_cache.py:286-289). Four layers are cycled.
    bytes = read + write of the K and V rows + the int64 slots.
    """
    import torch

    from engine import paged_ops, workloads

    pb = workloads.build_prefix_batch(dev, seed=0, num_layers=4)
    ctx = pb.cache.packed_prefill_context(pb.children, pb.suffix_lens)
    n = sum(pb.suffix_lens)
    hkv, d = 2, 64
    gen = torch.Generator(device=dev).manual_seed(9)
    ks = [torch.randn(1, hkv, n, d, generator=gen, device=dev).half() for _ in range(4)]
    vs = [torch.randn(1, hkv, n, d, generator=gen, device=dev).half() for _ in range(4)]
    calls = [paged_ops.prepare_kv_append(pb.cache.k[i], pb.cache.v[i], ks[i][0].transpose(0, 1),
                                         vs[i][0].transpose(0, 1), ctx.slot_mapping) for i in range(4)]
    it = [0]

    def call():
        calls[it[0] % 4]()
        it[0] += 1

    for _ in range(4):
        call()
    torch.cuda.synchronize()
    t = time_loop(call, iters)
    nbytes = 2 * (2 * n * hkv * d * 2) + 8 * n
    gbs = nbytes / t / 1e9
    floor = copy_floor(dev, nbytes, sets=4)
    return {
        "workload": f"packed prefill append: {n} new tokens of {len(pb.children)} forks into one layer's pool, "
                    "fp16, 2 kv heads d64, block 16",
        "kernel": "kv_append_kernel",
        "us_per_layer": round(t * 1e6, 2),
        "copy_floor_us": round(floor * 1e6, 2),
        "bound": "hbm",
        "achieved": round(gbs, 1),
        "peak": 8000.0,
        "unit": "GB/s",
        "frac": round(gbs / 8000.0, 4),
        "bytes": nbytes,
    }


def copy_floor(dev, nbytes: int, sets: int, iters: int = 40) -> float:
    """Seconds a plain device copy (``torch.Tensor.copy_``) takes to move ``nbytes`` of traffic
    (half read, half written) in one launch, cycling ``sets`` disjoint buffer pairs as the
    measurement it is set beside does: the floor for a data-movement kernel of that size."""
    import torch

    half = nbytes // 2
    pairs = [(torch.empty(half, dtype=torch.uint8, device=dev), torch.empty(half, dtype=torch.uint8, device=dev))
             for _ in range(sets)]
    it = [0]

    def call():
        src, dst = pairs[it[0] % sets]
        dst.copy_(src)
        it[0] += 1

    for _ in range(sets):
        call()
    torch.cuda.synchronize()
    t = time_loop(call, iters)
    del pairs
    return t


def copy_measure(dev, iters: int = 40, sets: int = 8) -> dict:
    """Copy-on-write of the shared-prefix workload: each of 64 forks copies its partially
    filled last shared block, every layer, K and V, in one launch for all pairs. Timed as
    PagedKVCache.copy_blocks issues it, with the pairs built on the host and passed in the
    kernel arguments (``mip_copy_blocks_host``); ``device_pairs`` times the same copies with
    the pairs read from device memory (``mip_copy_blocks``). Pools of 24 layers at the
    Qwen2.5-0.5B shape (fp16, 2 kv heads, d64, block 16); ``sets`` disjoint sets of 64
    (src, dst) pairs are cycled so no launch re-reads what the last one touched. bytes = read
    + write of 24 * 2 * 2 KiB per pair.
    """
    import random

    import torch

    from engine import paged_ops

    layers, hkv, bs, d, pairs_per = 24, 2, 16, 64, 64
    nb = 2 * sets * pairs_per + 8
    k = torch.empty(layers, nb + 1, hkv, bs, d, dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    gen = torch.Generator(device=dev).manual_seed(5)
    k.normal_(0.0, 1.0, generator=gen)
    v.normal_(0.0, 1.0, generator=gen)
    ids = list(range(nb))
    random.Random(5).shuffle(ids)
    host_sets = [[(ids[2 * (i * pairs_per + j)], ids[2 * (i * pairs_per + j) + 1]) for j in range(pairs_per)]
                 for i in range(sets)]

    def timed(pair_sets) -> float:
        calls = [paged_ops.prepare_copy_blocks(k, v, p) for p in pair_sets]
        it = [0]

        def call():
            calls[it[0] % sets]()
            it[0] += 1

        for _ in range(sets):
            call()
        torch.cuda.synchronize()
        return time_loop(call, iters)

    t = timed(host_sets)
    t_dev = timed([torch.tensor(p, dtype=torch.int64, device=dev) for p in host_sets])
    nbytes = 2 * pairs_per * layers * 2 * hkv * bs * d * 2
    gbs = nbytes / t / 1e9
    floor = copy_floor(dev, nbytes, sets=sets)
    return {
        "workload": f"copy-on-write of {pairs_per} partially filled shared blocks (one per fork), {layers} layers, "
                    "K and V, fp16, 2 kv heads d64, block 16",
        "kernel": "copy_blocks_kernel<16, InlinePairs> (pairs in the kernel arguments)",
        "us": round(t * 1e6, 2),
        "device_pairs_us": round(t_dev * 1e6, 2),
        "copy_floor_us": round(floor * 1e6, 2),
        "bound": "hbm",
        "achieved": round(gbs, 1),
        "peak": 8000.0,
        "unit": "GB/s",
        "frac": round(gbs / 8000.0, 4),
        "bytes": nbytes,
    }


PROBE_MODES = {"grid_stride": 0, "span_lds": 1, "span_lds_nt": 2}


def hbm_ceiling(dev, nbytes: int, chunk: int = 2048, sets: int = 24, iters: int = 48,
                grids: dict | None = None) -> dict:
    """What this GPU streams for ``nbytes`` (one decode call's algorithmic bytes): the library's
    read probe (``mip_hbm_read_probe``) over randomly placed ``chunk``-byte chunks of a 4 GiB
    buffer; over random chunks drawn from a window of twice the bytes, as one layer's K and V
    pools are read (a window per set, each of its chunks used once); and over one contiguous
    run. Each pattern is read three ways (grid-stride register loads; contiguous spans per
    wavefront through an LDS ring of direct loads, the decode kernel's path; the same with the
    nontemporal cache policy, as the decode kernel's K/V loads), each at a few grids
    (workgroups of 256 threads), and cycles ``sets`` disjoint chunk sets so nothing is served
    from the 256 MB last-level cache. The fastest launch of each pattern is reported, with the
    best of each read path beside it. HIP events."""
    import torch

    from engine import _native

    grids = grids or {"grid_stride": (512, 1024, 1536, 2048), "span_lds": (512, 768), "span_lds_nt": (512, 768)}
    lib = _native.load()
    pool_bytes = 4 << 30
    buf = torch.zeros(pool_bytes // 4, dtype=torch.int32, device=dev)
    total = pool_bytes // chunk
    per = nbytes // chunk
    gen = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randperm(total, generator=gen, device=dev)[:per * sets].to(torch.int32).view(sets, per).contiguous()
    # Windows of twice the bytes (one layer's K and V pools, about); the sets reuse the buffer's
    # windows in turn, so a window comes back only after several others (far more than the
    # last-level cache holds) have been read.
    win = 2 * per
    nwin = max(1, total // win)
    windowed = [((i % nwin) * win + torch.randperm(win, generator=gen, device=dev)[:per]).to(torch.int32)
                for i in range(sets)]
    seq = [torch.arange(i * per, (i + 1) * per, dtype=torch.int32, device=dev) for i in range(sets)]
    sink = torch.empty(max(max(g) for g in grids.values()) * 256, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    out = {}
    for name, chunks in (("random_chunks", [ids[i] for i in range(sets)]), ("random_chunks_layer_window", windowed),
                         ("sequential", seq)):
        by_mode = {}
        for mode, mode_grids in grids.items():
            by_grid = {}
            for grid in mode_grids:
                args = [(buf.data_ptr(), pool_bytes, c.data_ptr(), per, chunk, sink.data_ptr(), grid, PROBE_MODES[mode],
                         st) for c in chunks]
                it = [0]

                def call():
                    a = args[it[0] % sets]
                    it[0] += 1
                    rc = lib.mip_hbm_read_probe(*a)
                    if rc:
                        _native.check(rc, "mip_hbm_read_probe")

                for _ in range(sets):
                    call()
                torch.cuda.synchronize()
                by_grid[grid] = time_loop(call, iters)
            grid, t = min(by_grid.items(), key=lambda kv: kv[1])
            by_mode[mode] = {"us": round(t * 1e6, 2), "grid": grid,
                             "us_by_grid": {str(g): round(v * 1e6, 2) for g, v in by_grid.items()}}
        mode = min(by_mode, key=lambda m: by_mode[m]["us"])
        t = by_mode[mode]["us"] * 1e-6
        out[name] = {"us": round(t * 1e6, 2), "GBps": round(per * chunk / t / 1e9, 1),
                     "frac": round(per * chunk / t / 1e9 / HBM_PEAK_GBPS, 4), "mode": mode,
                     "grid": by_mode[mode]["grid"], "by_mode": by_mode}
    del buf, ids, windowed, seq, sink
    torch.cuda.empty_cache()
    out.update({"kernel": "hbm_read_probe_kernel / hbm_read_probe_ring_kernel", "bytes": per * chunk,
                "chunk_bytes": chunk,
                "workload": f"read {per * chunk} B as {per} randomly placed {chunk}-byte chunks of a 4 GiB buffer, "
                            f"as {per} random chunks of a {win * chunk}-byte window (one per set), and as one "
                            f"contiguous run; {sets} disjoint sets cycled; each by grid-stride register loads, by "
                            f"contiguous spans per wavefront through an LDS ring of direct loads, and the same "
                            f"with the nontemporal policy; the fastest launch reported"})
    return out


def small_batch_decode(dev, steps: int, warmup: int) -> dict:
    """Full decode step at the 32-sequence fp16 shape: random-init Qwen2.5-0.5B, 24 layers,
    contexts U[128, 1024], block 16, tables randomly permuted over a 16,384-block pool; graphed
    and eager, as decode_tok_s (tok_s through the unchanged call protocol, fused_rope_* with
    the RoPE fused into the append)."""
    import torch

    from engine import workloads

    batch = workloads.build_decode_batch(workloads.SHAPES[2], dev, seed=0)
    dm = decode_tok_s(batch, steps=steps, warmup=warmup)
    del batch
    torch.cuda.empty_cache()
    return {
        "workload": "full decode step, random-init Qwen2.5-0.5B, fp16, B=32, ctx U[128,1024], block 16, "
                    "tables permuted over 16384 blocks",
        "tok_s": round(dm["attend_tok_s"], 1), "ms_per_step": round(dm["attend_ms_per_step"], 3),
        "eager_tok_s": round(dm["eager_attend_tok_s"], 1),
        "eager_ms_per_step": round(dm["eager_attend_ms_per_step"], 3),
        "fused_rope_tok_s": round(dm["tok_s"], 1), "fused_rope_ms_per_step": round(dm["ms_per_step"], 3),
        "eager_fused_rope_tok_s": round(dm["eager_tok_s"], 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline work (about)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-model", action="store_true", help="skip the full-model decode tok/s measurement")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the packed prefill attention, packed append and block-copy measurements")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the long-context decode measurement (28q/4kv heads d128, B=128, ctx up to 8192)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 512 MiB device copy three times (HBM counter scale for rocprofv3 --pmc)")
    ap.add_argument("--decode-algo", choices=("auto", "stream", "mfma", "valu"), default="auto",
                    help="force the decode attention kernel (kernel comparison; the headline uses auto = stream)")
    ap.add_argument("--no-probe", action="store_true", help="skip the HBM read-probe ceiling")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the headline decode call (no model, prefill, long-context, probe or CPU legs)")
    args = ap.parse_args()
    if args.headline_only:
        args.no_model = args.no_prefill = args.no_long_context = args.no_probe = args.no_cpu_baseline = True

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the paged decode path runs on a single GPU here "
              "(--gpus 1); multi-GPU runs are not supported.", file=sys.stderr)
        return 2

    import torch

    from engine import paged_ops, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    if args.decode_algo != "auto":
        from engine import _native

        _native.set_decode_algo(args.decode_algo)
    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.bfloat16, device=dev)  # 512 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    shape = workloads.SHAPES[3]
    t0 = time.perf_counter()
    batch = workloads.build_decode_batch(shape, dev, seed=0)
    cache = batch.cache
    log(f"workload ready in {time.perf_counter() - t0:.1f}s: B={shape.batch} layers={shape.num_layers} "
        f"pool={cache.num_blocks} blocks, mean ctx {statistics.mean(batch.ctx):.0f}")

    layers = shape.num_layers
    hot_step, (qs, ks, vs) = decode_step(batch, dev)
    for _ in range(args.warmup):
        hot_step()
    torch.cuda.synchronize()
    step_s = time_loop(hot_step, args.steps)
    call_s = step_s / layers  # the step is the plan + 24 calls, back to back on one stream
    lens = [n + 1 for n in batch.ctx]
    a_bytes = attention_bytes(lens, shape)
    p_bytes = append_bytes(shape)
    value = (a_bytes + p_bytes) * layers / step_s / 1e9
    achieved = (a_bytes + p_bytes) / call_s / 1e9
    log(f"step {step_s * 1e3:.3f} ms ({value:.0f} GB/s); append + attention call {call_s * 1e6:.2f} us "
        f"({achieved:.0f} GB/s, {achieved / HBM_PEAK_GBPS:.1%} of peak)")

    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V pool and q/k/v, seeded; churned block tables",
        "config": {
            "workload": "paged decode step (KV append + paged attention) x 24 layers, Qwen2.5-0.5B attention "
                        "shape 14q/2kv heads d64, bf16, B=256, ctx log-uniform[128,4096], block 16, pool of "
                        f"{cache.num_blocks} blocks fragmented by 5000 alloc/free events",
            "batch": shape.batch,
            "layers": layers,
            "mean_ctx": round(statistics.mean(batch.ctx), 1),
            "attn_bytes_per_layer": a_bytes,
            "append_bytes_per_layer": p_bytes,
        },
        "frac_of_peak": round(value / HBM_PEAK_GBPS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_stream_tiles<bf16, D=64, QR=8, NS=3> (planned, with the fused append) + "
                      "paged_decode_stream_merge<bf16, D=64>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "avg_launch_us": round(call_s * 1e6, 3),
        },
    }

    if args.decode_algo != "auto":
        result["decode_algo"] = args.decode_algo
        result["roofline"]["kernel"] = f"forced decode algorithm: {args.decode_algo}"

    if not args.no_probe:
        try:
            hc = hbm_ceiling(dev, a_bytes + p_bytes)
            hc["decode_call_frac_of_random_chunks"] = round(achieved / hc["random_chunks"]["GBps"], 4)
            hc["decode_call_frac_of_layer_window"] = round(achieved / hc["random_chunks_layer_window"]["GBps"], 4)
            result["hbm_ceiling"] = hc
            log(f"hbm probe: {hc['bytes']} B as random 2 KiB chunks {hc['random_chunks']['us']} us "
                f"({hc['random_chunks']['GBps']} GB/s, {hc['random_chunks']['mode']}), within a layer-sized window "
                f"{hc['random_chunks_layer_window']['us']} us ({hc['random_chunks_layer_window']['GBps']} GB/s, the "
                f"decode call reaches {hc['decode_call_frac_of_layer_window']:.1%} of it), sequential "
                f"{hc['sequential']['us']} us ({hc['sequential']['GBps']} GB/s, {hc['sequential']['mode']}); the decode "
                f"call reaches {hc['decode_call_frac_of_random_chunks']:.1%} of the random-chunk rate")
        except Exception as exc:
            log(f"hbm probe failed: {exc!r}")
            result["hbm_ceiling"] = None

    if not args.no_model:
        try:
            dm = decode_tok_s(batch, steps=max(10, min(args.steps, 30)), warmup=3)
            # The headline keys time the model's unchanged call protocol (apply_rope, then
            # ctx.attend); the *_fused_rope keys time the opt-in RoPE + append kernel.
            result["decode_tok_s"] = round(dm["attend_tok_s"], 1)
            result["decode_ms_per_step"] = round(dm["attend_ms_per_step"], 3)
            result["decode_tok_s_eager"] = round(dm["eager_attend_tok_s"], 1)
            result["decode_tok_s_fused_rope"] = round(dm["tok_s"], 1)
            result["decode_ms_per_step_fused_rope"] = round(dm["ms_per_step"], 3)
            result["decode_tok_s_eager_fused_rope"] = round(dm["eager_tok_s"], 1)
            log(f"full-model decode, reference protocol (apply_rope + ctx.attend): graph "
                f"{dm['attend_ms_per_step']:.2f} ms/step ({dm['attend_tok_s']:.0f} tok/s), eager "
                f"{dm['eager_attend_ms_per_step']:.2f} ms/step ({dm['eager_attend_tok_s']:.0f} tok/s)")
            log(f"full-model decode, RoPE fused into the append (attend_rope): graph {dm['ms_per_step']:.2f} ms/step "
                f"({dm['tok_s']:.0f} tok/s), eager {dm['eager_ms_per_step']:.2f} ms/step ({dm['eager_tok_s']:.0f} tok/s)")
        except Exception as exc:  # the headline kernel numbers stand on their own
            log(f"full-model decode failed: {exc!r}")
            result["decode_tok_s"] = None
        try:
            sb = small_batch_decode(dev, steps=max(10, min(args.steps, 30)), warmup=3)
            result["small_batch_decode"] = sb
            log(f"full-model decode B=32 fp16: graph {sb['ms_per_step']} ms/step ({sb['tok_s']} tok/s), "
                f"eager {sb['eager_ms_per_step']} ms/step ({sb['eager_tok_s']} tok/s)")
        except Exception as exc:
            log(f"B=32 full-model decode failed: {exc!r}")
            result["small_batch_decode"] = None

    if not args.no_prefill:
        try:
            result["prefill"] = prefill_measure(dev)
            pf = result["prefill"]
            log(f"prefill attention: {pf['us_per_layer']} us/layer sustained, {pf['achieved']} TFLOP/s ({pf['frac']:.1%} of "
                f"peak); {pf['us_per_layer_cold']} us/layer right after the other legs")
            # The same workload in bf16, right after the fp16 figure (so at the clocks that one
            # raised: only its sustained figure is reported).
            pb16 = prefill_measure(dev, dtype="bfloat16")
            pf["bf16"] = {k: pb16[k] for k in ("kernel", "us_per_layer", "achieved", "frac")}
            log(f"prefill attention bf16: {pb16['us_per_layer']} us/layer sustained, {pb16['achieved']} TFLOP/s "
                f"({pb16['frac']:.1%} of peak)")
        except Exception as exc:
            log(f"prefill measurement failed: {exc!r}")
            result["prefill"] = None
        try:
            result["packed_append"] = append_measure(dev)
            pa = result["packed_append"]
            log(f"packed append: {pa['us_per_layer']} us/layer, {pa['achieved']} GB/s ({pa['frac']:.1%} of peak); "
                f"a device copy of the same bytes takes {pa['copy_floor_us']} us")
        except Exception as exc:
            log(f"packed append measurement failed: {exc!r}")
            result["packed_append"] = None
        try:
            result["block_copy"] = copy_measure(dev)
            bc = result["block_copy"]
            log(f"block copy: {bc['us']} us, {bc['achieved']} GB/s ({bc['frac']:.1%} of peak; pairs read from "
                f"device memory {bc['device_pairs_us']} us); a device copy of the same bytes takes "
                f"{bc['copy_floor_us']} us")
        except Exception as exc:
            log(f"block copy measurement failed: {exc!r}")
            result["block_copy"] = None

    if not args.no_long_context:
        try:
            result["long_context"] = long_context_measure(dev)
            lc = result["long_context"]
            log(f"long-context decode: {lc['us_per_layer']} us/layer, {lc['achieved']} GB/s ({lc['frac']:.1%} of peak)")
            if not args.no_probe:
                # The same bytes through the read probe, as 8 KiB chunks (one block's K or V rows of
                # one kv head at this shape); 4 disjoint sets of the 4 GiB buffer, cycled.
                lh = hbm_ceiling(dev, lc["bytes_per_layer"], chunk=8192, sets=4, iters=12)
                lh["decode_call_frac_of_layer_window"] = round(lc["achieved"] / lh["random_chunks_layer_window"]["GBps"], 4)
                lc["hbm_ceiling"] = lh
                log(f"long-context hbm probe: {lh['bytes']} B as random 8 KiB chunks {lh['random_chunks']['us']} us "
                    f"({lh['random_chunks']['GBps']} GB/s), within a layer-sized window "
                    f"{lh['random_chunks_layer_window']['us']} us ({lh['random_chunks_layer_window']['GBps']} GB/s; the "
                    f"call reaches {lh['decode_call_frac_of_layer_window']:.1%} of it), sequential "
                    f"{lh['sequential']['us']} us ({lh['sequential']['GBps']} GB/s)")
        except Exception as exc:
            log(f"long-context decode measurement failed: {exc!r}")
            result["long_context"] = None

    if not args.no_cpu_baseline:
        cb = cpu_baseline(batch, qs[0], ks[0], vs[0], args.cpu_budget)
        cpu_gbps = (a_bytes + p_bytes) / cb["per_layer_s"] / 1e9
        result["cpu_baseline"] = {
            "value": round(cpu_gbps, 3),
            "unit": "GB/s",
            "cores": cb["cores"],
            "kind": "port",
            "sample": f"reference torch CPU path (index_put_ append + table gather + SDPA), fp32, one layer of the "
                      f"same B=256 workload, median of {cb['runs']} after {cb['warmup']} warm-ups: "
                      f"{cb['per_layer_s'] * 1e3:.1f} ms/layer ({cb['per_layer_s'] * layers * 1e3:.0f} ms per "
                      f"24-layer step); {cb['cpu_model']}",
        }
        log(f"cpu baseline: {cb['per_layer_s'] * 1e3:.1f} ms/layer on {cb['cores']} cores ({cpu_gbps:.2f} GB/s)")

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

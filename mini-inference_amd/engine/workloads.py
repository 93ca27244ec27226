"""Seeded synthetic workloads for the paged decode path (no datasets, no checkpoints).

Seeds: ``random.Random(seed)`` drives lengths, block permutations and the alloc/free churn
trace; tensors come from a seeded ``torch.Generator`` (CPU for small inputs, the device for
pool-sized fills). The five shapes:

  1  fp32, 1 layer, 14q/2kv heads, D 64, pool 512 blocks of 16, B 8, ctx U[16, 256],
     block tables = consecutive chunks of a permutation of the pool (golden-vector case)
  2  fp16, 24 layers, B 32, ctx U[128, 1024], block size 16, tables randomly permuted over
     a 16,384-block pool, K/V ~ 0.5 N(0, 1)
  3  bf16, 24 layers, B 256, ctx log-uniform [128, 4096], block size 16, pool fragmented
     by 5,000 alloc/free events before the 256 sequences are allocated
  4  fp16, 64 requests sharing a 520-token prefix (32 full blocks + a partial one, forked,
     so the partial block is copied on write), unique suffixes U[32, 512], packed append
     (:func:`build_prefix_batch`)
  5  bf16, 28q/4kv heads, D 128, 28 layers, B 128, ctx log-uniform [512, 8192], block 32,
     tables randomly permuted over a pool of about 60 % of the 288 GB HBM (94,168 blocks of
     1.835 MB each over the 28 layers' K and V: 172.8 GB)

"ctx" is the number of tokens already cached; a decode step appends one, so a sequence
attends ctx + 1 keys.
"""

from __future__ import annotations

import math
import random
from dataclasses import dataclass

import torch

from .kv_cache import PagedKVCache


@dataclass(frozen=True)
class DecodeShape:
    name: str
    dtype: torch.dtype
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    batch: int
    ctx_lo: int
    ctx_hi: int
    log_uniform: bool
    num_blocks: int
    churn_events: int = 0
    kv_scale: float = 1.0
    table_mode: str = "allocator"  # "chunks" | "permuted" | "allocator"


HBM_BYTES = 288e9  # MI355X


def pool_blocks_for(fraction: float, num_layers: int, num_kv_heads: int, block_size: int, head_dim: int,
                    elem_bytes: int) -> int:
    """Blocks of a pool that fills ``fraction`` of the HBM with every layer's K and V."""
    per_block = 2 * num_layers * num_kv_heads * block_size * head_dim * elem_bytes
    return int(fraction * HBM_BYTES // per_block)


SHAPES = {
    1: DecodeShape("cfg1-fp32-b8", torch.float32, 1, 14, 2, 64, 16, 8, 16, 256, False, 512, table_mode="chunks"),
    2: DecodeShape("cfg2-fp16-b32", torch.float16, 24, 14, 2, 64, 16, 32, 128, 1024, False, 16384, kv_scale=0.5,
                   table_mode="permuted"),
    3: DecodeShape("cfg3-bf16-b256", torch.bfloat16, 24, 14, 2, 64, 16, 256, 128, 4096, True, 32768,
                   churn_events=5000),
    5: DecodeShape("cfg5-bf16-b128-d128", torch.bfloat16, 28, 28, 4, 128, 32, 128, 512, 8192, True,
                   pool_blocks_for(0.6, 28, 4, 32, 128, 2), table_mode="permuted"),
}


def context_lengths(shape: DecodeShape, seed: int = 0) -> list[int]:
    rng = random.Random(seed)
    if shape.log_uniform:
        lo, hi = math.log(shape.ctx_lo), math.log(shape.ctx_hi)
        return [min(shape.ctx_hi, max(shape.ctx_lo, int(round(math.exp(rng.uniform(lo, hi))))))
                for _ in range(shape.batch)]
    return [rng.randint(shape.ctx_lo, shape.ctx_hi) for _ in range(shape.batch)]


def churn(cache: PagedKVCache, events: int, rng: random.Random, max_tokens: int) -> None:
    """Seeded alloc / grow / free trace on the allocator, then free everything it allocated.

    Leaves the pool empty but its free queue in a scrambled order, so later allocations
    receive scattered block ids, as in a long-running server.
    """
    live: list[int] = []
    for _ in range(events):
        r = rng.random()
        if live and r < 0.35:
            slot = live.pop(rng.randrange(len(live)))
            cache.free(slot)
        elif live and r < 0.55:
            slot = live[rng.randrange(len(live))]
            target = min(cache.max_len, cache.lengths[slot] + rng.randint(1, 256))
            if cache.ensure_capacity(slot, target):
                cache.lengths[slot] = target
        else:
            n = int(math.exp(rng.uniform(math.log(16), math.log(max_tokens))))
            if cache.can_allocate(n):
                slot = cache.allocate(n)
                cache.lengths[slot] = n
                live.append(slot)
    for slot in live:
        cache.free(slot)


@dataclass
class DecodeBatch:
    shape: DecodeShape
    cache: PagedKVCache
    slots: list[int]
    ctx: list[int]


def build_decode_batch(shape: DecodeShape, device: torch.device | str, seed: int = 0,
                       fill_pool: bool = True) -> DecodeBatch:
    """Allocate a cache and ``shape.batch`` sequences holding ``ctx`` tokens each (room for one more).

    Block tables follow ``shape.table_mode``: consecutive chunks of one random permutation
    of the pool ("chunks" / "permuted"), or whatever the allocator hands out after
    ``churn_events`` of churn ("allocator"). With ``fill_pool``
    the whole pool is filled with ``kv_scale * N(0, 1)`` (stale data included).
    """
    ctx = context_lengths(shape, seed)
    max_len = max(ctx) + 1
    cache = PagedKVCache(shape.num_layers, shape.num_kv_heads, shape.head_dim, shape.num_blocks, shape.block_size,
                         max_seqs=max(shape.batch, 1024), max_len=max(max_len, 8192), dtype=shape.dtype,
                         device=device)
    rng = random.Random(seed + 1)
    slots: list[int] = []
    if shape.table_mode == "allocator":
        if shape.churn_events:
            churn(cache, shape.churn_events, rng, max_tokens=shape.ctx_hi)
        for n in ctx:
            slot = cache.allocate(n + 1)
            cache.lengths[slot] = n
            slots.append(slot)
    else:
        perm = list(range(shape.num_blocks))
        rng.shuffle(perm)
        need = sum(cache.blocks_for(n + 1) for n in ctx)
        if need > shape.num_blocks:
            raise ValueError("pool too small for the batch")
        cursor = 0
        for n in ctx:
            slot = cache.allocate(0)
            nblk = cache.blocks_for(n + 1)
            blocks = perm[cursor:cursor + nblk]
            cursor += nblk
            # Hand the chosen blocks to the sequence through the allocator's own bookkeeping.
            for blk in blocks:
                cache._share(blk)
            cache.block_tables[slot] = list(blocks)
            cache.lengths[slot] = n
            slots.append(slot)
    if fill_pool:
        gen = torch.Generator(device=cache.k.device).manual_seed(seed + 2)
        for pool in (cache.k, cache.v):
            for layer in range(pool.shape[0]):
                pool[layer].normal_(0.0, shape.kv_scale, generator=gen)
    return DecodeBatch(shape, cache, slots, ctx)


@dataclass
class PrefixBatch:
    """A shared-prefix packed prefill: one parent holding the prefix, ``requests`` forks of it."""
    cache: PagedKVCache
    parent: int
    children: list[int]
    suffix_lens: list[int]
    prefix_len: int


def build_prefix_batch(device: torch.device | str, seed: int = 0, requests: int = 64, prefix_len: int = 520,
                       suffix_lo: int = 32, suffix_hi: int = 512, num_layers: int = 24, num_kv_heads: int = 2,
                       head_dim: int = 64, block_size: int = 16, dtype: torch.dtype = torch.float16,
                       num_blocks: int | None = None) -> PrefixBatch:
    """Shape 4: ``requests`` sequences forked from one parent whose ``prefix_len`` tokens are cached.

    With the default 520 tokens the prefix fills 32 blocks of 16 and part of a 33rd, so every
    fork shares 32 full blocks and one partially filled block; the first write of each fork's
    suffix copies that partial block (copy-on-write). The pool holds N(0, 1) data and the
    parent's prefix rows are part of it. Suffix lengths are U[suffix_lo, suffix_hi].
    """
    rng = random.Random(seed)
    suffix_lens = [rng.randint(suffix_lo, suffix_hi) for _ in range(requests)]
    bs = block_size
    need = -(-prefix_len // bs) + sum(-(-(prefix_len + n) // bs) - prefix_len // bs for n in suffix_lens)
    nb = num_blocks if num_blocks is not None else need + 64
    max_len = prefix_len + suffix_hi
    cache = PagedKVCache(num_layers, num_kv_heads, head_dim, nb, bs, max_seqs=requests + 1, max_len=max_len,
                         dtype=dtype, device=device)
    gen = torch.Generator(device=cache.k.device).manual_seed(seed + 2)
    for pool in (cache.k, cache.v):
        for layer in range(pool.shape[0]):
            pool[layer].normal_(0.0, 1.0, generator=gen)
    parent = cache.allocate(prefix_len)
    cache.lengths[parent] = prefix_len
    children = [cache.fork(parent) for _ in range(requests)]
    return PrefixBatch(cache, parent, children, suffix_lens, prefix_len)


def step_inputs(batch: DecodeBatch, seed: int = 0, device: torch.device | str | None = None):
    """q ``[B, Hq, 1, D]``, k/v ``[B, Hkv, 1, D]`` ~ N(0,1) (K/V scaled by ``kv_scale``) for one layer."""
    s = batch.shape
    dev = device if device is not None else batch.cache.k.device
    gen = torch.Generator(device="cpu").manual_seed(seed + 3)
    q = torch.randn(s.batch, s.num_heads, 1, s.head_dim, generator=gen)
    k = torch.randn(s.batch, s.num_kv_heads, 1, s.head_dim, generator=gen) * s.kv_scale
    v = torch.randn(s.batch, s.num_kv_heads, 1, s.head_dim, generator=gen) * s.kv_scale
    return q.to(s.dtype).to(dev), k.to(s.dtype).to(dev), v.to(s.dtype).to(dev)

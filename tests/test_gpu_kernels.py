"""GPU parity of the three HIP kernels against the CPU oracle, through the C ABI.

Bar: KV append and block copy bit-exact (every byte of the pool, touched or not);
paged decode attention within 2e-3 max-abs of the float64 oracle for fp16/bf16 (the
fp32-accumulate bound), 2e-5 for fp32.
"""

from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
TOL = {"float32": 2e-5, "float16": 2e-3, "bfloat16": 2e-3}


def storage(t: torch.Tensor) -> np.ndarray:
    """CPU numpy view of a tensor's storage: float32 values, or uint16 bits for 16-bit dtypes."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def values(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def dname(dtype: torch.dtype) -> str:
    return {v: k for k, v in DTYPES.items()}[dtype]


MANTISSA_BITS = {"float32": 23, "float16": 10, "bfloat16": 7}


def half_ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    """Half the spacing of ``dtype`` at |x|: the error of rounding an exact result once to the output dtype."""
    ax = np.maximum(np.abs(x), np.finfo(np.float32).tiny)
    return 0.5 * np.exp2(np.floor(np.log2(ax)) - MANTISSA_BITS[dtype])


def attention_error(got: np.ndarray, want: np.ndarray, dtype: str) -> float:
    """Max error beyond the output's own final rounding (the fp32-accumulate error, bounded by TOL)."""
    return float((np.abs(got - want) - half_ulp(want, dtype)).max())


# ----------------------------------------------------------------------------- append


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_append_decode_bit_exact(gpu, dtype):
    from engine import paged_ops

    announce(f"append decode {dtype}")
    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(1)
    nb, hkv, bs, d, batch = 64, 2, 16, 64, 40
    k_cache = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt).to(gpu)
    v_cache = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt).to(gpu)
    slots = torch.tensor(random.Random(2).sample(range((nb + 1) * bs), batch), dtype=torch.int64)
    # k as a contiguous [B, Hkv, D]; v as a strided view out of a wider row (like the qkv split).
    k_new = torch.randn(batch, hkv, d, generator=g).to(dt)
    wide = torch.randn(batch, 3 * hkv * d, generator=g).to(dt)
    v_new = wide[:, 2 * hkv * d:].view(batch, hkv, d)
    kc, vc = storage(k_cache), storage(v_cache)
    ref.append(kc, vc, (slots // bs).numpy(), (slots % bs).numpy(), storage(k_new), storage(v_new))
    paged_ops.kv_append(k_cache, v_cache, k_new.to(gpu), wide.to(gpu)[:, 2 * hkv * d:].view(batch, hkv, d),
                        slots.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(storage(k_cache), kc)
    assert np.array_equal(storage(v_cache), vc)


def test_append_packed_prefill_views(gpu):
    """The packed-prefill scatter: k[0].transpose(0, 1) and a v view of the fused qkv output."""
    from engine import paged_ops

    announce("append packed fp16")
    dt = torch.float16
    g = torch.Generator().manual_seed(3)
    nb, hkv, bs, d, n, hq = 300, 2, 16, 64, 3000, 14
    width = (hq + 2 * hkv) * d
    k_cache = torch.zeros(nb + 1, hkv, bs, d, dtype=dt, device=gpu)
    v_cache = torch.zeros_like(k_cache)
    qkv = torch.randn(1, n, width, generator=g).to(dt)
    k = qkv[..., hq * d:(hq + hkv) * d].reshape(1, n, hkv, d).transpose(1, 2).contiguous()  # post-RoPE k is contiguous
    v = qkv[..., (hq + hkv) * d:].view(1, n, hkv, d).transpose(1, 2)                         # v stays a view
    perm = list(range(nb))
    random.Random(4).shuffle(perm)
    blocks = np.asarray([perm[i // bs] for i in range(n)], dtype=np.int64)
    offsets = np.arange(n, dtype=np.int64) % bs
    slots = torch.from_numpy(blocks * bs + offsets)
    kc, vc = storage(k_cache), storage(v_cache)
    ref.append(kc, vc, blocks, offsets, storage(k[0].transpose(0, 1)), storage(v[0].transpose(0, 1)))
    kg, qkvg = k.to(gpu), qkv.to(gpu)
    vg = qkvg[..., (hq + hkv) * d:].view(1, n, hkv, d).transpose(1, 2)
    paged_ops.kv_append(k_cache, v_cache, kg[0].transpose(0, 1), vg[0].transpose(0, 1), slots.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(storage(k_cache), kc)
    assert np.array_equal(storage(v_cache), vc)


@pytest.mark.parametrize("dtype,d", [("bfloat16", 4), ("float16", 6), ("float32", 3), ("float32", 128)])
def test_append_narrow_rows_and_skipped_slots(gpu, dtype, d):
    from engine import paged_ops

    announce(f"append narrow {dtype} d={d}")
    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(5)
    nb, hkv, bs = 10, 3, 4
    k_cache = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt).to(gpu)
    v_cache = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt).to(gpu)
    slots = torch.tensor([5, -1, 43, (nb + 1) * bs, 0, 17, 10 ** 9], dtype=torch.int64)
    k_new = torch.randn(len(slots), hkv, d, generator=g).to(dt)
    v_new = torch.randn(len(slots), hkv, d, generator=g).to(dt)
    kc, vc = storage(k_cache), storage(v_cache)
    keep = [(i, int(s)) for i, s in enumerate(slots) if 0 <= s < (nb + 1) * bs]
    idx = np.asarray([i for i, _ in keep])
    sl = np.asarray([s for _, s in keep])
    ref.append(kc, vc, sl // bs, sl % bs, storage(k_new)[idx], storage(v_new)[idx])
    paged_ops.kv_append(k_cache, v_cache, k_new.to(gpu), v_new.to(gpu), slots.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(storage(k_cache), kc)
    assert np.array_equal(storage(v_cache), vc)


# ----------------------------------------------------------------------------- block copy


@pytest.mark.parametrize("where", ["device", "host"])
@pytest.mark.parametrize("dtype,hkv,bs,d", [("bfloat16", 2, 16, 64), ("float32", 2, 16, 64),
                                            ("bfloat16", 4, 32, 128), ("float32", 1, 1, 3)])
def test_copy_blocks_bit_exact(gpu, dtype, hkv, bs, d, where):
    """Whole-block copies, all layers, K and V; a 32 KiB block (4 kv heads x 32 x 128) takes
    several chunk rounds per thread, a 12-byte block the 4-byte chunk width. Pairs in device
    memory (mip_copy_blocks) and on the host (mip_copy_blocks_host, in the kernel arguments)."""
    from engine import paged_ops

    announce(f"copy_blocks {dtype} hkv={hkv} bs={bs} d={d} pairs on the {where}")
    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(6)
    layers, nb = 3, 40
    k = torch.randn(layers, nb + 1, hkv, bs, d, generator=g).to(dt).to(gpu)
    v = torch.randn(layers, nb + 1, hkv, bs, d, generator=g).to(dt).to(gpu)
    rng = random.Random(7)
    ids = rng.sample(range(nb + 1), 24)
    pairs = [(ids[i], ids[i + 12]) for i in range(12)] + [(3, -1), (nb + 5, 4)]  # last two are skipped
    kc, vc = storage(k), storage(v)
    ref.copy_blocks(kc, vc, pairs[:12])
    paged_ops.copy_blocks(k, v, torch.tensor(pairs, dtype=torch.int64, device=gpu) if where == "device" else pairs)
    torch.cuda.synchronize()
    assert np.array_equal(storage(k), kc)
    assert np.array_equal(storage(v), vc)


def test_copy_blocks_host_pairs_over_several_launches(gpu):
    """300 host pairs (three launches of at most 128 pairs in the kernel arguments), ids past
    the int32 range and negative ones skipped, against the oracle; then the same copy through
    PagedKVCache.copy_blocks with a list and with a CPU tensor."""
    from engine import paged_ops
    from engine.kv_cache import PagedKVCache

    announce("copy_blocks_host: 300 pairs, 3 launches")
    g = torch.Generator().manual_seed(8)
    layers, nb, hkv, bs, d = 2, 700, 2, 16, 64
    k = torch.randn(layers, nb + 1, hkv, bs, d, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(layers, nb + 1, hkv, bs, d, generator=g).to(torch.bfloat16).to(gpu)
    ids = random.Random(9).sample(range(nb + 1), 600)
    pairs = [(ids[i], ids[i + 300]) for i in range(300)]
    pairs[5] = (pairs[5][0], 1 << 40)   # skipped: past the pool (and past int32)
    pairs[200] = (-3, pairs[200][1])    # skipped
    kc, vc = storage(k), storage(v)
    ref.copy_blocks(kc, vc, [p for i, p in enumerate(pairs) if i not in (5, 200)])
    paged_ops.copy_blocks(k, v, np.asarray(pairs, dtype=np.int64))
    torch.cuda.synchronize()
    assert np.array_equal(storage(k), kc)
    assert np.array_equal(storage(v), vc)

    cache = PagedKVCache(num_layers=layers, num_kv_heads=hkv, head_dim=d, num_blocks=nb, block_size=bs, max_seqs=4,
                         max_len=64, dtype=torch.bfloat16, device=gpu)
    cache.k.copy_(k)
    cache.v.copy_(v)
    more = [(ids[i], ids[i + 1]) for i in range(0, 20, 2)]
    kc2, vc2 = storage(cache.k), storage(cache.v)
    ref.copy_blocks(kc2, vc2, more)
    cache.copy_blocks(more[:5])
    cache.copy_blocks(torch.tensor(more[5:], dtype=torch.int64))
    torch.cuda.synchronize()
    assert np.array_equal(storage(cache.k), kc2)
    assert np.array_equal(storage(cache.v), vc2)


def test_copy_blocks_device_pairs_over_several_launches(gpu):
    """A device-pairs call with more (pair, layer, K|V) units than one launch's grid may hold
    (2^24 - 1 workgroups of 256 threads): 2^22 + 1 pairs at 2 layers is split into two launches,
    and every destination block equals its source afterwards."""
    from engine import paged_ops

    announce("copy_blocks device pairs: 2^22 + 1 pairs x 2 layers, two launches")
    n = (1 << 22) + 1
    layers, nb = 2, 2 * n
    g = torch.Generator(device=gpu).manual_seed(10)
    k = torch.randn(layers, nb + 1, 1, 1, 4, generator=g, device=gpu)  # 16-byte blocks
    v = torch.randn(layers, nb + 1, 1, 1, 4, generator=g, device=gpu)
    src = torch.arange(n, dtype=torch.int64, device=gpu)
    pairs = torch.stack([src, src + n], dim=1).contiguous()
    k_src, v_src = k[:, :n].clone(), v[:, :n].clone()
    k_tail, v_tail = k[:, 2 * n:].clone(), v[:, 2 * n:].clone()
    paged_ops.copy_blocks(k, v, pairs)
    torch.cuda.synchronize()
    assert torch.equal(k[:, n:2 * n], k_src) and torch.equal(v[:, n:2 * n], v_src)
    assert torch.equal(k[:, :n], k_src) and torch.equal(v[:, :n], v_src)
    assert torch.equal(k[:, 2 * n:], k_tail) and torch.equal(v[:, 2 * n:], v_tail)
    del k, v, pairs, k_src, v_src
    torch.cuda.empty_cache()


# ----------------------------------------------------------------------------- paged decode attention


def _random_case(dtype, batch, hq, hkv, d, bs, lens, nb_extra=3, seed=0, stale=None):
    """Pool with scattered tables; returns device tensors and the CPU float pools for the oracle."""
    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(seed)
    need = [math.ceil(n / bs) for n in lens]
    nb = sum(need) + nb_extra
    perm = list(range(nb))
    random.Random(seed + 1).shuffle(perm)
    tables, cur = [], 0
    for n in need:
        tables.append(perm[cur:cur + n])
        cur += n
    width = max(max(need), 1)
    bt = np.zeros((batch, width + 2), dtype=np.int32)  # extra columns never read
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    k_pool = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt)
    v_pool = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt)
    if stale is not None:
        # Poison every row that no query may read: padding, tails of last blocks, free blocks.
        live = np.zeros((nb + 1, bs), dtype=bool)
        for t, n in zip(tables, lens):
            for j in range(n):
                live[t[j // bs], j % bs] = True
        dead = torch.from_numpy(~live)
        k_pool[dead.nonzero(as_tuple=True)[0], :, dead.nonzero(as_tuple=True)[1]] = stale
        v_pool[dead.nonzero(as_tuple=True)[0], :, dead.nonzero(as_tuple=True)[1]] = stale
    q = torch.randn(batch, hq, d, generator=g).to(dt)
    return q, k_pool, v_pool, tables, bt, width


def _check_decode(gpu, dtype, batch, hq, hkv, d, bs, lens, seed=0, stale=None, max_blocks=None):
    from engine import paged_ops

    q, k_pool, v_pool, tables, bt, width = _random_case(dtype, batch, hq, hkv, d, bs, lens, seed=seed, stale=stale)
    mb = width if max_blocks is None else max_blocks
    out = paged_ops.paged_decode(q.to(gpu), k_pool.to(gpu), v_pool.to(gpu), torch.from_numpy(bt).to(gpu),
                                 torch.tensor(lens, dtype=torch.int32, device=gpu), max_blocks=mb)
    torch.cuda.synchronize()
    want = ref.attention_f64(values(q), values(k_pool), values(v_pool), tables, lens, bs)
    got = values(out)
    assert np.isfinite(got).all()
    err = attention_error(got, want, dtype)
    assert err <= TOL[dtype], f"error beyond output rounding {err:.3g} > {TOL[dtype]}"
    return err


@pytest.fixture(params=["default", "valu", "mfma", "stream"])
def algo(request):
    """Which decode kernel the library runs (mip_set_decode_algo; ignored where a kernel does not apply)."""
    from engine import _native

    prev = _native.set_decode_algo("auto" if request.param == "default" else request.param)
    yield request.param
    _native.set_decode_algo(prev)


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("d,hq,hkv,bs", [(64, 14, 2, 16), (128, 28, 4, 32), (8, 4, 2, 4), (64, 8, 8, 16),
                                         (32, 6, 2, 8), (256, 8, 1, 16), (16, 5, 1, 2), (64, 14, 2, 4),
                                         (128, 16, 1, 8), (64, 24, 2, 64), (32, 11, 1, 16), (64, 13, 1, 16),
                                         (64, 27, 3, 16)])
def test_paged_decode_shapes(gpu, dtype, d, hq, hkv, bs, algo):
    announce(f"paged_decode {dtype} d={d} hq={hq} hkv={hkv} bs={bs} algo={algo}")
    lens = [1, bs - 1 if bs > 1 else 1, bs, bs + 1, 37, 511, 512, 513, 1200, 2049]
    _check_decode(gpu, dtype, len(lens), hq, hkv, d, bs, lens, seed=d + hq)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_paged_decode_never_reads_stale_rows(gpu, dtype, algo):
    """NaN in every row a query may not see (padding, last-block tails, free blocks) must not leak."""
    announce(f"paged_decode stale NaN {dtype} algo={algo}")
    lens = [3, 16, 17, 100, 700, 1500]
    _check_decode(gpu, dtype, len(lens), 14, 2, 64, 16, lens, seed=11, stale=float("nan"))


@pytest.mark.parametrize("dtype,d,hq,hkv,bs", [("bfloat16", 64, 14, 2, 16), ("float16", 128, 28, 4, 32),
                                               ("bfloat16", 64, 14, 2, 4), ("float32", 64, 14, 2, 16),
                                               ("bfloat16", 128, 16, 1, 8), ("float16", 64, 8, 8, 64)])
def test_fused_append_decode_equals_two_calls(gpu, dtype, d, hq, hkv, bs, algo):
    """mip_paged_decode_append == mip_kv_append then mip_paged_decode: pools and outputs bit-identical.

    Rows cover: the newest key in the first / middle / last row of its tile, a one-key
    sequence, an empty sequence, a padding row (slot -1) and a row whose slot is a free block
    (not the newest key's slot), which the fused kernel must write without redirecting.
    """
    from engine import paged_ops

    announce(f"fused append+decode {dtype} d={d} hq={hq} hkv={hkv} bs={bs} algo={algo}")
    lens = [1, bs, bs + 1, 37, 513, 1200, 2049, 5, 0, 64, 17]  # keys after the append (positions + 1)
    batch = len(lens)
    q, k_pool, v_pool, tables, bt, width = _random_case(dtype, batch, hq, hkv, d, bs, lens, nb_extra=4, seed=d + bs)
    nb = k_pool.shape[0] - 1
    used = {blk for t in tables for blk in t}
    free = [blk for blk in range(nb) if blk not in used]
    slots = []
    for b, n in enumerate(lens):
        if n == 0 or b == 7:
            slots.append(-1)                                  # no append for this row
        elif b == 9:
            slots.append(free[0] * bs + 3)                    # valid slot, but not the newest key's
        else:
            slots.append(tables[b][(n - 1) // bs] * bs + (n - 1) % bs)
    g = torch.Generator().manual_seed(99)
    dt = DTYPES[dtype]
    wide = torch.randn(batch, 3 * hkv * d, generator=g).to(dt).to(gpu)
    k_new = wide[:, hkv * d:2 * hkv * d].view(batch, hkv, d)  # strided view, as from a fused projection
    v_new = torch.randn(batch, hkv, d, generator=g).to(dt).to(gpu)
    slot_t = torch.tensor(slots, dtype=torch.int64, device=gpu)
    bt_t = torch.from_numpy(bt).to(gpu)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    qg = q.to(gpu)
    ka, va = k_pool.to(gpu), v_pool.to(gpu)
    kb, vb = ka.clone(), va.clone()
    paged_ops.kv_append(ka, va, k_new, v_new, slot_t)
    out_a = paged_ops.paged_decode(qg, ka, va, bt_t, lens_t, max_blocks=width)
    out_b = paged_ops.paged_decode_append(qg, k_new, v_new, kb, vb, slot_t, bt_t, lens_t, max_blocks=width)
    torch.cuda.synchronize()
    assert torch.equal(ka, kb) and torch.equal(va, vb), "pools differ"
    assert torch.equal(out_a, out_b), "outputs differ"
    want = ref.attention_f64(values(q), values(ka), values(va), tables, lens, bs)
    assert attention_error(values(out_b), want, dtype) <= TOL[dtype]


def _plan_restated(plan: np.ndarray, lens, tables, hkv, bs, cap):
    """Host restatement of the work plan from its header (T, W, offsets, slots per wavefront):
    wavefront ranges, segment descriptors for the merge and one descriptor per tile (pool row,
    sequence, kv head, valid keys, segment edges) in its wavefront's slots, in tile order."""
    u = plan.view(np.uint32)
    L = [min(max(n, 0), cap) for n in lens]
    tiles = [(n + 15) // 16 for n in L]
    pre = np.concatenate([[0], np.cumsum(tiles)]).astype(np.int64)
    T, W = int(plan[0]), int(plan[1])
    assert T == hkv * pre[-1] and plan[2] == len(lens) and plan[3] == hkv
    assert (T == 0) == (W == 0) and W <= T
    tile_off, seg_off, cap = int(plan[4]), int(plan[5]), int(plan[6])
    assert tile_off % 2 == 0 and seg_off >= 8 + 2 * W and tile_off >= seg_off + 4 * len(lens) * hkv
    tw = (seg_off - 8) // 2  # wavefront records reserved: one per wavefront of the grid
    assert plan.shape[0] >= tile_off + 2 * (tw * cap + 64) and W <= tw
    for g in range(W):
        assert list(plan[8 + 2 * g: 10 + 2 * g]) == [g * T // W, (g + 1) * T // W], g
        assert (g + 1) * T // W - g * T // W <= cap, g
    for b in range(len(lens)):
        for kvh in range(hkv):
            r = plan[seg_off + 4 * (b * hkv + kvh): seg_off + 4 * (b * hkv + kvh) + 4]
            if tiles[b] == 0:
                assert list(r) == [0, 0, 0, L[b]]
                continue
            s0 = hkv * pre[b] + kvh * tiles[b]
            e1 = s0 + tiles[b] - 1
            g_lo, g_hi = ((s0 + 1) * W - 1) // T, ((e1 + 1) * W - 1) // T
            assert list(r) == [g_lo, g_hi - g_lo + 1, int(g_lo * T // W < s0), L[b]]
            for t in range(tiles[b]):
                x = s0 + t
                g = ((x + 1) * W - 1) // T  # the wavefront whose range holds tile x
                assert g * T // W <= x < (g + 1) * T // W
                slot = g * cap + x - g * T // W
                blk = tables[b][16 * t // bs]
                row0 = (blk * hkv + kvh) * bs + (16 * t) % bs
                meta = b | kvh << 16 | min(16, L[b] - 16 * t) << 24 | int(t == 0) << 29 | int(t == tiles[b] - 1) << 30
                assert [int(u[tile_off + 2 * slot]), int(u[tile_off + 2 * slot + 1])] == [row0, meta], (b, kvh, t)


@pytest.mark.parametrize("dtype,d,hq,hkv,bs", [("bfloat16", 64, 14, 2, 16), ("float16", 128, 28, 4, 32),
                                               ("bfloat16", 64, 14, 2, 4), ("bfloat16", 128, 16, 1, 8)])
def test_decode_plan(gpu, dtype, d, hq, hkv, bs):
    """The per-step work plan: its contents vs the host restatement; decode and fused calls
    with the plan bit-identical to the same calls deriving the split in-kernel."""
    from engine import paged_ops

    announce(f"decode plan {dtype} d={d} hq={hq} hkv={hkv} bs={bs}")
    lens = [1, bs, bs + 1, 37, 513, 1200, 2049, 5, 0, 64, 17, 3000]
    batch = len(lens)
    q, k_pool, v_pool, tables, bt, width = _random_case(dtype, batch, hq, hkv, d, bs, lens, seed=5 * d + bs)
    bt_t = torch.from_numpy(bt).to(gpu)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    plan = paged_ops.decode_plan(lens_t, bt_t, hq, hkv, d, bs, DTYPES[dtype], max_blocks=width)
    if bs < 16:  # tiles span several blocks: no plan (the calls derive their split themselves)
        assert plan is None
        return
    assert plan is not None
    torch.cuda.synchronize()
    _plan_restated(plan.cpu().numpy(), lens, tables, hkv, bs, width * bs)
    qg, kg, vg = q.to(gpu), k_pool.to(gpu), v_pool.to(gpu)
    out0 = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width)
    out1 = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(out0, out1)
    # fused append + decode with the plan vs without
    g = torch.Generator().manual_seed(3)
    k_new = torch.randn(batch, hkv, d, generator=g).to(DTYPES[dtype]).to(gpu)
    v_new = torch.randn(batch, hkv, d, generator=g).to(DTYPES[dtype]).to(gpu)
    slots = torch.tensor([tables[b][(n - 1) // bs] * bs + (n - 1) % bs if n > 0 else -1 for b, n in enumerate(lens)],
                         dtype=torch.int64, device=gpu)
    ka, va, kb, vb = kg.clone(), vg.clone(), kg.clone(), vg.clone()
    fa = paged_ops.paged_decode_append(qg, k_new, v_new, ka, va, slots, bt_t, lens_t, max_blocks=width)
    fb = paged_ops.paged_decode_append(qg, k_new, v_new, kb, vb, slots, bt_t, lens_t, max_blocks=width, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(fa, fb) and torch.equal(ka, kb) and torch.equal(va, vb)


def test_paged_decode_edge_batches(gpu):
    """A batch above the stream kernel's limit (falls back to the partition kernel), one long
    sequence (32k keys, many pieces per segment), and lengths beyond max_blocks * block_size
    (clamped, per the ABI)."""
    from engine import paged_ops

    announce("paged_decode B=4100 short contexts")
    lens = [(i * 37) % 60 + 1 for i in range(4100)]
    _check_decode(gpu, "bfloat16", len(lens), 14, 2, 64, 16, lens, seed=21)
    announce("paged_decode B=1 ctx 32768")
    _check_decode(gpu, "bfloat16", 1, 14, 2, 64, 16, [32768], seed=22)
    announce("paged_decode clamped context lengths")
    lens = [40, 100, 64]
    q, k_pool, v_pool, tables, bt, width = _random_case("float16", 3, 8, 2, 64, 16, lens, seed=23)
    mb = 3  # 48 keys: the first two sequences are clamped to 48
    out = paged_ops.paged_decode(q.to(gpu), k_pool.to(gpu), v_pool.to(gpu), torch.from_numpy(bt).to(gpu),
                                 torch.tensor(lens, dtype=torch.int32, device=gpu), max_blocks=mb)
    torch.cuda.synchronize()
    want = ref.attention_f64(values(q), values(k_pool), values(v_pool), tables, [min(n, 48) for n in lens], 16)
    assert attention_error(values(out), want, "float16") <= TOL["float16"]


@pytest.mark.parametrize("batch", [1, 8, 32, 33, 40])
def test_paged_decode_merge_streams(gpu, batch):
    """One long sequence among short ones: its segments split into many pieces. At batch 1
    and 8 (2 and 16 segments) the merge cuts a long segment into runs folded by a second
    kernel, at 32 (64 segments) it runs two streams per workgroup, at 33 and 40 one; all
    against float64, and the planned call bit-identical to the one deriving its split
    in-kernel."""
    from engine import paged_ops

    announce(f"paged_decode merge streams B={batch}")
    lens = [20000] + [17 + (i * 53) % 190 for i in range(batch - 1)]
    q, k_pool, v_pool, tables, bt, width = _random_case("bfloat16", batch, 14, 2, 64, 16, lens, seed=31 + batch)
    qg, kg, vg = q.to(gpu), k_pool.to(gpu), v_pool.to(gpu)
    bt_t = torch.from_numpy(bt).to(gpu)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    out0 = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width)
    plan = paged_ops.decode_plan(lens_t, bt_t, 14, 2, 64, 16, DTYPES["bfloat16"], max_blocks=width)
    out1 = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width, plan=plan)
    torch.cuda.synchronize()
    want = ref.attention_f64(values(q), values(k_pool), values(v_pool), tables, lens, 16)
    assert attention_error(values(out0), want, "bfloat16") <= TOL["bfloat16"]
    assert torch.equal(out0, out1)


@pytest.mark.parametrize("dtype,d,hq,hkv,bs,batch", [("bfloat16", 64, 14, 2, 16, 96), ("float16", 128, 28, 4, 32, 40),
                                                     ("bfloat16", 128, 16, 1, 16, 80), ("float16", 64, 8, 8, 64, 12),
                                                     ("bfloat16", 64, 14, 2, 16, 300)])
def test_decode_many_segments_planned(gpu, dtype, d, hq, hkv, bs, batch):
    """Planned calls of more than 64 segments (the one-stream merge, as at the benchmark shapes).

    Lengths include empty sequences, single keys, block edges and one long sequence whose
    segments split into hundreds of pieces (several merge chunks). Checked: the planned call
    bit-identical to the unplanned one, three planned calls in a row identical, against
    float64 with stale NaN rows planted, and the fused planned call equal to kv_append
    followed by the unplanned decode, pools and outputs bit for bit."""
    from engine import paged_ops

    announce(f"planned decode, many segments {dtype} d={d} hq={hq} hkv={hkv} bs={bs} B={batch}")
    rng = random.Random(batch + d)
    lens = [0, 1, bs, bs + 1, 16, 17, 30000] + [rng.randint(1, 900) for _ in range(batch - 7)]
    q, k_pool, v_pool, tables, bt, width = _random_case(dtype, batch, hq, hkv, d, bs, lens, seed=batch + 7 * d,
                                                        stale=float("nan"))
    qg, kg, vg = q.to(gpu), k_pool.to(gpu), v_pool.to(gpu)
    bt_t = torch.from_numpy(bt).to(gpu)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    plan = paged_ops.decode_plan(lens_t, bt_t, hq, hkv, d, bs, DTYPES[dtype], max_blocks=width)
    assert plan is not None
    out0 = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width)
    outs = [paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width, plan=plan) for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, out0)
    want = ref.attention_f64(values(q), values(k_pool), values(v_pool), tables, lens, bs)
    got = values(out0)
    assert np.isfinite(got).all()
    assert attention_error(got, want, dtype) <= TOL[dtype]
    # fused: the planned call against kv_append + the unplanned decode
    g = torch.Generator().manual_seed(batch)
    k_new = torch.randn(batch, hkv, d, generator=g).to(DTYPES[dtype]).to(gpu)
    v_new = torch.randn(batch, hkv, d, generator=g).to(DTYPES[dtype]).to(gpu)
    slots = torch.tensor([tables[b][(n - 1) // bs] * bs + (n - 1) % bs if n > 0 else -1 for b, n in enumerate(lens)],
                         dtype=torch.int64, device=gpu)
    ka, va, kb, vb = kg.clone(), vg.clone(), kg.clone(), vg.clone()
    paged_ops.kv_append(ka, va, k_new, v_new, slots)
    fa = paged_ops.paged_decode(qg, ka, va, bt_t, lens_t, max_blocks=width)
    fb = paged_ops.paged_decode_append(qg, k_new, v_new, kb, vb, slots, bt_t, lens_t, max_blocks=width, plan=plan)
    torch.cuda.synchronize()
    # bit patterns: the planted NaN rows compare unequal as values
    assert np.array_equal(storage(ka), storage(kb)) and np.array_equal(storage(va), storage(vb)), "pools differ"
    assert torch.equal(fa, fb), "outputs differ"


def test_paged_decode_large_logits_rescale(gpu):
    """Scores spanning hundreds of units exercise the lazy running-max rescale."""
    from engine import paged_ops

    announce("paged_decode large logits")
    lens = [50, 600, 1800]
    q, k_pool, v_pool, tables, bt, width = _random_case("float32", 3, 14, 2, 64, 16, lens, seed=12)
    q = q * 40.0
    ramp = torch.linspace(-3, 3, k_pool.shape[0]).view(-1, 1, 1, 1)
    k_pool = k_pool * ramp
    out = paged_ops.paged_decode(q.to(gpu), k_pool.to(gpu), v_pool.to(gpu), torch.from_numpy(bt).to(gpu),
                                 torch.tensor(lens, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    want = ref.attention_f64(values(q), values(k_pool), values(v_pool), tables, lens, 16)
    assert np.abs(values(out) - want).max() < 1e-4


def test_paged_decode_config1_golden(gpu):
    """Config 1 (fp32, B=8, 14q/2kv, D=64, pool 512x16): append then attention, vs the reference path."""
    from engine import workloads

    announce("config1 decode step fp32")
    batch = workloads.build_decode_batch(workloads.SHAPES[1], gpu, seed=0)
    cache = batch.cache
    q, k, v = workloads.step_inputs(batch, seed=0)
    k_cpu, v_cpu = cache.k[0].cpu().clone(), cache.v[0].cpu().clone()
    tables = [list(cache.block_tables[s]) for s in batch.slots]
    inputs = ref.decode_inputs(batch.ctx, tables, cache.block_size)
    want_t = ref.paged_decode_torch(q.cpu(), k_cpu, v_cpu, k.cpu(), v.cpu(), inputs)
    ctx = cache.decode_context(batch.slots)
    got = ctx.attend(0, q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(cache.k[0].cpu(), k_cpu) and torch.equal(cache.v[0].cpu(), v_cpu)  # append bit-exact
    want64 = ref.attention_f64(values(q[:, :, 0]), k_cpu.numpy(), v_cpu.numpy(), tables, inputs["context_lens"], 16)
    assert np.abs(values(got[:, :, 0]) - want64).max() < 2e-5
    assert np.abs(values(got) - want_t.numpy()).max() < 2e-5


def test_paged_decode_golden_fixture(gpu):
    """The committed golden case (tests/golden): append + attention through the C ABI vs the fixture."""
    import json

    import cfg1
    from engine import paged_ops

    announce("golden fixture cfg1 fp32 decode step")
    meta = json.loads(cfg1.META.read_text())
    gold = np.load(cfg1.NPZ)
    inp = cfg1.make_inputs()
    assert cfg1.inputs_sha256(inp) == meta["inputs_sha256"]
    k_pool = torch.from_numpy(inp["k_pool"]).to(gpu)
    v_pool = torch.from_numpy(inp["v_pool"]).to(gpu)
    slot_mapping = torch.from_numpy(gold["slot_mapping"]).to(gpu)
    paged_ops.kv_append(k_pool, v_pool, torch.from_numpy(inp["k_new"]).to(gpu), torch.from_numpy(inp["v_new"]).to(gpu),
                        slot_mapping)
    nb = max(len(t) for t in inp["tables"])
    tables = np.zeros((cfg1.BATCH, nb), dtype=np.int32)
    for i, t in enumerate(inp["tables"]):
        tables[i, :len(t)] = t
    out = paged_ops.paged_decode(torch.from_numpy(inp["q"]).to(gpu), k_pool, v_pool, torch.from_numpy(tables).to(gpu),
                                 torch.from_numpy(gold["context_lens"]).to(gpu))
    torch.cuda.synchronize()
    blocks = cfg1.touched_blocks(inp["tables"])
    assert cfg1.blocks_sha256(k_pool.cpu().numpy(), v_pool.cpu().numpy(), blocks) == meta["pool_after_append_sha256"]
    assert np.abs(values(out) - gold["out"]).max() < 2e-5


@pytest.mark.parametrize("cfg", [2, 3, 5])
def test_decode_step_full_size(gpu, cfg):
    """Configs 2 (fp16 B=32), 3 (bf16 B=256, churned pool) and 5 (bf16 28q/4kv D=128 BS=32 B=128,
    tables permuted over one layer of the 94k-block pool): one layer's append + attention vs
    float64."""
    from engine import workloads

    announce(f"config{cfg} decode step")
    shape = workloads.SHAPES[cfg]
    small = workloads.DecodeShape(**{**shape.__dict__, "num_layers": 1})
    batch = workloads.build_decode_batch(small, gpu, seed=0)
    cache = batch.cache
    q, k, v = workloads.step_inputs(batch, seed=1)
    ctx = cache.decode_context(batch.slots)
    out = ctx.attend(0, q, k, v)
    torch.cuda.synchronize()
    # The oracle reads a compact copy of the blocks the batch owns (config 5's pool is 94k blocks).
    used = sorted({b for s in batch.slots for b in cache.block_tables[s]})
    remap = {b: i for i, b in enumerate(used)}
    tables = [[remap[b] for b in cache.block_tables[s]] for s in batch.slots]
    idx = torch.tensor(used, device=gpu)
    kp, vp = values(cache.k[0].index_select(0, idx)), values(cache.v[0].index_select(0, idx))
    lens = [n + 1 for n in batch.ctx]
    # the append wrote the new rows where the reference index math says
    inputs = ref.decode_inputs(batch.ctx, tables, cache.block_size)
    assert np.array_equal(kp[inputs["write_blocks"], :, inputs["write_offsets"]], values(k[:, :, 0]))
    assert np.array_equal(vp[inputs["write_blocks"], :, inputs["write_offsets"]], values(v[:, :, 0]))
    want = ref.attention_f64(values(q[:, :, 0]), kp, vp, tables, lens, cache.block_size)
    got = values(out[:, :, 0])
    err = np.abs(got - want).max()
    print(f"config{cfg} max-abs err {err:.3g}, max |out| {np.abs(want).max():.3g}")
    assert err <= 2e-3  # plain max-abs: at these context lengths |out| < 1, where half a bf16 ulp is <= 1.95e-3
    assert attention_error(got, want, dname(shape.dtype)) <= 2e-3


def test_prefix_fork_packed_append_copy_on_write(gpu):
    """Config 4: 64 forks of a 520-token prefix, packed append of their suffixes (about 17k
    tokens per layer) after copy-on-write of the shared partial block; every byte of both
    pools (2 layers) vs the oracle replaying the same copies and appends."""
    from engine import paged_ops, workloads

    announce("config4 prefix fork + packed append + copy-on-write")
    pb = workloads.build_prefix_batch(gpu, seed=0, num_layers=2)
    cache = pb.cache
    before_k, before_v = storage(cache.k), storage(cache.v)
    parent_table = list(cache.block_tables[pb.parent])
    assert len(parent_table) == 33 and all(cache.ref_count(b) == 65 for b in parent_table)
    ctx = cache.packed_prefill_context(pb.children, pb.suffix_lens)  # ensure_capacity + copy-on-write
    n_tok = sum(pb.suffix_lens)
    gen = torch.Generator().manual_seed(7)
    ks = [torch.randn(n_tok, 2, 64, generator=gen).to(torch.float16).to(gpu) for _ in range(2)]
    vs = [torch.randn(n_tok, 2, 64, generator=gen).to(torch.float16).to(gpu) for _ in range(2)]
    for layer in range(2):
        paged_ops.kv_append(cache.k[layer], cache.v[layer], ks[layer], vs[layer], ctx.slot_mapping)
    torch.cuda.synchronize()
    # bookkeeping: 32 full prefix blocks still shared by all, the partial one now private per fork
    for c in pb.children:
        t = cache.block_tables[c]
        assert t[:32] == parent_table[:32] and t[32] != parent_table[32]
    assert all(cache.ref_count(b) == 65 for b in parent_table[:32]) and cache.ref_count(parent_table[32]) == 1
    pairs = [(parent_table[32], cache.block_tables[c][32]) for c in pb.children]
    assert len({d for _, d in pairs}) == len(pairs)
    want_k, want_v = before_k.copy(), before_v.copy()
    ref.copy_blocks(want_k, want_v, pairs)
    blocks, offsets = ref.write_index(cache.block_tables, pb.children, [pb.prefix_len] * len(pb.children),
                                      pb.suffix_lens, cache.block_size)
    assert np.array_equal(blocks * cache.block_size + offsets, ctx.slot_mapping.cpu().numpy())
    for layer in range(2):
        ref.append(want_k[layer], want_v[layer], blocks, offsets, storage(ks[layer]), storage(vs[layer]))
    assert np.array_equal(storage(cache.k), want_k) and np.array_equal(storage(cache.v), want_v)


def test_decode_context_matches_per_sequence_sdpa(gpu):
    """Reference tests/test_kv_cache.py:179-207 restated on the GPU path."""
    from engine.kv_cache import PagedKVCache

    announce("decode context vs per-sequence sdpa")
    torch.manual_seed(0)
    cache = PagedKVCache(num_layers=1, num_kv_heads=2, head_dim=8, num_blocks=12, block_size=4, max_seqs=4,
                         max_len=32, dtype=torch.float32, device=gpu)
    heads, kv_heads, dim = 4, 2, 8
    lengths = [6, 9, 3]
    slots = [cache.allocate(0) for _ in lengths]
    for n_blocks in range(1, 4):
        for s, n in zip(slots, lengths):
            cache.ensure_capacity(s, min(n + 1, n_blocks * 4))
    keys_by_seq = []
    for s, n in zip(slots, lengths):
        k = torch.randn(1, kv_heads, n, dim, device=gpu)
        v = torch.randn(1, kv_heads, n, dim, device=gpu)
        ctx = cache.packed_prefill_context([s], [n])
        ctx.attend(0, torch.randn(1, heads, n, dim, device=gpu), k, v)
        ctx.commit()
        keys_by_seq.append((k, v))
    assert cache.block_tables[slots[0]] != list(range(cache.block_tables[slots[0]][0],
                                                      cache.block_tables[slots[0]][0] + 2))
    q = torch.randn(3, heads, 1, dim, device=gpu)
    k_new, v_new = torch.randn(3, kv_heads, 1, dim, device=gpu), torch.randn(3, kv_heads, 1, dim, device=gpu)
    ctx = cache.decode_context(slots)
    out = ctx.attend(0, q, k_new, v_new)
    for b, (k, v) in enumerate(keys_by_seq):
        full_k = torch.cat([k, k_new[b:b + 1]], dim=2).cpu()
        full_v = torch.cat([v, v_new[b:b + 1]], dim=2).cpu()
        want = ref.sdpa_attention(q[b:b + 1].cpu(), full_k, full_v)
        torch.testing.assert_close(out[b:b + 1].cpu(), want, rtol=1e-5, atol=1e-6)
    ctx.commit()
    assert [cache.lengths[s] for s in slots] == [7, 10, 4]


@torch.inference_mode()
def test_paged_decode_graph_replay(gpu):
    """Append + attention captured in a HIP graph: every replay equals the eager result."""
    from engine import paged_ops

    announce("graph capture append+decode")
    lens = [40, 700, 1300, 5]
    q, k_pool, v_pool, tables, bt, width = _random_case("bfloat16", 4, 14, 2, 64, 16, lens, seed=21)
    qg, kg, vg = q.to(gpu), k_pool.to(gpu), v_pool.to(gpu)
    btg = torch.from_numpy(bt).to(gpu)
    cl = torch.tensor(lens, dtype=torch.int32, device=gpu)
    slots = torch.tensor([tables[i][(n - 1) // 16] * 16 + (n - 1) % 16 for i, n in enumerate(lens)],
                         dtype=torch.int64, device=gpu)
    k_new = torch.randn(4, 2, 64, device=gpu).to(torch.bfloat16)
    v_new = torch.randn(4, 2, 64, device=gpu).to(torch.bfloat16)
    out = torch.empty_like(qg)
    ws = torch.empty(paged_ops.decode_workspace_bytes(4, 14, 2, 64, 16, width, torch.bfloat16), dtype=torch.uint8,
                     device=gpu)
    paged_ops.kv_append(kg, vg, k_new, v_new, slots)
    eager = paged_ops.paged_decode(qg, kg, vg, btg, cl, workspace=ws).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_ops.kv_append(kg, vg, k_new, v_new, slots)
        paged_ops.paged_decode(qg, kg, vg, btg, cl, out=out, workspace=ws)
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        _ = (qg.float() * 2).sum().item()  # unrelated eager work between replays


@torch.inference_mode()
def test_planned_fused_decode_graph_replay_config3_padded_matches_oracle(gpu):
    """The graphed decode's attention call at the config-3 shape (bf16, 14q/2kv heads d64,
    block 16, churned pool): 250 sequences padded to a bucket of 256 with rows on the scratch
    block, the step's plan and the fused append + attention captured in one graph. Every
    replay's outputs match the float64 oracle, and the pool (scratch block aside) equals the
    oracle's append of the new rows, bit for bit."""
    from engine import paged_ops, workloads

    announce("graph replay config-3 shape, 250 sequences in a 256 bucket, vs oracle")
    shape = workloads.DecodeShape(**{**workloads.SHAPES[3].__dict__, "num_layers": 1})
    batch = workloads.build_decode_batch(shape, gpu, seed=0)
    cache, bs = batch.cache, shape.block_size
    real, top = 250, 256
    slots = batch.slots[:real]
    ctx_lens = batch.ctx[:real]
    tables = [list(cache.block_tables[s]) for s in slots]
    nb = max(len(t) for t in tables)
    bt = np.full((top, nb), cache.scratch_block, dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    lens = np.ones(top, dtype=np.int32)
    lens[:real] = np.asarray(ctx_lens) + 1
    slot_map = np.full(top, cache.scratch_block * bs, dtype=np.int64)
    for i, (t, n) in enumerate(zip(tables, ctx_lens)):
        slot_map[i] = t[n // bs] * bs + n % bs
    gen = torch.Generator().manual_seed(31)
    q = torch.randn(top, 14, 64, generator=gen).to(torch.bfloat16).to(gpu)
    k_new = torch.randn(top, 2, 64, generator=gen).to(torch.bfloat16).to(gpu)
    v_new = torch.randn(top, 2, 64, generator=gen).to(torch.bfloat16).to(gpu)
    bt_t, lens_t = torch.from_numpy(bt).to(gpu), torch.from_numpy(lens).to(gpu)
    slot_t = torch.from_numpy(slot_map).to(gpu)
    k_layer, v_layer = cache.k[0], cache.v[0]
    k_before, v_before = storage(k_layer), storage(v_layer)
    ws = torch.empty(paged_ops.decode_workspace_bytes(top, 14, 2, 64, bs, nb, torch.bfloat16), dtype=torch.uint8,
                     device=gpu)
    out = torch.empty(top, 14, 64, dtype=torch.bfloat16, device=gpu)
    plan_call, plan = paged_ops.prepare_decode_plan(lens_t, bt_t, 14, 2, 64, bs, torch.bfloat16, max_blocks=nb)
    assert plan is not None
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_ops.decode_plan(lens_t, bt_t, 14, 2, 64, bs, torch.bfloat16, max_blocks=nb, plan=plan)
        paged_ops.paged_decode_append(q, k_new, v_new, k_layer, v_layer, slot_t, bt_t, lens_t, max_blocks=nb,
                                      workspace=ws, plan=plan, out=out)
    torch.cuda.synchronize()
    want_k, want_v = k_before.copy(), v_before.copy()
    ref.append(want_k, want_v, slot_map[:real] // bs, slot_map[:real] % bs, storage(k_new[:real]),
               storage(v_new[:real]))
    want = None
    sc = cache.scratch_block
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        kp, vp = storage(k_layer), storage(v_layer)
        assert np.array_equal(kp[:sc], want_k[:sc]) and np.array_equal(vp[:sc], want_v[:sc]), f"replay {i}: pool"
        if want is None:
            want = ref.attention_f64(values(q[:real]), values(k_layer), values(v_layer), tables,
                                     lens[:real].tolist(), bs)
        got = values(out[:real])
        err = attention_error(got, want, "bfloat16")
        assert np.isfinite(got).all() and err <= TOL["bfloat16"], f"replay {i}: {err}"
        _ = (q.float() * 2).sum().item()  # unrelated eager work between replays


@pytest.mark.parametrize("batch", [4, 70])
def test_mismatched_plan_fails_visibly(gpu, batch):
    """A plan made for another batch: the Python layer refuses it, and through the C ABI the
    call writes NaN to every output row and leaves the pool unchanged (no silent garbage).
    Batch 4 (8 segments) takes the two-stream merge with runs; batch 70 (140 segments) the
    one-stream merge."""
    from engine import paged_ops

    announce(f"decode with a plan of another batch size, B={batch}")
    lens = ([40, 700, 1300, 5] * 18)[:batch]
    q, k_pool, v_pool, tables, bt, width = _random_case("bfloat16", batch, 14, 2, 64, 16, lens, seed=23)
    qg, kg, vg = q.to(gpu), k_pool.to(gpu), v_pool.to(gpu)
    btg = torch.from_numpy(bt).to(gpu)
    cl = torch.tensor(lens, dtype=torch.int32, device=gpu)
    slots = torch.tensor([tables[i][(n - 1) // 16] * 16 + (n - 1) % 16 for i, n in enumerate(lens)],
                         dtype=torch.int64, device=gpu)
    k_new = torch.randn(batch, 2, 64, device=gpu).to(torch.bfloat16)
    v_new = torch.randn(batch, 2, 64, device=gpu).to(torch.bfloat16)
    lib = paged_ops._native.load()
    need4 = lib.mip_paged_decode_plan_bytes(batch, 14, 2, 64, 16, width, paged_ops.dtype_code(torch.bfloat16))
    need3 = lib.mip_paged_decode_plan_bytes(batch - 1, 14, 2, 64, 16, width, paged_ops.dtype_code(torch.bfloat16))
    buf = torch.zeros(-(-max(need4, need3) // 4), dtype=torch.int32, device=gpu)
    paged_ops.decode_plan(cl[:-1], btg[:-1], 14, 2, 64, 16, torch.bfloat16, max_blocks=width, plan=buf)
    with pytest.raises(ValueError, match="plan was made for"):
        paged_ops.paged_decode_append(qg, k_new, v_new, kg, vg, slots, btg, cl, max_blocks=width, plan=buf)
    del buf._mip_plan_key  # reach the library as a caller of the C ABI would
    before_k, before_v = kg.clone(), vg.clone()
    out = paged_ops.paged_decode_append(qg, k_new, v_new, kg, vg, slots, btg, cl, max_blocks=width, plan=buf)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all(), "a mismatched plan must not leave plausible outputs"
    assert torch.equal(kg, before_k) and torch.equal(vg, before_v), "a mismatched plan must not append"


@torch.inference_mode()
def test_eager_decode_context_device_tables_match_oracle(gpu):
    """The eager PagedDecodeContext on the device-resident tables: 40 steps over 8 sequences
    that cross block boundaries, a sequence freed and its slot reused at step 12, a fork with
    copy-on-write of its shared partial block at step 24. Each step's outputs match the float64
    oracle over the host tables, and the pool equals the oracle's append, bit for bit."""
    from engine.kv_cache import PagedKVCache

    announce("eager decode context, device tables under growth, slot reuse and fork, vs oracle")
    lengths = [13, 30, 47, 5, 62, 16, 31, 100]
    cache = PagedKVCache(1, 2, 64, num_blocks=160, block_size=16, max_seqs=16, max_len=512, dtype=torch.bfloat16,
                         device=gpu)
    slots = []
    for n in lengths:
        s = cache.allocate(n + 1)
        cache.lengths[s] = n
        slots.append(s)
    gen = torch.Generator(device=gpu).manual_seed(2)
    cache.k.normal_(0.0, 1.0, generator=gen)
    cache.v.normal_(0.0, 1.0, generator=gen)
    for step in range(40):
        if step == 12:
            cache.free(slots[3])
            s = cache.allocate(40)
            cache.lengths[s] = 33
            slots[3] = s
        if step == 24:
            cache.free(slots[5])
            slots[5] = cache.fork(slots[2])
        for s in slots:
            assert cache.ensure_capacity(s, cache.lengths[s] + 1)
        pos = [cache.lengths[s] for s in slots]
        ctx = cache.decode_context(slots)  # copy-on-write happens here
        tables = [list(cache.block_tables[s]) for s in slots]
        k_before, v_before = storage(cache.k[0]), storage(cache.v[0])
        q = torch.randn(8, 14, 1, 64, generator=gen, device=gpu).to(torch.bfloat16)
        k = torch.randn(8, 2, 1, 64, generator=gen, device=gpu).to(torch.bfloat16)
        v = torch.randn(8, 2, 1, 64, generator=gen, device=gpu).to(torch.bfloat16)
        out = ctx.attend(0, q, k, v)
        torch.cuda.synchronize()
        blocks = np.asarray([t[p // 16] for t, p in zip(tables, pos)])
        offs = np.asarray(pos) % 16
        ref.append(k_before, v_before, blocks, offs, storage(k[:, :, 0]), storage(v[:, :, 0]))
        assert np.array_equal(storage(cache.k[0]), k_before), f"step {step}: K pool"
        assert np.array_equal(storage(cache.v[0]), v_before), f"step {step}: V pool"
        want = ref.attention_f64(values(q[:, :, 0]), values(cache.k[0]), values(cache.v[0]), tables,
                                 [p + 1 for p in pos], 16)
        err = attention_error(values(out[:, :, 0]), want, "bfloat16")
        assert err <= TOL["bfloat16"], f"step {step}: {err}"
        ctx.commit()
    assert cache.cow_copies >= 1


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@torch.inference_mode()
def test_decode_context_layer_calls_equal_checked_calls(gpu, dtype):
    """PagedDecodeContext checks the step's shared arguments on its first layer call and then
    only swaps addresses (paged_ops.DecodeStepCalls). Over 4 layers, with a q layout change at
    layer 2 (re-checked) and back at layer 3, and one layer issued on a side stream, both
    protocols (attend; attend_rope) give outputs and pools bit-equal to the fully checked
    paged_ops calls on the same inputs."""
    from engine import paged_ops
    from engine.kv_cache import PagedKVCache
    from engine.model import rope_cos_sin

    announce(f"decode context layer calls vs checked calls, {dtype}")
    dt = DTYPES[dtype]
    lengths = [13, 30, 47, 5, 62, 16, 31, 100]
    cache = PagedKVCache(4, 2, 64, num_blocks=160, block_size=16, max_seqs=16, max_len=512, dtype=dt, device=gpu)
    slots = []
    for n in lengths:
        s = cache.allocate(n + 1)
        cache.lengths[s] = n
        slots.append(s)
    gen = torch.Generator(device=gpu).manual_seed(7)
    cache.k.normal_(0.0, 1.0, generator=gen)
    cache.v.normal_(0.0, 1.0, generator=gen)
    k0, v0 = cache.k.clone(), cache.v.clone()
    b = len(slots)
    qs = [torch.randn(b, 14, 1, 64, generator=gen, device=gpu).to(dt) for _ in range(4)]
    qs[2] = torch.randn(b, 14, 1, 128, generator=gen, device=gpu).to(dt)[..., :64]  # other strides
    ks = [torch.randn(b, 2, 1, 64, generator=gen, device=gpu).to(dt) for _ in range(4)]
    vs = [torch.randn(b, 2, 1, 64, generator=gen, device=gpu).to(dt) for _ in range(4)]
    side = torch.cuda.Stream(device=gpu)
    assert paged_ops._stream_ptr(gpu) == torch.cuda.current_stream(gpu).cuda_stream
    with torch.cuda.stream(side):
        assert paged_ops._stream_ptr(gpu) == side.cuda_stream

    def run_context(rope: bool):
        cache.k.copy_(k0)
        cache.v.copy_(v0)
        ctx = cache.decode_context(slots)
        cos, sin = rope_cos_sin(ctx.positions.unsqueeze(1), 64, 1e6, dt)
        outs = []
        for layer in range(4):
            q, k, v = qs[layer].clone(), ks[layer].clone(), vs[layer].clone()
            if layer == 2:  # keep the wider strides of this layer's q (clone() would compact them)
                q = torch.empty_strided(qs[2].shape, qs[2].stride(), dtype=dt, device=gpu).copy_(qs[2])
            if layer == 1:
                side.wait_stream(torch.cuda.current_stream(gpu))
                with torch.cuda.stream(side):
                    out = ctx.attend_rope(layer, q, k, v, cos, sin) if rope else ctx.attend(layer, q, k, v)
                torch.cuda.current_stream(gpu).wait_stream(side)
            else:
                out = ctx.attend_rope(layer, q, k, v, cos, sin) if rope else ctx.attend(layer, q, k, v)
            outs.append(out[:, :, 0].clone())
        torch.cuda.synchronize()
        return ctx, cos, sin, outs, cache.k.clone(), cache.v.clone()

    def run_checked(ctx, cos, sin, rope: bool):
        cache.k.copy_(k0)
        cache.v.copy_(v0)
        plan = ctx.plan(14, dt)
        outs = []
        for layer in range(4):
            q = torch.empty_strided(qs[layer].shape, qs[layer].stride(), dtype=dt, device=gpu).copy_(qs[layer])
            k, v = ks[layer].clone(), vs[layer].clone()
            kl, vl = cache.k[layer], cache.v[layer]
            if rope:
                paged_ops.rope_kv_append(q[:, :, 0], k[:, :, 0], v[:, :, 0], cos[:, 0, 0], sin[:, 0, 0], kl, vl,
                                         ctx.slot_mapping)
                out = paged_ops.paged_decode(q[:, :, 0], kl, vl, ctx.block_tables, ctx.context_lens, scale=ctx.scale,
                                             max_blocks=ctx.num_blocks, plan=plan)
            else:
                out = paged_ops.paged_decode_append(q[:, :, 0], k[:, :, 0], v[:, :, 0], kl, vl, ctx.slot_mapping,
                                                    ctx.block_tables, ctx.context_lens, scale=ctx.scale,
                                                    max_blocks=ctx.num_blocks, plan=plan)
            outs.append(out.clone())
        torch.cuda.synchronize()
        return outs, cache.k.clone(), cache.v.clone()

    for rope in (False, True):
        ctx, cos, sin, got, kg, vg = run_context(rope)
        assert ctx.calls._cached, "the layer calls went through the step's call cache"
        want, kw, vw = run_checked(ctx, cos, sin, rope)
        for layer in range(4):
            assert torch.equal(got[layer], want[layer]), f"rope={rope} layer {layer}: output"
        assert torch.equal(kg, kw) and torch.equal(vg, vw), f"rope={rope}: pools"
        assert not torch.equal(kg, k0), "the calls appended"

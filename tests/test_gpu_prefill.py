"""GPU parity of the paged prefill attention kernel (``mip_paged_prefill``) through the C ABI.

Bar: within 2e-3 beyond the output's own final rounding (half an ulp) of the float64 oracle
(oracle/paged_ref.py ``prefill_attention_f64``) on the same 16-bit inputs, as for decode;
2e-5 for fp32 (the VALU path). The cache context's output also matches the reference's own
formulation (prefix read-back + dense mask + SDPA, engine/kv_cache.py:262-294) evaluated by
the oracle on the CPU.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
MANTISSA_BITS = {"float16": 10, "bfloat16": 7, "float32": 23}
TOL = {"float16": 2e-3, "bfloat16": 2e-3, "float32": 2e-5}


def half_ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    ax = np.maximum(np.abs(x), np.finfo(np.float32).tiny)
    return 0.5 * np.exp2(np.floor(np.log2(ax)) - MANTISSA_BITS[dtype])


def build(gpu, dtype, d, hq, hkv, bs, starts, lengths, seed=0, stale_nan=False, extra_blocks=3, edit_v=None):
    """Scattered pool holding every sequence's keys 0..end-1; padded int32 tables; packed q.
    edit_v(v_pool, tables), if given, changes the host V pool before it is copied and checked."""
    rnd = random.Random(seed)
    ends = [a + n for a, n in zip(starts, lengths)]
    need = [(e + bs - 1) // bs for e in ends]
    nb = sum(need) + extra_blocks
    ids = list(range(nb))
    rnd.shuffle(ids)
    tables, cur = [], 0
    for k in need:
        tables.append(ids[cur:cur + k])
        cur += k
    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(seed)
    k_pool = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt)
    v_pool = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt)
    if stale_nan:  # rows past each sequence's last key must never be read
        for t, e in zip(tables, ends):
            last, used = t[-1], e - (len(t) - 1) * bs
            k_pool[last, :, used:] = float("nan")
            v_pool[last, :, used:] = float("nan")
    if edit_v is not None:
        edit_v(v_pool, tables)
    # q as the packed [N, Hq, D] view of a wider qkv row, like the model's projection output.
    n_all = sum(lengths)
    qkv = torch.randn(n_all, (hq + 2 * hkv) * d, generator=g).to(dt)
    q = qkv[:, :hq * d].view(n_all, hq, d)
    width = max(need) + 1
    tab = torch.full((len(lengths), width), 0, dtype=torch.int32)
    for i, t in enumerate(tables):
        tab[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    cu = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lengths), 0)
    dev = dict(q=qkv.to(gpu)[:, :hq * d].view(n_all, hq, d), k=k_pool.to(gpu), v=v_pool.to(gpu), tab=tab.to(gpu),
               cu=cu.to(gpu), st=torch.tensor(starts, dtype=torch.int32).to(gpu))
    want = ref.prefill_attention_f64(q.float().numpy(), k_pool.float().numpy(), v_pool.float().numpy(), tables,
                                     starts, lengths, bs)
    return dev, want


CASES = [
    ([0, 0, 0], [1, 17, 40]),             # fresh prompts, block-diagonal causal
    ([37, 0, 512, 3], [5, 33, 100, 1]),   # cached prefixes at unaligned positions
    ([16], [64]),                         # one sequence, block-aligned prefix
]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d,hq,hkv,bs", [(64, 14, 2, 16), (128, 28, 4, 32), (64, 8, 8, 16), (64, 16, 1, 16),
                                         (128, 7, 1, 4)])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_paged_prefill_matches_f64(gpu, dtype, d, hq, hkv, bs, case):
    from engine import paged_ops

    starts, lengths = CASES[case]
    announce(f"paged_prefill {dtype} d={d} hq={hq} hkv={hkv} bs={bs} starts={starts} lengths={lengths}")
    dev, want = build(gpu, dtype, d, hq, hkv, bs, starts, lengths, seed=case)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    err = float((np.abs(got - want) - half_ulp(want, dtype)).max())
    assert err <= 2e-3, err


@pytest.mark.parametrize("dtype,d,hq,hkv,bs", [("float32", 64, 14, 2, 16), ("float32", 128, 8, 2, 32),
                                               ("float16", 32, 8, 2, 16), ("bfloat16", 256, 4, 2, 16),
                                               ("float32", 8, 4, 4, 4), ("float16", 16, 5, 1, 2),
                                               ("float32", 64, 16, 1, 16), ("float16", 32, 24, 2, 8),
                                               ("bfloat16", 16, 11, 1, 16), ("float32", 64, 27, 3, 16)])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_paged_prefill_valu_shapes(gpu, dtype, d, hq, hkv, bs, case):
    """Shapes without an MFMA prefill kernel (fp32, head sizes other than 64/128) run the VALU
    decode kernel, one workgroup per (new token, kv head, group of at most 8 query heads: 16 =
    2 x 8, 12 = 2 x 6, 11 = 6 + 5, 9 = 5 + 4 with the last workgroup masking a head slot);
    same bar against float64."""
    from engine import paged_ops

    starts, lengths = CASES[case]
    announce(f"paged_prefill VALU {dtype} d={d} hq={hq} hkv={hkv} bs={bs} starts={starts} lengths={lengths}")
    dev, want = build(gpu, dtype, d, hq, hkv, bs, starts, lengths, seed=case + 40)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    err = float((np.abs(got - want) - half_ulp(want, dtype)).max())
    assert err <= TOL[dtype], err


def test_paged_prefill_valu_stale_rows_and_loose_grid(gpu):
    """VALU path: NaN rows past every sequence's keys never leak; a loose max_q_len and an empty
    sequence write nothing extra."""
    from engine import paged_ops

    announce("paged_prefill VALU fp32 stale NaN rows, loose max_q_len, empty sequence")
    starts, lengths = [21, 0, 7, 3], [11, 29, 0, 2]
    dev, want = build(gpu, "float32", 64, 14, 2, 16, starts, lengths, seed=8, stale_nan=True)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], 100)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert float((np.abs(got - want) - half_ulp(want, "float32")).max()) <= TOL["float32"]


def test_paged_prefill_unsupported_shape_raises(gpu):
    """No kernel for a head size that is not a power of two: the call raises (no fallback)."""
    from engine import _native, paged_ops

    announce("paged_prefill fp32 head_dim 96: unsupported")
    dev, _ = build(gpu, "float32", 96, 16, 1, 16, [0], [4], seed=1)
    with pytest.raises(_native.NativeError, match="unsupported"):
        paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], 4)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_paged_prefill_never_reads_stale_rows(gpu, dtype):
    from engine import paged_ops

    announce(f"paged_prefill stale NaN rows {dtype}")
    starts, lengths = [21, 0, 7], [11, 29, 2]
    dev, want = build(gpu, dtype, 64, 14, 2, 16, starts, lengths, seed=7, stale_nan=True)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert float((np.abs(got - want) - half_ulp(want, dtype)).max()) <= 2e-3


def test_paged_prefill_max_q_len_larger_than_needed_and_empty_sequences(gpu):
    """Extra grid blocks (a loose max_q_len) and sequences with no new tokens write nothing."""
    from engine import paged_ops

    announce("paged_prefill loose max_q_len, empty sequences")
    starts, lengths = [4, 9, 0], [6, 0, 3]
    dev, want = build(gpu, "bfloat16", 64, 14, 2, 16, starts, lengths, seed=9)
    out = torch.full((sum(lengths), 14, 64), 7.0, dtype=torch.bfloat16, device=gpu)
    paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], 200, out=out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert float((np.abs(got - want) - half_ulp(want, "bfloat16")).max()) <= 2e-3


def test_paged_prefill_config4_prefix_hits(gpu):
    """Config 4's prefill: 64 requests on a 512-token cached prefix + suffix U[32, 512], fp16,
    Qwen2.5-0.5B attention shape; rows of 8 sampled sequences checked against float64."""
    from engine import paged_ops

    announce("paged_prefill config 4 (64 x (512 prefix + U[32,512]) fp16)")
    rnd = random.Random(4)
    lengths = [rnd.randint(32, 512) for _ in range(64)]
    starts = [512] * 64
    dtype, d, hq, hkv, bs = "float16", 64, 14, 2, 16
    # Full-size inputs (the oracle runs on a sample of sequences).
    ends = [a + n for a, n in zip(starts, lengths)]
    need = [(e + bs - 1) // bs for e in ends]
    nb = sum(need) + 8
    ids = list(range(nb))
    rnd.shuffle(ids)
    tables, cur = [], 0
    for k in need:
        tables.append(ids[cur:cur + k])
        cur += k
    g = torch.Generator(device=gpu).manual_seed(11)
    k_pool = torch.randn(nb + 1, hkv, bs, d, generator=g, device=gpu).half()
    v_pool = torch.randn(nb + 1, hkv, bs, d, generator=g, device=gpu).half()
    n_all = sum(lengths)
    qkv = torch.randn(n_all, (hq + 2 * hkv) * d, generator=g, device=gpu).half()
    q = qkv[:, :hq * d].view(n_all, hq, d)
    tab = torch.zeros(64, max(need), dtype=torch.int32)
    for i, t in enumerate(tables):
        tab[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    cu = torch.zeros(65, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lengths), 0)
    out = paged_ops.paged_prefill(q, k_pool, v_pool, tab.to(gpu), cu.to(gpu), torch.tensor(starts, dtype=torch.int32,
                                  device=gpu), max(lengths))
    torch.cuda.synchronize()
    kp, vp = k_pool.float().cpu().numpy(), v_pool.float().cpu().numpy()
    qc, oc = q.float().cpu().numpy(), out.float().cpu().numpy()
    for s in (0, 5, 17, 30, 41, 50, 58, 63):
        r0, r1 = int(cu[s]), int(cu[s + 1])
        want = ref.prefill_attention_f64(qc[r0:r1], kp, vp, [tables[s]], [starts[s]], [lengths[s]], bs)
        err = float((np.abs(oc[r0:r1] - want) - half_ulp(want, dtype)).max())
        assert err <= 2e-3, (s, err)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("prefix", [False, True])
@torch.inference_mode()
def test_prefill_context_matches_reference_formulation(gpu, prefix, dtype):
    """PackedPrefillContext.attend (append + paged prefill kernel) against the reference's own
    formulation, prefix read-back + dense mask + SDPA (engine/kv_cache.py:262-294), which the
    oracle evaluates in fp32 on the CPU over the pool the context appended to."""
    from engine.kv_cache import PagedKVCache

    announce(f"prefill context vs the reference formulation, prefix={prefix} {dtype}")
    dt, d, hq, hkv, bs = DTYPES[dtype], 64, 14, 2, 16
    starts = [40, 0, 17] if prefix else [0, 0, 0]
    new = [23, 50, 9]
    cache = PagedKVCache(1, hkv, d, num_blocks=64, block_size=bs, max_seqs=4, max_len=256, dtype=dt, device=gpu)
    slots = []
    for st, n in zip(starts, new):
        s = cache.allocate(st + n)
        cache.lengths[s] = st
        slots.append(s)
    gen = torch.Generator(device=gpu).manual_seed(5)
    cache.k.normal_(0.0, 1.0, generator=gen)
    cache.v.normal_(0.0, 1.0, generator=gen)
    ctx = cache.packed_prefill_context(slots, new)
    n = sum(new)
    qkv = torch.randn(1, n, (hq + 2 * hkv) * d, generator=gen, device=gpu).to(dt)
    q, k, v = qkv.split([hq * d, hkv * d, hkv * d], dim=-1)
    q = q.view(1, n, hq, d).transpose(1, 2)
    k = k.view(1, n, hkv, d).transpose(1, 2)
    v = v.view(1, n, hkv, d).transpose(1, 2)
    got = ctx.attend(0, q, k, v).float().cpu()
    torch.cuda.synchronize()
    tables = [list(cache.block_tables[s]) for s in slots]
    want = ref.packed_prefill_torch(q.float().cpu(), cache.k[0].float().cpu(), cache.v[0].float().cpu(), tables,
                                    starts, new, bs)
    w = want.numpy()
    err = float((np.abs(got.numpy() - w) - half_ulp(w, dtype)).max())
    assert err <= TOL[dtype], err
    ctx.commit()
    assert [cache.lengths[s] for s in slots] == [a + b for a, b in zip(starts, new)]


def _long_sequence_rows(gpu, rnd, start, n, seed, dtype="bfloat16"):
    """One sequence of n new tokens after start cached ones (14q/2kv, d64, block 16); rows
    sampled at the ends and in the middle against float64."""
    from engine import paged_ops

    d, hq, hkv, bs = 64, 14, 2, 16
    nblk = (start + n + bs - 1) // bs
    ids = list(range(nblk + 4))
    rnd.shuffle(ids)
    table = ids[:nblk]
    g = torch.Generator(device=gpu).manual_seed(seed)
    tdt = getattr(torch, dtype)
    k_pool = torch.randn(nblk + 5, hkv, bs, d, generator=g, device=gpu).to(tdt)
    v_pool = torch.randn(nblk + 5, hkv, bs, d, generator=g, device=gpu).to(tdt)
    qkv = torch.randn(n, (hq + 2 * hkv) * d, generator=g, device=gpu).to(tdt)
    q = qkv[:, :hq * d].view(n, hq, d)
    tab = torch.tensor([table], dtype=torch.int32, device=gpu)
    cu = torch.tensor([0, n], dtype=torch.int32, device=gpu)
    out = paged_ops.paged_prefill(q, k_pool, v_pool, tab, cu, torch.tensor([start], dtype=torch.int32, device=gpu), n)
    torch.cuda.synchronize()
    kp, vp = k_pool.float().cpu().numpy(), v_pool.float().cpu().numpy()
    qc, oc = q.float().cpu().numpy(), out.float().cpu().numpy()
    for r0 in (0, 31, n // 2, n - 200, n - 33):
        rows = slice(r0, r0 + 32)
        want = ref.prefill_attention_f64(qc[rows], kp, vp, [table], [start + r0], [32], bs)
        err = float((np.abs(oc[rows] - want) - half_ulp(want, dtype)).max())
        assert err <= 2e-3, (n, r0, err)


def test_paged_prefill_grid_fallbacks(gpu):
    """The one-workgroup-per-item grid, taken past the persistent kernel's work-list limits:
    more than 1024 sequences, and one sequence with more than 255 blocks of new tokens (rows
    of the long one sampled against float64)."""
    from engine import paged_ops

    announce("paged_prefill 1100 short sequences (per-item grid)")
    rnd = random.Random(13)
    lengths = [rnd.randint(1, 3) for _ in range(1100)]
    starts = [rnd.randint(0, 40) for _ in range(1100)]
    dev, want = build(gpu, "float16", 64, 14, 2, 16, starts, lengths, seed=13)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert float((np.abs(got - want) - half_ulp(want, "float16")).max()) <= 2e-3

    # 9,300 tokens at 36 per work item (14q/2kv) are 259 blocks: past the persistent list's 255.
    announce("paged_prefill one sequence of 9300 new tokens after 100 cached (per-item grid)")
    _long_sequence_rows(gpu, rnd, 100, 9300, seed=17)


def test_paged_prefill_persistent_limits(gpu):
    """The persistent kernel exactly at its work-list limits: 1024 sequences (the largest
    index of the sequence arrays), and one sequence of 255 blocks of 36 new tokens (the top
    level of the block histogram)."""
    from engine import paged_ops

    announce("paged_prefill 1024 short sequences (persistent grid, sequence limit)")
    rnd = random.Random(29)
    lengths = [rnd.randint(1, 3) for _ in range(1024)]
    starts = [rnd.randint(0, 40) for _ in range(1024)]
    dev, want = build(gpu, "float16", 64, 14, 2, 16, starts, lengths, seed=29)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert float((np.abs(got - want) - half_ulp(want, "float16")).max()) <= 2e-3

    announce("paged_prefill one sequence of 9180 new tokens after 100 cached (persistent grid, 255 blocks)")
    _long_sequence_rows(gpu, rnd, 100, 255 * 36, seed=31, dtype="float16")


# bf16 V is staged as fp16 (exact up to 65280, the largest bf16 value below 65536); an item
# that reaches a larger magnitude runs again with bf16 V and a split P. (planted values,
# sequences (starts, lengths), (d, hq, hkv, bs)): the largest values that convert; values that
# force the second pass, in one sequence of several and in many; the per-item grid (1100
# sequences) with values that force it; head_dim 128.
_RND = random.Random(41)
_D64 = (64, 14, 2, 16)
BF16_RANGE_CASES = [
    ([65280.0, -65280.0], ([37, 0, 512, 3], [5, 33, 100, 1]), _D64),
    ([1.0e5, -3.0e4], ([37, 0, 512, 3], [5, 33, 100, 1]), _D64),
    ([1.0e30, -7.0e5, 70000.0], ([_RND.randint(0, 300) for _ in range(40)], [_RND.randint(1, 200) for _ in range(40)]),
     _D64),
    ([2.0e5, -65536.0], ([_RND.randint(0, 40) for _ in range(1100)], [_RND.randint(1, 3) for _ in range(1100)]), _D64),
    ([65280.0, 1.0e5], ([37, 0, 512, 3], [5, 33, 100, 1]), (128, 28, 4, 32)),
]


@pytest.mark.parametrize("case", range(len(BF16_RANGE_CASES)))
def test_paged_prefill_bf16_values_beyond_fp16(gpu, case):
    """Values near and beyond fp16's range in a bf16 V pool, against float64: every output
    finite, and within 2e-3 + 2^-11 M beyond half an ulp, M the largest planted magnitude
    (P is rounded to 16 bits, 2^-11 relative at fp16, which moves an output by at most
    2^-11 times the values' spread; the 2e-3 bound is for values of unit scale)."""
    from engine import paged_ops

    values, (starts, lengths), (d, hq, hkv, bs) = BF16_RANGE_CASES[case]
    rnd = random.Random(100 + case)
    # Only the first of several sequences gets the planted values, unless there is just one
    # kind of case to show (many sequences: spread over all of them).
    few = len(lengths) <= 4

    def plant(v_pool, tables):
        chosen = tables[:1] if few else tables
        for i in range(24):
            t = rnd.choice(chosen)
            v_pool[rnd.choice(t), rnd.randrange(hkv), rnd.randrange(bs), rnd.randrange(d)] = values[i % len(values)]

    announce(f"paged_prefill bf16 V values {values}, {len(lengths)} sequences")
    dev, want = build(gpu, "bfloat16", d, hq, hkv, bs, starts, lengths, seed=200 + case, edit_v=plant)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert np.abs(want).max() > 1000.0  # some planted value reaches an output
    err = float((np.abs(got - want) - half_ulp(want, "bfloat16")).max())
    assert err <= TOL["bfloat16"] + 2.0 ** -11 * max(abs(x) for x in values), err


# Work lists whose last, partial round of the persistent grid takes each form on a device of
# 512 resident workgroups (256 CUs, two each): (starts, lengths, hq, hkv, d, bs).
LAST_ROUND_CASES = [
    ([0] * 58, [252] * 58, 14, 2, 64, 16),    # 812 items: one whole round, then 212 items halved + 88 whole
    ([100] * 64, [288] * 64, 14, 2, 64, 16),  # 1024 items: two whole rounds, nothing left over
    ([7] * 30, [36] * 30, 14, 2, 64, 16),     # 60 items, all halved (grid of 120)
    ([0] * 21, [200] * 21, 10, 2, 64, 16),    # group 5: 51 tokens per item do not fit two halves of 25
    ([40] * 9, [130] * 9, 28, 4, 128, 32),    # head_dim 128: items of 18 tokens in halves of 9
]


@pytest.mark.parametrize("case", range(len(LAST_ROUND_CASES)))
def test_paged_prefill_last_round_pieces(gpu, case):
    """The persistent kernel cuts items of its last, partial round into two halves of half the
    rows where workgroups would otherwise idle; every row of every sequence is checked against
    float64, whichever way its item ran."""
    from engine import paged_ops

    starts, lengths, hq, hkv, d, bs = LAST_ROUND_CASES[case]
    announce(f"paged_prefill last-round pieces: {len(lengths)} x {lengths[0]} after {starts[0]}, hq={hq} hkv={hkv} d={d}")
    dev, want = build(gpu, "float16", d, hq, hkv, bs, starts, lengths, seed=40 + case)
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"], max(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert float((np.abs(got - want) - half_ulp(want, "float16")).max()) <= 2e-3

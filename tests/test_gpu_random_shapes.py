"""Seeded random shapes through the C ABI against the float64 oracle.

Decode attention (planned where the stream kernel runs, and unplanned), the fused append +
decode call, and packed prefill, over dtypes, head sizes, query groups (groups of more than
8 heads included, which the VALU kernel splits over workgroups), block sizes, batch sizes,
empty sequences, sequences at their table's capacity and q / k / v taken as strided views of
a fused projection. Every draw is printed before it runs. Bar: attention within TOL beyond
the output's own rounding; pools after the fused call bit-exact against the oracle append.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import paged_ref as ref
from test_gpu_kernels import DTYPES, TOL, _random_case, attention_error, storage, values

pytestmark = pytest.mark.gpu

N_DECODE = 64
N_PREFILL = 32
ALGOS = ["auto", "auto", "auto", "valu", "mfma", "stream"]


def _decode_draw(i: int):
    r = random.Random(1000 + i)
    dtype = r.choice(list(DTYPES))
    d = r.choice([64, 64, 128, 128, 32, 16, 256, 8])
    hkv = r.choice([1, 2, 2, 4, 8])
    group = r.choice([1, 2, 4, 7, 7, 8, 12, 16, 11, 24])
    bs = r.choice([1, 2, 4, 8, 16, 16, 32, 64, 256])
    batch = r.choice([1, 3, 17, 64, 130, 257])
    width = max(1, r.choice([1, 2, 8, 40]) * max(1, 64 // bs))  # table width in blocks
    cap = width * bs
    lens = []
    for _ in range(batch):
        u = r.random()
        lens.append(0 if u < 0.08 else cap if u < 0.16 else 1 if u < 0.22 else r.randint(1, cap))
    # At most 2e7 pool elements per case (and so a quick float64 oracle).
    limit = max(1, min(1500, int(2e7 / (hkv * d * batch))))
    lens = [min(n, limit) for n in lens]
    return dict(dtype=dtype, d=d, hkv=hkv, hq=hkv * group, bs=bs, lens=lens, algo=r.choice(ALGOS), seed=i)


@pytest.mark.parametrize("i", range(N_DECODE))
def test_random_decode_shapes(gpu, i):
    from engine import _native, paged_ops

    c = _decode_draw(i)
    dtype, d, hq, hkv, bs, lens = c["dtype"], c["d"], c["hq"], c["hkv"], c["bs"], c["lens"]
    batch = len(lens)
    announce(f"random decode #{i}: {dtype} d={d} hq={hq} hkv={hkv} bs={bs} B={batch} "
             f"max_len={max(lens)} empty={lens.count(0)} algo={c['algo']}")
    q, k_pool, v_pool, tables, bt, width = _random_case(dtype, batch, hq, hkv, d, bs, lens, nb_extra=3, seed=c["seed"])
    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(c["seed"])
    # q, k and v as strided views of one fused projection row per sequence.
    qkv = torch.randn(batch, (hq + 2 * hkv) * d, generator=g).to(dt)
    qkv[:, :hq * d] = q.reshape(batch, hq * d)
    qkv_g = qkv.to(gpu)
    qg = qkv_g[:, :hq * d].view(batch, hq, d)
    k_new = qkv_g[:, hq * d:(hq + hkv) * d].view(batch, hkv, d)
    v_new = qkv_g[:, (hq + hkv) * d:].view(batch, hkv, d)
    bt_t = torch.from_numpy(bt).to(gpu)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    live = [b for b, n in enumerate(lens) if n > 0]
    slots = [tables[b][(n - 1) // bs] * bs + (n - 1) % bs if n > 0 else -1 for b, n in enumerate(lens)]
    slot_t = torch.tensor(slots, dtype=torch.int64, device=gpu)

    prev = _native.set_decode_algo(c["algo"])
    try:
        kg, vg = k_pool.to(gpu), v_pool.to(gpu)
        plan = paged_ops.decode_plan(lens_t, bt_t, hq, hkv, d, bs, dt, max_blocks=width)
        out_u = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width)
        out_p = paged_ops.paged_decode(qg, kg, vg, bt_t, lens_t, max_blocks=width, plan=plan)
        ka, va = kg.clone(), vg.clone()
        out_f = paged_ops.paged_decode_append(qg, k_new, v_new, ka, va, slot_t, bt_t, lens_t, max_blocks=width,
                                              plan=plan)
        torch.cuda.synchronize()
    finally:
        _native.set_decode_algo(prev)

    want = ref.attention_f64(values(q), values(k_pool), values(v_pool), tables, lens, bs)
    for name, out in (("unplanned", out_u), ("planned", out_p)):
        got = values(out)
        assert np.isfinite(got).all(), name
        assert not got[[b for b, n in enumerate(lens) if n == 0]].any(), f"{name}: empty rows are zero"
        err = attention_error(got[live], want[live], dtype) if live else 0.0
        assert err <= TOL[dtype], f"{name}: error beyond output rounding {err:.3g}"

    # Fused call: the oracle appends the new rows, then attends.
    kc, vc = storage(k_pool), storage(v_pool)
    rows = [b for b in range(batch) if slots[b] >= 0]
    blocks = np.array([slots[b] // bs for b in rows], dtype=np.int64)
    offs = np.array([slots[b] % bs for b in rows], dtype=np.int64)
    ref.append(kc, vc, blocks, offs, storage(k_new)[rows], storage(v_new)[rows])
    assert np.array_equal(storage(ka), kc) and np.array_equal(storage(va), vc), "pools after the fused append"
    want_f = ref.attention_f64(values(q), values(ka), values(va), tables, lens, bs)
    got_f = values(out_f)
    err = attention_error(got_f[live], want_f[live], dtype) if live else 0.0
    assert err <= TOL[dtype], f"fused: error beyond output rounding {err:.3g}"


def _prefill_draw(i: int):
    r = random.Random(5000 + i)
    dtype = r.choice(list(DTYPES))
    d = r.choice([64, 64, 128, 128, 32, 16])
    hkv = r.choice([1, 2, 4])
    group = r.choice([1, 2, 7, 7, 8, 12, 16, 24])
    bs = r.choice([1, 4, 16, 16, 32, 64])
    n = r.choice([1, 2, 5, 9])
    starts = [r.choice([0, 0, r.randint(1, 700)]) for _ in range(n)]
    lengths = [r.choice([1, r.randint(1, 40), r.randint(40, 300)]) for _ in range(n)]
    return dict(dtype=dtype, d=d, hkv=hkv, hq=hkv * group, bs=bs, starts=starts, lengths=lengths, seed=i)


@pytest.mark.parametrize("i", range(N_PREFILL))
def test_random_prefill_shapes(gpu, i):
    from engine import paged_ops
    from test_gpu_prefill import build, half_ulp

    c = _prefill_draw(i)
    announce(f"random prefill #{i}: {c['dtype']} d={c['d']} hq={c['hq']} hkv={c['hkv']} bs={c['bs']} "
             f"starts={c['starts']} lengths={c['lengths']}")
    dev, want = build(gpu, c["dtype"], c["d"], c["hq"], c["hkv"], c["bs"], c["starts"], c["lengths"],
                      seed=c["seed"] + 77)
    # A loose max_q_len (the grid may be larger than needed).
    out = paged_ops.paged_prefill(dev["q"], dev["k"], dev["v"], dev["tab"], dev["cu"], dev["st"],
                                  max(c["lengths"]) + 3)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = float((np.abs(got - want) - half_ulp(want, c["dtype"])).max())
    assert err <= TOL[c["dtype"]], f"error beyond output rounding {err:.3g}"

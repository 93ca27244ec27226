"""GPU parity of the fused rotary-embedding + KV-append kernel (``mip_rope_kv_append``).

Bar: bit-exact. The rotated q and k (in place) and every byte of both pools equal the
oracle (oracle/paged_ref.py ``rope_append``), and the rotated q and k also equal torch's own
GPU evaluation of the reference expression (``apply_rope``, engine/model.py:216-224). The
cache contexts' ``attend_rope`` gives the same outputs and pools as ``apply_rope`` followed
by ``attend``.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def storage(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def _case(gpu, dtype, n, d, hq, hkv, bs, seed=11, padding=(1,)):
    from engine.model import rope_cos_sin

    dt = DTYPES[dtype]
    g = torch.Generator().manual_seed(seed)
    nb = max(64, 2 * n // bs + 8)
    k_cache = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt)
    v_cache = torch.randn(nb + 1, hkv, bs, d, generator=g).to(dt)
    qkv = torch.randn(n, (hq + 2 * hkv) * d, generator=g).to(dt)  # rows of a fused qkv projection
    positions = torch.randint(0, 32768, (n,), generator=g)
    slots = torch.tensor(random.Random(seed).sample(range((nb + 1) * bs), n), dtype=torch.int64)
    for i in padding:
        if i < n:
            slots[i] = -1
    cos, sin = rope_cos_sin(positions.to(gpu).unsqueeze(1), d, 1_000_000.0, dt)  # [n, 1, 1, d], as the model
    return k_cache, v_cache, qkv, slots, cos, sin


def _views(qkv, n, d, hq, hkv):
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(n, hkv, d)
    return q, k, v


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("n,d,hq,hkv,bs", [(40, 64, 14, 2, 16), (33, 128, 28, 4, 32), (7, 16, 4, 2, 4),
                                           (256, 64, 14, 2, 16)])
def test_rope_kv_append_bit_exact(gpu, dtype, n, d, hq, hkv, bs):
    from engine import paged_ops
    from engine.model import apply_rope

    announce(f"rope_kv_append {dtype} n={n} d={d} hq={hq} hkv={hkv} bs={bs}")
    k_cache, v_cache, qkv, slots, cos, sin = _case(gpu, dtype, n, d, hq, hkv, bs)
    q0, k0, v0 = _views(qkv, n, d, hq, hkv)
    kc, vc = storage(k_cache), storage(v_cache)
    qr, kr = ref.rope_append(storage(q0), storage(k0), storage(v0), storage(cos[:, 0, 0]), storage(sin[:, 0, 0]),
                             dtype, kc, vc, slots.numpy(), bs)

    qkv_g, kg, vg, sg = qkv.to(gpu), k_cache.to(gpu), v_cache.to(gpu), slots.to(gpu)
    q, k, v = _views(qkv_g, n, d, hq, hkv)
    want_q, want_k = apply_rope(q.unsqueeze(2).clone(), k.unsqueeze(2).clone(), cos, sin)  # torch on the GPU
    paged_ops.rope_kv_append(q, k, v, cos[:, 0, 0], sin[:, 0, 0], kg, vg, sg)
    torch.cuda.synchronize()
    assert np.array_equal(storage(q), qr)
    assert np.array_equal(storage(k), kr)
    assert np.array_equal(storage(v), storage(v0))
    assert np.array_equal(storage(kg), kc)
    assert np.array_equal(storage(vg), vc)
    assert torch.equal(q, want_q[:, :, 0]) and torch.equal(k, want_k[:, :, 0])


@pytest.mark.parametrize("dtype,d,hq", [("bfloat16", 6, 3), ("float16", 10, 2), ("float32", 6, 1), ("float32", 2, 2),
                                        ("bfloat16", 64, 0)])
def test_rope_kv_append_narrow_rows_and_no_q(gpu, dtype, d, hq):
    """Rows whose halves are not 16-byte multiples take the narrow chunks; hq = 0 passes q = None."""
    from engine import paged_ops

    announce(f"rope_kv_append narrow {dtype} d={d} hq={hq}")
    n, hkv, bs = 9, 2, 4
    k_cache, v_cache, qkv, slots, cos, sin = _case(gpu, dtype, n, d, hq, hkv, bs, seed=5, padding=(0, 4))
    q0, k0, v0 = _views(qkv, n, d, hq, hkv)
    kc, vc = storage(k_cache), storage(v_cache)
    qr, kr = ref.rope_append(storage(q0), storage(k0), storage(v0), storage(cos[:, 0, 0]), storage(sin[:, 0, 0]),
                             dtype, kc, vc, slots.numpy(), bs)
    qkv_g, kg, vg = qkv.to(gpu), k_cache.to(gpu), v_cache.to(gpu)
    q, k, v = _views(qkv_g, n, d, hq, hkv)
    paged_ops.rope_kv_append(q if hq else None, k, v, cos[:, 0, 0], sin[:, 0, 0], kg, vg, slots.to(gpu))
    torch.cuda.synchronize()
    if hq:
        assert np.array_equal(storage(q), qr)
    assert np.array_equal(storage(k), kr)
    assert np.array_equal(storage(kg), kc) and np.array_equal(storage(vg), vc)


def _two_caches(gpu, dtype, d, hkv, bs, lengths, num_layers=2, seed=3):
    from engine.kv_cache import PagedKVCache

    out = []
    for _ in range(2):
        c = PagedKVCache(num_layers, hkv, d, num_blocks=sum(n // bs + 2 for n in lengths) + 16, block_size=bs,
                         max_seqs=len(lengths) + 2, max_len=max(lengths) + 2 * bs, dtype=DTYPES[dtype], device=gpu)
        slots = []
        for n in lengths:
            s = c.allocate(n + 1)
            c.lengths[s] = n
            slots.append(s)
        out.append((c, slots))
    gen = torch.Generator(device=gpu).manual_seed(seed)
    for pool in (out[0][0].k, out[0][0].v):
        pool.normal_(0.0, 1.0, generator=gen)
    out[1][0].k.copy_(out[0][0].k)
    out[1][0].v.copy_(out[0][0].v)
    return out


@pytest.mark.parametrize("dtype,d,hq,hkv,bs", [("bfloat16", 64, 14, 2, 16), ("float16", 128, 28, 4, 32),
                                               ("float32", 64, 8, 2, 16)])
@torch.inference_mode()
def test_decode_context_attend_rope_equals_apply_rope_then_attend(gpu, dtype, d, hq, hkv, bs):
    from engine.model import apply_rope, rope_cos_sin

    announce(f"decode attend_rope vs apply_rope + attend {dtype} d={d}")
    lengths = [1, 15, 16, 17, 200, 513, 1000, 64, 3, 777]
    (ca, sa), (cb, sb) = _two_caches(gpu, dtype, d, hkv, bs, lengths)
    dt, b = DTYPES[dtype], len(lengths)
    g = torch.Generator(device=gpu).manual_seed(9)
    qkv = torch.randn(b, 1, (hq + 2 * hkv) * d, generator=g, device=gpu).to(dt)
    for layer in range(2):
        ctx_a, ctx_b = ca.decode_context(sa), cb.decode_context(sb)
        cos, sin = rope_cos_sin(ctx_a.positions.unsqueeze(1), d, 1_000_000.0, dt)

        def split(t):
            q, k, v = t.split([hq * d, hkv * d, hkv * d], dim=-1)
            return (q.view(b, 1, hq, d).transpose(1, 2), k.view(b, 1, hkv, d).transpose(1, 2),
                    v.view(b, 1, hkv, d).transpose(1, 2))

        q, k, v = split(qkv.clone())
        q, k = apply_rope(q, k, cos, sin)
        out_a = ctx_a.attend(layer, q, k, v)
        q2, k2, v2 = split(qkv.clone())
        out_b = ctx_b.attend_rope(layer, q2, k2, v2, cos, sin)
        torch.cuda.synchronize()
        assert torch.equal(q2, q) and torch.equal(k2, k)  # rotated in place, same bits
        assert torch.equal(out_b, out_a), f"layer {layer}: max diff {(out_b.float() - out_a.float()).abs().max()}"
        assert torch.equal(cb.k, ca.k) and torch.equal(cb.v, ca.v)


@pytest.mark.parametrize("prefix", [False, True])
@torch.inference_mode()
def test_prefill_context_attend_rope_equals_apply_rope_then_attend(gpu, prefix):
    from engine.model import apply_rope, rope_cos_sin

    announce(f"prefill attend_rope vs apply_rope + attend, prefix={prefix}")
    dtype, d, hq, hkv, bs = "float16", 64, 14, 2, 16
    dt = DTYPES[dtype]
    start = [40, 0, 17] if prefix else [0, 0, 0]
    new = [23, 50, 9]
    (ca, sa), (cb, sb) = _two_caches(gpu, dtype, d, hkv, bs, [s + n + bs for s, n in zip(start, new)])
    for c, slots in ((ca, sa), (cb, sb)):
        for s, st in zip(slots, start):
            c.lengths[s] = st
    ctx_a = ca.packed_prefill_context(sa, new)
    ctx_b = cb.packed_prefill_context(sb, new)
    n = sum(new)
    g = torch.Generator(device=gpu).manual_seed(4)
    qkv = torch.randn(1, n, (hq + 2 * hkv) * d, generator=g, device=gpu).to(dt)
    cos, sin = rope_cos_sin(ctx_a.positions.unsqueeze(0), d, 1_000_000.0, dt)  # [1, 1, N, D]

    def split(t):
        q, k, v = t.split([hq * d, hkv * d, hkv * d], dim=-1)
        return (q.view(1, n, hq, d).transpose(1, 2), k.view(1, n, hkv, d).transpose(1, 2),
                v.view(1, n, hkv, d).transpose(1, 2))

    q, k, v = split(qkv.clone())
    q, k = apply_rope(q, k, cos, sin)
    out_a = ctx_a.attend(0, q, k, v)
    q2, k2, v2 = split(qkv.clone())
    out_b = ctx_b.attend_rope(0, q2, k2, v2, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q2, q) and torch.equal(k2, k)
    assert torch.equal(out_b, out_a)
    assert torch.equal(cb.k, ca.k) and torch.equal(cb.v, ca.v)

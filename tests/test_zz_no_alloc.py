"""mip_paged_decode_append_noalloc (static scratch, no allocation) against mip_paged_decode_append
(caller workspace), through the C ABI: the same kernels, so pools and outputs are bit-identical.
Two calls in a row, the second with a smaller batch; a shape whose scratch need exceeds the
static array is refused with MIP_E2BIG before anything is launched.
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


def _case(gpu, lens, seed, hq=14, hkv=2, d=64, bs=16, dtype=torch.bfloat16):
    """Scattered pool, tables, q, the step's new rows and their slots (the newest key of each sequence)."""
    g = torch.Generator().manual_seed(seed)
    need = [math.ceil(n / bs) for n in lens]
    nb = sum(need) + 4
    perm = list(range(nb))
    random.Random(seed).shuffle(perm)
    tables, cur = [], 0
    for n in need:
        tables.append(perm[cur:cur + n])
        cur += n
    width = max(need)
    bt = np.zeros((len(lens), width), dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    slots = [t[(n - 1) // bs] * bs + (n - 1) % bs for t, n in zip(tables, lens)]
    b = len(lens)
    return dict(
        q=torch.randn(b, hq, d, generator=g).to(dtype).to(gpu),
        k=torch.randn(nb + 1, hkv, bs, d, generator=g).to(dtype).to(gpu),
        v=torch.randn(nb + 1, hkv, bs, d, generator=g).to(dtype).to(gpu),
        k_new=torch.randn(b, hkv, d, generator=g).to(dtype).to(gpu),
        v_new=torch.randn(b, hkv, d, generator=g).to(dtype).to(gpu),
        bt=torch.from_numpy(bt).to(gpu), lens=torch.tensor(lens, dtype=torch.int32, device=gpu),
        slots=torch.tensor(slots, dtype=torch.int64, device=gpu), tables=tables, width=width,
        shape=(b, hq, hkv, d, bs), dtype=dtype)


def _args(c, k_pool, v_pool, out, plan):
    from engine import paged_ops

    b, hq, hkv, d, bs = c["shape"]
    st = torch.cuda.current_stream().cuda_stream
    head = (c["k_new"].data_ptr(), c["v_new"].data_ptr(), c["k_new"].stride(0), c["k_new"].stride(1),
            c["v_new"].stride(0), c["v_new"].stride(1), c["slots"].data_ptr(), out.data_ptr(), out.stride(0),
            out.stride(1), c["q"].data_ptr(), c["q"].stride(0), c["q"].stride(1), k_pool.data_ptr(),
            v_pool.data_ptr(), k_pool.shape[0], c["bt"].data_ptr(), c["bt"].stride(0), c["lens"].data_ptr(), b, hq,
            hkv, d, bs, c["width"], 1.0 / math.sqrt(d))
    tail = (plan.data_ptr() if plan is not None else None, plan.numel() * 4 if plan is not None else 0,
            paged_ops.dtype_code(c["dtype"]), st)
    return head, tail


@torch.inference_mode()
def test_noalloc_entry_point_matches_workspace_entry_point(gpu):
    from engine import _native, paged_ops

    lib = _native.load()
    rnd = random.Random(3)
    big = [int(math.exp(rnd.uniform(math.log(128), math.log(4096)))) for _ in range(256)]
    for step, lens in enumerate((big, [3, 90, 1300])):
        announce(f"no-alloc fused decode vs workspace entry point, call {step}, batch {len(lens)}")
        c = _case(gpu, lens, seed=10 + step)
        b, hq, hkv, d, bs = c["shape"]
        plan = paged_ops.decode_plan(c["lens"], c["bt"], hq, hkv, d, bs, c["dtype"], max_blocks=c["width"])
        need = paged_ops.decode_workspace_bytes(b, hq, hkv, d, bs, c["width"], c["dtype"])
        assert 0 < need <= _native.MIP_NOALLOC_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        ka, va, kb, vb = c["k"].clone(), c["v"].clone(), c["k"].clone(), c["v"].clone()
        out_a = torch.full_like(c["q"], float("nan"))
        out_b = torch.full_like(c["q"], float("nan"))
        head, tail = _args(c, ka, va, out_a, plan)
        st = lib.mip_paged_decode_append(*head, ws.data_ptr(), need, *tail)
        assert st == _native.MIP_OK, st
        head, tail = _args(c, kb, vb, out_b, plan)
        st = lib.mip_paged_decode_append_noalloc(*head, *tail)
        assert st == _native.MIP_OK, st
        torch.cuda.synchronize()
        assert torch.equal(ka, kb) and torch.equal(va, vb), f"call {step}: pools differ"
        assert torch.equal(out_a, out_b), f"call {step}: outputs differ"
        want = ref.attention_f64(c["q"].float().cpu().numpy(), kb.float().cpu().numpy(),
                                 vb.float().cpu().numpy(), c["tables"], lens, bs)
        got = out_b.float().cpu().numpy()
        half = 0.5 * np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
        assert float((np.abs(got - want) - half).max()) <= 2e-3


@torch.inference_mode()
def test_noalloc_entry_point_refuses_oversized_scratch(gpu):
    """fp32 decode runs the partition kernels, whose workspace grows with the batch and the
    longest table: 4096 sequences of up to 65,536 keys need far more than the static array."""
    from engine import _native, paged_ops

    announce("no-alloc fused decode: oversized scratch refused")
    lib = _native.load()
    b, hq, hkv, d, bs, width = 4096, 8, 1, 256, 16, 4096
    need = paged_ops.decode_workspace_bytes(b, hq, hkv, d, bs, width, torch.float32)
    assert need > _native.MIP_NOALLOC_SCRATCH_BYTES
    c = dict(q=torch.zeros(b, hq, d, device=gpu), k=torch.zeros(3, hkv, bs, d, device=gpu),
             v=torch.zeros(3, hkv, bs, d, device=gpu), k_new=torch.zeros(b, hkv, d, device=gpu),
             v_new=torch.zeros(b, hkv, d, device=gpu), bt=torch.zeros(b, width, dtype=torch.int32, device=gpu),
             lens=torch.zeros(b, dtype=torch.int32, device=gpu),
             slots=torch.full((b,), -1, dtype=torch.int64, device=gpu), width=width, shape=(b, hq, hkv, d, bs),
             dtype=torch.float32)
    out = torch.zeros_like(c["q"])
    head, tail = _args(c, c["k"], c["v"], out, None)
    assert lib.mip_paged_decode_append_noalloc(*head, *tail) == _native.MIP_E2BIG
    assert b"static array" in lib.mip_status_string(_native.MIP_E2BIG)

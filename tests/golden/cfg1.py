"""Seeded inputs of the golden decode case (fp32, one layer) and the fixture's file names.

Case: 14 query / 2 kv heads, head_dim 64, a pool of 512 blocks of 16 tokens (plus the
scratch block), batch 8, cached contexts U[16, 256]; block tables are consecutive chunks of
one permutation of the pool. Pool, q and the step's new k/v are N(0, 1). One decode step =
append the new k/v at each sequence's next position, then attend context + 1 keys.

Random streams (both stable across library versions):
  random.Random(0)                       context lengths, then the block permutation
  numpy Generator(PCG64(0)), float32     pool K, pool V, q, new k, new v (in that order)

The fixture (``cfg1_decode.npz`` + ``cfg1_decode.json``) is written by ``make_golden.py``
from the float64 oracle; tests regenerate these inputs and compare against it.
"""

from __future__ import annotations

import hashlib
import random
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
NPZ = HERE / "cfg1_decode.npz"
META = HERE / "cfg1_decode.json"

BATCH, HQ, HKV, D, BS, NB = 8, 14, 2, 64, 16, 512
CTX_LO, CTX_HI = 16, 256


def make_inputs() -> dict:
    rnd = random.Random(0)
    ctx = [rnd.randint(CTX_LO, CTX_HI) for _ in range(BATCH)]
    perm = list(range(NB))
    rnd.shuffle(perm)
    tables, cursor = [], 0
    for n in ctx:
        nblk = (n + 1 + BS - 1) // BS  # room for the token appended this step
        tables.append(perm[cursor:cursor + nblk])
        cursor += nblk
    g = np.random.Generator(np.random.PCG64(0))
    k_pool = g.standard_normal((NB + 1, HKV, BS, D), dtype=np.float32)
    v_pool = g.standard_normal((NB + 1, HKV, BS, D), dtype=np.float32)
    q = g.standard_normal((BATCH, HQ, D), dtype=np.float32)
    k_new = g.standard_normal((BATCH, HKV, D), dtype=np.float32)
    v_new = g.standard_normal((BATCH, HKV, D), dtype=np.float32)
    return {"ctx": ctx, "tables": tables, "k_pool": k_pool, "v_pool": v_pool, "q": q, "k_new": k_new,
            "v_new": v_new}


def touched_blocks(tables) -> list[int]:
    return sorted({b for t in tables for b in t})


def blocks_sha256(k_pool: np.ndarray, v_pool: np.ndarray, blocks) -> str:
    """SHA-256 over the bytes of the listed blocks, K then V, in block order."""
    h = hashlib.sha256()
    idx = np.asarray(blocks, dtype=np.int64)
    h.update(np.ascontiguousarray(k_pool[idx]).tobytes())
    h.update(np.ascontiguousarray(v_pool[idx]).tobytes())
    return h.hexdigest()


def inputs_sha256(inp: dict) -> str:
    """Fingerprint of the generated inputs (guards against a changed random stream)."""
    h = hashlib.sha256()
    h.update(np.asarray(inp["ctx"], dtype=np.int64).tobytes())
    for t in inp["tables"]:
        h.update(np.asarray(t, dtype=np.int64).tobytes())
    for key in ("k_pool", "v_pool", "q", "k_new", "v_new"):
        h.update(np.ascontiguousarray(inp[key]).tobytes())
    return h.hexdigest()

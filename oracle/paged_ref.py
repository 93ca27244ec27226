"""Oracle: CPU restatement of the reference's paged KV-cache path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the reference results are checked
against or as the timed CPU baseline. The product (``mini-inference_amd/engine``) never calls it.

Each function restates one piece of the reference (Ham12-3/mini-inference) and cites it:

  write_index          engine/kv_cache.py:562-573   (block, offset) of tokens start..start+n-1
  decode_inputs        engine/kv_cache.py:592-609   per-step positions / write index / padded tables / mask
  append               engine/kv_cache.py:613-614   k_layer[write_blocks, :, write_offsets] = k[:, :, 0]
                       engine/kv_cache.py:286-289   packed prefill scatter (same indexing, N tokens)
  rope                 engine/model.py:216-224      x * cos + rotate_half(x) * sin, rounded op by op in the dtype
  rope_append          engine/model.py:249 + kv_cache.py:613-614   rotate q and k, append the rotated k and v
  gather_kv            engine/kv_cache.py:615-619   k_layer[tables].permute(0, 2, 1, 3, 4).reshape(...)
  decode_attention     engine/model.py:126-147      GQA regroup + SDPA with a [B,1,1,kv_len] bool mask
  sdpa_attention       engine/model.py:101-123      GQA by repeat_interleave + SDPA
  paged_decode_torch   engine/kv_cache.py:611-620   append + gather + decode_attention (the reference path)
  packed_prefill_torch engine/kv_cache.py:262-294   prefix read-back + dense [N, keys] mask + SDPA
  attention_f64        (independent)                float64 brute force over each sequence's own keys
  prefill_attention_f64  engine/kv_cache.py:268-294  float64 packed prefill: each new token over its own
                                                    sequence's keys 0..position (prefix + new tokens)
  copy_blocks          (no reference counterpart)   bitwise k[:, dst] = k[:, src] for every layer

Arrays: the pool of one layer is ``[num_blocks + 1, Hkv, block_size, D]`` (reference layout,
engine/kv_cache.py:426-428). 16-bit pools are handled as raw ``uint16`` bit patterns so that
append and copy are checked bit for bit; ``bf16_to_f32`` / ``f16_to_f32`` widen them exactly.

Pinning (tests/test_oracle.py): every function above is checked against the reference's
own known-answer tests restated (tests/test_kv_cache.py:40-46, :120-141, :179-207) and
against closed forms (L = 1 gives the value row, constant keys give the mean of the values,
block relabelling and stale padding leave the output unchanged, G = 1 is plain MHA), plus
planted mistakes that those checks must catch. ``rope`` is checked against a float64
complex-number rotation, the angle-0 and quarter-turn special cases, torch's own CPU
arithmetic in each dtype (the rounding sequence), and planted sign, half-swap and
rounding mistakes. ``paged_decode_torch`` and ``attention_f64``
are two independent formulations and are checked against each other.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import numpy as np
import torch
import torch.nn.functional as F

# --------------------------------------------------------------------------- dtype helpers


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bfloat16 bit patterns (uint16) to float32."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (torch's rounding)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> float16 bit patterns, round to nearest even; values beyond 65504 round to inf."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def widen(a: np.ndarray, dtype: str) -> np.ndarray:
    """Storage array (float32, or uint16 bits of 'float16'/'bfloat16') -> float32 values."""
    if dtype == "float32":
        return np.asarray(a, dtype=np.float32)
    if dtype == "float16":
        return f16_to_f32(a)
    if dtype == "bfloat16":
        return bf16_to_f32(a)
    raise ValueError(dtype)


def narrow(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values -> storage array for ``dtype`` (RNE for the 16-bit types)."""
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return f32_to_f16(x)
    if dtype == "bfloat16":
        return f32_to_bf16(x)
    raise ValueError(dtype)


# --------------------------------------------------------------------------- index math


def write_index(block_tables: dict[int, list[int]] | Sequence[Sequence[int]], slots: Sequence[int],
                starts: Sequence[int], counts: Sequence[int], block_size: int) -> tuple[np.ndarray, np.ndarray]:
    """engine/kv_cache.py:562-573: token p of a sequence lives at (table[p // bs], p % bs)."""
    blocks, offsets = [], []
    for slot, a, n in zip(slots, starts, counts):
        table = list(block_tables[slot])
        for p in range(a, a + n):
            blocks.append(table[p // block_size])
            offsets.append(p % block_size)
    return np.asarray(blocks, dtype=np.int64), np.asarray(offsets, dtype=np.int64)


def decode_inputs(lengths: Sequence[int], tables: Sequence[Sequence[int]], block_size: int) -> dict:
    """engine/kv_cache.py:592-609 for a batch whose sequences hold ``lengths`` tokens.

    positions[b] = lengths[b] (where the new token goes); write_blocks/offsets locate it;
    tables are padded with block 0 to the longest sequence's block count; kv_len =
    num_blocks * block_size; mask[b, j] = j <= positions[b].
    """
    pos = [int(x) for x in lengths]
    if any(p // block_size >= len(t) for p, t in zip(pos, tables)):
        raise ValueError("a sequence has no block for its next token (call ensure_capacity first)")
    write_blocks = [t[p // block_size] for t, p in zip(tables, pos)]
    write_offsets = [p % block_size for p in pos]
    nb = max(pos) // block_size + 1
    padded = [list(t[:nb]) + [0] * (nb - len(t[:nb])) for t in tables]
    kv_len = nb * block_size
    mask = np.arange(kv_len)[None, :] <= np.asarray(pos)[:, None]
    return {
        "positions": np.asarray(pos, dtype=np.int64),
        "write_blocks": np.asarray(write_blocks, dtype=np.int64),
        "write_offsets": np.asarray(write_offsets, dtype=np.int64),
        "slot_mapping": np.asarray(write_blocks, dtype=np.int64) * block_size + np.asarray(write_offsets),
        "tables": np.asarray(padded, dtype=np.int64),
        "num_blocks": nb,
        "kv_len": kv_len,
        "mask": mask,
        "context_lens": np.asarray(pos, dtype=np.int32) + 1,
    }


# --------------------------------------------------------------------------- data movement


def append(k_layer: np.ndarray, v_layer: np.ndarray, blocks: np.ndarray, offsets: np.ndarray,
           k_rows: np.ndarray, v_rows: np.ndarray) -> None:
    """In place: ``layer[blocks[i], :, offsets[i], :] = rows[i]`` (engine/kv_cache.py:613-614, :286-289).

    ``rows`` is ``[N, Hkv, D]`` in the pool's storage dtype (bit patterns for 16-bit).
    """
    k_layer[blocks, :, offsets] = k_rows
    v_layer[blocks, :, offsets] = v_rows


# --------------------------------------------------------------------------- rotary embedding


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """``x * cos + _rotate_half(x) * sin`` evaluated op by op in ``dtype`` (engine/model.py:216-224).

    ``_rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])``. Each torch op on ``dtype``
    tensors computes in fp32 and rounds its result to ``dtype`` (RNE), so the value stored is
    ``rnd(rnd(x * cos) + rnd(rotate_half(x) * sin))``. Arrays are storage arrays (float32, or
    uint16 bit patterns for the 16-bit types); ``cos``/``sin`` broadcast against ``x``.
    Returns a new storage array.
    """
    xf, cf, sf = widen(x, dtype), widen(cos, dtype), widen(sin, dtype)
    half = xf.shape[-1] // 2
    rot = np.concatenate([-xf[..., half:], xf[..., :half]], axis=-1)
    t1 = widen(narrow(xf * cf, dtype), dtype)
    t2 = widen(narrow(rot * sf, dtype), dtype)
    return narrow(t1 + t2, dtype)


def rope_append(q: np.ndarray, k: np.ndarray, v: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str,
                k_layer: np.ndarray, v_layer: np.ndarray, slots: np.ndarray, block_size: int):
    """``apply_rope`` (engine/model.py:249) then the append of the rotated k and v.

    ``q`` ``[N, Hq, D]``, ``k``/``v`` ``[N, Hkv, D]``, ``cos``/``sin`` ``[N, D]``. Slots outside
    the pool (padding rows) are not written. Returns the rotated ``(q, k)``; the pool is
    updated in place.
    """
    qr = rope(q, cos[:, None, :], sin[:, None, :], dtype)
    kr = rope(k, cos[:, None, :], sin[:, None, :], dtype)
    slots = np.asarray(slots, dtype=np.int64)
    ok = (slots >= 0) & (slots < (k_layer.shape[0] * block_size))
    append(k_layer, v_layer, slots[ok] // block_size, slots[ok] % block_size, kr[ok], v[ok])
    return qr, kr


def copy_blocks(k_pool: np.ndarray, v_pool: np.ndarray, pairs: Sequence[tuple[int, int]]) -> None:
    """In place: every layer's K and V copy of block dst becomes that of block src."""
    for src, dst in pairs:
        k_pool[:, dst] = k_pool[:, src]
        v_pool[:, dst] = v_pool[:, src]


# --------------------------------------------------------------------------- attention (torch, fp32)


def sdpa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask=None, is_causal: bool = False):
    """engine/model.py:101-123: repeat each kv head for its query group, then SDPA."""
    groups = q.shape[1] // k.shape[1]
    if groups > 1:
        k = k.repeat_interleave(groups, dim=1)
        v = v.repeat_interleave(groups, dim=1)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal)


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask=None) -> torch.Tensor:
    """engine/model.py:126-147: q [B, Hq, 1, D] regrouped to [B, Hkv, G, D], one SDPA call."""
    batch, heads, _, dim = q.shape
    kv_heads = k.shape[1]
    qg = q.reshape(batch, kv_heads, heads // kv_heads, dim)
    out = F.scaled_dot_product_attention(qg, k, v, attn_mask=attn_mask)
    return out.reshape(batch, heads, 1, dim)


def gather_kv(layer: torch.Tensor, tables: torch.Tensor, kv_len: int) -> torch.Tensor:
    """engine/kv_cache.py:615-619: [B, nb, Hkv, bs, D] -> [B, Hkv, nb * bs, D] in table order."""
    batch = tables.shape[0]
    heads = layer.shape[1]
    return layer[tables].permute(0, 2, 1, 3, 4).reshape(batch, heads, kv_len, -1)


def paged_decode_torch(q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor, k_new: torch.Tensor,
                       v_new: torch.Tensor, inputs: dict) -> torch.Tensor:
    """The reference decode step for one layer (engine/kv_cache.py:611-620), on CPU tensors.

    Mutates ``k_layer``/``v_layer`` (the append) and returns ``[B, Hq, 1, D]``.
    ``q`` ``[B, Hq, 1, D]``, ``k_new``/``v_new`` ``[B, Hkv, 1, D]``.
    """
    wb = torch.as_tensor(inputs["write_blocks"])
    wo = torch.as_tensor(inputs["write_offsets"])
    k_layer[wb, :, wo] = k_new[:, :, 0]
    v_layer[wb, :, wo] = v_new[:, :, 0]
    tables = torch.as_tensor(inputs["tables"])
    kv_len = int(inputs["kv_len"])
    mask = torch.as_tensor(inputs["mask"])[:, None, None, :]
    keys = gather_kv(k_layer, tables, kv_len)
    values = gather_kv(v_layer, tables, kv_len)
    return decode_attention(q, keys, values, attn_mask=mask)


def packed_prefill_torch(q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                         tables: Sequence[Sequence[int]], starts: Sequence[int], lengths: Sequence[int],
                         block_size: int) -> torch.Tensor:
    """The reference's packed prefill attention with cached prefixes (engine/kv_cache.py:262-294).

    Every sequence's keys ``0 .. end-1`` are read back from the pool (``write_index``), and
    SDPA runs over all of them with the dense mask ``key_seg == seg & key_pos <= position``.
    ``q`` ``[1, Hq, N, D]`` (float32), pools ``[NB, Hkv, bs, D]``; returns ``[1, Hq, N, D]``.
    """
    nseq = len(lengths)
    ends = [a + n for a, n in zip(starts, lengths)]
    seg = torch.repeat_interleave(torch.arange(nseq), torch.tensor(list(lengths)))
    positions = torch.cat([torch.arange(a, a + n) for a, n in zip(starts, lengths)])
    rb, ro = write_index(tables, range(nseq), [0] * nseq, ends, block_size)
    rb, ro = torch.from_numpy(rb), torch.from_numpy(ro)
    keys = k_layer[rb, :, ro].transpose(0, 1).unsqueeze(0)     # [1, Hkv, total keys, D]
    values = v_layer[rb, :, ro].transpose(0, 1).unsqueeze(0)
    key_seg = torch.repeat_interleave(torch.arange(nseq), torch.tensor(ends))
    key_pos = torch.cat([torch.arange(e) for e in ends])
    mask = (seg.unsqueeze(1) == key_seg.unsqueeze(0)) & (key_pos.unsqueeze(0) <= positions.unsqueeze(1))
    return sdpa_attention(q, keys, values, attn_mask=mask)


# --------------------------------------------------------------------------- attention (float64 brute force)


def attention_f64(q: np.ndarray, k_layer: np.ndarray, v_layer: np.ndarray, tables: Sequence[Sequence[int]],
                  context_lens: Sequence[int], block_size: int, scale: float | None = None) -> np.ndarray:
    """Independent float64 decode attention over each sequence's own keys.

    ``q`` ``[B, Hq, D]``, pools ``[NB, Hkv, bs, D]`` (float values). Query head h reads kv
    head h // (Hq // Hkv); key j of sequence b is pool row (tables[b][j // bs], ., j % bs).
    Returns ``[B, Hq, D]`` float64.
    """
    q = np.asarray(q, dtype=np.float64)
    batch, hq, d = q.shape
    hkv = k_layer.shape[1]
    group = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((batch, hq, d), dtype=np.float64)
    for b in range(batch):
        n = int(context_lens[b])
        if n <= 0:
            continue
        j = np.arange(n)
        blk = np.asarray(tables[b], dtype=np.int64)[j // block_size]
        off = j % block_size
        for kv in range(hkv):
            keys = np.asarray(k_layer[blk, kv, off], dtype=np.float64)    # [n, D]
            vals = np.asarray(v_layer[blk, kv, off], dtype=np.float64)
            heads = slice(kv * group, (kv + 1) * group)                   # query heads reading kv head `kv`
            s = q[b, heads] @ keys.T * scale                              # [G, n]
            s -= s.max(axis=1, keepdims=True)
            w = np.exp(s)
            out[b, heads] = (w @ vals) / w.sum(axis=1, keepdims=True)
    return out


def prefill_attention_f64(q: np.ndarray, k_layer: np.ndarray, v_layer: np.ndarray, tables: Sequence[Sequence[int]],
                          starts: Sequence[int], lengths: Sequence[int], block_size: int,
                          scale: float | None = None) -> np.ndarray:
    """Independent float64 packed prefill over paged keys (engine/kv_cache.py:268-294).

    ``q`` ``[N, Hq, D]`` packed rows, sequence s owning ``lengths[s]`` consecutive rows; its
    new token i sits at position ``starts[s] + i`` and attends keys ``0 .. starts[s] + i`` of
    its own sequence (prefix and earlier new tokens), read from the pool through ``tables[s]``
    (pools ``[NB, Hkv, bs, D]`` float values, already holding the new keys). Query head h reads
    kv head h // (Hq // Hkv). Returns ``[N, Hq, D]`` float64.
    """
    q = np.asarray(q, dtype=np.float64)
    n_all, hq, d = q.shape
    hkv = k_layer.shape[1]
    group = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((n_all, hq, d), dtype=np.float64)
    row = 0
    for s, (start, n) in enumerate(zip(starts, lengths)):
        end = start + n
        j = np.arange(end)
        blk = np.asarray(tables[s], dtype=np.int64)[j // block_size]
        off = j % block_size
        pos = start + np.arange(n)
        allowed = j[None, :] <= pos[:, None]                                  # [n, end] causal over positions
        for kv in range(hkv):
            keys = np.asarray(k_layer[blk, kv, off], dtype=np.float64)        # [end, D]
            vals = np.asarray(v_layer[blk, kv, off], dtype=np.float64)
            for g in range(group):
                h = kv * group + g
                sc = q[row:row + n, h] @ keys.T * scale                       # [n, end]
                sc = np.where(allowed, sc, -np.inf)
                sc -= sc.max(axis=1, keepdims=True)
                w = np.exp(sc)
                out[row:row + n, h] = (w @ vals) / w.sum(axis=1, keepdims=True)
        row += n
    return out

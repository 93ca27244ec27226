"""Paged KV cache whose attention contexts run the MI355X HIP kernels.

Drop-in for the paged half of the reference's engine/kv_cache.py:

* :class:`PagedKVCache` keeps the reference's pool tensors, public state and allocator
  API (engine/kv_cache.py:377-579) with the same block-reuse policy, so the scheduler,
  prefix caching and graph code see the same block ids. It adds :meth:`copy_blocks`
  and :meth:`fork` for copy-on-write of shared blocks.
* :class:`PagedDecodeContext` (engine/kv_cache.py:582-624): ``attend`` = KV append +
  paged decode attention in one fused call. No gathered copy of the history is made, and
  the block tables stay on the device (:class:`DeviceBlockTables`): a step uploads the
  batch's slot ids, positions and the table entries written since the last step.
* :class:`PackedPrefillContext` (engine/kv_cache.py:218-301): the packed scatter is the
  append kernel and the attention over cached prefixes is the paged prefill kernel.

Pool layout (reference engine/kv_cache.py:426-428):
``k, v: [num_layers, num_blocks + 1, num_kv_heads, block_size, head_dim]``; block
``num_blocks`` is the scratch block that graph padding rows point at.
"""

from __future__ import annotations

from collections import OrderedDict
from collections.abc import Sequence

import numpy as np
import torch

from . import paged_ops
from .model import Qwen2Config


class PagedKVCache:
    """Fixed-size blocks handed out to sequences; optional content-keyed prefix sharing.

    A sequence ("slot") owns a block table: token p lives in block ``table[p // block_size]``
    at offset ``p % block_size``. Block reuse order, reference counting and prefix keys
    follow engine/kv_cache.py:436-560 exactly:

    * free blocks form an LRU queue, least recently freed first; a released block that
      holds no cached prefix is put at the head so it is reused before cached ones;
    * a full block is keyed by ``(hash(previous key), its tokens)``; registered blocks
      stay findable while free until the queue hands them out again.
    """

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_blocks: int, block_size: int,
                 max_seqs: int, max_len: int, dtype: torch.dtype, device: torch.device | str,
                 enable_prefix_caching: bool = False) -> None:
        if block_size <= 0 or block_size & (block_size - 1):
            raise ValueError(f"block_size must be a power of two, got {block_size}")
        shape = (num_layers, num_blocks + 1, num_kv_heads, block_size, head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=device)
        self.v = torch.zeros(shape, dtype=dtype, device=device)
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_blocks = num_blocks
        self.scratch_block = num_blocks
        self.block_size = block_size
        self.max_len = max_len
        self.enable_prefix_caching = enable_prefix_caching
        self.lengths: dict[int, int] = {}
        self.block_tables: dict[int, list[int]] = {}
        self._free_ids = list(range(max_seqs - 1, -1, -1))  # pop() hands out slot 0 first
        self._free_blocks: OrderedDict[int, None] = OrderedDict.fromkeys(range(num_blocks))
        self._ref_counts = [0] * num_blocks
        self._block_key: dict[int, tuple] = {}
        self._cached: dict[tuple, int] = {}
        self.prefix_hit_tokens = 0
        self.cow_copies = 0  # blocks copied on write so far
        self.max_seqs = max_seqs
        # (slot, index, block) of every table entry written since the last drain; kept only
        # once a device mirror of the tables exists (enable_device_tables).
        self._journal: list[tuple[int, int, int]] | None = None
        self.device_tables: DeviceBlockTables | None = None

    @classmethod
    def for_model(cls, cfg: Qwen2Config, num_blocks: int, block_size: int, max_seqs: int, max_len: int,
                  dtype: torch.dtype, device: torch.device | str, enable_prefix_caching: bool = False) -> "PagedKVCache":
        return cls(cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, num_blocks, block_size, max_seqs, max_len, dtype,
                   device, enable_prefix_caching)

    # ----------------------------------------------------------------- capacity queries
    @property
    def num_free_slots(self) -> int:
        return len(self._free_ids)

    @property
    def num_free_blocks(self) -> int:
        return len(self._free_blocks)

    def blocks_for(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def can_allocate(self, num_tokens: int) -> bool:
        # Same conservative test as the reference: blocks a prefix hit would share are not counted.
        return (len(self._free_ids) > 0 and num_tokens <= self.max_len
                and self.blocks_for(num_tokens) <= len(self._free_blocks))

    # ----------------------------------------------------------------- block life cycle
    def _new_block(self) -> int:
        block = next(iter(self._free_blocks))
        del self._free_blocks[block]
        key = self._block_key.pop(block, None)
        if key is not None:
            del self._cached[key]  # its cached prefix is overwritten from now on
        self._ref_counts[block] = 1
        return block

    def _share(self, block: int) -> None:
        if self._ref_counts[block] == 0:
            del self._free_blocks[block]  # free but still cached: back in use
        self._ref_counts[block] += 1

    def _release(self, block: int) -> None:
        self._ref_counts[block] -= 1
        if self._ref_counts[block]:
            return
        self._free_blocks[block] = None  # newest free block: reused last ...
        if block not in self._block_key:
            self._free_blocks.move_to_end(block, last=False)  # ... unless it caches nothing

    @staticmethod
    def _chain_keys(token_ids: Sequence[int], block_size: int, count: int):
        parent = None
        for i in range(count):
            key = (parent, tuple(token_ids[i * block_size:(i + 1) * block_size]))
            yield key
            parent = hash(key)

    def _match_prefix(self, token_ids: Sequence[int]) -> list[int]:
        usable = (len(token_ids) - 1) // self.block_size  # at least one token is always computed
        found = []
        for key in self._chain_keys(token_ids, self.block_size, usable):
            block = self._cached.get(key)
            if block is None:
                break
            found.append(block)
        return found

    # ----------------------------------------------------------------- sequences
    def allocate(self, num_tokens: int = 0, token_ids: Sequence[int] | None = None) -> int:
        if not self.can_allocate(num_tokens):
            raise RuntimeError("not enough free KV cache blocks")
        shared = self._match_prefix(token_ids) if (self.enable_prefix_caching and token_ids) else []
        for block in shared:
            self._share(block)
        slot = self._free_ids.pop()
        fresh = [self._new_block() for _ in range(self.blocks_for(num_tokens) - len(shared))]
        self.block_tables[slot] = shared + fresh
        self._log_table(slot)
        self.lengths[slot] = len(shared) * self.block_size
        self.prefix_hit_tokens += self.lengths[slot]
        return slot

    def register_prefix(self, slot: int, token_ids: Sequence[int]) -> None:
        if not self.enable_prefix_caching:
            return
        table = self.block_tables[slot]
        full = self.lengths[slot] // self.block_size
        for i, key in enumerate(self._chain_keys(token_ids, self.block_size, full)):
            if key not in self._cached and table[i] not in self._block_key:
                self._cached[key] = table[i]
                self._block_key[table[i]] = key

    def ensure_capacity(self, slot: int, num_tokens: int) -> bool:
        if num_tokens > self.max_len:
            return False
        table = self.block_tables[slot]
        missing = self.blocks_for(num_tokens) - len(table)
        if missing > len(self._free_blocks):
            return False
        for _ in range(missing):
            table.append(self._new_block())
            if self._journal is not None:
                self._journal.append((slot, len(table) - 1, table[-1]))
        return True

    def free(self, slot: int) -> None:
        if slot not in self.block_tables:
            raise RuntimeError(f"slot {slot} freed twice")
        for block in reversed(self.block_tables.pop(slot)):
            self._release(block)
        del self.lengths[slot]
        self._free_ids.append(slot)

    def fork(self, slot: int) -> int:
        """New sequence sharing every block (and the length) of ``slot``.

        Shared blocks are reference counted; the first write into a shared, partially
        filled block copies it first (see :meth:`prepare_writes`). No reference
        counterpart: the reference only shares full prefix blocks.
        """
        if not self._free_ids:
            raise RuntimeError("no free sequence slot")
        table = self.block_tables[slot]
        for block in table:
            self._share(block)
        child = self._free_ids.pop()
        self.block_tables[child] = list(table)
        self.lengths[child] = self.lengths[slot]
        self._log_table(child)
        return child

    def ref_count(self, block: int) -> int:
        return self._ref_counts[block]

    def prepare_writes(self, slots: Sequence[int], starts: Sequence[int], counts: Sequence[int]) -> list[tuple[int, int]]:
        """Copy-on-write: give every sequence private copies of the shared blocks it is about to write.

        For each sequence, every block touched by tokens ``[start, start + count)`` whose
        reference count is above one is replaced in that sequence's table by a fresh block,
        and one :meth:`copy_blocks` call copies all of them (all layers, K and V; one launch
        per 128 pairs).
        Returns the ``(src, dst)`` pairs copied. Raises if the pool cannot supply them.
        """
        pairs: list[tuple[int, int]] = []
        for slot, start, n in zip(slots, starts, counts):
            if n <= 0:
                continue
            table = self.block_tables[slot]
            last = min((start + n - 1) // self.block_size, len(table) - 1)
            for i in range(start // self.block_size, last + 1):
                old = table[i]
                if self._ref_counts[old] > 1:
                    if not self._free_blocks:
                        raise RuntimeError("not enough free KV cache blocks for copy-on-write")
                    new = self._new_block()
                    table[i] = new
                    self._release(old)
                    pairs.append((old, new))
                    if self._journal is not None:
                        self._journal.append((slot, i, new))
        if pairs:
            self.copy_blocks(pairs)
            self.cow_copies += len(pairs)
        return pairs

    def copy_blocks(self, pairs: Sequence[tuple[int, int]] | torch.Tensor) -> None:
        """``k[:, dst] = k[:, src]`` and ``v[:, dst] = v[:, src]`` for every (src, dst), all layers, on device.

        Pairs built on the host (the copy-on-write pairs of :meth:`prepare_writes`) go to the
        kernel in its arguments (``mip_copy_blocks_host``), with no upload; a tensor on the
        pool's device is read there (``mip_copy_blocks``)."""
        if isinstance(pairs, torch.Tensor) and pairs.is_cuda:
            pairs = pairs.to(device=self.k.device, dtype=torch.int64).reshape(-1, 2).contiguous()
        elif len(pairs) == 0:
            return
        paged_ops.copy_blocks(self.k, self.v, pairs)

    # ----------------------------------------------------------------- device-resident tables
    def _log_table(self, slot: int) -> None:
        if self._journal is not None:
            self._journal.extend((slot, i, b) for i, b in enumerate(self.block_tables[slot]))

    def enable_device_tables(self) -> "DeviceBlockTables":
        """Keep a device mirror of every block table, updated from a journal of changes.

        The reference rebuilds the padded ``[B, nb]`` tables on the host and copies them to
        the device every step (engine/kv_cache.py:592-609). With the mirror, only the
        entries written since the last step travel (a new block every ``block_size`` tokens
        per sequence, copy-on-write replacements, new sequences).
        """
        if self.device_tables is None:
            self._journal = []
            for slot in self.block_tables:
                self._log_table(slot)
            self.device_tables = DeviceBlockTables(self)
        return self.device_tables

    def drain_journal(self) -> np.ndarray:
        """int64 ``[n, 3]`` rows ``(slot, index, block)`` logged since the last drain, oldest first."""
        if not self._journal:
            return np.zeros((0, 3), dtype=np.int64)
        out = np.asarray(self._journal, dtype=np.int64)
        self._journal.clear()
        return out

    # ----------------------------------------------------------------- index helpers
    def write_index(self, slots: Sequence[int], starts: Sequence[int],
                    counts: Sequence[int]) -> tuple[torch.Tensor, torch.Tensor]:
        """``(block, offset)`` of tokens ``start .. start+count-1`` of each sequence (kv_cache.py:562-573)."""
        blocks, offsets = self._write_index_np(slots, starts, counts)
        return torch.from_numpy(blocks).to(self.k.device), torch.from_numpy(offsets).to(self.k.device)

    def _write_index_np(self, slots, starts, counts) -> tuple[np.ndarray, np.ndarray]:
        parts_b, parts_o = [], []
        for slot, a, n in zip(slots, starts, counts):
            pos = np.arange(a, a + n, dtype=np.int64)
            table = np.asarray(self.block_tables[slot], dtype=np.int64)
            parts_b.append(table[pos // self.block_size])
            parts_o.append(pos % self.block_size)
        if not parts_b:
            return np.zeros(0, np.int64), np.zeros(0, np.int64)
        return np.concatenate(parts_b), np.concatenate(parts_o)

    def slot_mapping(self, slots: Sequence[int], starts: Sequence[int], counts: Sequence[int]) -> torch.Tensor:
        """Flat int64 slots ``block * block_size + offset`` for the same tokens as :meth:`write_index`."""
        blocks, offsets = self._write_index_np(slots, starts, counts)
        return torch.from_numpy(blocks * self.block_size + offsets).to(self.k.device)

    def packed_prefill_context(self, slots: Sequence[int], lengths: Sequence[int]) -> "PackedPrefillContext":
        return PackedPrefillContext(self, slots, lengths)

    def decode_context(self, slots: Sequence[int]) -> "PagedDecodeContext":
        return PagedDecodeContext(self, slots)


class DeviceBlockTables:
    """Device mirror of a cache's block tables: int32 ``rows [max_seqs + 1, max_blocks]``.

    Row ``slot`` holds that sequence's table; entries past its length are stale and never
    read (every kernel stops at the sequence's context length). The last row, ``spare_row``,
    only ever holds the scratch block: padding rows of a batch point at it, and unused
    entries of a fixed-size journal write into it.
    """

    def __init__(self, cache: PagedKVCache) -> None:
        self.cache = cache
        self.max_blocks = cache.blocks_for(cache.max_len)
        self.spare_row = cache.max_seqs
        self.rows = torch.full((cache.max_seqs + 1, self.max_blocks), cache.scratch_block, dtype=torch.int32,
                               device=cache.k.device)

    def flat_entries(self, journal: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """Distinct (flat index into ``rows``, block) pairs of a journal, the newest entry winning.

        A scatter with repeated indices leaves an unspecified winner, so an entry written
        twice (a slot freed and reused, a block replaced by copy-on-write) keeps only its last
        value here.
        """
        flat = journal[:, 0] * self.max_blocks + journal[:, 1]
        _, last = np.unique(flat[::-1], return_index=True)
        keep = len(flat) - 1 - last
        return flat[keep], journal[keep, 2]

    def apply_flat(self, flat: np.ndarray, blocks: np.ndarray) -> None:
        """Scatter distinct ``rows.view(-1)[flat] = blocks`` now, on the current stream."""
        if len(flat) == 0:
            return
        both = torch.from_numpy(np.concatenate([flat, blocks]).astype(np.int64)).to(self.rows.device)
        n = len(flat)
        self.rows.view(-1).scatter_(0, both[:n], both[n:].to(torch.int32))

    def sync(self) -> None:
        """Apply everything the cache logged since the last drain."""
        self.apply_flat(*self.flat_entries(self.cache.drain_journal()))



class PagedDecodeContext:
    """One batched decode step: B sequences, one new token each (engine/kv_cache.py:582-624).

    Built once per step; every layer's ``attend`` reuses its device tensors:

    * ``positions`` int64 ``[B]`` (RoPE positions, where each new token goes);
    * ``slot_mapping`` int64 ``[B]`` = ``write_blocks * block_size + write_offsets``;
    * ``block_tables`` int32 ``[B, nb]`` (``nb`` = blocks of the longest sequence), gathered
      on the device from the cache's :class:`DeviceBlockTables`. Entries past a sequence's
      own blocks are stale, where the reference pads with block 0; no kernel reads them;
    * ``context_lens`` int32 ``[B]`` = ``positions + 1`` (keys each query attends).

    The reference rebuilds the padded tables on the host and copies them every step
    (engine/kv_cache.py:597-607). Here the host does O(B) work: the batch's slot ids,
    positions and slots, plus the table entries logged since the previous step, go to the
    device in one copy; the mirror is updated there and the batch's rows gathered from it.

    With ``fuse_rope`` set (the default) the model hands over q and k before the rotary
    embedding and calls :meth:`attend_rope`; otherwise it rotates them itself and calls
    :meth:`attend`, the reference's protocol.
    """

    fuse_rope = True

    def __init__(self, cache: PagedKVCache, slots: Sequence[int]) -> None:
        self.cache = cache
        self.slots = list(slots)
        bs = cache.block_size
        pos = [cache.lengths[s] for s in self.slots]
        if any(p // bs >= len(cache.block_tables[s]) for p, s in zip(pos, self.slots)):
            raise ValueError("a sequence has no block for its next token (call ensure_capacity first)")
        cache.prepare_writes(self.slots, pos, [1] * len(self.slots))  # copy-on-write of shared blocks
        dt = cache.enable_device_tables()
        b = len(self.slots)
        write_blocks = [cache.block_tables[s][p // bs] for s, p in zip(self.slots, pos)]
        flat, blocks = dt.flat_entries(cache.drain_journal())
        m = len(flat)
        # One int64 upload: slot ids | positions | slots | journal (flat index, block) | context
        # lengths as int32 pairs.
        n32 = (b + 1) // 2
        stage = np.empty(3 * b + 2 * m + n32, dtype=np.int64)
        stage[:b] = self.slots
        stage[b:2 * b] = pos
        stage[2 * b:3 * b] = np.asarray(write_blocks, dtype=np.int64) * bs + np.asarray(pos, dtype=np.int64) % bs
        stage[3 * b:3 * b + m] = flat
        stage[3 * b + m:3 * b + 2 * m] = blocks
        lens32 = stage[3 * b + 2 * m:].view(np.int32)
        lens32[:b] = np.asarray(pos, dtype=np.int32) + 1
        lens32[b:] = 0
        dev = cache.k.device
        staged = torch.from_numpy(stage).to(dev)
        row_ids = staged[:b]
        self.positions = staged[b:2 * b]
        self.slot_mapping = staged[2 * b:3 * b]
        if m:
            dt.rows.view(-1).scatter_(0, staged[3 * b:3 * b + m], staged[3 * b + m:3 * b + 2 * m].to(torch.int32))
        self.context_lens = staged[3 * b + 2 * m:].view(torch.int32)[:b]
        nb = max(pos) // bs + 1 if b else 1
        self.block_tables = torch.index_select(dt.rows[:, :nb], 0, row_ids)
        self.num_blocks = nb
        self.kv_len = nb * bs
        self.scale = 1.0 / (cache.head_dim ** 0.5)
        self._mask: torch.Tensor | None = None
        self._plan: tuple[tuple, torch.Tensor | None] | None = None  # (shape key, work plan)
        self._calls: paged_ops.DecodeStepCalls | None = None

    @property
    def tables(self) -> torch.Tensor:
        """The batch's block tables (int32 here; int64 and zero-padded in the reference)."""
        return self.block_tables

    @property
    def write_blocks(self) -> torch.Tensor:
        """Block of each new token (engine/kv_cache.py:603), from ``slot_mapping``."""
        return torch.div(self.slot_mapping, self.cache.block_size, rounding_mode="floor")

    @property
    def write_offsets(self) -> torch.Tensor:
        """Offset of each new token in its block (engine/kv_cache.py:604)."""
        return self.slot_mapping % self.cache.block_size

    @property
    def mask(self) -> torch.Tensor:
        """``[B, 1, 1, kv_len]`` bool mask of the reference (built on demand; the kernel does not need it)."""
        if self._mask is None:
            keys = torch.arange(self.kv_len, device=self.positions.device)
            self._mask = (keys <= self.positions.unsqueeze(1))[:, None, None, :]
        return self._mask

    def plan(self, num_heads: int, dtype: torch.dtype) -> torch.Tensor | None:
        """The step's decode work plan (made by the first layer's call, shared by the rest)."""
        key = (num_heads, dtype)
        if self._plan is None or self._plan[0] != key:
            c = self.cache
            p = paged_ops.decode_plan(self.context_lens, self.block_tables, num_heads, c.num_kv_heads, c.head_dim,
                                      c.block_size, dtype, max_blocks=self.num_blocks)
            self._plan = (key, p)
        return self._plan[1]

    @property
    def calls(self) -> paged_ops.DecodeStepCalls:
        """The step's layer calls: the shared arguments are checked on the first layer only."""
        if self._calls is None:
            self._calls = paged_ops.DecodeStepCalls(self.block_tables, self.context_lens, self.slot_mapping,
                                                    self.scale, self.num_blocks, self.plan)
        return self._calls

    def attend(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Append this step's k/v and attend (engine/kv_cache.py:611-620) in one fused call."""
        k_layer, v_layer = self.cache.k[layer_idx], self.cache.v[layer_idx]
        return self.calls.decode_append(q[:, :, 0], k[:, :, 0], v[:, :, 0], k_layer, v_layer).unsqueeze(2)

    def attend_rope(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor) -> torch.Tensor:
        """``apply_rope`` (engine/model.py:249) + append + attend, on pre-rotation q and k.

        One kernel rotates q and k in place and writes the rotated k and v to the pool; the
        decode kernel then reads every key, the new one included, from the pool. ``cos`` and
        ``sin`` are the ``[B, 1, 1, D]`` tables of the step.
        """
        k_layer, v_layer = self.cache.k[layer_idx], self.cache.v[layer_idx]
        q1 = q[:, :, 0]
        self.calls.rope_append(q1, k[:, :, 0], v[:, :, 0], cos[:, 0, 0], sin[:, 0, 0], k_layer, v_layer)
        return self.calls.decode(q1, k_layer, v_layer).unsqueeze(2)

    def commit(self) -> None:
        for s in self.slots:
            self.cache.lengths[s] += 1


class PackedPrefillContext:
    """Several prompts packed end to end in one forward pass (engine/kv_cache.py:218-301).

    The scatter of the N packed tokens into the pool is the append kernel. Attention over
    the packed tokens (block-diagonal causal, plus any cached prefix of each sequence) is the
    paged prefill kernel (``mip_paged_prefill``), which reads every key in place through the
    block tables; there is no SDPA path. A shape the library has no kernel for raises.
    ``mask`` and ``read_at`` (the reference's dense mask and read-back index) are still built
    on demand for callers that read them. ``fuse_rope`` as for :class:`PagedDecodeContext`.
    """

    fuse_rope = True

    def __init__(self, cache: PagedKVCache, slots: Sequence[int], lengths: Sequence[int]) -> None:
        self.cache = cache
        self.slots = list(slots)
        self.lengths = list(lengths)
        self.starts = [cache.lengths[s] for s in self.slots]
        for s, start, n in zip(self.slots, self.starts, self.lengths):
            if not cache.ensure_capacity(s, start + n):
                raise ValueError(f"no room in the KV cache for {start + n} tokens")
        cache.prepare_writes(self.slots, self.starts, self.lengths)
        dev = cache.k.device
        self.positions = torch.from_numpy(np.concatenate(
            [np.arange(a, a + n, dtype=np.int64) for a, n in zip(self.starts, self.lengths)])).to(dev)
        blocks, offsets = cache._write_index_np(self.slots, self.starts, self.lengths)
        both = torch.from_numpy(np.concatenate([blocks, offsets, blocks * cache.block_size + offsets])).to(dev)
        n_tok = blocks.shape[0]
        self.write_at = (both[:n_tok], both[n_tok:2 * n_tok])
        self.slot_mapping = both[2 * n_tok:]
        self.has_prefix = any(self.starts)
        self.ends = [a + n for a, n in zip(self.starts, self.lengths)]
        # Inputs of the paged prefill kernel: packed row offsets, cached lengths, tables.
        self.max_q_len = max(self.lengths) if self.lengths else 0
        nb = max(1, cache.blocks_for(max(self.ends))) if self.ends else 1
        tables = np.zeros((len(self.slots), nb), dtype=np.int32)
        for i, s in enumerate(self.slots):
            row = cache.block_tables[s][:nb]
            tables[i, :len(row)] = row
        cu = np.zeros(len(self.slots) + 1, dtype=np.int32)
        cu[1:] = np.cumsum(self.lengths)
        i32 = torch.from_numpy(np.concatenate([cu, np.asarray(self.starts, dtype=np.int32), tables.reshape(-1)])).to(dev)
        s_n = len(self.slots)
        self.cu_q, self.ctx_start = i32[:s_n + 1], i32[s_n + 1:2 * s_n + 1]
        self.block_tables = i32[2 * s_n + 1:].view(s_n, nb)
        self._mask_built = False
        self._mask = None
        self._read_at = None
        self.last_index = torch.tensor(self.lengths, device=dev).cumsum(0) - 1

    def _build_mask(self) -> None:
        """The reference's mask and read-back index (engine/kv_cache.py:262-279), built on demand."""
        cache, dev = self.cache, self.cache.k.device
        seg = torch.repeat_interleave(torch.arange(len(self.slots), device=dev), torch.tensor(self.lengths, device=dev))
        if self.has_prefix:
            self._read_at = cache.write_index(self.slots, [0] * len(self.slots), self.ends)
            key_seg = torch.repeat_interleave(torch.arange(len(self.slots), device=dev),
                                              torch.tensor(self.ends, device=dev))
            key_pos = torch.cat([torch.arange(e, device=dev) for e in self.ends])
            self._mask = (seg[:, None] == key_seg[None, :]) & (key_pos[None, :] <= self.positions[:, None])
        elif len(self.slots) == 1:
            self._mask = None
        else:
            idx = torch.arange(seg.shape[0], device=dev)
            self._mask = (seg[:, None] == seg[None, :]) & (idx[None, :] <= idx[:, None])
        self._mask_built = True

    @property
    def mask(self) -> torch.Tensor | None:
        """The reference's ``[N, keys]`` bool mask (None for one fresh prompt); built on demand."""
        if not self._mask_built:
            self._build_mask()
        return self._mask

    @property
    def read_at(self) -> tuple[torch.Tensor, torch.Tensor] | None:
        """``(block, offset)`` of every sequence's keys ``0 .. end-1`` (prefix hits only)."""
        if not self._mask_built:
            self._build_mask()
        return self._read_at

    def attend(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        k_layer, v_layer = self.cache.k[layer_idx], self.cache.v[layer_idx]
        # k[0] is [Hkv, N, D]; the append kernel takes [N, Hkv, D] views with any strides.
        paged_ops.kv_append(k_layer, v_layer, k[0].transpose(0, 1), v[0].transpose(0, 1), self.slot_mapping)
        return self._attention(k_layer, v_layer, q, k, v)

    def attend_rope(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor) -> torch.Tensor:
        """``apply_rope`` (engine/model.py:249) + :meth:`attend`, with the rotation fused into the append.

        ``cos``/``sin`` are ``[1, 1, N, D]``; q and k are rotated in place, so the prefill
        attention below sees the same tensors as after ``apply_rope``.
        """
        k_layer, v_layer = self.cache.k[layer_idx], self.cache.v[layer_idx]
        paged_ops.rope_kv_append(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), cos[0, 0],
                                 sin[0, 0], k_layer, v_layer, self.slot_mapping)
        return self._attention(k_layer, v_layer, q, k, v)

    def _attention(self, k_layer, v_layer, q, k, v) -> torch.Tensor:
        # q is [1, Hq, N, D]; the kernel takes the [N, Hq, D] view and returns [N, Hq, D].
        out = paged_ops.paged_prefill(q[0].transpose(0, 1), k_layer, v_layer, self.block_tables, self.cu_q,
                                      self.ctx_start, self.max_q_len, scale=1.0 / (self.cache.head_dim ** 0.5))
        return out.transpose(0, 1).unsqueeze(0)

    def commit(self) -> None:
        for slot, start, n in zip(self.slots, self.starts, self.lengths):
            self.cache.lengths[slot] = start + n

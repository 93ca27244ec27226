"""HIP-graph capture of the paged decode step (engine/cuda_graphs.py:1-189 of the reference).

A decode step launches a few hundred small kernels (24 layers of norms, GEMMs, RoPE, the KV
append and the paged attention); replaying them as one captured graph removes the host
launch cost. As in the reference:

* inputs live in static device buffers that are overwritten before each replay;
* one graph per batch bucket (1, 2, 4, 8, then every 16 up to ``max_batch``); rows past
  the real batch point at the cache's scratch block, so their appends land there and their
  outputs are ignored;
* everything that depends on the inputs (slot mapping, context lengths) is computed inside
  the graph from the static buffers.

Block tables stay on the device (``PagedKVCache.enable_device_tables``). Each step uploads
only token ids, positions, the batch's sequence ids and the table entries written since the
previous step, in one copy from a pinned staging row. The graph first writes those entries
into the device mirror, then gathers the batch's rows from it. The reference instead
rebuilds and uploads the whole padded ``[B, nb]`` table every step
(engine/cuda_graphs.py:160-176, engine/kv_cache.py:592-609).

Unlike the reference, the attention kernel reads each sequence's pages in place and its
launch shape does not depend on the KV length, so one KV bucket (the cache's ``max_len``)
serves every step by default; ``kv_step`` restores per-length buckets (useful only for the
partition kernels, whose grid grows with the longest table).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from . import paged_ops
from .kv_cache import PagedKVCache
from .model import Qwen2ForCausalLM


def _batch_buckets(limit: int) -> list[int]:
    """1, 2, 4, 8, then every 16 up to ``limit`` (always including ``limit``); engine/cuda_graphs.py:34-43."""
    sizes = [b for b in (1, 2, 4, 8) if b < limit] + list(range(16, limit, 16))
    return sizes + [limit]


def _kv_buckets(limit: int, step: int | None, block_size: int) -> list[int]:
    """KV-length buckets in whole blocks: every ``step`` positions up to ``limit``, or just ``limit``."""
    raw = [limit] if step is None else list(range(step, limit, step)) + [limit]
    return sorted({-(-kv // block_size) * block_size for kv in raw})


class _GraphDecodeContext:
    """Attention for a captured decode step; reads everything from the static buffers."""

    def __init__(self, owner: "GraphedDecoder", batch: int, kv_len: int) -> None:
        self.owner = owner
        self.cache = owner.cache
        self.batch, self.kv_len = batch, kv_len
        self.num_blocks = kv_len // owner.cache.block_size
        self.positions = owner.positions[:batch]
        self.tables = owner.tables[:batch, :self.num_blocks]
        self.slot_mapping = owner.slot_mapping[:batch]
        self.context_lens = owner.context_lens[:batch]
        self.scale = 1.0 / (owner.cache.head_dim ** 0.5)
        self.num_heads = owner.model.cfg.num_heads
        self.fuse_rope = owner.fuse_rope
        # Buffer of the step's work plan; prepare() fills it inside the graph. (The launch is
        # issued there, not prepared here, so that it binds the capturing stream.)
        self.plan = paged_ops.prepare_decode_plan(self.context_lens, self.tables, self.num_heads,
                                                  owner.cache.num_kv_heads, owner.cache.head_dim,
                                                  owner.cache.block_size, owner.cache.k.dtype,
                                                  max_blocks=self.num_blocks)[1]

    def prepare(self) -> None:
        """Inside the graph, once per step: table updates, the batch's rows, slot mapping, context lengths."""
        owner = self.owner
        rows = owner.device_tables.rows
        rows.view(-1).scatter_(0, owner.journal_flat, owner.journal_block.to(torch.int32))
        torch.index_select(rows, 0, owner.row_ids[:self.batch], out=owner.tables[:self.batch])
        bs = self.cache.block_size
        write_blocks = self.tables.gather(1, torch.div(self.positions, bs, rounding_mode="floor").unsqueeze(1))
        self.slot_mapping.copy_(write_blocks.squeeze(1).to(torch.int64) * bs + self.positions % bs)
        self.context_lens.copy_(self.positions + 1)
        if self.plan is not None:
            c = self.cache
            paged_ops.decode_plan(self.context_lens, self.tables, self.num_heads, c.num_kv_heads, c.head_dim,
                                  c.block_size, c.k.dtype, max_blocks=self.num_blocks, plan=self.plan)

    def attend(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        k_layer, v_layer = self.cache.k[layer_idx], self.cache.v[layer_idx]
        out = paged_ops.paged_decode_append(q[:, :, 0], k[:, :, 0], v[:, :, 0], k_layer, v_layer, self.slot_mapping,
                                            self.tables, self.context_lens, scale=self.scale,
                                            max_blocks=self.num_blocks, workspace=self.owner.workspace,
                                            plan=self.plan)
        return out.unsqueeze(2)

    def attend_rope(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor) -> torch.Tensor:
        """Rotary embedding fused with the append, then the decode kernel (as ``PagedDecodeContext``)."""
        k_layer, v_layer = self.cache.k[layer_idx], self.cache.v[layer_idx]
        q1 = q[:, :, 0]
        paged_ops.rope_kv_append(q1, k[:, :, 0], v[:, :, 0], cos[:, 0, 0], sin[:, 0, 0], k_layer, v_layer,
                                 self.slot_mapping)
        out = paged_ops.paged_decode(q1, k_layer, v_layer, self.tables, self.context_lens, scale=self.scale,
                                     max_blocks=self.num_blocks, workspace=self.owner.workspace, plan=self.plan)
        return out.unsqueeze(2)


class GraphedDecoder:
    """Captures the decode step as HIP graphs and replays them (engine/cuda_graphs.py:95-189).

    Call :meth:`capture` once, then :meth:`decode` each step. ``decode`` returns ``None``
    when no captured graph fits, and the caller runs the eager step instead.
    """

    def __init__(self, model: Qwen2ForCausalLM, cache: PagedKVCache, max_batch: int, kv_step: int | None = None,
                 fuse_rope: bool = True) -> None:
        if not isinstance(cache, PagedKVCache):
            raise TypeError("GraphedDecoder drives the paged cache")
        self.model, self.cache = model, cache
        self.fuse_rope = fuse_rope  # rotary embedding inside the append kernel (attend_rope)
        self.device = cache.k.device
        self.batch_buckets = _batch_buckets(max_batch)
        self.kv_buckets = _kv_buckets(cache.max_len, kv_step, cache.block_size)
        top = self.batch_buckets[-1]
        self.device_tables = cache.enable_device_tables()
        dt = self.device_tables
        if self.kv_buckets[-1] // cache.block_size > dt.max_blocks:
            raise ValueError("KV bucket beyond the cache's max_len")
        dev = self.device
        # Per-step inputs, one int64 buffer: ids | positions | row ids | journal flat index |
        # journal block. The journal part has a fixed capacity; a step that logs more
        # applies the excess eagerly before its replay.
        self.journal_cap = max(64, 2 * top)
        j = self.journal_cap
        self._layout = (top, top, top, j, j)
        n_words = sum(self._layout)
        self._stage = torch.zeros(n_words, dtype=torch.long, pin_memory=True)
        self._stage_np = self._stage.numpy()
        self._inputs = torch.zeros(n_words, dtype=torch.long, device=dev)
        self.ids = self._inputs[:top].view(top, 1)
        self.positions = self._inputs[top:2 * top]
        self.row_ids = self._inputs[2 * top:3 * top]
        self.journal_flat = self._inputs[3 * top:3 * top + j]
        self.journal_block = self._inputs[3 * top + j:]
        self._pad_inputs(0)
        self.tables = torch.full((top, dt.max_blocks), cache.scratch_block, dtype=torch.int32, device=dev)
        self.slot_mapping = torch.zeros(top, dtype=torch.long, device=dev)
        self.context_lens = torch.ones(top, dtype=torch.int32, device=dev)
        # Decode scratch shared by every captured graph: sized for the largest need over all
        # (batch, kv length) buckets and allocated once, before any capture, so no graph is
        # ever left holding the address of a buffer that was replaced. (A call with few
        # sequences can need more than a full batch: its long segments are merged in runs.)
        hq = model.cfg.num_heads
        need = max(paged_ops.decode_workspace_bytes(b, hq, cache.num_kv_heads, cache.head_dim, cache.block_size,
                                                    kv // cache.block_size, cache.k.dtype)
                   for b in self.batch_buckets for kv in self.kv_buckets)
        self.workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        # (batch, kv_len) -> (graph, its output logits, its context); the context stays alive
        # with the graph because the graph reads its tensors.
        self.graphs: dict[tuple[int, int], tuple[torch.cuda.CUDAGraph, torch.Tensor, _GraphDecodeContext]] = {}
        self._pool = None
        self.replays = 0

    @torch.inference_mode()
    def capture(self, batches: Sequence[int] | None = None) -> None:
        """Record one graph per (batch, kv length) bucket, largest first so smaller ones reuse its memory."""
        wanted = self.batch_buckets if batches is None else sorted({self._bucket(b) for b in batches})
        for batch in reversed(wanted):
            for kv_len in reversed(self.kv_buckets):
                self._capture_one(batch, kv_len)
        torch.cuda.synchronize()

    def _bucket(self, n: int) -> int:
        b = next((b for b in self.batch_buckets if b >= n), None)
        if b is None:
            raise ValueError(f"batch {n} exceeds max_batch {self.batch_buckets[-1]}")
        return b

    def _pad_inputs(self, n: int, n_journal: int = 0) -> None:
        """Staging rows from ``n`` (and journal entries from ``n_journal``) on: padding values."""
        top, j = self.batch_buckets[-1], self.journal_cap
        st, dt = self._stage_np, self.device_tables
        st[n:top] = 0
        st[top + n:2 * top] = 0
        st[2 * top + n:3 * top] = dt.spare_row
        st[3 * top + n_journal:3 * top + j] = dt.spare_row * dt.max_blocks
        st[3 * top + j + n_journal:] = self.cache.scratch_block

    def _capture_one(self, batch: int, kv_len: int) -> None:
        ctx = _GraphDecodeContext(self, batch, kv_len)

        def step() -> torch.Tensor:
            ctx.prepare()
            hidden = self.model(self.ids[:batch], self.positions[:batch].unsqueeze(1), ctx)
            return self.model.compute_logits(hidden[:, -1]).float()

        # Every row points at the spare (all-scratch) table row while recording.
        self._pad_inputs(0)
        self._inputs.copy_(self._stage)
        self.device_tables.sync()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up outside the graph: kernel selection, workspace, allocator
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._pool):
            logits = step()
        self._pool = graph.pool()
        self.graphs[(batch, kv_len)] = (graph, logits, ctx)

    def decode(self, slots: Sequence[int], last_tokens: Sequence[int]) -> torch.Tensor | None:
        """One decode step via a captured graph; logits ``[len(slots), vocab]``, or None if none fits."""
        n = len(slots)
        positions = [self.cache.lengths[s] for s in slots]
        bs = self.cache.block_size
        batch = next((b for b in self.batch_buckets if b >= n), None)
        kv_len = next((k for k in self.kv_buckets if k > max(positions)), None)
        if batch is None or kv_len is None or (batch, kv_len) not in self.graphs:
            return None
        if any(p // bs >= len(self.cache.block_tables[s]) for p, s in zip(positions, slots)):
            raise ValueError("a sequence has no block for its next token (call ensure_capacity first)")
        self.cache.prepare_writes(list(slots), positions, [1] * n)  # copy-on-write of shared blocks
        graph, logits, _ = self.graphs[(batch, kv_len)]
        top, j = self.batch_buckets[-1], self.journal_cap
        flat, blocks = self.device_tables.flat_entries(self.cache.drain_journal())
        if len(flat) > j:  # more table changes than the graph's journal holds: the rest now
            self.device_tables.apply_flat(flat[j:], blocks[j:])
            flat, blocks = flat[:j], blocks[:j]
        st, m = self._stage_np, len(flat)
        st[:n] = last_tokens
        st[top:top + n] = positions
        st[2 * top:2 * top + n] = slots
        st[3 * top:3 * top + m] = flat
        st[3 * top + j:3 * top + j + m] = blocks
        self._pad_inputs(n, m)
        self._inputs.copy_(self._stage, non_blocking=True)
        graph.replay()
        torch.cuda.current_stream().synchronize()  # the pinned staging rows are reused next step
        self.replays += 1
        for s in slots:
            self.cache.lengths[s] += 1
        return logits[:n]

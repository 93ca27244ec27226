"""CPU tests of the host side: allocator, decode-context index math, copy-on-write
bookkeeping, the C-ABI library's exports and host-side argument checks, and the rule
that the product path never falls back to the CPU.

No kernel runs here (no GPU): ABI calls below only take paths that return before any
launch (empty work or rejected arguments).
"""

from __future__ import annotations

import ctypes
import importlib.util
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from engine import _native, paged_ops
from engine.kv_cache import PagedKVCache
from oracle import paged_ref as ref

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mipaged.h"
PROBE_HEADER = ROOT / "include" / "mipaged_probe.h"


def tiny_paged(num_blocks=12, block_size=4, max_seqs=4, max_len=32, **kw) -> PagedKVCache:
    return PagedKVCache(num_layers=1, num_kv_heads=2, head_dim=8, num_blocks=num_blocks, block_size=block_size,
                        max_seqs=max_seqs, max_len=max_len, dtype=torch.float32, device="cpu", **kw)


# ----------------------------------------------------------------------------- allocator (reference known answers)


def test_paged_block_bookkeeping():
    """tests/test_kv_cache.py:163-175 restated."""
    cache = tiny_paged(num_blocks=6, block_size=4)
    a = cache.allocate(5)
    assert len(cache.block_tables[a]) == 2 and cache.num_free_blocks == 4
    assert cache.ensure_capacity(a, 8) and len(cache.block_tables[a]) == 2
    assert cache.ensure_capacity(a, 9) and len(cache.block_tables[a]) == 3
    b = cache.allocate(12)
    assert cache.num_free_blocks == 0
    assert not cache.can_allocate(1) and not cache.ensure_capacity(b, 13)
    cache.free(a)
    assert cache.num_free_blocks == 3 and cache.can_allocate(12)
    with pytest.raises(RuntimeError):
        cache.free(a)


def test_prefix_blocks_are_shared_refcounted_and_evicted_lru():
    """tests/test_kv_cache.py:210-242 restated."""
    cache = PagedKVCache(num_layers=1, num_kv_heads=1, head_dim=4, num_blocks=16, block_size=4, max_seqs=4,
                         max_len=64, dtype=torch.float32, device="cpu", enable_prefix_caching=True)
    shared = list(range(100, 116))
    a_tokens = shared + [1, 2, 3]
    a = cache.allocate(len(a_tokens), token_ids=a_tokens)
    assert cache.lengths[a] == 0
    cache.lengths[a] = len(a_tokens)
    cache.register_prefix(a, a_tokens)
    b_tokens = shared + [7, 8]
    b = cache.allocate(len(b_tokens), token_ids=b_tokens)
    assert cache.lengths[b] == 16
    assert cache.block_tables[b][:4] == cache.block_tables[a][:4]
    assert cache.block_tables[b][4] != cache.block_tables[a][4]
    c = cache.allocate(16, token_ids=shared)
    assert cache.lengths[c] == 12
    cache.free(a)
    cache.free(b)
    cache.free(c)
    assert cache.num_free_blocks == 16
    d = cache.allocate(18, token_ids=shared + [5, 6])
    assert cache.lengths[d] == 16
    cache.free(d)
    e = cache.allocate(64, token_ids=list(range(64)))
    cache.free(e)
    f = cache.allocate(18, token_ids=shared + [5, 6])
    assert cache.lengths[f] == 0


def test_slot_ids_and_lru_reuse_order():
    """Slots from 0 upward; a freed uncached block is reused before older free blocks (kv_cache.py:468-488)."""
    cache = tiny_paged(num_blocks=8, block_size=4)
    s0, s1 = cache.allocate(8), cache.allocate(4)
    assert (s0, s1) == (0, 1)
    assert cache.block_tables[s0] == [0, 1] and cache.block_tables[s1] == [2]
    cache.free(s0)  # releases 1 then 0, each to the head of the queue
    s2 = cache.allocate(12)
    assert cache.block_tables[s2] == [0, 1, 3]
    assert s2 == 0  # the freed slot id is handed out again


# ----------------------------------------------------------------------------- decode context index math


GOLDEN = ROOT / "tests" / "golden"


def _alloc_fixture():
    import json
    import sys

    if str(GOLDEN) not in sys.path:
        sys.path.insert(0, str(GOLDEN))
    import alloc_trace

    meta = json.loads((GOLDEN / "alloc_churn.json").read_text())
    with np.load(GOLDEN / "alloc_churn.npz") as z:
        lengths, flat = z["table_lengths"], z["table_blocks"]
    tables = np.split(flat, np.cumsum(lengths)[:-1])
    return alloc_trace, meta, [t.tolist() for t in tables]


def _prefix_cache(cls=PagedKVCache):
    import alloc_trace

    pool = alloc_trace.PREFIX_POOL
    return cls(1, 1, 1, pool["num_blocks"], pool["block_size"], pool["max_seqs"], pool["max_len"], torch.float16,
               "cpu", enable_prefix_caching=True)


def test_allocator_matches_reference_under_config3_churn():
    """The bf16 B=256 workload's 256 block tables (after 5,000 seeded alloc / grow / free events
    on a 32,768-block pool) equal the ones the reference allocator hands out for the same calls
    (tests/golden/make_alloc_golden.py, engine/kv_cache.py:468-560)."""
    import dataclasses

    from engine import workloads

    _, meta, want = _alloc_fixture()
    shape = dataclasses.replace(workloads.SHAPES[3], num_layers=1, head_dim=8)  # same allocator calls, tiny pool
    batch = workloads.build_decode_batch(shape, "cpu", seed=0, fill_pool=False)
    got = [list(batch.cache.block_tables[s]) for s in batch.slots]
    assert len(got) == meta["config3"]["sequences"] == 256
    for i, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"sequence {i}: first differing block at {next(j for j, (a, b) in enumerate(zip(g, w)) if a != b)}"


def test_allocator_matches_reference_under_prefix_caching_trace():
    """3,000 events of admissions with shared prompt prefixes (prefix hits), growth, preemption
    and frees: every event's observation (slot, table, length, hit tokens, free blocks) equals
    the reference allocator's, by digest."""
    alloc_trace, meta, _ = _alloc_fixture()
    cache = _prefix_cache()
    got = alloc_trace.prefix_churn(cache)
    want = meta["prefix_trace"]["digests"]
    first = next((i for i, (g, w) in enumerate(zip(got, want)) if g != w), None)
    assert first is None, f"first divergence at event {first}"
    assert cache.prefix_hit_tokens == meta["prefix_trace"]["prefix_hit_tokens"] > 0


def test_prefix_trace_catches_a_policy_change():
    """The trace is sensitive to the reuse policy: an allocator that queues released blocks
    without a cached prefix at the back (reused last), instead of the front, diverges."""
    alloc_trace, meta, _ = _alloc_fixture()

    class BackOfQueue(PagedKVCache):
        def _release(self, block: int) -> None:
            self._ref_counts[block] -= 1
            if self._ref_counts[block] == 0:
                self._free_blocks[block] = None

    got = alloc_trace.prefix_churn(_prefix_cache(BackOfQueue))
    assert got != meta["prefix_trace"]["digests"]


def test_decode_context_matches_oracle_inputs():
    cache = tiny_paged(num_blocks=12, block_size=4)
    lengths = [6, 9, 3]
    slots = [cache.allocate(0) for _ in lengths]
    for n_blocks in range(1, 4):
        for s, n in zip(slots, lengths):
            cache.ensure_capacity(s, min(n + 1, n_blocks * 4))
    for s, n in zip(slots, lengths):
        cache.lengths[s] = n
    ctx = cache.decode_context(slots)
    tables = [cache.block_tables[s] for s in slots]
    want = ref.decode_inputs(lengths, tables, 4)
    assert ctx.positions.tolist() == want["positions"].tolist()
    assert ctx.slot_mapping.tolist() == want["slot_mapping"].tolist()
    assert ctx.write_blocks.tolist() == want["write_blocks"].tolist()
    assert ctx.write_offsets.tolist() == want["write_offsets"].tolist()
    assert ctx.context_lens.tolist() == want["context_lens"].tolist()
    # The device-resident rows hold each sequence's blocks; entries past them are stale (the
    # reference pads with block 0) and no kernel reads them.
    assert ctx.block_tables.shape == want["tables"].shape
    for row, t, n in zip(ctx.block_tables.tolist(), want["tables"].tolist(), lengths):
        used = n // 4 + 1
        assert row[:used] == t[:used]
    assert ctx.block_tables.dtype == torch.int32 and ctx.context_lens.dtype == torch.int32
    assert torch.equal(ctx.mask, torch.as_tensor(want["mask"])[:, None, None, :])
    ctx.commit()
    assert [cache.lengths[s] for s in slots] == [7, 10, 4]


def test_decode_context_requires_capacity():
    cache = tiny_paged(num_blocks=4, block_size=4)
    s = cache.allocate(4)
    cache.lengths[s] = 4  # next token needs a second block
    with pytest.raises(ValueError):
        cache.decode_context([s])


def test_fork_copy_on_write_bookkeeping(monkeypatch):
    """A write into a shared, partially filled block gets a private copy (one copy_blocks call)."""
    cache = tiny_paged(num_blocks=10, block_size=4)
    copies = []
    monkeypatch.setattr(cache, "copy_blocks", lambda pairs: copies.append(list(pairs)))
    parent = cache.allocate(7)
    cache.lengths[parent] = 6  # blocks [0, 1]; block 1 holds tokens 4..5
    child = cache.fork(parent)
    assert cache.block_tables[child] == cache.block_tables[parent]
    assert cache.ref_count(cache.block_tables[parent][1]) == 2
    ctx = cache.decode_context([child])  # token 6 goes into shared block 1 -> copied
    old = cache.block_tables[parent][1]
    new = cache.block_tables[child][1]
    assert copies == [[(old, new)]] and new != old
    assert cache.ref_count(old) == 1 and cache.ref_count(new) == 1
    assert cache.block_tables[child][0] == cache.block_tables[parent][0]  # full block stays shared
    assert ctx.slot_mapping.tolist() == [new * 4 + 2]
    cache.decode_context([parent])  # the parent's block is now private: no copy
    assert len(copies) == 1


def _mirror_matches(cache):
    rows = cache.device_tables.rows.numpy()
    for slot, table in cache.block_tables.items():
        assert rows[slot, :len(table)].tolist() == table, f"slot {slot}"
    assert (rows[cache.device_tables.spare_row] == cache.scratch_block).all()


def test_device_tables_follow_every_table_change(monkeypatch):
    """The journal replayed into the mirror reproduces every live table after allocate (with
    prefix hits), ensure_capacity, fork, copy-on-write, free and slot reuse, in any batching
    of the drains. (The mirror is an ordinary tensor, so this runs on the CPU.)"""
    import random

    rnd = random.Random(3)
    cache = tiny_paged(num_blocks=40, block_size=4, max_seqs=6, max_len=48, enable_prefix_caching=True)
    monkeypatch.setattr(cache, "copy_blocks", lambda pairs: None)
    prompt = list(range(13))
    first = cache.allocate(13, prompt)
    cache.lengths[first] = 13
    cache.register_prefix(first, prompt)
    cache.enable_device_tables()  # initial upload of the existing table via the journal
    cache.device_tables.sync()
    _mirror_matches(cache)
    live = [first]
    for step in range(300):
        op = rnd.random()
        if op < 0.25 and cache.num_free_slots and cache.can_allocate(20):
            s = cache.allocate(rnd.randint(1, 20), prompt if rnd.random() < 0.5 else None)
            cache.lengths[s] = max(cache.lengths[s], 1)
            live.append(s)
        elif op < 0.35 and live and cache.num_free_slots:
            live.append(cache.fork(rnd.choice(live)))
        elif op < 0.45 and len(live) > 1:
            s = live.pop(rnd.randrange(len(live)))
            cache.free(s)
        elif live:
            s = rnd.choice(live)
            n = cache.lengths[s]
            if cache.ensure_capacity(s, n + 1):
                try:
                    cache.prepare_writes([s], [n], [1])
                except RuntimeError:
                    continue
                cache.lengths[s] = n + 1
        if rnd.random() < 0.3:  # drains at irregular intervals
            cache.device_tables.sync()
            _mirror_matches(cache)
    cache.device_tables.sync()
    _mirror_matches(cache)


def test_device_table_journal_last_write_wins():
    cache = tiny_paged(num_blocks=12, block_size=4)
    dt = cache.enable_device_tables()
    journal = np.array([[1, 0, 5], [1, 1, 6], [1, 0, 7], [2, 0, 3], [1, 0, 9]], dtype=np.int64)
    flat, blocks = dt.flat_entries(journal)
    got = dict(zip(flat.tolist(), blocks.tolist()))
    assert got == {1 * dt.max_blocks + 0: 9, 1 * dt.max_blocks + 1: 6, 2 * dt.max_blocks: 3}


def test_packed_prefill_slot_mapping():
    cache = tiny_paged(num_blocks=12, block_size=4)
    slots = [cache.allocate(0) for _ in range(2)]
    ctx = cache.packed_prefill_context(slots, [5, 3])
    blocks, offsets = ref.write_index(cache.block_tables, slots, [0, 0], [5, 3], 4)
    assert ctx.slot_mapping.tolist() == (blocks * 4 + offsets).tolist()
    assert ctx.positions.tolist() == [0, 1, 2, 3, 4, 0, 1, 2]


# ----------------------------------------------------------------------------- C ABI


def header_functions(header=None) -> list[str]:
    text = (HEADER if header is None else header).read_text()
    return re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t)\s+(mip_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        spec = importlib.util.spec_from_file_location("mip_build", ROOT / "mini-inference_amd" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _native.load()


def test_header_declares_the_bound_entry_points():
    assert sorted(header_functions()) == sorted(_native.EXPORTED)
    assert sorted(header_functions(PROBE_HEADER)) == sorted(_native.PROBE_EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(_native.LIB_PATH))
    for name in header_functions() + header_functions(PROBE_HEADER):
        assert hasattr(raw, name), f"{name} declared in a header but not exported"
    assert lib.mip_version() >> 16 == 0 and lib.mip_version() & 0xFFFF >= 1
    assert lib.mip_status_string(_native.MIP_OK) == b"ok"
    assert lib.mip_status_string(_native.MIP_EINVAL) == b"invalid argument"
    assert b"unsupported" in lib.mip_status_string(_native.MIP_EUNSUPPORTED)


def test_abi_host_checks_return_before_launch(lib):
    """Empty work returns OK and rejected arguments return EINVAL, with nothing launched."""
    E, OK = _native.MIP_EINVAL, _native.MIP_OK
    app = lib.mip_kv_append
    args = [None, None, 128, 64, 128, 64, None, None, 16, None, 0, 2, 64, 16, _native.MIP_BF16, None]
    assert app(*args) == OK                             # n_tokens = 0
    assert app(*(args[:14] + [7, None])) == E           # unknown dtype
    bad_bs = list(args); bad_bs[13] = 12
    assert app(*bad_bs) == E                            # block size not a power of two
    null = list(args); null[10] = 4
    assert app(*null) == E                              # tokens but null pointers
    dec = lib.mip_paged_decode
    dargs = [None, 896, 64, None, 896, 64, None, None, 64, None, 8, None, 0, 14, 2, 64, 16, 8, 0.125, None, 0,
             None, 0, _native.MIP_BF16, None]
    assert dec(*dargs) == OK                            # batch 0
    g = list(dargs); g[12], g[14] = 4, 3
    assert dec(*g) == E                                 # 14 heads do not split over 3 kv heads
    st = list(dargs); st[12], st[10] = 4, 4
    assert dec(*st) == E                                # table stride below max_blocks
    nul = list(dargs); nul[12] = 4
    assert dec(*nul) == E                               # null pointers
    assert lib.mip_paged_decode_workspace(0, 14, 2, 64, 16, 8, _native.MIP_BF16) == 0
    fused = lib.mip_paged_decode_append
    app = [None, None, 128, 64, 128, 64, None]
    assert fused(*(app + dargs)) == OK                  # batch 0
    nul = list(dargs); nul[12] = 4
    assert fused(*(app + nul)) == E                     # new rows missing
    bad = list(dargs); bad[23] = 9
    assert fused(*(app + bad)) == E                     # unknown dtype
    plan = lib.mip_paged_decode_plan
    assert plan(None, None, 8, 4, 14, 2, 64, 16, 8, _native.MIP_BF16, None, 0, None) == E  # no buffers
    assert plan(None, None, 4, 4, 14, 2, 64, 16, 8, _native.MIP_BF16, None, 0, None) == E  # stride < max_blocks
    assert lib.mip_paged_decode_plan_bytes(0, 14, 2, 64, 16, 8, _native.MIP_BF16) == 0
    rope = lib.mip_rope_kv_append
    rargs = [None, 1152, 64, None, 1152, 64, None, 1152, 64, None, None, 64, None, None, 64, None, 0, 14, 2, 64, 16,
             _native.MIP_BF16, None]
    assert rope(*rargs) == OK                           # n_tokens = 0
    odd = list(rargs); odd[19] = 63
    assert rope(*odd) == E                              # odd head_dim has no rotation pairs
    nul = list(rargs); nul[16] = 4
    assert rope(*nul) == E                              # tokens but null pointers
    dt = list(rargs); dt[21] = 5
    assert rope(*dt) == E                               # unknown dtype
    bs = list(rargs); bs[20] = 24
    assert rope(*bs) == E                               # block size not a power of two
    pf = lib.mip_paged_prefill
    pargs = [None, 896, 64, None, 1152, 64, None, None, 64, None, 8, None, None, 0, 16, 14, 2, 64, 16, 8, 0.125,
             _native.MIP_BF16, None]
    assert pf(*pargs) == OK                             # no sequences
    g = list(pargs); g[13], g[16] = 2, 3
    assert pf(*g) == E                                  # 14 heads do not split over 3 kv heads
    st = list(pargs); st[13], st[10] = 2, 4
    assert pf(*st) == E                                 # table stride below max_blocks
    nul = list(pargs); nul[13] = 2
    assert pf(*nul) == E                                # null pointers
    for cp in (lib.mip_copy_blocks, lib.mip_copy_blocks_host):
        assert cp(None, None, None, 0, 24, 100, 8192, None) == OK  # no pairs
        assert cp(None, None, None, 3, 0, 100, 8192, None) == E    # no layers
        assert cp(None, None, None, -1, 24, 100, 8192, None) == E  # negative count
        assert cp(None, None, None, 3, 24, 100, 8192, None) == E   # pairs but null pointers
        assert cp(16, 16, 16, 3, 1 << 23, 100, 16, None) == E      # one pair alone exceeds a launch's grid


def test_probe_argument_checks(lib):
    """mip_hbm_read_probe refuses bad arguments before it launches anything: an unknown read
    path, chunk sizes that are not whole KiB, and (the LDS-ring paths) a wavefront span of more
    than the 128 chunk ids a wavefront holds."""
    E, OK = _native.MIP_EINVAL, _native.MIP_OK
    probe = lib.mip_hbm_read_probe
    assert probe(16, 1 << 30, 16, 0, 2048, 16, 1, 0, None) == OK        # no chunks: nothing to read
    assert probe(16, 1 << 30, 16, 10, 2048, 16, 1, 3, None) == E        # unknown read path
    assert probe(16, 1 << 30, 16, 10, 1000, 16, 1, 0, None) == E        # not a multiple of 1 KiB
    assert probe(None, 1 << 30, 16, 10, 2048, 16, 1, 0, None) == E      # null base
    for mode in (1, 2):
        assert probe(16, 1 << 30, 16, 1000, 2048, 16, 1, mode, None) == E  # 250 chunks per wavefront


def test_decode_algo_setting(lib):
    """mip_set_decode_algo: returns the previous setting, refuses unknown values, host-only."""
    prev = _native.set_decode_algo("valu")
    try:
        assert _native.set_decode_algo("mfma") == "valu"
        assert _native.set_decode_algo("stream") == "mfma"
        assert lib.mip_set_decode_algo(7) == _native.MIP_EINVAL
        assert lib.mip_set_decode_algo(-1) == _native.MIP_EINVAL
        assert _native.set_decode_algo("auto") == "stream"
    finally:
        _native.set_decode_algo(prev)


# ----------------------------------------------------------------------------- no CPU fallback


def test_kernels_refuse_cpu_tensors():
    k = torch.zeros(5, 2, 4, 8)
    v = torch.zeros_like(k)
    with pytest.raises(RuntimeError):
        paged_ops.kv_append(k, v, torch.zeros(1, 2, 8), torch.zeros(1, 2, 8), torch.zeros(1, dtype=torch.int64))
    with pytest.raises(RuntimeError):
        paged_ops.paged_decode(torch.zeros(1, 4, 8), k, v, torch.zeros(1, 1, dtype=torch.int32),
                               torch.ones(1, dtype=torch.int32))
    with pytest.raises(RuntimeError):
        paged_ops.copy_blocks(k[None], v[None], torch.zeros(1, 2, dtype=torch.int64))
    with pytest.raises(RuntimeError):
        paged_ops.rope_kv_append(torch.zeros(1, 4, 8), torch.zeros(1, 2, 8), torch.zeros(1, 2, 8), torch.ones(1, 8),
                                 torch.zeros(1, 8), k, v, torch.zeros(1, dtype=torch.int64))


def test_host_copy_pairs_are_a_private_copy():
    """Pairs for mip_copy_blocks_host: any host form becomes a contiguous int64 [n, 2] copy, so
    a prepared call keeps the pairs it was prepared with."""
    a = np.array([[1, 2], [3, 4]], dtype=np.int64)
    b = paged_ops._host_pairs(a)
    a[0, 0] = 9
    assert b.tolist() == [[1, 2], [3, 4]] and b.flags["C_CONTIGUOUS"] and b.dtype == np.int64
    assert paged_ops._host_pairs([(5, 6)]).tolist() == [[5, 6]]
    assert paged_ops._host_pairs(torch.tensor([[7, 8]], dtype=torch.int32)).dtype == np.int64
    assert paged_ops._host_pairs(torch.arange(8).view(2, 4)[:, ::2]).tolist() == [[0, 2], [4, 6]]
    assert paged_ops._host_pairs([]).shape == (0, 2)


def test_missing_library_raises(tmp_path):
    with pytest.raises(_native.NativeLibraryMissing):
        _native.load(tmp_path / "absent.so")


def test_product_never_imports_the_oracle():
    for src in (ROOT / "mini-inference_amd").rglob("*.py"):
        text = src.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, flags=re.M), src
        assert "paged_ref" not in text, src


# ----------------------------------------------------------------------------- graph buckets


def test_graph_buckets():
    """engine/cuda_graphs.py:34-47: batch buckets 1, 2, 4, 8, then every 16; KV buckets in whole blocks."""
    from engine.cuda_graphs import _batch_buckets, _kv_buckets

    assert _batch_buckets(256) == [1, 2, 4, 8] + list(range(16, 256, 16)) + [256]
    assert _batch_buckets(5) == [1, 2, 4, 5]
    assert _batch_buckets(8) == [1, 2, 4, 8]
    assert _kv_buckets(1000, None, 16) == [1008]
    assert _kv_buckets(1000, 256, 16) == [256, 512, 768, 1008]
    assert _kv_buckets(520, 256, 32) == [256, 512, 544]

"""HIP-graph decode (engine/cuda_graphs.py) against the eager decode step, on the GPU.

Two caches start from identical contents. Each step runs the eager path on one, replays the
captured graph on the other, and compares the logits and the pools. Replays are separated by
eager work and synchronisations, and every replay is checked.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


def _setup(gpu, lengths, seed=0):
    from engine.kv_cache import PagedKVCache
    from engine.model import Qwen2Config, Qwen2ForCausalLM, random_init_

    cfg = Qwen2Config(vocab_size=512, hidden_size=896, intermediate_size=1024, num_layers=2, num_heads=14,
                      num_kv_heads=2, head_dim=64)
    with torch.device(gpu):
        model = Qwen2ForCausalLM(cfg)
    model = random_init_(model.to(gpu, torch.bfloat16), seed=seed)
    caches = []
    for _ in range(2):
        c = PagedKVCache(cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, num_blocks=256, block_size=16, max_seqs=16,
                         max_len=512, dtype=torch.bfloat16, device=gpu)
        slots = []
        for n in lengths:
            s = c.allocate(n + 8)  # room for the steps below
            c.lengths[s] = n
            slots.append(s)
        caches.append((c, slots))
    gen = torch.Generator(device=gpu).manual_seed(seed + 1)
    for pool in (caches[0][0].k, caches[0][0].v):
        pool.normal_(0.0, 1.0, generator=gen)
    caches[1][0].k.copy_(caches[0][0].k)
    caches[1][0].v.copy_(caches[0][0].v)
    return model, caches


@torch.inference_mode()
def _run(gpu, lengths, batches, exact, graph_rope=True, eager_rope=True):
    from engine.cuda_graphs import GraphedDecoder

    model, ((ec, eslots), (gc, gslots)) = _setup(gpu, lengths)
    assert eslots == gslots
    gd = GraphedDecoder(model, gc, max_batch=16, fuse_rope=graph_rope)
    gd.capture(batches=batches)
    tokens = [(7 * i + 3) % 512 for i in range(len(lengths))]
    nb = ec.num_blocks  # the scratch block (index nb) takes the graph's padding rows
    for step in range(4):
        ctx = ec.decode_context(eslots)
        ctx.fuse_rope = eager_rope
        ids = torch.tensor(tokens, device=gpu).unsqueeze(1)
        want = model.compute_logits(model(ids, ctx.positions.unsqueeze(1), ctx)[:, -1]).float()
        ctx.commit()
        torch.cuda.synchronize()
        got = gd.decode(gslots, tokens)
        assert got is not None
        torch.cuda.synchronize()
        if exact:
            assert torch.equal(got, want), f"step {step}: graph logits differ from eager"
            assert torch.equal(gc.k[:, :nb], ec.k[:, :nb]) and torch.equal(gc.v[:, :nb], ec.v[:, :nb])
        else:
            # padded batch: the GEMMs see a different M, so allow their rounding differences
            err = (got - want).abs().max().item()
            assert err <= 1e-2 * want.abs().max().item() + 1e-3, f"step {step}: {err}"
        assert [gc.lengths[s] for s in gslots] == [ec.lengths[s] for s in eslots]
        tokens = want.argmax(dim=-1).tolist()
    assert gd.replays == 4


def test_graphed_decode_full_bucket_equals_eager(gpu):
    announce("graphed decode, batch 8 = bucket 8, exact")
    _run(gpu, [37, 100, 5, 64, 250, 17, 128, 300], batches=[8], exact=True)


def test_graphed_decode_padded_bucket(gpu):
    announce("graphed decode, batch 5 in bucket 8 (scratch-block padding rows)")
    _run(gpu, [37, 100, 5, 64, 250], batches=[5], exact=False)


def test_graphed_fused_rope_equals_eager_reference_protocol(gpu):
    """Graph with the rotary embedding inside the append kernel vs the eager step that rotates
    q and k in torch (``apply_rope``) and calls ``attend``: identical logits and pools."""
    announce("graphed decode with fused rope vs eager apply_rope + attend, exact")
    _run(gpu, [37, 100, 5, 64, 250, 17, 128, 300], batches=[8], exact=True, graph_rope=True, eager_rope=False)


def test_graphed_unfused_rope_equals_eager(gpu):
    announce("graphed decode, apply_rope + fused append/decode call, vs eager fused rope, exact")
    _run(gpu, [37, 100, 5, 64, 250, 17, 128, 300], batches=[8], exact=True, graph_rope=False, eager_rope=True)


@torch.inference_mode()
def test_graphed_decode_device_tables_follow_growth_fork_and_reuse(gpu):
    """40 steps over 8 sequences that cross block boundaries (new blocks every 16 tokens), with
    a sequence freed and its slot reused at step 12 and a fork (copy-on-write on its first
    write) at step 24. The graph reads the device-resident tables, updated only through the
    cache's journal; the eager step rebuilds them on the host. Logits and pools must match."""
    from engine.cuda_graphs import GraphedDecoder

    announce("graphed decode, device tables under growth, slot reuse and fork")
    lengths = [13, 30, 47, 5, 62, 16, 31, 100]
    model, ((ec, eslots), (gc, gslots)) = _setup(gpu, lengths)
    gd = GraphedDecoder(model, gc, max_batch=8)
    gd.capture(batches=[8])
    tokens = [(5 * i + 1) % 512 for i in range(len(lengths))]
    for step in range(40):
        if step == 12:  # free one sequence, start a new one in its slot
            for c, slots in ((ec, eslots), (gc, gslots)):
                c.free(slots[3])
                s = c.allocate(40)
                c.lengths[s] = 33
                slots[3] = s
        if step == 24:  # replace sequence 5 by a fork of sequence 2 (shared partial block)
            for c, slots in ((ec, eslots), (gc, gslots)):
                c.free(slots[5])
                slots[5] = c.fork(slots[2])
        assert eslots == gslots
        for c, slots in ((ec, eslots), (gc, gslots)):
            for s in slots:
                assert c.ensure_capacity(s, c.lengths[s] + 1)
        ctx = ec.decode_context(eslots)
        ids = torch.tensor(tokens, device=gpu).unsqueeze(1)
        want = model.compute_logits(model(ids, ctx.positions.unsqueeze(1), ctx)[:, -1]).float()
        ctx.commit()
        got = gd.decode(gslots, tokens)
        torch.cuda.synchronize()
        assert got is not None
        assert torch.equal(got, want), f"step {step}: graph logits differ from eager"
        nb = ec.num_blocks
        assert torch.equal(gc.k[:, :nb], ec.k[:, :nb]) and torch.equal(gc.v[:, :nb], ec.v[:, :nb]), f"step {step}"
        assert [gc.lengths[s] for s in gslots] == [ec.lengths[s] for s in eslots]
        tokens = want.argmax(dim=-1).tolist()
    assert gc.cow_copies == ec.cow_copies >= 1

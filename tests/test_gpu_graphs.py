"""HIP-graph decode (engine/cuda_graphs.py) against the eager decode step and the oracle, on the GPU.

Two caches start from identical contents. Each step runs the eager path on one, replays the
captured graph on the other, and compares the logits and the pools. Replays are separated by
eager work and synchronisations, and every replay is checked. With an attention-probe model
(its "logits" are the attention outputs of every layer) the replays are also checked against
the float64 oracle and the oracle's append.
"""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import paged_ref as ref

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
def _run(gpu, lengths, batches, exact, graph_rope=True, eager_rope=True, gd_out=None):
    from engine.cuda_graphs import GraphedDecoder

    model, ((ec, eslots), (gc, gslots)) = _setup(gpu, lengths)
    assert eslots == gslots
    gd = GraphedDecoder(model, gc, max_batch=16, fuse_rope=graph_rope)
    gd.capture(batches=batches)
    if gd_out is not None:
        gd_out.append(gd)
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


def test_graphed_decode_all_buckets_replay_16_and_8(gpu):
    """capture() of every bucket of a max_batch=16 decoder (1, 2, 4, 8, 16), as the reference
    engine calls it (engine/engine.py:87), then replays of bucket 16 and of bucket 8: every
    graph shares one workspace sized for all buckets, allocated before the first capture."""
    announce("graphed decode, all buckets of max_batch 16, replay bucket 16")
    lens16 = [37, 100, 5, 64, 250, 17, 128, 300, 3, 77, 190, 45, 9, 260, 31, 140]
    kept = []
    _run(gpu, lens16, batches=None, exact=True, gd_out=kept)
    gd = kept[0]
    assert sorted(b for b, _ in gd.graphs) == [1, 2, 4, 8, 16]
    ws = gd.workspace.data_ptr()
    assert all(ctx.owner.workspace.data_ptr() == ws for _, _, ctx in gd.graphs.values())
    announce("graphed decode, all buckets of max_batch 16, replay bucket 8")
    _run(gpu, lens16[:8], batches=None, exact=True)


class _AttentionProbe(torch.nn.Module):
    """Stand-in for the model whose per-step output is the paged attention itself.

    Token t gives q = ``q_tab[t]`` and, per layer, k = ``k_tab[t, l]``, v = ``v_tab[t, l]``;
    ``forward`` returns every layer's ``ctx.attend`` output, so a graph replay's "logits" are
    ``[B, layers * Hq * D]`` attention outputs that the oracle can check.
    """

    def __init__(self, vocab, hq, hkv, d, layers, dtype, device, seed=0):
        super().__init__()
        self.cfg = types.SimpleNamespace(num_heads=hq)
        g = torch.Generator().manual_seed(seed)
        self.q_tab = torch.randn(vocab, hq, d, generator=g).to(dtype).to(device)
        self.k_tab = torch.randn(vocab, layers, hkv, d, generator=g).to(dtype).to(device)
        self.v_tab = torch.randn(vocab, layers, hkv, d, generator=g).to(dtype).to(device)
        self.layers = layers

    def forward(self, ids, positions, ctx):
        t = ids[:, 0]
        q = self.q_tab[t].unsqueeze(2)
        outs = [ctx.attend(layer, q, self.k_tab[t, layer].unsqueeze(2), self.v_tab[t, layer].unsqueeze(2))
                for layer in range(self.layers)]
        return torch.stack(outs, 1).reshape(t.shape[0], 1, -1)

    def compute_logits(self, hidden):
        return hidden


def _storage(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


@torch.inference_mode()
def test_graphed_attention_replays_match_oracle_and_eager(gpu):
    """All buckets of a max_batch=16 decoder captured; replays at batch 16 (bucket 16), batch
    8 (bucket 8) and batch 5 (bucket 8, three padding rows on the scratch block). Each replay:
    attention outputs within the bf16 bound of the float64 oracle, the pool (scratch block
    aside) equal to the oracle's append of the step's k/v rows, and, for full buckets, outputs
    and pool bit-identical to the eager PagedDecodeContext on a twin cache."""
    from engine.cuda_graphs import GraphedDecoder
    from engine.kv_cache import PagedKVCache

    hq, hkv, d, bs, layers, vocab = 14, 2, 64, 16, 2, 64
    probe = _AttentionProbe(vocab, hq, hkv, d, layers, torch.bfloat16, gpu, seed=3)
    lengths = [37, 100, 5, 64, 250, 17, 128, 300, 3, 77, 190, 45, 9, 260, 31, 140]
    caches = []
    for _ in range(2):
        c = PagedKVCache(layers, hkv, d, num_blocks=320, block_size=bs, max_seqs=16, max_len=512,
                         dtype=torch.bfloat16, device=gpu)
        sl = []
        for n in lengths:
            s = c.allocate(n + 8)
            c.lengths[s] = n
            sl.append(s)
        caches.append((c, sl))
    (ec, eslots), (gc, gslots) = caches
    gen = torch.Generator(device=gpu).manual_seed(4)
    ec.k.normal_(0.0, 1.0, generator=gen)
    ec.v.normal_(0.0, 1.0, generator=gen)
    gc.k.copy_(ec.k)
    gc.v.copy_(ec.v)
    gd = GraphedDecoder(probe, gc, max_batch=16, fuse_rope=False)
    gd.capture()
    sc = gc.scratch_block
    plan = [(16, 2), (8, 2), (5, 1)]
    step = 0
    for n, reps in plan:
        for _ in range(reps):
            tokens = [(11 * i + 5 * step + 1) % vocab for i in range(n)]
            es, gs = eslots[:n], gslots[:n]
            announce(f"graphed attention probe, batch {n}, step {step}")
            pos = [gc.lengths[s] for s in gs]
            tables = [list(gc.block_tables[s]) for s in gs]
            before = [(_storage(gc.k[layer]), _storage(gc.v[layer])) for layer in range(layers)]
            ctx = ec.decode_context(es)
            ids = torch.tensor(tokens, device=gpu).unsqueeze(1)
            want_eager = probe(ids, ctx.positions.unsqueeze(1), ctx)[:, -1].float()
            ctx.commit()
            got = gd.decode(gs, tokens)
            torch.cuda.synchronize()
            assert got is not None
            t = torch.tensor(tokens, device=gpu)
            blocks = np.asarray([tb[p // bs] for tb, p in zip(tables, pos)])
            offs = np.asarray(pos) % bs
            for layer in range(layers):
                wk, wv = before[layer]
                ref.append(wk, wv, blocks, offs, _storage(probe.k_tab[t, layer]), _storage(probe.v_tab[t, layer]))
                assert np.array_equal(_storage(gc.k[layer])[:sc], wk[:sc]), f"step {step} layer {layer}: K pool"
                assert np.array_equal(_storage(gc.v[layer])[:sc], wv[:sc]), f"step {step} layer {layer}: V pool"
                want = ref.attention_f64(probe.q_tab[t].float().cpu().numpy(), gc.k[layer].float().cpu().numpy(),
                                         gc.v[layer].float().cpu().numpy(), tables, [p + 1 for p in pos], bs)
                g = got.view(n, layers, hq, d)[:, layer].cpu().numpy()
                half = 0.5 * np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
                err = float((np.abs(g - want) - half).max())
                assert err <= 2e-3, f"step {step} layer {layer}: {err}"
            if n in (16, 8):  # full buckets: the graph runs exactly the eager kernels
                assert torch.equal(got, want_eager), f"step {step}: graph differs from eager"
                assert torch.equal(gc.k[:, :sc], ec.k[:, :sc]) and torch.equal(gc.v[:, :sc], ec.v[:, :sc])
            _ = (got * 2).sum().item()  # unrelated eager work between replays
            step += 1
    assert gd.replays == step

"""The model through mini-inference_amd's contexts against the same model through the reference's own
formulation of attention, logits compared.

A random-init Qwen2 (2 layers of the Qwen2.5-0.5B attention shape) prefills four prompts in
one packed pass and then decodes six steps, teacher-forced, twice:
  A. through PagedKVCache's PackedPrefillContext and PagedDecodeContext (the HIP kernels);
  B. through two small contexts that do what the reference's contexts do
     (engine/kv_cache.py:252-294 and :611-620): write the new K/V rows at their slots, then
     read the keys back through the block tables and run SDPA with the reference's masks,
     restated by the oracle (paged_ref.packed_prefill_torch / paged_decode_torch) on a CPU
     copy of the pool.
Same weights, same tokens, same block tables and positions; only the attention path differs.
Bar: max |A - B| over every logit, relative to max |B|.
"""

from __future__ import annotations

import random

import pytest
import torch

from conftest import announce
from oracle import paged_ref as ref
from test_gpu_engine_flow import BS, _model

pytestmark = pytest.mark.gpu

# fp32: both paths accumulate in fp32 (measured 8.6e-7 on the logits). bf16: the reference's
# SDPA on the CPU rounds its intermediate products to bf16, the kernels do not (measured 1.4e-2).
REL_TOL = {torch.float32: 1e-5, torch.bfloat16: 3e-2}


class RefPrefill:
    """engine/kv_cache.py:252-294 with a prefix of ``starts`` tokens: append, then read back and SDPA."""

    def __init__(self, pool_k, pool_v, tables, starts, lengths, bs):
        self.pool_k, self.pool_v, self.tables = pool_k, pool_v, tables
        self.starts, self.lengths, self.bs = starts, lengths, bs
        blocks, offs = ref.write_index(tables, range(len(lengths)), starts, lengths, bs)
        self.blocks, self.offs = torch.from_numpy(blocks), torch.from_numpy(offs)

    def attend(self, layer_idx, q, k, v):
        kl, vl = self.pool_k[layer_idx], self.pool_v[layer_idx]
        kl[self.blocks, :, self.offs] = k[0].transpose(0, 1).cpu()
        vl[self.blocks, :, self.offs] = v[0].transpose(0, 1).cpu()
        out = ref.packed_prefill_torch(q.cpu(), kl, vl, self.tables, self.starts, self.lengths, self.bs)
        return out.to(q.device)


class RefDecode:
    """engine/kv_cache.py:592-620: append the new token, gather the padded tables, masked SDPA."""

    def __init__(self, pool_k, pool_v, lengths, tables, bs):
        self.pool_k, self.pool_v = pool_k, pool_v
        self.inputs = ref.decode_inputs(lengths, tables, bs)

    def attend(self, layer_idx, q, k, v):
        out = ref.paged_decode_torch(q.cpu(), self.pool_k[layer_idx], self.pool_v[layer_idx], k.cpu(), v.cpu(),
                                     self.inputs)
        return out.to(q.device)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@torch.inference_mode()
def test_model_logits_match_reference_attention_path(gpu, dtype):
    from engine.kv_cache import PagedKVCache

    announce(f"model parity: kernels vs the reference attention path, {dtype}")
    cfg, model = _model(gpu, dtype)
    rnd = random.Random(3)
    prompt_lens = [5, 17, 33, 70]
    prompts = [[rnd.randrange(cfg.vocab_size) for _ in range(n)] for n in prompt_lens]
    forced = [[rnd.randrange(cfg.vocab_size) for _ in range(6)] for _ in prompt_lens]
    cache = PagedKVCache.for_model(cfg, num_blocks=48, block_size=BS, max_seqs=4, max_len=128, dtype=dtype,
                                   device=gpu)
    slots = [cache.allocate(n) for n in prompt_lens]
    pool_k = torch.zeros(cache.k.shape, dtype=dtype)  # the reference path's own pool (CPU)
    pool_v = torch.zeros(cache.v.shape, dtype=dtype)

    worst = {"logits": 0.0, "rows": 0.0}

    def compare(a, b, what, kind="logits"):
        scale = float(b.abs().max())
        err = float((a - b).abs().max()) / scale
        worst[kind] = max(worst[kind], err)
        assert err <= REL_TOL[dtype], f"{what}: max |kernels - reference| / max |reference| = {err:.3g}"

    # Packed prefill of every prompt (no cached prefix).
    tables = [list(cache.block_tables[s]) for s in slots]
    ids = torch.tensor([[t for p in prompts for t in p]], device=gpu)
    ctx = cache.packed_prefill_context(slots, prompt_lens)
    hidden_a = model(ids, ctx.positions.unsqueeze(0), ctx)
    logits_a = model.compute_logits(hidden_a[0, ctx.last_index]).float()
    positions = ctx.positions.clone()
    last = ctx.last_index.clone()
    ctx.commit()
    rctx = RefPrefill(pool_k, pool_v, tables, [0] * len(slots), prompt_lens, BS)
    hidden_b = model(ids, positions.unsqueeze(0), rctx)
    logits_b = model.compute_logits(hidden_b[0, last]).float()
    compare(logits_a, logits_b, "prefill")

    # Decode steps, teacher-forced.
    for step in range(6):
        lengths = [cache.lengths[s] for s in slots]
        for s, n in zip(slots, lengths):
            assert cache.ensure_capacity(s, n + 1)
        tables = [list(cache.block_tables[s]) for s in slots]
        ids = torch.tensor([f[step] for f in forced], device=gpu).unsqueeze(1)
        ctx = cache.decode_context(slots)
        pos = ctx.positions.unsqueeze(1)
        logits_a = model.compute_logits(model(ids, pos, ctx)[:, -1]).float()
        ctx.commit()
        rctx = RefDecode(pool_k, pool_v, lengths, tables, BS)
        logits_b = model.compute_logits(model(ids, pos, rctx)[:, -1]).float()
        compare(logits_a, logits_b, f"decode step {step}")

    # Every token both paths appended sits at the same slot. Layer 0's rows depend only on the
    # embeddings, so they are bit-identical; later layers' rows carry the attention difference.
    for layer in range(cfg.num_layers):
        for s in slots:
            blocks, offs = ref.write_index([cache.block_tables[s]], [0], [0], [cache.lengths[s]], BS)
            rows = (torch.from_numpy(blocks), slice(None), torch.from_numpy(offs))
            for pa, pb in ((cache.k, pool_k), (cache.v, pool_v)):
                ra = pa[layer].cpu()[rows]
                rb = pb[layer][rows]
                if layer == 0:
                    assert torch.equal(ra, rb), f"sequence {s}: layer-0 K/V rows differ"
                else:
                    compare(ra.float(), rb.float(), f"layer {layer} sequence {s} K/V rows", "rows")
    announce(f"model parity {dtype}: worst relative difference, logits {worst['logits']:.3g}, "
             f"K/V rows past layer 0 {worst['rows']:.3g}")

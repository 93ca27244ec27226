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
Bar: max |A - B| over every logit, relative to max |B|. In bf16 the reference's CPU SDPA rounds
its intermediate products to bf16, so B carries an error of its own; a third run C does what B
does with the attention in fp32 (q, K and V widened, the output rounded back to bf16).

Logits of a bf16 model amplify every last-bit difference of an attention output through the
layers after it, so the logit bounds stay loose. The sharp check is layer 0, whose q, K and V
depend only on the tokens and positions and so are the same in A and C: there every attention
output of A is within one bf16 ulp of C's (both round a near-exact fp32 result once), and the
mean signed difference is far below an ulp (no systematic bias).
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
# bf16 against the reference path with fp32 attention (C): both keep the softmax and the
# weighted sum in fp32 and round once to bf16, so only that rounding and what it feeds differ.
REL_TOL_FP32_ATTN = 2e-2  # measured 8.9e-3


class Layer0:
    """Passes ``attend`` through to a context and keeps layer 0's output."""

    def __init__(self, inner):
        self.inner, self.out = inner, None
        self.fuse_rope = getattr(inner, "fuse_rope", False)  # keep the context's protocol

    def _keep(self, layer_idx, out):
        if layer_idx == 0:
            self.out = out.float().cpu()
        return out

    def attend(self, layer_idx, q, k, v):
        return self._keep(layer_idx, self.inner.attend(layer_idx, q, k, v))

    def attend_rope(self, layer_idx, q, k, v, cos, sin):
        return self._keep(layer_idx, self.inner.attend_rope(layer_idx, q, k, v, cos, sin))


def check_layer0(a: torch.Tensor, c: torch.Tensor, dtype, what: str, stats: dict) -> None:
    """Layer-0 attention outputs of the kernels (a) against the fp32-attention reference (c)."""
    d = a - c
    if dtype == torch.float32:
        err = float(d.abs().max()) / float(c.abs().max())
        stats["l0_max"] = max(stats["l0_max"], err)
        assert err <= 1e-5, f"{what}: layer-0 attention differs by {err:.3g} relative"
        return
    # One bf16 ulp of c, elementwise (8 significant bits: 2^(e - 7) for |c| in [2^e, 2^(e+1))),
    # plus a floor for outputs near zero, where the sum of p * v cancels and the two fp32 sums'
    # own errors (a few 2^-24 of the terms' size) exceed the output's ulp.
    ulp = torch.exp2(torch.floor(torch.log2(c.abs().clamp_min(2.0 ** -120))) - 7)
    slack = 2.0 ** -14 * float(c.abs().max())
    ratio = (d.abs() - slack).clamp_min(0.0) / ulp
    over = float(ratio.max())
    stats["l0_max"] = max(stats["l0_max"], over)
    i = int(ratio.flatten().argmax())
    assert over <= 1.0, (f"{what}: a layer-0 attention output is {over:.3g} bf16 ulps (beyond {slack:.3g}) from the "
                         f"fp32 reference: kernels {float(a.flatten()[i]):.6g}, reference {float(c.flatten()[i]):.6g}, "
                         f"max |reference| {float(c.abs().max()):.4g}; raw max {float((d.abs() / ulp).max()):.3g} ulps")
    bias = float(d.mean()) / float(c.abs().mean())
    stats["l0_bias"] = max(stats["l0_bias"], abs(bias))
    stats["l0_frac"] = max(stats["l0_frac"], float((d != 0).float().mean()))
    assert abs(bias) <= 2e-4, f"{what}: layer-0 attention outputs are biased by {bias:.3g} of their mean magnitude"


class RefPrefill:
    """engine/kv_cache.py:252-294 with a prefix of ``starts`` tokens: append, then read back and SDPA."""

    def __init__(self, pool_k, pool_v, tables, starts, lengths, bs, wide=False):
        self.pool_k, self.pool_v, self.tables, self.wide = pool_k, pool_v, tables, wide
        self.starts, self.lengths, self.bs = starts, lengths, bs
        blocks, offs = ref.write_index(tables, range(len(lengths)), starts, lengths, bs)
        self.blocks, self.offs = torch.from_numpy(blocks), torch.from_numpy(offs)

    def attend(self, layer_idx, q, k, v):
        kl, vl = self.pool_k[layer_idx], self.pool_v[layer_idx]
        kl[self.blocks, :, self.offs] = k[0].transpose(0, 1).cpu()
        vl[self.blocks, :, self.offs] = v[0].transpose(0, 1).cpu()
        if self.wide:  # the same formulation with the attention in fp32, rounded back once
            out = ref.packed_prefill_torch(q.cpu().float(), kl.float(), vl.float(), self.tables, self.starts,
                                           self.lengths, self.bs).to(q.dtype)
        else:
            out = ref.packed_prefill_torch(q.cpu(), kl, vl, self.tables, self.starts, self.lengths, self.bs)
        return out.to(q.device)


class RefDecode:
    """engine/kv_cache.py:592-620: append the new token, gather the padded tables, masked SDPA."""

    def __init__(self, pool_k, pool_v, lengths, tables, bs, wide=False):
        self.pool_k, self.pool_v, self.wide = pool_k, pool_v, wide
        self.inputs = ref.decode_inputs(lengths, tables, bs)

    def attend(self, layer_idx, q, k, v):
        kl, vl = self.pool_k[layer_idx], self.pool_v[layer_idx]
        if self.wide:
            # paged_decode_torch writes the new rows into the pool it is given: write them into
            # this path's own pool in its dtype first, then attend over a widened copy.
            wk, wv = kl.float(), vl.float()
            out = ref.paged_decode_torch(q.cpu().float(), wk, wv, k.cpu().float(), v.cpu().float(), self.inputs)
            kl.copy_(wk.to(kl.dtype))
            vl.copy_(wv.to(vl.dtype))
            return out.to(q.dtype).to(q.device)
        out = ref.paged_decode_torch(q.cpu(), kl, vl, k.cpu(), v.cpu(), self.inputs)
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
    wide = dtype != torch.float32  # run C: the reference path with the attention in fp32
    pool_kc, pool_vc = pool_k.clone(), pool_v.clone()

    worst = {"logits": 0.0, "rows": 0.0, "logits_fp32_attn": 0.0}
    l0 = {"l0_max": 0.0, "l0_bias": 0.0, "l0_frac": 0.0}

    def compare(a, b, what, kind="logits"):
        scale = float(b.abs().max())
        err = float((a - b).abs().max()) / scale
        worst[kind] = max(worst[kind], err)
        tol = REL_TOL_FP32_ATTN if kind == "logits_fp32_attn" else REL_TOL[dtype]
        assert err <= tol, f"{what} ({kind}): max |kernels - reference| / max |reference| = {err:.3g}"

    # Packed prefill of every prompt (no cached prefix).
    tables = [list(cache.block_tables[s]) for s in slots]
    ids = torch.tensor([[t for p in prompts for t in p]], device=gpu)
    ctx = cache.packed_prefill_context(slots, prompt_lens)
    actx = Layer0(ctx)
    hidden_a = model(ids, ctx.positions.unsqueeze(0), actx)
    logits_a = model.compute_logits(hidden_a[0, ctx.last_index]).float()
    positions = ctx.positions.clone()
    last = ctx.last_index.clone()
    ctx.commit()
    rctx = Layer0(RefPrefill(pool_k, pool_v, tables, [0] * len(slots), prompt_lens, BS))
    hidden_b = model(ids, positions.unsqueeze(0), rctx)
    logits_b = model.compute_logits(hidden_b[0, last]).float()
    compare(logits_a, logits_b, "prefill")
    if wide:
        cctx = Layer0(RefPrefill(pool_kc, pool_vc, tables, [0] * len(slots), prompt_lens, BS, wide=True))
        logits_c = model.compute_logits(model(ids, positions.unsqueeze(0), cctx)[0, last]).float()
        compare(logits_a, logits_c, "prefill", "logits_fp32_attn")
    check_layer0(actx.out, (cctx if wide else rctx).out, dtype, "prefill", l0)

    # Decode steps, teacher-forced.
    for step in range(6):
        lengths = [cache.lengths[s] for s in slots]
        for s, n in zip(slots, lengths):
            assert cache.ensure_capacity(s, n + 1)
        tables = [list(cache.block_tables[s]) for s in slots]
        ids = torch.tensor([f[step] for f in forced], device=gpu).unsqueeze(1)
        ctx = cache.decode_context(slots)
        pos = ctx.positions.unsqueeze(1)
        actx = Layer0(ctx)
        logits_a = model.compute_logits(model(ids, pos, actx)[:, -1]).float()
        ctx.commit()
        rctx = Layer0(RefDecode(pool_k, pool_v, lengths, tables, BS))
        logits_b = model.compute_logits(model(ids, pos, rctx)[:, -1]).float()
        compare(logits_a, logits_b, f"decode step {step}")
        if wide:
            cctx = Layer0(RefDecode(pool_kc, pool_vc, lengths, tables, BS, wide=True))
            logits_c = model.compute_logits(model(ids, pos, cctx)[:, -1]).float()
            compare(logits_a, logits_c, f"decode step {step}", "logits_fp32_attn")
        check_layer0(actx.out, (cctx if wide else rctx).out, dtype, f"decode step {step}", l0)

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
             f"logits against fp32 attention {worst['logits_fp32_attn']:.3g}, K/V rows past layer 0 {worst['rows']:.3g}; "
             f"layer-0 attention: max {l0['l0_max']:.3g} ({'ulps' if wide else 'relative'}), "
             f"bias {l0['l0_bias']:.3g}, differing outputs {l0['l0_frac']:.3g}")

"""Write the golden decode fixture (cfg1_decode.npz / .json) from the float64 oracle.

    python tests/golden/make_golden.py

The reference ships no on-disk vectors for this path, so the fixture is the oracle's own
output on the seeded case of ``cfg1.py``, cross-checked at generation time against the
oracle's restatement of the reference torch path (append + gather + SDPA, fp32) and
against per-sequence SDPA on contiguous keys (the check of the reference's
tests/test_kv_cache.py:179-207).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT, HERE):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import cfg1  # noqa: E402
from oracle import paged_ref as ref  # noqa: E402


def compute(inp: dict) -> dict:
    k_pool, v_pool = inp["k_pool"].copy(), inp["v_pool"].copy()
    di = ref.decode_inputs(inp["ctx"], inp["tables"], cfg1.BS)
    ref.append(k_pool, v_pool, di["write_blocks"], di["write_offsets"], inp["k_new"], inp["v_new"])
    out64 = ref.attention_f64(inp["q"], k_pool, v_pool, inp["tables"], di["context_lens"], cfg1.BS)
    return {"k_pool": k_pool, "v_pool": v_pool, "out": out64, "inputs": di}


def main() -> None:
    inp = cfg1.make_inputs()
    res = compute(inp)
    # Cross-check 1: the reference's torch path (fp32 CPU) on the same inputs.
    di = res["inputs"]
    t_out = ref.paged_decode_torch(torch.from_numpy(inp["q"])[:, :, None], torch.from_numpy(inp["k_pool"].copy()),
                                   torch.from_numpy(inp["v_pool"].copy()), torch.from_numpy(inp["k_new"])[:, :, None],
                                   torch.from_numpy(inp["v_new"])[:, :, None], di)[:, :, 0].numpy()
    err = float(np.abs(t_out - res["out"]).max())
    assert err < 2e-5, f"torch path vs float64 oracle: {err}"
    # Cross-check 2: each sequence alone over its contiguous keys.
    for b, n in enumerate(inp["ctx"]):
        j = np.arange(n + 1)
        blk = np.asarray(inp["tables"][b])[j // cfg1.BS]
        keys = torch.from_numpy(res["k_pool"][blk, :, j % cfg1.BS]).permute(1, 0, 2)[None]
        vals = torch.from_numpy(res["v_pool"][blk, :, j % cfg1.BS]).permute(1, 0, 2)[None]
        one = ref.sdpa_attention(torch.from_numpy(inp["q"][b:b + 1])[:, :, None], keys, vals)[0, :, 0].numpy()
        assert float(np.abs(one - res["out"][b]).max()) < 2e-5
    blocks = cfg1.touched_blocks(inp["tables"])
    np.savez(cfg1.NPZ, out=res["out"], context_lens=di["context_lens"], slot_mapping=di["slot_mapping"])
    meta = {
        "case": "fp32, 1 layer, Hq 14 / Hkv 2, D 64, 512 blocks of 16, B 8, ctx U[16,256], chunked permutation tables",
        "inputs_sha256": cfg1.inputs_sha256(inp),
        "touched_blocks": len(blocks),
        "pool_after_append_sha256": cfg1.blocks_sha256(res["k_pool"], res["v_pool"], blocks),
        "oracle": "attention_f64 (float64); cross-checked: torch path max-abs %.3g" % err,
    }
    cfg1.META.write_text(json.dumps(meta, indent=1) + "\n")
    print(json.dumps(meta, indent=1))


if __name__ == "__main__":
    main()

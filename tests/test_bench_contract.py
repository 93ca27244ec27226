"""bench.py's contract on the CPU: the single-GPU refusal, the algorithmic-byte formulas the
bench line's `value` and `roofline.achieved` rest on (checked against hand counts), and the
committed traffic summary it reads for `roofline.traffic`."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "single GPU" in r.stderr and r.stdout == ""


def _shape(**kw):
    base = dict(dtype=torch.bfloat16, batch=2, num_heads=4, num_kv_heads=2, head_dim=8, block_size=4)
    base.update(kw)
    return SimpleNamespace(**base)


def test_attention_bytes_hand_count():
    # K and V rows attended: 2 (K, V) x 2 kv heads x (5 + 9) keys x 8 dims x 2 bytes = 896;
    # q read + output written: 2 x 2 sequences x 4 heads x 8 dims x 2 bytes = 256;
    # block-table entries: (ceil(5/4) + ceil(9/4)) x 4 bytes = 20; context lengths 2 x 4 = 8.
    assert bench.attention_bytes([5, 9], _shape()) == 896 + 256 + 20 + 8
    # fp32 doubles the data terms only.
    assert bench.attention_bytes([5, 9], _shape(dtype=torch.float32)) == 2 * (896 + 256) + 20 + 8


def test_append_bytes_hand_count():
    # Read and write of each sequence's new K and V rows (2 x 2 x 2 kv heads x 8 dims x 2 bytes
    # per sequence, for 2 sequences) plus one 8-byte slot per sequence.
    assert bench.append_bytes(_shape()) == 2 * (2 * 2 * 2 * 8 * 2) + 8 * 2


def test_config3_bytes_per_call_match_the_formula_in_words():
    # 512 bytes per attended key at the Qwen2.5-0.5B shape in bf16 (2 kv heads x 64 dims x 2
    # bytes, K and V), 3,584 bytes of q and output per sequence, 1,032 bytes of append per token.
    s = _shape(batch=1, num_heads=14, num_kv_heads=2, head_dim=64, block_size=16)
    assert bench.attention_bytes([16], s) - bench.attention_bytes([0], s) == 16 * 512 + 4
    assert bench.attention_bytes([0], s) == 3584 + 4
    assert bench.append_bytes(s) == 1032


def test_traffic_summary_is_readable_and_plausible():
    d = json.loads(bench.TRAFFIC_FILE.read_text())
    t, alg = d["hbm_bytes_per_launch"], d["algorithmic_bytes_per_call"]
    kernels = d["kernels"]
    assert t == sum(kernels[k]["fetch_bytes"] + kernels[k]["write_bytes"] for k in ("main", "merge"))
    # Copy-calibrated counters of the append + attention call: at least the algorithmic bytes,
    # and within a fifth above them.
    assert alg <= t <= 1.2 * alg

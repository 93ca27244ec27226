"""Pins the oracle's packed prefill attention (oracle/paged_ref.py ``prefill_attention_f64``).

Checks, by kind:
  * the reference's own formulation restated (``packed_prefill_torch``: prefix read-back and
    the dense ``[N, keys]`` mask of engine/kv_cache.py:262-294, torch fp32 SDPA) against the
    float64 per-sequence loop, with and without cached prefixes;
  * one new token per sequence at position L-1 is decode attention over L keys
    (``attention_f64``, pinned by tests/test_oracle.py);
  * closed forms: a fresh sequence's first token returns value row 0;
  * invariants: splitting a sequence's new tokens over two passes (the second one with the
    first one's tokens as its cached prefix), and reordering the sequences in the pack, leave
    every output unchanged;
  * planted mistakes (``<`` for ``<=``, positions that ignore the cached prefix, GQA
    ``h % Hkv``) that at least one check must catch.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref


def case(starts, lengths, hq=4, hkv=2, d=8, bs=4, seed=0):
    """Pool with every sequence's keys 0 .. end-1 in scattered blocks; data N(0, 1)."""
    rnd = random.Random(seed)
    ends = [a + n for a, n in zip(starts, lengths)]
    need = [(e + bs - 1) // bs for e in ends]
    nb = sum(need) + 3
    ids = list(range(nb))
    rnd.shuffle(ids)
    tables, cur = [], 0
    for k in need:
        tables.append(ids[cur:cur + k])
        cur += k
    g = torch.Generator().manual_seed(seed)
    k_pool = torch.randn(nb + 1, hkv, bs, d, generator=g)
    v_pool = torch.randn(nb + 1, hkv, bs, d, generator=g)
    q = torch.randn(sum(lengths), hq, d, generator=g)
    return tables, k_pool, v_pool, q


def f64(q, k_pool, v_pool, tables, starts, lengths, bs):
    return ref.prefill_attention_f64(q.numpy(), k_pool.numpy(), v_pool.numpy(), tables, starts, lengths, bs)


@pytest.mark.parametrize("starts,lengths", [([0, 0, 0], [5, 1, 9]), ([7, 0, 12], [3, 6, 1]), ([16, 3], [17, 4])])
@pytest.mark.parametrize("hq,hkv", [(4, 2), (6, 1), (3, 3)])
def test_prefill_matches_reference_formulation(starts, lengths, hq, hkv):
    tables, kp, vp, q = case(starts, lengths, hq, hkv)
    want = ref.packed_prefill_torch(q.transpose(0, 1).unsqueeze(0), kp, vp, tables, starts, lengths, 4)
    got = f64(q, kp, vp, tables, starts, lengths, 4)
    assert np.abs(got - want[0].transpose(0, 1).double().numpy()).max() < 1e-5


def test_single_new_token_is_decode_attention():
    starts, lengths = [9, 0, 30, 4], [1, 1, 1, 1]
    tables, kp, vp, q = case(starts, lengths, seed=2)
    got = f64(q, kp, vp, tables, starts, lengths, 4)
    want = ref.attention_f64(q.numpy(), kp.numpy(), vp.numpy(), tables, [a + 1 for a in starts], 4)
    assert np.abs(got - want).max() < 1e-12


def test_first_fresh_token_returns_value_row_zero():
    tables, kp, vp, q = case([0, 0], [3, 2], seed=3)
    got = f64(q, kp, vp, tables, [0, 0], [3, 2], 4)
    for s, row in ((0, 0), (1, 3)):
        v0 = vp[tables[s][0], :, 0].double().numpy()  # [Hkv, D]
        assert np.abs(got[row] - np.repeat(v0, 2, axis=0)).max() < 1e-12


def test_split_passes_and_sequence_order_are_invariant():
    starts, lengths = [5, 0, 11], [9, 13, 6]
    tables, kp, vp, q = case(starts, lengths, seed=4)
    full = f64(q, kp, vp, tables, starts, lengths, 4)
    # First pass: the first 4 new tokens of each sequence; second pass: the rest, their prefix now cached.
    first = [4, 4, 4]
    rows1 = np.concatenate([np.arange(sum(lengths[:s]), sum(lengths[:s]) + first[s]) for s in range(3)])
    rows2 = np.concatenate([np.arange(sum(lengths[:s]) + first[s], sum(lengths[:s + 1])) for s in range(3)])
    a = f64(q[rows1], kp, vp, tables, starts, first, 4)
    b = f64(q[rows2], kp, vp, tables, [st + f for st, f in zip(starts, first)],
            [n - f for n, f in zip(lengths, first)], 4)
    assert np.abs(a - full[rows1]).max() < 1e-12
    assert np.abs(b - full[rows2]).max() < 1e-12
    order = [2, 0, 1]
    rows = np.concatenate([np.arange(sum(lengths[:s]), sum(lengths[:s + 1])) for s in order])
    c = f64(q[rows], kp, vp, [tables[s] for s in order], [starts[s] for s in order], [lengths[s] for s in order], 4)
    assert np.abs(c - full[rows]).max() < 1e-12


def _mutant(kind):
    orig = ref.prefill_attention_f64

    def f(q, k_layer, v_layer, tables, starts, lengths, block_size, scale=None):
        if kind == "strict":  # j < position: every cached-prefix token position shifted down one
            return orig(q, k_layer, v_layer, tables, [max(st - 1, 0) for st in starts], lengths, block_size, scale)
        if kind == "no_prefix":  # positions restart at 0: the cached prefix is ignored
            return orig(q, k_layer, v_layer, tables, [0] * len(starts), lengths, block_size, scale)
        if kind == "gqa_mod":  # head h reads kv head h % Hkv
            hq, hkv = np.shape(q)[1], k_layer.shape[1]
            perm = [(h % hkv) * (hq // hkv) + h // hkv for h in range(hq)]
            return orig(np.asarray(q)[:, perm], k_layer, v_layer, tables, starts, lengths, block_size, scale)[:, np.argsort(perm)]
        raise ValueError(kind)
    return f


@pytest.mark.parametrize("mutant", ["strict", "no_prefix", "gqa_mod"])
def test_planted_prefill_mistakes_are_caught(monkeypatch, mutant):
    monkeypatch.setattr(ref, "prefill_attention_f64", _mutant(mutant))
    checks = [lambda: test_prefill_matches_reference_formulation([7, 0, 12], [3, 6, 1], 4, 2),
              test_single_new_token_is_decode_attention, test_first_fresh_token_returns_value_row_zero]
    caught = 0
    for check in checks:
        try:
            check()
        except AssertionError:
            caught += 1
    assert caught >= 1, f"mutant {mutant} passed every check"

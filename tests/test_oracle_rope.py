"""Pins the oracle's rotary embedding (oracle/paged_ref.py ``rope`` / ``rope_append``).

The reference rotates q and k with ``x * cos + _rotate_half(x) * sin`` (engine/model.py:
216-224) on tensors of the model dtype, the cos/sin rows being the half-table of angles
``position * inv_freq`` repeated twice (engine/model.py:185-213). Checks, by kind:
  * the rotation itself against a float64 complex-number formulation (pair (j, j + D/2) is
    the complex number x[j] + i x[j + D/2], multiplied by exp(i theta_j));
  * the special angles 0, a quarter turn and a half turn, which give x, rotate_half(x) and -x
    exactly in every dtype;
  * the rounding sequence (each product and the sum rounded to the dtype) against torch's
    own CPU arithmetic on tensors of that dtype, bit for bit;
  * ``rope_append``: pool rows at the slots hold the rotated k and the unrotated v, padding
    slots write nothing;
  * planted mistakes (sign flip, unswapped halves, interleaved pairs, one rounding instead of
    three) that at least one check must catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref

DTYPES = ["float32", "float16", "bfloat16"]
TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def tables(positions, dim, theta=1_000_000.0):
    """float64 angles [N, D/2] and the cos/sin rows [N, D] (half-table repeated, engine/model.py:196-199)."""
    half = dim // 2
    inv_freq = 1.0 / theta ** (np.arange(half, dtype=np.float64) * 2.0 / dim)
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv_freq[None, :]
    full = np.concatenate([ang, ang], axis=-1)
    return ang, np.cos(full), np.sin(full)


def to_storage(x: np.ndarray, dtype: str) -> np.ndarray:
    return ref.narrow(np.asarray(x, dtype=np.float32), dtype)


def case(n=6, heads=3, dim=16, dtype="float32", seed=0, positions=None):
    rng = np.random.default_rng(seed)
    pos = rng.integers(0, 5000, n) if positions is None else np.asarray(positions)
    ang, c, s = tables(pos, dim)
    x = to_storage(rng.standard_normal((n, heads, dim)), dtype)
    return x, to_storage(c, dtype), to_storage(s, dtype), ang


# ----------------------------------------------------------------------------- checks


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_matches_complex_rotation(dtype):
    x, c, s, _ = case(n=32, heads=4, dim=64, dtype=dtype)
    got = ref.widen(ref.rope(x, c[:, None], s[:, None], dtype), dtype).astype(np.float64)
    xf = ref.widen(x, dtype).astype(np.float64)
    cf = ref.widen(c, dtype).astype(np.float64)[:, None, :32]  # the tables as stored in the dtype
    sf = ref.widen(s, dtype).astype(np.float64)[:, None, :32]
    z = (xf[..., :32] + 1j * xf[..., 32:]) * (cf + 1j * sf)
    want = np.concatenate([z.real, z.imag], axis=-1)
    ulp = {"float32": 2.0 ** -23, "float16": 2.0 ** -10, "bfloat16": 2.0 ** -7}[dtype]
    bound = 3 * ulp * (np.abs(xf[..., :32]) + np.abs(xf[..., 32:]))
    assert (np.abs(got - want) <= np.concatenate([bound, bound], axis=-1) + 1e-30).all()


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_special_angles(dtype):
    rng = np.random.default_rng(3)
    x = to_storage(rng.standard_normal((5, 2, 8)) + 0.25, dtype)  # no zeros: keep the signs of zero out of it
    xf = ref.widen(x, dtype)
    one, zero = to_storage(np.ones((5, 8)), dtype), to_storage(np.zeros((5, 8)), dtype)
    ident = ref.widen(ref.rope(x, one[:, None], zero[:, None], dtype), dtype)
    assert (ident == xf).all()
    quarter = ref.widen(ref.rope(x, zero[:, None], one[:, None], dtype), dtype)
    assert (quarter == np.concatenate([-xf[..., 4:], xf[..., :4]], axis=-1)).all()
    minus = to_storage(-np.ones((5, 8)), dtype)
    half = ref.widen(ref.rope(x, minus[:, None], zero[:, None], dtype), dtype)
    assert (half == -xf).all()


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_rounding_matches_torch_cpu(dtype):
    """The reference's expression run by torch on CPU tensors of the dtype, bit for bit."""
    x, c, s, _ = case(n=64, heads=7, dim=64, dtype=dtype, seed=5)
    tdt = TORCH[dtype]

    def t(a):
        arr = torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a)
        return arr.view(tdt)

    xt, ct, st = t(x), t(c)[:, None], t(s)[:, None]
    rot = torch.cat((-xt[..., 32:], xt[..., :32]), dim=-1)
    want = xt * ct + rot * st
    want_bits = want.view(torch.int16).numpy().view(np.uint16) if dtype != "float32" else want.numpy()
    got = ref.rope(x, c[:, None], s[:, None], dtype)
    assert (got.view(np.uint32 if dtype == "float32" else np.uint16) ==
            want_bits.view(np.uint32 if dtype == "float32" else np.uint16)).all()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_rope_append_pool_rows(dtype):
    rng = np.random.default_rng(7)
    n, hq, hkv, d, bs, nb = 5, 4, 2, 16, 4, 6
    q, c, s, _ = case(n=n, heads=hq, dim=d, dtype=dtype, seed=8)
    k = to_storage(rng.standard_normal((n, hkv, d)), dtype)
    v = to_storage(rng.standard_normal((n, hkv, d)), dtype)
    shape = (nb + 1, hkv, bs, d)
    k_pool, v_pool = to_storage(rng.standard_normal(shape), dtype), to_storage(rng.standard_normal(shape), dtype)
    k0, v0 = k_pool.copy(), v_pool.copy()
    slots = np.array([3, 9, -1, 27, nb * bs + bs], dtype=np.int64)  # a padding row and one past the pool
    qr, kr = ref.rope_append(q, k, v, c, s, dtype, k_pool, v_pool, slots, bs)
    assert (qr == ref.rope(q, c[:, None], s[:, None], dtype)).all()
    touched = np.zeros(shape[0] * bs, dtype=bool)
    for i, sl in enumerate(slots):
        if 0 <= sl < (nb + 1) * bs:
            touched[sl] = True
            assert (k_pool[sl // bs, :, sl % bs] == kr[i]).all()
            assert (v_pool[sl // bs, :, sl % bs] == v[i]).all()
    # Every other row is untouched (the padding row and the out-of-pool slot wrote nothing).
    untouched = ~touched.reshape(nb + 1, bs)
    assert (k_pool.transpose(0, 2, 1, 3)[untouched] == k0.transpose(0, 2, 1, 3)[untouched]).all()
    assert (v_pool.transpose(0, 2, 1, 3)[untouched] == v0.transpose(0, 2, 1, 3)[untouched]).all()
    # The rotation of k matches the complex formulation (pins kr independently of rope itself).
    kf, cf, sf = ref.widen(kr, dtype), ref.widen(c, dtype), ref.widen(s, dtype)
    k_in = ref.widen(k, dtype).astype(np.float64)
    z = (k_in[..., :8] + 1j * k_in[..., 8:]) * (cf[:, None, :8] + 1j * sf[:, None, :8])
    tol = 4 * (2.0 ** -7 if dtype == "bfloat16" else 2.0 ** -23) * (np.abs(k_in[..., :8]) + np.abs(k_in[..., 8:]))
    assert (np.abs(kf[..., :8] - z.real) <= tol + 1e-30).all()
    assert (np.abs(kf[..., 8:] - z.imag) <= tol + 1e-30).all()


# ----------------------------------------------------------------------------- planted mistakes


def _mutant(kind):
    def f(x, cos, sin, dtype):
        xf, cf, sf = ref.widen(x, dtype), ref.widen(cos, dtype), ref.widen(sin, dtype)
        h = xf.shape[-1] // 2
        if kind == "sign":  # rotate_half with the minus on the wrong half
            rot = np.concatenate([xf[..., h:], -xf[..., :h]], axis=-1)
        elif kind == "no_swap":  # negates without swapping the halves
            rot = np.concatenate([-xf[..., :h], xf[..., h:]], axis=-1)
        elif kind == "interleaved":  # pairs (2i, 2i + 1) instead of (i, i + D/2)
            rot = np.stack([-xf[..., 1::2], xf[..., 0::2]], axis=-1).reshape(xf.shape)
        elif kind == "one_rounding":  # fp32 all the way, one rounding at the end
            rot = np.concatenate([-xf[..., h:], xf[..., :h]], axis=-1)
            return ref.narrow(xf * cf + rot * sf, dtype)
        else:
            raise ValueError(kind)
        t1 = ref.widen(ref.narrow(xf * cf, dtype), dtype)
        t2 = ref.widen(ref.narrow(rot * sf, dtype), dtype)
        return ref.narrow(t1 + t2, dtype)
    return f


@pytest.mark.parametrize("mutant", ["sign", "no_swap", "interleaved", "one_rounding"])
def test_planted_rope_mistakes_are_caught(monkeypatch, mutant):
    monkeypatch.setattr(ref, "rope", _mutant(mutant))
    checks = [lambda: test_rope_matches_complex_rotation("float32"), lambda: test_rope_special_angles("float32"),
              lambda: test_rope_rounding_matches_torch_cpu("bfloat16")]
    caught = 0
    for check in checks:
        try:
            check()
        except AssertionError:
            caught += 1
    assert caught >= 1, f"mutant {mutant} passed every check"

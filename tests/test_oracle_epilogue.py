"""Pins the oracle's SiLU-gate epilogue (CPU).

The oracle defines out[m, j] = silu(gu[m, j]) * gu[m, F + j] with
silu(v) = v / (1 + expf(-v)) in fp32.  What fixes it independently of that
formula: silu(0) = 0; silu(v) - silu(-v) = v for every v (sigmoid(v) +
sigmoid(-v) = 1); silu(ln 3) = (3/4) ln 3 (sigmoid(ln 3) = 3/4); silu(v) -> v
for large v and -> 0 for very negative v; a float64 evaluation through
numpy's exp; and one-hot inputs that expose a wrong gate/up pairing or row
stride.
"""
import math

import numpy as np


def _silu(orc, v):
    v = np.asarray(v, np.float32).reshape(1, -1)
    return orc.silu_mul(np.concatenate([v, np.ones_like(v)], axis=1))[0]


def test_silu_closed_forms(orc):
    assert _silu(orc, [0.0])[0] == 0.0
    ln3 = np.float32(math.log(3.0))
    assert abs(float(_silu(orc, [ln3])[0]) - 0.75 * float(ln3)) <= 2e-7
    big = _silu(orc, [30.0, 60.0, -60.0, -110.0])
    assert big[0] == np.float32(30.0) and big[1] == np.float32(60.0)
    assert -1e-23 < big[2] <= 0.0 and big[3] == 0.0


def test_silu_odd_part_identity(orc):
    v = np.linspace(-20, 20, 4001, dtype=np.float32)
    d = _silu(orc, v).astype(np.float64) - _silu(orc, -v).astype(np.float64)
    # each silu value carries a few fp32 roundings of its own magnitude
    tol = 4 * np.spacing(np.abs(v).astype(np.float32)).astype(np.float64) + 1e-30
    assert np.all(np.abs(d - v) <= tol)


def test_silu_matches_float64(orc):
    v = np.random.default_rng(7).standard_normal(20000).astype(np.float32) * 6
    ref = v.astype(np.float64) / (1.0 + np.exp(-v.astype(np.float64)))
    got = _silu(orc, v).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 4e-7 * np.maximum(np.abs(ref), 1e-3))


def test_silu_mul_pairs_gate_j_with_up_j(orc):
    f, m = 13, 3
    gate = np.arange(m * f, dtype=np.float32).reshape(m, f) / 7 - 2
    up = np.full((m, f), 1.0, np.float32)
    out = orc.silu_mul(np.concatenate([gate, up], axis=1))
    assert np.array_equal(out, _silu(orc, gate.ravel()).reshape(m, f))
    gate1 = np.ones((m, f), np.float32)
    up1 = (np.arange(m * f, dtype=np.float32).reshape(m, f) + 1)
    out1 = orc.silu_mul(np.concatenate([gate1, up1], axis=1))
    assert np.array_equal(out1, np.float32(_silu(orc, [1.0])[0]) * up1)

"""The oracle reproduces the committed golden vectors bit for bit (CPU)."""
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def test_fp8_golden(orc):
    g = load("fp8_small.npz")
    q, s = orc.fp8_quantize_rows(g["w"])
    assert np.array_equal(q, g["q"]) and np.array_equal(s, g["s"])
    assert np.array_equal(orc.fp8_gemv(g["x_bf16"], q, s)[0], g["y32"])


def test_aq4_golden(orc):
    g = load("aq4_small.npz")
    p, sc, z = orc.aq4_quantize(g["w"])
    assert np.array_equal(p, g["packed"])
    assert np.array_equal(sc, g["scales"]) and np.array_equal(z, g["zeros"])
    assert np.array_equal(orc.aq4_gemv(g["x_bf16"], p, sc, z)[0], g["y32"])


def test_gemm_golden(orc):
    g = load("gemm_small.npz")
    q, s = orc.fp8_quantize_rows(g["w"])
    xq, xs = orc.act_quantize(g["x_bf16"])
    assert np.array_equal(xq, g["xq"]) and np.array_equal(xs, g["xs"])
    assert np.array_equal(orc.fp8_gemm(xq, xs, q, s)[0], g["y32"])

"""Pins the oracle's quantizers and contractions (CPU only).

Each check is chosen so that a plausible mistake fails it: a transposed
operand (shape/identity checks), a wrong nibble order (hand-built
known-answer words), a dropped zero point or scale (closed-form
reconstruction of constructed groups), a wrong rounding mode (idempotence
and error bounds), a wrong accumulation index (fp64 brute force through an
independent numpy contraction, one-hot and all-ones identities).
"""
import numpy as np
import pytest

from helpers import activations_bf16, weights


# ----------------------------------------------------------- FP8 rows

def test_fp8_rows_scale_and_peak_code(orc):
    w = weights(37, 255, tag=1)
    q, s = orc.fp8_quantize_rows(w)
    assert np.array_equal(s, (np.abs(w).max(axis=1) / np.float32(448)).astype(np.float32))
    # the row maximum maps to +-448 exactly
    peak = np.take_along_axis(q, np.abs(w).argmax(axis=1)[:, None], 1)[:, 0]
    assert np.all((peak & 0x7F) == 0x7E)


def test_fp8_rows_error_bound_and_idempotence(orc):
    w = weights(64, 512, tag=2)
    q, s = orc.fp8_quantize_rows(w)
    d = orc.fp8_dequantize(q, s)
    # E4M3 relative spacing is 2^-3 in the normal range, absolute 2^-9 below
    bound = np.maximum(np.abs(w) * 2.0 ** -4, 2.0 ** -10 * s[:, None]) * (1 + 1e-6)
    assert np.all(np.abs(d - w) <= bound)
    q2, s2 = orc.fp8_quantize_rows(d)
    d2 = orc.fp8_dequantize(q2, s2)
    assert np.array_equal(d2, d)


def test_fp8_rows_zero_row_and_exact_dequant(orc):
    w = weights(3, 64, tag=3)
    w[1] = 0.0
    q, s = orc.fp8_quantize_rows(w)
    assert s[1] == 0 and np.all(q[1] == 0)
    d = orc.fp8_dequantize(q, s)
    assert np.array_equal(d, (orc.e4m3_to_f32(q) * s[:, None]).astype(np.float32))


# ------------------------------------------------------------- AQ4 g128

def test_aq4_known_answer_words(orc):
    # Group [lo, lo + 15 s] built from exact codes 0..15: z = 8 gives lo = -8 s
    # with s = 1/64 (exact in f16); codes repeat 0..15 along k.
    s = 1.0 / 64
    codes = np.tile(np.arange(16), 8)
    w = ((codes - 8) * s).astype(np.float32)[None, :]
    p, sc, z = orc.aq4_quantize(w)
    assert orc.f16_to_f32(sc)[0, 0] == s and orc.f16_to_f32(z)[0, 0] == 8.0
    # nibble j of word w is k = 8w + j, low nibble first
    assert p[0, 0] == 0x76543210 and p[0, 1] == 0xFEDCBA98
    assert np.array_equal(orc.aq4_dequantize(p, sc, z), w)


def test_aq4_nibble_order_single_code(orc):
    w = np.zeros((1, 128), np.float32)
    w[0, 13] = 1.0  # lo = 0, hi = 1: s = f16(1/15), z = 0, q[13] = 15
    p, sc, z = orc.aq4_quantize(w)
    assert p[0, 1] == 0xF << 4 * 5 and np.count_nonzero(p) == 1
    assert z[0, 0] == 0 or z[0, 0] == 0x8000


def test_aq4_error_bound_and_idempotence(orc):
    w = weights(33, 512, tag=4)
    p, sc, z = orc.aq4_quantize(w)
    d = orc.aq4_dequantize(p, sc, z)
    sf = np.repeat(orc.f16_to_f32(sc), 128, axis=1)
    g = w.reshape(33, 4, 128)
    rng_ = np.repeat(g.max(axis=2) - g.min(axis=2), 128, axis=1)
    assert np.all(np.abs(d - w) <= 0.5 * sf + 0.01 * sf + 2.0 ** -10 * rng_)
    # re-quantizing the dequantized values with the same s, z reproduces q
    zf = np.repeat(orc.f16_to_f32(z), 128, axis=1)
    q = np.clip(np.rint(d / sf + zf), 0, 15)
    codes = (p[:, :, None] >> (4 * np.arange(8))) & 0xF
    assert np.array_equal(q.astype(np.uint32), codes.reshape(33, 512))


def test_aq4_degenerate_groups(orc):
    w = weights(4, 256, tag=5)
    w[0, :128] = 0.0            # all-zero group: s = 1, z = 0, q = 0
    w[1, :128] = 0.3            # constant group
    w[2, 128:] = -0.7           # constant negative group
    w[3, :128] = np.linspace(0.01, 0.05, 128)  # all-positive group: z < 0
    p, sc, z = orc.aq4_quantize(w)
    d = orc.aq4_dequantize(p, sc, z)
    assert sc[0, 0] == 0x3C00 and orc.f16_to_f32(z[0, 0]) == 0 and np.all(d[0, :128] == 0)
    assert np.all(np.abs(d[1, :128] - 0.3) <= 2e-4)
    assert np.all(np.abs(d[2, 128:] + 0.7) <= 4e-4)
    assert orc.f16_to_f32(z[3, 0]) < 0
    assert np.max(np.abs(d[3, :128] - w[3, :128])) <= 0.51 * orc.f16_to_f32(sc[3, 0])


# ------------------------------------------------------------ contractions

@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (1, 3, 17), (2, 17, 128),
                                   (3, 7, 255), (7, 16, 384)])
def test_fp8_gemv_bruteforce_fp64(orc, m, n, k):
    w = weights(n, k, tag=m + n)
    q, s = orc.fp8_quantize_rows(w)
    xb = activations_bf16(orc, m, k, tag=k)
    y32, y64 = orc.fp8_gemv(xb, q, s, want64=True)
    xf = orc.bf16_to_f32(xb).astype(np.float64)
    # the scale multiplies the exact E4M3 sum (it is factored out of the sum)
    ref = (xf @ orc.e4m3_to_f32(q).astype(np.float64).T) * s.astype(np.float64)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12)
    assert np.max(np.abs(y32 - ref)) <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("m,n,k", [(1, 1, 128), (2, 17, 256), (3, 7, 384), (7, 16, 128)])
def test_aq4_gemv_bruteforce_fp64(orc, m, n, k):
    w = weights(n, k, tag=m * n)
    p, sc, z = orc.aq4_quantize(w)
    xb = activations_bf16(orc, m, k, tag=k + 1)
    y32, y64 = orc.aq4_gemv(xb, p, sc, z, want64=True)
    ref = orc.bf16_to_f32(xb).astype(np.float64) @ orc.aq4_dequantize(p, sc, z).astype(np.float64).T
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12)
    assert np.max(np.abs(y32 - ref)) <= 1e-5 * max(1.0, np.abs(ref).max())


def test_gemv_identities(orc):
    n, k = 9, 256
    w = weights(n, k, tag=11)
    q, s = orc.fp8_quantize_rows(w)
    p, sc, z = orc.aq4_quantize(w)
    d8 = orc.fp8_dequantize(q, s)
    d4 = orc.aq4_dequantize(p, sc, z)
    onehot = np.zeros((1, k), np.float32)
    onehot[0, 77] = 1.0
    xb = orc.bf16_from_f32(onehot)
    assert np.array_equal(orc.fp8_gemv(xb, q, s)[0][0], d8[:, 77])
    assert np.array_equal(orc.aq4_gemv(xb, p, sc, z)[0][0], d4[:, 77])
    ones = orc.bf16_from_f32(np.ones((1, k), np.float32))
    assert np.allclose(orc.fp8_gemv(ones, q, s, want64=True)[1][0],
                       orc.e4m3_to_f32(q).astype(np.float64).sum(1) * s, rtol=1e-12)
    # alpha scales linearly; row stride is honoured
    xb = activations_bf16(orc, 2, k + 8)
    y_view = orc.fp8_gemv(xb[:, :k].copy(), q, s, alpha=0.25)[0]
    y_full = orc.fp8_gemv(np.ascontiguousarray(xb[:, :k]), q, s)[0]
    assert np.array_equal(y_view, np.float32(0.25) * y_full)


def test_act_quant_and_gemm(orc):
    m, n, k = 5, 12, 300
    xb = activations_bf16(orc, m, k, tag=12)
    xb[2] = 0
    xq, xs = orc.act_quantize(xb)
    xf = orc.bf16_to_f32(xb)
    assert np.array_equal(xs, (np.abs(xf).max(1) / np.float32(448)).astype(np.float32))
    assert xs[2] == 0 and np.all(xq[2] == 0)
    peak = np.take_along_axis(xq, np.abs(xf).argmax(1)[:, None], 1)[:, 0]
    assert np.all((peak[[0, 1, 3, 4]] & 0x7F) == 0x7E)
    w = weights(n, k, tag=13)
    q, s = orc.fp8_quantize_rows(w)
    y32, y64 = orc.fp8_gemm(xq, xs, q, s, want64=True)
    ref = (orc.e4m3_to_f32(xq).astype(np.float64) @ orc.e4m3_to_f32(q).astype(np.float64).T) \
        * xs.astype(np.float64)[:, None] * s.astype(np.float64)[None, :]
    assert np.allclose(y64, ref, rtol=1e-9, atol=1e-12)
    # GEMM with per-token quantized x stays close to the exact bf16 product
    exact = xf.astype(np.float64) @ orc.fp8_dequantize(q, s).astype(np.float64).T
    rms = np.sqrt(np.mean(exact ** 2))
    assert np.max(np.abs(y32 - exact)) <= 0.15 * rms

"""Pins the oracle's scalar number formats (CPU only).

E4M3FN, bf16 and f16 are checked against three independent sources:
  * the closed forms of the formats, evaluated here in Python from sign,
    exponent and mantissa fields (all 256 E4M3 codes, every bf16 / f16 class);
  * library casts: torch.float8_e4m3fn and torch.bfloat16, numpy.float16
    (round-to-nearest-even implementations maintained outside this repo);
  * the committed table tests/golden/e4m3_table.npz written by torch.
Special cases (ties to even, saturation at 448, NaN, signed zero, subnormals)
are enumerated so that a wrong rounding mode, bias or field width fails.
"""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def e4m3_closed_form(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8) * 2.0 ** (e - 7)


def test_e4m3_decode_all_codes_closed_form(orc):
    got = orc.e4m3_to_f32(np.arange(256))
    for c in range(256):
        want = e4m3_closed_form(c)
        if np.isnan(want):
            assert np.isnan(got[c]), c
        else:
            assert got[c] == np.float32(want), (c, got[c], want)
    assert got[0x7E] == 448.0 and got[0xFE] == -448.0
    assert got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_e4m3_decode_matches_torch_and_golden(orc):
    import torch
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = orc.e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(got), np.isnan(t))
    assert np.array_equal(got[~np.isnan(got)], t[~np.isnan(t)])
    table = np.load(GOLDEN / "e4m3_table.npz")
    assert np.array_equal(table["codes"], codes)
    v = table["values"]
    assert np.array_equal(np.isnan(v), np.isnan(got))
    assert np.array_equal(v[~np.isnan(v)], got[~np.isnan(got)])


def test_e4m3_encode_roundtrip_every_code(orc):
    vals = orc.e4m3_to_f32(np.arange(256))
    finite = ~np.isnan(vals)
    codes = np.arange(256)[finite]
    back = orc.e4m3_from_f32(vals[finite])
    assert np.array_equal(back, codes.astype(np.uint8))


def test_e4m3_encode_ties_to_even_and_neighbours(orc):
    pos = orc.e4m3_to_f32(np.arange(0x00, 0x7F))  # 0 .. 448 ascending
    for c in range(0x7E):
        lo, hi = float(pos[c]), float(pos[c + 1])
        mid = (lo + hi) / 2
        even = c if c % 2 == 0 else c + 1
        assert orc.e4m3_from_f32(np.float32(mid))[()] == even, (c, mid)
        below = np.nextafter(np.float32(mid), np.float32(0))
        above = np.nextafter(np.float32(mid), np.float32(1000))
        assert orc.e4m3_from_f32(below)[()] == c
        assert orc.e4m3_from_f32(above)[()] == c + 1
        assert orc.e4m3_from_f32(-np.float32(mid))[()] == 0x80 | even


@pytest.mark.parametrize("x,code", [(448.0, 0x7E), (449.0, 0x7E), (464.0, 0x7E),
                                    (480.0, 0x7E), (1e30, 0x7E),
                                    (float("inf"), 0x7E), (-float("inf"), 0xFE),
                                    (-500.0, 0xFE), (0.0, 0x00), (-0.0, 0x80),
                                    (2.0 ** -10, 0x00), (3 * 2.0 ** -11, 0x01),
                                    (1e-30, 0x00)])
def test_e4m3_encode_saturation_and_specials(orc, x, code):
    assert orc.e4m3_from_f32(np.float32(x))[()] == code


def test_e4m3_encode_nan(orc):
    assert orc.e4m3_from_f32(np.float32("nan"))[()] & 0x7F == 0x7F


def test_e4m3_encode_matches_torch_in_range(orc):
    import torch
    rs = np.random.default_rng(7)
    x = np.concatenate([rs.standard_normal(200000) * s
                        for s in (1e-3, 0.05, 1.0, 30.0, 150.0)]).astype(np.float32)
    x = x[np.abs(x) < 448]
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.e4m3_from_f32(x), want)


def test_bf16_matches_torch(orc):
    import torch
    rs = np.random.default_rng(8)
    x = np.concatenate([rs.standard_normal(100000) * s for s in (1e-38, 1e-3, 1.0, 1e30)])
    x = np.concatenate([x, [0.0, -0.0, 3.4e38, -3.4e38, 1e-45, 2.0 ** -126]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.bf16_from_f32(x), want)
    assert np.array_equal(orc.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_bf16_ties_overflow_nan(orc):
    # 1 + 2^-8 is the midpoint between 1 and 1 + 2^-7: ties go to even (1.0)
    assert orc.bf16_from_f32(np.float32(1 + 2.0 ** -8))[()] == 0x3F80
    assert orc.bf16_from_f32(np.float32(1 + 3 * 2.0 ** -8))[()] == 0x3F82
    assert orc.bf16_from_f32(np.float32(3.4028235e38))[()] == 0x7F80  # rounds up to inf
    assert orc.bf16_from_f32(np.float32("nan"))[()] & 0x7FC0 == 0x7FC0


def test_f16_matches_numpy(orc):
    rs = np.random.default_rng(9)
    x = np.concatenate([rs.standard_normal(100000) * s for s in (1e-7, 1e-3, 1.0, 3e4)])
    x = np.concatenate([x, [65504.0, 65519.0, 65520.0, 1e6, -0.0, 2.0 ** -24, 2.0 ** -25,
                            3 * 2.0 ** -26]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f16_from_f32(x), want)
    assert np.array_equal(orc.f16_to_f32(want), want.view(np.float16).astype(np.float32))


# ---------------------------------------------------------------- bf16 add

def _bf16(values):
    import torch
    return torch.tensor(values, dtype=torch.float32).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def test_bf16_add_closed_forms(orc):
    """Ties, overflow, signed zeros and the IEEE specials of the bf16 add."""
    one, tie, ulp = 0x3F80, 0x3B80, 0x3C00      # 1.0, 2^-8, 2^-7
    cases = [
        (one, tie, 0x3F80),                      # 1 + 2^-8: tie, to even (1.0)
        (0x3F81, tie, 0x3F82),                   # (1 + 2^-7) + 2^-8: tie, to even
        (one, ulp, 0x3F81),                      # exact
        (0x4040, 0x4000, 0x40A0),                # 3 + 2 = 5
        (0x7F7F, 0x7F7F, 0x7F80),                # max + max overflows to inf
        (0xFF7F, 0xFF7F, 0xFF80),                # and to -inf
        (0x7F80, 0xFF80, None),                  # inf + -inf: NaN
        (0x8000, 0x8000, 0x8000),                # -0 + -0 = -0
        (0x8000, 0x0000, 0x0000),                # -0 + +0 = +0
        (0x4049, 0xC049, 0x0000),                # x + (-x) = +0
        (0x0001, 0x0001, 0x0002),                # subnormals add exactly
    ]
    a = np.array([c[0] for c in cases], np.uint16)
    b = np.array([c[1] for c in cases], np.uint16)
    got = orc.bf16_add(a, b)
    for (x, y, want), g in zip(cases, got):
        if want is None:
            assert (g & 0x7F80) == 0x7F80 and (g & 0x7F) != 0, (hex(x), hex(y), hex(g))
        else:
            assert g == want, (hex(x), hex(y), hex(g))
    assert np.array_equal(orc.bf16_add(b, a), got)  # commutative


def test_bf16_add_matches_torch(orc):
    """Against torch's bfloat16 add (fp32 sum rounded to nearest even) over
    mixed magnitudes, including sums that cancel, overflow and underflow."""
    import torch
    rs = np.random.default_rng(31)
    parts = [rs.standard_normal(50000) * s for s in (1e-38, 1e-3, 1.0, 1e3, 3e38)]
    with np.errstate(over="ignore"):  # the 3e38 part overflows to inf on purpose
        x = np.concatenate(parts).astype(np.float32)
    y = np.concatenate([rs.standard_normal(x.size - 20000) * 1.0,
                        -x[:10000], x[10000:20000] * 1e-3]).astype(np.float32)
    a, b = _bf16(x), _bf16(y)
    ta = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    want = (ta + tb).view(torch.int16).numpy().view(np.uint16)
    got = orc.bf16_add(a, b)
    nan = (want & 0x7FFF) > 0x7F80
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7FFF) > 0x7F80)


def test_add_act_quantize_is_quantize_of_sum(orc):
    rs = np.random.default_rng(32)
    a = _bf16(rs.standard_normal((6, 300)))
    b = _bf16(rs.standard_normal((6, 300)) * 4)
    xq, xs, s = orc.add_act_quantize(a, b)
    assert np.array_equal(s, orc.bf16_add(a, b))
    q2, s2 = orc.act_quantize(s)
    assert np.array_equal(xq, q2) and np.array_equal(xs, s2)

"""GPU parity of the HIP linear path against the C oracle, through the C ABI.

Bit-exact: weight quantization (FP8 rows, AQ4 g128), the canonical export of
the device tile layout, dequantization, per-token activation quantization.
Within 1e-2 x RMS of the fp32-accumulated oracle: the decode GEMV (FP8, AQ4)
and the prefill FP8 GEMM.  Shapes cover the boundary policy of the reference
(0/1/3/7, B-1/B/B+1 around the 16-row stripe, 64-k tile and 128-k group,
17/37/73) at sizes the oracle finishes in seconds.
"""
import numpy as np
import pytest
import torch

from helpers import (activations_bf16, assert_close, bf16_tensor_to_f32,
                     check_gemv_plan, to_torch_bf16, weights)

pytestmark = pytest.mark.gpu

FP8_SHAPES = [(1, 1), (3, 17), (15, 63), (16, 64), (17, 65), (37, 255),
              (73, 513), (64, 4096)]
AQ4_SHAPES = [(1, 128), (3, 256), (15, 384), (16, 128), (17, 640), (73, 1024),
              (64, 4096)]


def _fp8_weight(uh, w, dev):
    return uh.LinearWeight.quantize(torch.from_numpy(w).to(dev),
                                    uh.ENCODING_FP8_E4M3_ROW)


def _aq4_weight(uh, w, dev):
    return uh.LinearWeight.quantize(torch.from_numpy(w).to(dev),
                                    uh.ENCODING_AQ4_G128)


@pytest.mark.parametrize("n,k", FP8_SHAPES)
def test_fp8_quantize_export_dequant_bit_exact(uh, orc, gpu, n, k):
    w = weights(n, k, tag=n * 7 + k)
    w[0, : min(k, 5)] = 0.0
    if n > 2:
        w[2, :] = 0.0  # all-zero row: s = 0, q = 0
    q_ref, s_ref = orc.fp8_quantize_rows(w)
    lw = _fp8_weight(uh, w, gpu)
    q, s = lw.export()
    assert np.array_equal(q, q_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    d = lw.dequantize().cpu().numpy()
    d_ref = orc.fp8_dequantize(q_ref, s_ref)
    assert np.array_equal(d.view(np.uint32), d_ref.view(np.uint32))
    # upload of canonical bytes reproduces the same device weight
    lw2 = uh.LinearWeight.from_fp8(q_ref, s_ref)
    q2, s2 = lw2.export()
    assert np.array_equal(q2, q_ref) and np.array_equal(s2, s_ref)


@pytest.mark.parametrize("n,k", AQ4_SHAPES)
def test_aq4_quantize_export_dequant_bit_exact(uh, orc, gpu, n, k):
    w = weights(n, k, tag=n * 11 + k)
    w[0, :128] = 0.25  # constant group: degenerate scale
    if n > 1:
        w[1, :128] = np.linspace(0.01, 0.05, 128)  # all-positive group
    p_ref, s_ref, z_ref = orc.aq4_quantize(w)
    lw = _aq4_weight(uh, w, gpu)
    p, s, z = lw.export()
    assert np.array_equal(s, s_ref)
    assert np.array_equal(z, z_ref)
    assert np.array_equal(p, p_ref)
    d = lw.dequantize().cpu().numpy()
    d_ref = orc.aq4_dequantize(p_ref, s_ref, z_ref)
    assert np.array_equal(d.view(np.uint32), d_ref.view(np.uint32))
    lw2 = uh.LinearWeight.from_aq4(p_ref, s_ref, z_ref)
    p2, s2, z2 = lw2.export()
    assert np.array_equal(p2, p_ref) and np.array_equal(s2, s_ref) \
        and np.array_equal(z2, z_ref)


@pytest.mark.parametrize("m", [1, 2, 3, 7, 16, 17, 24, 27, 32, 33, 70])
@pytest.mark.parametrize("n,k", [(17, 65), (64, 4096), (129, 640), (16, 4096)])
def test_fp8_gemv_parity(uh, orc, gpu, m, n, k):
    w = weights(n, k, tag=3)
    q, s = orc.fp8_quantize_rows(w)
    xb = activations_bf16(orc, m, k, tag=m)
    y_ref, _ = orc.fp8_gemv(xb, q, s)
    lw = uh.LinearWeight.from_fp8(q, s)
    x = to_torch_bf16(xb, gpu)
    y32 = lw.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(y32.cpu().numpy(), y_ref, what="fp8 gemv f32")
    yb = lw.forward(x)
    assert_close(bf16_tensor_to_f32(yb), y_ref, bf16_out=True, what="fp8 gemv bf16")


@pytest.mark.parametrize("m", [1, 2, 3, 7, 9, 16, 20, 27, 32, 33])
@pytest.mark.parametrize("n,k", [(17, 128), (64, 4096), (129, 640), (16, 1024)])
def test_aq4_gemv_parity(uh, orc, gpu, m, n, k):
    w = weights(n, k, tag=5)
    p, s, z = orc.aq4_quantize(w)
    xb = activations_bf16(orc, m, k, tag=m + 100)
    y_ref, _ = orc.aq4_gemv(xb, p, s, z)
    lw = uh.LinearWeight.from_aq4(p, s, z)
    x = to_torch_bf16(xb, gpu)
    y32 = lw.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(y32.cpu().numpy(), y_ref, what="aq4 gemv f32")
    yb = lw.forward(x)
    assert_close(bf16_tensor_to_f32(yb), y_ref, bf16_out=True, what="aq4 gemv bf16")


# (variant, waves, stripes per group, row classes) on a 256-CU device.
MANY_STRIPES_PLAN = {
    (1, 9000): (("single_lds", 8, 1, 1), ("multi", 8, 1, 4)),
    (2, 9000): (("single_lds", 8, 1, 1), ("multi", 8, 1, 4)),
    (1, 25000): (("single_lds", 8, 1, 1), ("multi", 4, 1, 4)),
    (2, 25000): (("single_lds", 8, 1, 1), ("multi", 4, 1, 4)),
    (2, 13000): (("single_lds", 8, 1, 1), ("multi", 4, 1, 4)),
    (3, 25000): (("single_lds", 8, 1, 1), ("multi", 8, 1, 4)),
    (4, 25000): (("single_lds", 8, 1, 1), ("rs", 4, 4, 1)),
    (8, 12500): (("multi", 8, 1, 1), ("rs", 4, 1, 2)),
    (16, 12500): (("multi", 8, 1, 1), ("rs", 4, 2, 1)),
}


@pytest.mark.parametrize("m,n", list(MANY_STRIPES_PLAN))
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_gemv_parity_many_stripes(uh, orc, gpu, enc, m, n):
    """Grids of 563 to 1563 16-row stripes (the last one ragged), K = 4096 as
    in the Llama shapes: more stripes than CUs.  On a 256-CU device AQ4
    M <= 3 takes the multi-stripe kernel (one stripe per wave at M = 1 from
    1536 stripes and at M = 2 from 768), AQ4 M >= 4 the register-staged
    kernel, FP8 M >= 8 the multi-stripe kernel and FP8 M < 8 the
    single-stripe LDS kernel; the test checks that plan, then the output."""
    k = 4096
    w = weights(n, k, tag=21)
    xb = activations_bf16(orc, m, k, tag=m + 200)
    if enc == "fp8":
        q, s = orc.fp8_quantize_rows(w)
        y_ref, _ = orc.fp8_gemv(xb, q, s)
        lw = uh.LinearWeight.from_fp8(q, s)
    else:
        p, s, z = orc.aq4_quantize(w)
        y_ref, _ = orc.aq4_gemv(xb, p, s, z)
        lw = uh.LinearWeight.from_aq4(p, s, z)
    x = to_torch_bf16(xb, gpu)
    y32 = lw.forward(x, out_dtype=torch.float32)
    check_gemv_plan(lw, x, y32, MANY_STRIPES_PLAN[(m, n)][enc == "aq4"])
    torch.cuda.synchronize()
    assert_close(y32.cpu().numpy(), y_ref, what=f"{enc} gemv f32 many stripes")
    yb = lw.forward(x)
    assert_close(bf16_tensor_to_f32(yb), y_ref, bf16_out=True,
                 what=f"{enc} gemv bf16 many stripes")


# Shapes that select each tier, and the plan on a 256-CU device:
# (m, n, k): (FP8 plan, AQ4 plan), plan = (variant, waves, stripes, classes).
TIER_PLAN = {
    # two m-tiles, 388 stripes: register-staged, groups of 2
    (17, 6200, 4096): (("rs", 8, 2, 1), ("rs", 4, 2, 1)),
    # 388 stripes, AQ4 M <= 8: single stripes, two classes
    (8, 6200, 1024): (("rs", 8, 2, 1), ("rs", 4, 1, 2)),
    # the same, four classes (FP8: its activation block fits LDS)
    (4, 6200, 1024): (("single_lds", 8, 1, 1), ("rs", 4, 1, 4)),
    # 1025 stripes: groups of 4
    (32, 16400, 1024): (("rs", 4, 4, 1), ("rs", 4, 4, 1)),
    # 4100 stripes: the wide configuration
    (8, 65600, 1024): (("rs", 8, 4, 1), ("rs", 8, 4, 1)),
    # 63 stripes, long K: single stripes (16 waves AQ4, 8 FP8)
    (8, 1000, 8192): (("rs", 8, 1, 2), ("rs", 16, 1, 2)),
    # a second 32-row block of one row
    (33, 6200, 1024): (("rs", 8, 2, 1), ("rs", 4, 2, 1)),
    # small grid, 16 <= M <= 32: single stripes, wide rows
    (23, 1000, 4096): (("rs", 8, 1, 1), ("rs", 4, 1, 1)),
    # FP8 M = 17 on a small grid: the single-stripe LDS kernel
    (17, 1000, 4096): (("single_lds", 8, 1, 1), ("rs", 4, 1, 1)),
    # AQ4 single stripes, rows packed in four classes
    (4, 1000, 8192): (("multi", 8, 1, 1), ("rs", 16, 1, 4)),
    # AQ4 single stripes, two classes, a ragged class
    (7, 1000, 8192): (("multi", 8, 1, 1), ("rs", 16, 1, 2)),
    # AQ4 groups of 4 at M = 5
    (5, 16400, 1024): (("single_lds", 8, 1, 1), ("rs", 4, 4, 1)),
    # AQ4 wide configuration at M = 6
    (6, 65600, 1024): (("single_lds", 8, 1, 1), ("rs", 8, 4, 1)),
    # AQ4 small grid: single stripes, 8 waves, packed
    (8, 1000, 4096): (("multi", 8, 1, 1), ("rs", 8, 1, 2)),
    # AQ4 small grid, ragged last stripe
    (5, 300, 2048): (("multi", 8, 1, 1), ("rs", 8, 1, 2)),
    # 1792 stripes: AQ4 groups of 7 (7 per CU on 256 CUs)
    (8, 28672, 1024): (("rs", 4, 4, 1), ("rs", 4, 7, 1)),
    # the same with a ragged 16-row tile
    (13, 28672, 1024): (("rs", 4, 4, 1), ("rs", 4, 7, 1)),
    # groups of 7 with two m-tiles (FP8 too: its activation block exceeds
    # LDS), the second ragged
    (16, 28672, 1024): (("rs", 4, 7, 1), ("rs", 4, 7, 1)),
    (20, 28672, 1024): (("rs", 4, 7, 1), ("rs", 4, 7, 1)),
    (32, 28672, 1024): (("rs", 4, 7, 1), ("rs", 4, 7, 1)),
}


@pytest.mark.parametrize("m,n,k", list(TIER_PLAN))
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_gemv_parity_register_staged_tiers(uh, orc, gpu, enc, m, n, k):
    """Shapes that select each grid-size tier of the register-staged
    multi-stripe kernels (M >= 8 for FP8, M >= 4 for AQ4; FP8 only where its
    activation block does not fit LDS), including the two-m-tile variant and
    a ragged last stripe and stripe group; the launch plan is checked
    against TIER_PLAN, then the output against the oracle."""
    w = weights(n, k, tag=31)
    xb = activations_bf16(orc, m, k, tag=m + 300)
    if enc == "fp8":
        q, s = orc.fp8_quantize_rows(w)
        y_ref, _ = orc.fp8_gemv(xb, q, s)
        lw = uh.LinearWeight.from_fp8(q, s)
    else:
        p, s, z = orc.aq4_quantize(w)
        y_ref, _ = orc.aq4_gemv(xb, p, s, z)
        lw = uh.LinearWeight.from_aq4(p, s, z)
    x = to_torch_bf16(xb, gpu)
    y32 = lw.forward(x, out_dtype=torch.float32)
    check_gemv_plan(lw, x, y32, TIER_PLAN[(m, n, k)][enc == "aq4"])
    torch.cuda.synchronize()
    assert_close(y32.cpu().numpy(), y_ref, what=f"{enc} gemv f32 {m}x{n}x{k}")
    yb = lw.forward(x)
    assert_close(bf16_tensor_to_f32(yb), y_ref, bf16_out=True,
                 what=f"{enc} gemv bf16 {m}x{n}x{k}")


@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_gemv_seven_stripe_groups_strided_rows(uh, orc, gpu, enc):
    """The 7-stripes-per-CU tier with two m-tiles (the second ragged) reading
    x as a column slice of a wider buffer; plan checked, then the oracle."""
    m, n, k = 20, 28672, 1024
    w = weights(n, k, tag=41)
    wide = activations_bf16(orc, m, k + 136, tag=m + 320)
    xb = np.ascontiguousarray(wide[:, 8:8 + k])
    if enc == "fp8":
        q, s = orc.fp8_quantize_rows(w)
        y_ref, _ = orc.fp8_gemv(xb, q, s)
        lw = uh.LinearWeight.from_fp8(q, s)
    else:
        p, s, z = orc.aq4_quantize(w)
        y_ref, _ = orc.aq4_gemv(xb, p, s, z)
        lw = uh.LinearWeight.from_aq4(p, s, z)
    x = to_torch_bf16(wide, gpu)[:, 8:8 + k]
    assert x.stride(0) == k + 136 and x.data_ptr() % 16 == 0
    y32 = lw.forward(x, out_dtype=torch.float32)
    check_gemv_plan(lw, x, y32, ("rs", 4, 7, 1))
    torch.cuda.synchronize()
    assert_close(y32.cpu().numpy(), y_ref, what=f"{enc} seven-stripe strided")


@pytest.mark.parametrize("m", [4, 8])
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_gemv_register_staged_strided_rows(uh, orc, gpu, enc, m):
    """Packed register-staged launches reading x as a column slice of a wider
    buffer (the decode stack reads the q slice of the qkv output and the gate
    half of the gate_up output this way)."""
    # K = 16384: at M = 8 the FP8 activation block exceeds LDS, so FP8 too
    # takes the register-staged kernel.
    n, k = 1000, 16384
    w = weights(n, k, tag=37)
    wide = activations_bf16(orc, m, k + 264, tag=m + 310)
    xb = np.ascontiguousarray(wide[:, :k])
    if enc == "fp8":
        q, s = orc.fp8_quantize_rows(w)
        y_ref, _ = orc.fp8_gemv(xb, q, s)
        lw = uh.LinearWeight.from_fp8(q, s)
    else:
        p, s, z = orc.aq4_quantize(w)
        y_ref, _ = orc.aq4_gemv(xb, p, s, z)
        lw = uh.LinearWeight.from_aq4(p, s, z)
    x = to_torch_bf16(wide, gpu)[:, :k]
    assert x.stride(0) == k + 264
    y32 = lw.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(y32.cpu().numpy(), y_ref, what=f"{enc} gemv strided m={m}")


def test_gemv_strided_activation_and_alpha(uh, orc, gpu):
    n, k, m = 48, 384, 5
    w = weights(n, k, tag=9)
    q, s = orc.fp8_quantize_rows(w)
    p, sz, z = orc.aq4_quantize(w)
    wide = activations_bf16(orc, m, k + 40, tag=9)
    xb = np.ascontiguousarray(wide[:, 8:8 + k])
    big = to_torch_bf16(wide, gpu)
    view = big[:, 8:8 + k]  # row stride k + 40, 16-byte aligned start
    odd = big[:, 3:3 + k]  # unaligned start
    for lw, ref in ((uh.LinearWeight.from_fp8(q, s), orc.fp8_gemv(xb, q, s, alpha=0.5)[0]),
                    (uh.LinearWeight.from_aq4(p, sz, z), orc.aq4_gemv(xb, p, sz, z, alpha=0.5)[0])):
        y = lw.forward(view, out_dtype=torch.float32, alpha=0.5)
        assert_close(y.cpu().numpy(), ref, what="strided")
    xo = np.ascontiguousarray(wide[:, 3:3 + k])
    y = uh.LinearWeight.from_fp8(q, s).forward(odd, out_dtype=torch.float32)
    assert_close(y.cpu().numpy(), orc.fp8_gemv(xo, q, s)[0], what="unaligned")


@pytest.mark.parametrize("m,k", [(1, 1), (3, 17), (7, 255), (16, 4096), (33, 513),
                                 # 16-byte vector path: one, two, eight chunks
                                 # per thread; nine falls back to scalar loads
                                 (5, 8), (64, 2048), (3, 16384), (3, 16392),
                                 (2048, 4096)])
def test_activation_quant_bit_exact(uh, orc, gpu, m, k):
    xb = activations_bf16(orc, m, k, tag=k)
    if m > 2:
        xb[1, :] = 0  # all-zero token
        xb[2, 0] = orc.bf16_from_f32(np.array([1e-30], np.float32))[0]
    xq_ref, xs_ref = orc.act_quantize(xb)
    xq, xs = uh.quantize_activations(to_torch_bf16(xb, gpu))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), xs_ref.view(np.uint32))


def test_activation_quant_special_rows(uh, orc, gpu):
    """Rows that pin the encode: exact E4M3 ties (row max 448 makes the scale
    1.0, so the midpoints between codes are quotients as they stand), the
    subnormal range, rows holding inf and NaN (inf max gives a NaN quotient
    for inf and zero for finite values), NaN beside finite values, and the
    bf16 extremes."""
    k = 1024
    codes = np.arange(0x7e, dtype=np.uint8)
    vals = orc.e4m3_to_f32(codes).astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    rows = []
    r = np.zeros(k, np.float32)
    r[0] = 448.0
    r[1:1 + mids.size] = mids
    r[1 + mids.size:1 + 2 * mids.size] = -mids
    rows.append(r)
    rows.append(np.linspace(-1e-3, 1e-3, k).astype(np.float32))
    r = np.linspace(-3, 3, k).astype(np.float32); r[5] = np.inf; rows.append(r)
    r = np.linspace(-3, 3, k).astype(np.float32); r[9] = np.nan; rows.append(r)
    r = np.linspace(-3, 3, k).astype(np.float32); r[9] = np.nan; r[700] = -np.inf
    rows.append(r)
    r = np.full(k, 3.3895314e38, np.float32); r[::2] *= -1; r[3] = 1e-38; rows.append(r)
    xb = orc.bf16_from_f32(np.stack(rows))
    xq_ref, xs_ref = orc.act_quantize(xb)
    xq, xs = uh.quantize_activations(to_torch_bf16(xb, gpu))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), xs_ref.view(np.uint32))


def test_activation_quant_strided_view(uh, orc, gpu):
    """A 16-byte aligned view with a padded row stride takes the vector path;
    an odd column offset the scalar one.  Both match the oracle."""
    m, k = 9, 1024
    wide = activations_bf16(orc, m, k + 24, tag=77)
    big = to_torch_bf16(wide, gpu)
    for off in (8, 3):
        xb = np.ascontiguousarray(wide[:, off:off + k])
        xq_ref, xs_ref = orc.act_quantize(xb)
        xq, xs = uh.quantize_activations(big[:, off:off + k])
        assert np.array_equal(xq.cpu().numpy(), xq_ref)
        assert np.array_equal(xs.cpu().numpy().view(np.uint32), xs_ref.view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(1, 16, 64), (7, 17, 65), (64, 64, 512),
                                   (130, 100, 1000), (256, 256, 4096),
                                   (200, 300, 512), (128, 17, 128),
                                   (513, 1040, 1024),
                                   # 256 x 256 blocks fill one round exactly,
                                   # so the 256-column block is chosen
                                   (256, 65536, 256),
                                   # one round of 256 x 192 blocks beats the
                                   # two rounds of 128 x 128 ones
                                   (1024, 8448, 256),
                                   # M below one 128-row block: the LDS
                                   # kernel with its single ragged block
                                   (1, 300, 128), (33, 1000, 256),
                                   (96, 4096, 512), (127, 520, 384)])
def test_fp8_gemm_parity(uh, orc, gpu, m, n, k):
    w = weights(n, k, tag=13)
    q, s = orc.fp8_quantize_rows(w)
    xb = activations_bf16(orc, m, k, tag=14)
    xq, xs = orc.act_quantize(xb)
    y_ref, _ = orc.fp8_gemm(xq, xs, q, s)
    lw = uh.LinearWeight.from_fp8(q, s)
    x = to_torch_bf16(xb, gpu)
    y = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    assert_close(y.cpu().numpy(), y_ref, what="fp8 gemm (quantize inside)")
    # pre-quantized activations
    xq_t = torch.from_numpy(xq).to(gpu)
    xs_t = torch.from_numpy(xs).to(gpu)
    y2 = lw.forward(xq_t, x_scales=xs_t)
    assert_close(bf16_tensor_to_f32(y2), y_ref, bf16_out=True, what="fp8 gemm bf16")


def test_workspace_size_and_caller_workspace(uh, orc, gpu):
    """Per-token FP8 prefill from bf16 without a K split needs the 1 KiB
    counter region plus M*K + 4*M bytes (each part rounded to 256); exact mode
    and pre-quantized input need none.  A caller-provided workspace of that
    size (counter region zeroed) gives the same result as the library
    buffer."""
    m, n, k = 300, 64, 512
    q, s = orc.fp8_quantize_rows(weights(n, k, tag=41))
    lw = uh.LinearWeight.from_fp8(q, s)
    rup = lambda v: (v + 255) // 256 * 256
    need = lw.workspace_size(m, mode=uh.ACT_FP8_PER_TOKEN)
    assert need == 1024 + rup(m * k) + rup(4 * m)
    assert lw.workspace_size(m) == 0
    assert lw.workspace_size(m, x_dtype=uh.DTYPE_F8E4M3FN) == 0
    x = to_torch_bf16(activations_bf16(orc, m, k, tag=42), gpu)
    wsb = torch.zeros((need,), dtype=torch.uint8, device=gpu)
    y1 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN, workspace=wsb)
    y2 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    assert torch.equal(y1, y2)


def test_zero_rows_is_noop(uh, orc, gpu):
    q, s = orc.fp8_quantize_rows(weights(16, 64))
    lw = uh.LinearWeight.from_fp8(q, s)
    x = torch.empty((0, 64), dtype=torch.bfloat16, device=gpu)
    y = lw.forward(x)
    assert y.shape == (0, 16)

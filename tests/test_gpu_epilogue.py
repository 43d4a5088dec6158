"""GPU parity of the fused output epilogues through the C ABI.

* Gated-pair weights (ULLM_LINEAR_LAYOUT_GATED_PAIRS): export and dequantize
  give back the canonical [2F][K] rows bit for bit, and a forward with
  SILU_MUL matches the oracle's gate/up product followed by its SiLU-gate
  epilogue, within 1e-2 x RMS (plus half a bf16 ulp for bf16 output).
* RESIDUAL_ADD: Y = alpha X W^T + R for bf16 and f32 R, also in place.

Shapes reach each kernel family: the LDS-staged and register-staged decode
kernels (M = 1, 3, 8, 17; few and many stripes; long K), and the FP8 prefill
GEMM (both its LDS-staged bf16 epilogue and its scalar f32 one).
"""
import numpy as np
import pytest
import torch

from helpers import (activations_bf16, assert_close, bf16_tensor_to_f32,
                     to_torch_bf16, weights)

pytestmark = pytest.mark.gpu


def _encode(orc, enc, w):
    if enc == "fp8":
        return orc.fp8_quantize_rows(w)
    return orc.aq4_quantize(w)


def _upload(uh, enc, parts, gated):
    if enc == "fp8":
        return uh.LinearWeight.from_fp8(*parts, gated=gated)
    return uh.LinearWeight.from_aq4(*parts, gated=gated)


def _gemv_ref(orc, enc, xb, parts, alpha=1.0):
    f = orc.fp8_gemv if enc == "fp8" else orc.aq4_gemv
    return f(xb, *parts, alpha=alpha)[0]


@pytest.mark.parametrize("enc", ["fp8", "aq4"])
@pytest.mark.parametrize("f,k", [(20, 256), (72, 1024)])
def test_gated_weight_keeps_canonical_rows(uh, orc, gpu, enc, f, k):
    w = weights(2 * f, k, tag=f + k)
    parts = _encode(orc, enc, w)
    lw = _upload(uh, enc, parts, gated=True)
    assert lw.info().layout == uh.LAYOUT_GATED_PAIRS and lw.n_out == f
    for got, ref in zip(lw.export(), parts):
        assert np.array_equal(got, ref)
    deq = (orc.fp8_dequantize if enc == "fp8" else orc.aq4_dequantize)(*parts)
    assert np.array_equal(lw.dequantize().cpu().numpy().view(np.uint32),
                          deq.view(np.uint32))
    # quantized on the device from f32 rows: same canonical encoding
    lq = uh.LinearWeight.quantize(torch.from_numpy(w).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW if enc == "fp8"
                                  else uh.ENCODING_AQ4_G128, gated=True)
    for got, ref in zip(lq.export(), parts):
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("m,f,k", [
    (1, 20, 256), (3, 72, 1024), (8, 72, 1024), (17, 40, 512),
    (1, 6200, 4096),     # multi-stripe LDS-staged, M = 1
    (8, 6200, 4096),     # register-staged groups of stripes
    (8, 500, 8192),      # long K: single-stripe groups
    (8, 8200, 1024),     # 1025 stripes: groups of 4
    (8, 33000, 1024),    # 4125 stripes: the wide configuration
])
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_silu_mul_decode(uh, orc, gpu, enc, m, f, k):
    w = weights(2 * f, k, tag=3 * f + m)
    parts = _encode(orc, enc, w)
    xb = activations_bf16(orc, m, k, tag=m + 500)
    alpha = 1.0 / (0.02 * np.sqrt(k))
    ref = orc.silu_mul(_gemv_ref(orc, enc, xb, parts, alpha=alpha))
    lw = _upload(uh, enc, parts, gated=True)
    x = to_torch_bf16(xb, gpu)
    y32 = lw.forward(x, out_dtype=torch.float32, alpha=alpha)
    torch.cuda.synchronize()
    assert y32.shape == (m, f)
    assert_close(y32.cpu().numpy(), ref, what=f"{enc} silu_mul f32 {m}x{f}x{k}")
    yb = lw.forward(x, alpha=alpha)
    assert_close(bf16_tensor_to_f32(yb), ref, bf16_out=True,
                 what=f"{enc} silu_mul bf16 {m}x{f}x{k}")


@pytest.mark.parametrize("m,f,k", [(256, 1000, 512), (130, 37, 256), (40, 100, 256)])
def test_silu_mul_prefill_gemm(uh, orc, gpu, m, f, k):
    w = weights(2 * f, k, tag=f)
    q, s = orc.fp8_quantize_rows(w)
    xb = activations_bf16(orc, m, k, tag=m + 600)
    xq, xs = orc.act_quantize(xb)
    ref = orc.silu_mul(orc.fp8_gemm(xq, xs, q, s)[0])
    lw = uh.LinearWeight.from_fp8(q, s, gated=True)
    x = to_torch_bf16(xb, gpu)
    yb = lw.forward(x, mode=uh.ACT_FP8_PER_TOKEN)       # LDS-staged bf16 stores
    y32 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(yb), ref, bf16_out=True, what="gemm silu bf16")
    assert_close(y32.cpu().numpy(), ref, what="gemm silu f32")


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (8, 300, 1024), (8, 4096, 14336),
                                   (33, 96, 512)])
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
@pytest.mark.parametrize("rdtype", ["bf16", "f32"])
def test_residual_add_decode(uh, orc, gpu, enc, rdtype, m, n, k):
    w = weights(n, k, tag=n + m)
    parts = _encode(orc, enc, w)
    xb = activations_bf16(orc, m, k, tag=m + 700)
    rb = activations_bf16(orc, m, n, tag=m + 800)
    r32 = orc.bf16_to_f32(rb)
    ref = _gemv_ref(orc, enc, xb, parts) + r32
    lw = _upload(uh, enc, parts, gated=False)
    x = to_torch_bf16(xb, gpu)
    res = to_torch_bf16(rb, gpu)
    if rdtype == "f32":
        res = res.float()
    y = lw.forward(x, out_dtype=torch.float32, residual=res)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), ref, what=f"{enc} residual {rdtype}")
    # in place: y is the residual
    yi = res.clone()
    lw.forward(x, yi, residual=yi)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(yi), ref, bf16_out=rdtype == "bf16",
                 what=f"{enc} residual in place {rdtype}")


def test_residual_add_prefill_gemm(uh, orc, gpu):
    m, n, k = 256, 448, 512
    q, s = orc.fp8_quantize_rows(weights(n, k, tag=9))
    xb = activations_bf16(orc, m, k, tag=901)
    rb = activations_bf16(orc, m, n, tag=902)
    xq, xs = orc.act_quantize(xb)
    ref = orc.fp8_gemm(xq, xs, q, s)[0] + orc.bf16_to_f32(rb)
    lw = uh.LinearWeight.from_fp8(q, s)
    x = to_torch_bf16(xb, gpu)
    y = to_torch_bf16(rb, gpu)
    lw.forward(x, y, residual=y, mode=uh.ACT_FP8_PER_TOKEN)   # in place, bf16
    y32 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN,
                     residual=to_torch_bf16(rb, gpu).float())
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(y), ref, bf16_out=True, what="gemm residual bf16")
    assert_close(y32.cpu().numpy(), ref, what="gemm residual f32")


@pytest.mark.parametrize("m,n,k,rdtype,pad", [(300, 1000, 512, "f32", 0),
                                              (130, 37, 256, "bf16", 3),
                                              (257, 448, 384, "bf16", 0),
                                              (256, 300, 256, "f32", 1),
                                              (1024, 8448, 256, "bf16", 0),
                                              (50, 300, 256, "bf16", 2)])
def test_residual_add_prefill_gemm_bf16_out(uh, orc, gpu, m, n, k, rdtype, pad):
    """bf16 output through the staged GEMM epilogue: residual as 4-column
    vectors (aligned rows) or element by element (odd row strides), ragged
    M and N, f32 and bf16 residuals."""
    q, s = orc.fp8_quantize_rows(weights(n, k, tag=n + k))
    xb = activations_bf16(orc, m, k, tag=m + 910)
    rb = activations_bf16(orc, m, n, tag=m + 920)
    xq, xs = orc.act_quantize(xb)
    ref = orc.fp8_gemm(xq, xs, q, s)[0] + orc.bf16_to_f32(rb)
    lw = uh.LinearWeight.from_fp8(q, s)
    x = to_torch_bf16(xb, gpu)
    wide = torch.zeros((m, n + pad), dtype=torch.float32 if rdtype == "f32" else torch.bfloat16,
                       device=gpu)
    res = wide[:, :n]
    res.copy_(to_torch_bf16(rb, gpu).to(wide.dtype))
    y = lw.forward(x, mode=uh.ACT_FP8_PER_TOKEN, residual=res)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(y), ref, bf16_out=True,
                 what=f"gemm residual {rdtype} pad {pad} {m}x{n}x{k}")


def test_epilogue_validation(uh, orc, gpu):
    import ctypes
    q, s = orc.fp8_quantize_rows(weights(32, 64))
    plain = uh.LinearWeight.from_fp8(q, s)
    gated = uh.LinearWeight.from_fp8(q, s, gated=True)
    x = torch.zeros((2, 64), dtype=torch.bfloat16, device=gpu)
    y = torch.zeros((2, 32), dtype=torch.bfloat16, device=gpu)

    def fwd(w, **kw):
        d = uh.new(uh.ForwardDesc, weight=w.handle, m=2, x=x.data_ptr(),
                   y=y.data_ptr(), x_dtype=uh.DTYPE_BF16, y_dtype=uh.DTYPE_BF16,
                   alpha=1.0, stream=torch.cuda.current_stream().cuda_stream)
        for k_, v in kw.items():
            setattr(d, k_, v)
        return uh.lib().ullm_linear_forward(ctypes.byref(d), None)

    assert fwd(plain) == uh.Status.OK
    assert fwd(gated) == uh.Status.INVALID_ARGUMENT                 # needs SILU_MUL
    assert fwd(gated, epilogue=uh.EPILOGUE_SILU_MUL) == uh.Status.OK
    assert fwd(plain, epilogue=uh.EPILOGUE_SILU_MUL) == uh.Status.INVALID_ARGUMENT
    assert fwd(plain, epilogue=9) == uh.Status.INVALID_ARGUMENT
    assert fwd(plain, epilogue=uh.EPILOGUE_RESIDUAL_ADD,
               residual_dtype=uh.DTYPE_BF16) == uh.Status.INVALID_ARGUMENT  # null R
    assert fwd(plain, epilogue=uh.EPILOGUE_RESIDUAL_ADD, residual=y.data_ptr(),
               residual_dtype=uh.DTYPE_F8E4M3FN) == uh.Status.UNSUPPORTED
    assert fwd(plain, epilogue=uh.EPILOGUE_RESIDUAL_ADD, residual=y.data_ptr(),
               residual_dtype=uh.DTYPE_F32) == uh.Status.INVALID_ARGUMENT  # in place, dtype
    assert fwd(plain, residual=y.data_ptr()) == uh.Status.INVALID_ARGUMENT
    assert fwd(plain, epilogue=uh.EPILOGUE_RESIDUAL_ADD, residual=y.data_ptr(),
               residual_dtype=uh.DTYPE_BF16) == uh.Status.OK
    torch.cuda.synchronize()

"""GPU parity at the exact BASELINE configurations #1-#3, at full size.

Configurations (the benchmark's own data distributions: weights ~N(0, 0.02)
quantized on the device, activations ~N(0, 1) in bf16, fp32 accumulation,
bf16 output):
  #1  FP8-E4M3 matvec, M=1, K=4096, N=4096;
  #2  AQ4 g128 matvec, M=1, K=4096, N=14336;
  #3  the FP8 small-batch sweep, M in {1, 2, 4, 8, 16, 32} over the Llama-3-8B
      layer shapes 4096->6144, 4096->4096, 4096->28672, 14336->4096.
Every output element is checked against the oracle's fp32-accumulated product
over the canonical encoding read back from the device weight (whose bit
exactness with the oracle's own quantizer is checked in test_gpu_linear.py):
max |Y - Y_ref| <= 1e-2 x RMS(Y_ref) + half a bf16 ulp of |Y_ref|.  The plan
query records which kernel family served each point.
"""
import pytest
import torch

from helpers import (activations_bf16, assert_close, bf16_tensor_to_f32, check_gemv_plan,
                     to_torch_bf16)

pytestmark = pytest.mark.gpu

SWEEP_SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]
SWEEP_M = [1, 2, 4, 8, 16, 32]


def _weight(uh, gpu, encoding, n, k, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    w = torch.randn((n, k), generator=g, device=gpu) * 0.02
    lw = uh.LinearWeight.quantize(w, encoding)
    del w
    return lw


def _check(uh, orc, gpu, lw, parts, enc, m, k, tag, what, plan=None):
    xb = activations_bf16(orc, m, k, tag=tag)
    x = to_torch_bf16(xb, gpu)
    y = lw.forward(x)
    if plan is not None:
        check_gemv_plan(lw, x, y, plan)
    torch.cuda.synchronize()
    ref = (orc.fp8_gemv if enc == "fp8" else orc.aq4_gemv)(xb, *parts)[0]
    assert_close(bf16_tensor_to_f32(y), ref, bf16_out=True, what=what)
    return lw.plan(x, y).kernel


def test_config1_fp8_matvec_4096(uh, orc, gpu):
    lw = _weight(uh, gpu, uh.ENCODING_FP8_E4M3_ROW, 4096, 4096, seed=1)
    # The multi-stripe kernel, 8 waves (the benchmarked launch).
    assert _check(uh, orc, gpu, lw, lw.export(), "fp8", 1, 4096, 11,
                  "config #1", ("multi", 8, 1, 1)) == uh.KERNEL_GEMV
    lw.destroy()


def test_config2_aq4_matvec_14336(uh, orc, gpu):
    lw = _weight(uh, gpu, uh.ENCODING_AQ4_G128, 14336, 4096, seed=2)
    # The multi-stripe kernel, 8 waves, rows packed in four classes.
    assert _check(uh, orc, gpu, lw, lw.export(), "aq4", 1, 4096, 12,
                  "config #2", ("multi", 8, 1, 4)) == uh.KERNEL_GEMV
    lw.destroy()


@pytest.mark.parametrize("k,n", SWEEP_SHAPES)
def test_config3_fp8_sweep(uh, orc, gpu, k, n):
    lw = _weight(uh, gpu, uh.ENCODING_FP8_E4M3_ROW, n, k, seed=k + n)
    parts = lw.export()
    for m in SWEEP_M:
        kind = _check(uh, orc, gpu, lw, parts, "fp8", m, k, m + n,
                      f"config #3 {k}->{n} M={m}")
        assert kind == uh.KERNEL_GEMV
    lw.destroy()

"""The bf16 encode the kernels use, checked on the device.

Every kernel rounds its fp32 results to bf16 with gfx950's packed convert
(device_common.hpp).  The contract is round-to-nearest-even on the 16 dropped
bits with NaN kept quiet (the oracle's f32_to_bf16, itself checked against
torch's bfloat16 cast in test_oracle_formats.py).  Two checks:

- libullm_bench.so's ullm_bench_bf16_convert_check runs the scalar and the
  packed encode over all 2^32 f32 bit patterns against that rule spelled out
  in integer arithmetic, and counts mismatches (must be none);
- end to end, a bf16 GEMM and GEMV output must equal the same call's fp32
  output rounded by torch (the two outputs share every fp32 operation before
  the encode), bit for bit.
"""
import ctypes

import pytest
import torch

from helpers import activations_bf16, to_torch_bf16, weights

pytestmark = pytest.mark.gpu


def test_encode_matches_rule_on_all_inputs(uh, gpu):
    lib = ctypes.CDLL(str(uh.LIB_PATH.parent / "libullm_bench.so"))
    fn = lib.ullm_bench_bf16_convert_check
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    counts = torch.zeros(3, dtype=torch.int64, device=gpu)
    stream = torch.cuda.current_stream(gpu)
    assert fn(ctypes.c_void_p(counts.data_ptr()), ctypes.c_void_p(stream.cuda_stream)) == 0
    stream.synchronize()
    finite, nan, first = (int(v) for v in counts.cpu())
    assert (finite, nan) == (0, 0), f"first mismatching input: {first - 1:#010x}"


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (8, 6144, 4096),
                                   (256, 2048, 1024), (2048, 1792, 512)])
def test_bf16_output_is_rounded_f32_output(uh, orc, gpu, m, n, k):
    """FP8 weights: decode GEMV (M <= 32) and the prefill GEMM (M >= 256,
    activations quantized per token first)."""
    q, s = orc.fp8_quantize_rows(weights(n, k, tag=61))
    lw = uh.LinearWeight.from_fp8(q, s)
    x = to_torch_bf16(activations_bf16(orc, m, k, tag=m + 600), gpu)
    if m >= 256:
        xq, xs = uh.quantize_activations(x)
        y32 = lw.forward(xq, x_scales=xs, out_dtype=torch.float32)
        y16 = lw.forward(xq, x_scales=xs)
    else:
        y32 = lw.forward(x, out_dtype=torch.float32)
        y16 = lw.forward(x)
    torch.cuda.synchronize()
    want = y32.to(torch.bfloat16).view(torch.int16)
    assert torch.equal(y16.view(torch.int16), want)
    lw.destroy()

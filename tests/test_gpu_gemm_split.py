"""GPU parity of the prefill FP8 GEMM when it splits K over workgroups.

Grids of few output tiles (at most half of the CUs busy, K of at least 32
k-steps of 128, 16 in 64 x 64 blocks) run each
tile's K in parts on otherwise idle CUs; the last part of a tile to finish
adds the fp32 partial sums in part order and runs the epilogue.  Checked
against the oracle on sampled rows (rows of a GEMM are independent), for each
epilogue, bf16 and f32 outputs, bf16 and pre-quantized activations, the
library-owned and a caller workspace.  Repeated calls are bit-identical: the
sum order does not depend on which part finishes last, and every call leaves
the tile counters zero for the next.

Tolerance: max |Y - Y_ref| <= 1e-2 x RMS(Y_ref) (+ half a bf16 ulp of |Y_ref|
for bf16 outputs), Y_ref the oracle's fp32-accumulated product.
"""
import numpy as np
import pytest
import torch

from helpers import (activations_bf16, assert_close, bf16_tensor_to_f32, rng,
                     to_torch_bf16)

pytestmark = pytest.mark.gpu

# (M, N, K, K parts expected on a 256-CU device)
SPLIT = [
    (256, 4096, 4096, 2),    # 128 tiles of 128 x 64, 16 k-steps per part
    (300, 2000, 4096, 2),    # ragged M and N (128 x 64)
    (300, 2000, 4224, 2),    # 33 k-steps: parts of 17 and 16
    (256, 1024, 8320, 4),    # 64 x 64; 65 k-steps: parts of 17, 17, 17, 14
    (256, 256, 4096, 4),     # 16 tiles of 64 x 64: four parts of 8
    (256, 4480, 6144, 3),    # 70 tiles of 256 x 64, 48 k-steps: three of 16
    (256, 2304, 14336, 3),   # 72 tiles of 128 x 64: parts of 38, 38, 36
    (64, 2048, 14336, 8),    # 32 tiles of 64 x 64: eight parts of 14
    (256, 2048, 14208, 4),   # 128 x 64; 111 k-steps: three of 28, one of 27
    (256, 2560, 14208, 3),   # 80 tiles of 128 x 64; parts of 37, 37, 37
    (64, 2560, 14208, 6),    # the same split on 64 x 64 blocks
    (16, 4096, 4096, 4),     # M below one MFMA tile
]


def _sample_rows(m, tag, per_block=8):
    r = rng(tag)
    rows = {0, m - 1}
    for b0 in range(0, m, 256):
        hi = min(m, b0 + 256)
        rows.update(int(v) for v in r.integers(b0, hi, size=min(per_block, hi - b0)))
    return np.array(sorted(rows))


def _fp8_weight(uh, n, k, tag, gpu, gated=False):
    w = torch.randn((n, k), generator=torch.Generator().manual_seed(tag)) * 0.02
    lw = uh.LinearWeight.quantize(w.to(gpu), uh.ENCODING_FP8_E4M3_ROW, gated=gated)
    q, s = lw.export()
    return lw, q, s


def _check_split(uh, lw, x, y, parts, **kw):
    p = lw.plan(x, y, mode=uh.ACT_FP8_PER_TOKEN, **kw)
    assert p.kernel == uh.KERNEL_GEMM_LDS, p.kernel
    if torch.cuda.get_device_properties(x.device).multi_processor_count == 256:
        assert p.split_k == parts, (p.split_k, parts)
        assert p.grid == p.tiles * parts, (p.grid, p.tiles)


@pytest.mark.parametrize("m,n,k,parts", SPLIT)
def test_split_gemm_parity(uh, orc, gpu, m, n, k, parts):
    lw, q, s = _fp8_weight(uh, n, k, tag=m + n + 11, gpu=gpu)
    xb = activations_bf16(orc, m, k, tag=m + 12)
    xq, xs = orc.act_quantize(xb)
    rows = _sample_rows(m, tag=m + 13)
    ref = orc.fp8_gemm(xq[rows], xs[rows], q, s)[0]
    x = to_torch_bf16(xb, gpu)
    yb = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    _check_split(uh, lw, x, yb, parts)
    lw.forward(x, yb, mode=uh.ACT_FP8_PER_TOKEN)
    y32 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    yb2 = torch.empty_like(yb)
    lw.forward(x, yb2, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(yb[rows]), ref, bf16_out=True,
                 what=f"split bf16 {m}x{n}x{k}")
    assert_close(y32[rows].cpu().numpy(), ref, what=f"split f32 {m}x{n}x{k}")
    assert torch.equal(yb, yb2)   # deterministic, counters left zero
    # pre-quantized activations: the same launch, its own split scratch
    xq_t = torch.from_numpy(xq).to(gpu)
    xs_t = torch.from_numpy(xs).to(gpu)
    y3 = lw.forward(xq_t, x_scales=xs_t, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y3, y32)


def test_split_gemm_epilogues(uh, orc, gpu):
    m, n, k = 256, 4096, 4096
    # SiLU-gate on a gated-pair weight
    lw, q, s = _fp8_weight(uh, n, k, tag=21, gpu=gpu, gated=True)
    xb = activations_bf16(orc, m, k, tag=22)
    xq, xs = orc.act_quantize(xb)
    rows = _sample_rows(m, tag=23)
    ref = orc.silu_mul(orc.fp8_gemm(xq[rows], xs[rows], q, s)[0])
    x = to_torch_bf16(xb, gpu)
    yb = torch.empty((m, n // 2), dtype=torch.bfloat16, device=gpu)
    p = lw.plan(x, yb, mode=uh.ACT_FP8_PER_TOKEN)
    assert p.split_k > 1 or torch.cuda.get_device_properties(gpu).multi_processor_count != 256
    lw.forward(x, yb, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(yb[rows]), ref, bf16_out=True, what="split silu")
    lw.destroy()
    # residual add, in place over the residual
    lw, q, s = _fp8_weight(uh, n, k, tag=24, gpu=gpu)
    rb = activations_bf16(orc, m, n, tag=25)
    ref = orc.fp8_gemm(xq[rows], xs[rows], q, s)[0] + orc.bf16_to_f32(rb[rows])
    y = to_torch_bf16(rb, gpu)
    lw.forward(x, y, residual=y, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(y[rows]), ref, bf16_out=True, what="split residual")


def test_split_gemm_caller_workspace(uh, orc, gpu):
    m, n, k = 300, 2000, 4096
    lw, q, s = _fp8_weight(uh, n, k, tag=31, gpu=gpu)
    x = to_torch_bf16(activations_bf16(orc, m, k, tag=32), gpu)
    need = lw.workspace_size(m, mode=uh.ACT_FP8_PER_TOKEN)
    rup = lambda v: (v + 255) // 256 * 256
    y0 = torch.empty((m, n), dtype=torch.float32, device=gpu)
    p = lw.plan(x, y0, mode=uh.ACT_FP8_PER_TOKEN)
    parts = p.tiles * p.split_k * p.block_m * p.block_n * 4 if p.split_k > 1 else 0
    assert need == 1024 + parts + rup(m * k) + rup(4 * m), (need, parts)
    ws = torch.zeros((need,), dtype=torch.uint8, device=gpu)
    y1 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN, workspace=ws)
    y2 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN, workspace=ws)
    y3 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    assert int(ws[:1024].count_nonzero()) == 0   # counters left zero
    # pre-quantized input needs only the split scratch
    assert lw.workspace_size(m, x_dtype=uh.DTYPE_F8E4M3FN) == 1024 + parts


def test_split_plan_invariants(uh, gpu):
    """Every plan over a sweep of prefill shapes: a split has at least two
    parts of at least 16 k-steps each (8 in 64 x 64 blocks; none empty), one workgroup per part,
    at most one round of the CUs, counters within their 1 KiB region, and the
    workspace size that holds its partial sums."""
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    rup = lambda v: (v + 255) // 256 * 256
    seen = set()
    for n, k in ((256, 4096), (2000, 4096), (4096, 14336), (4480, 6144),
                 (6144, 2048), (28672, 4096), (1024, 8320)):
        lw = uh.LinearWeight.quantize(torch.zeros((n, k), device=gpu),
                                      uh.ENCODING_FP8_E4M3_ROW)
        for m in (33, 64, 128, 200, 256, 300, 512, 768, 1024, 2048):
            x = torch.empty((m, k), dtype=torch.bfloat16, device=gpu)
            y = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
            p = lw.plan(x, y, mode=uh.ACT_FP8_PER_TOKEN)
            need = lw.workspace_size(m, mode=uh.ACT_FP8_PER_TOKEN)
            steps = k // 128
            if p.split_k > 1:
                seen.add(p.split_k)
                kpp = -(-steps // p.split_k)
                assert p.kernel == uh.KERNEL_GEMM_LDS
                assert p.block_m in (64, 128, 256) and p.block_n == 64 or \
                    p.block_m == 256, (m, n, k, p.block_m, p.block_n)
                floor = 8 if p.block_m * p.block_n <= 64 * 64 else 16
                assert kpp >= floor and (p.split_k - 1) * kpp < steps, (m, n, k, p.split_k)
                assert p.grid == p.tiles * p.split_k <= cus, (m, n, k, p.grid)
                assert p.tiles * 4 <= 1024
                parts = p.tiles * p.split_k * p.block_m * p.block_n * 4
                assert parts < 2 ** 31
            else:
                assert p.split_k == 1
                parts = 0
            assert need == 1024 + parts + rup(m * k) + rup(4 * m), (m, n, k, need)
        lw.destroy()
    if cus == 256:
        assert seen >= {2, 3, 4}, seen

"""GPU parity of the prefill FP8 GEMM on its persistent multi-tile launches
and on the one-round 256 x 128 launches of the N = 4096 prefill shapes.

Each shape below makes the launcher pick one block configuration with more
output tiles than workgroups, so every workgroup walks several tiles and
issues the next tile's first copies during the current tile's epilogue.  The
test asks the library which launch it makes (ullm_linear_forward_plan) and
fails if the shape no longer reaches the configuration it names, so a later
tuning change cannot drop the coverage silently.

Rows of a GEMM are independent, so the oracle runs on a stratified sample of
rows (some from every 256-row block, the first and last rows included) over
all columns; every output tile is checked on its sampled rows.  The full-size
prefill configuration (M=2048, K=4096, N=28672, bf16 activations quantized
per token inside the call) is checked the same way.

Tolerance: max |Y - Y_ref| <= 1e-2 x RMS(Y_ref) (+ half a bf16 ulp of |Y_ref|
for bf16 outputs), Y_ref the oracle's fp32-accumulated product.
"""
import numpy as np
import pytest
import torch

from helpers import (activations_bf16, assert_close, bf16_tensor_to_f32, rng,
                     to_torch_bf16)

pytestmark = pytest.mark.gpu

# (configuration, M, N, K): block 256 x N_b, or 128 x 128 two per CU.
PERSISTENT = [
    ("256x224", 1024, 28672, 256),   # 512 tiles on 256 workgroups
    ("256x256", 200, 131072, 128),   # 512 tiles, one ragged 256-row block
    ("256x192", 250, 98304, 256),    # 512 tiles
    ("128x128", 1100, 14000, 256),   # 990 tiles on 512 workgroups, ragged N
]
# One round of ping-pong blocks (the N = 4096 and 6144 prefill shapes, a
# 256-column one, and the 128 x 64 and 64 x 64 blocks of short prompts) with
# several k-steps, so the three-stage rings wrap: the launch is not
# persistent, so only the block is asserted.
ONE_ROUND = [
    ("256x128", 2048, 4096, 256),    # 256 tiles on 256 CUs
    ("256x64", 1024, 4000, 128),     # 252 tiles, ragged N
    ("256x256", 2048, 8192, 512),    # 256 tiles, four k-steps
    ("256x192", 2048, 6144, 384),    # 256 tiles, three k-steps
    ("64x64", 256, 4096, 512),       # 256 tiles of the short-prompt blocks
    ("64x64", 300, 2000, 256),       # 160 tiles, ragged M and N
    ("128x64", 120, 14336, 512),     # 224 tiles, one ragged 128-row block
    ("128x64", 100, 6000, 4096),     # 94 tiles, K split in two
    ("64x128", 40, 28672, 512),      # 224 tiles, chunks past the stages
    ("128x128", 128, 28672, 384),    # 224 tiles of the 128-column short blocks
]
CASES = [c + (True,) for c in PERSISTENT] + [c + (False,) for c in ONE_ROUND]


def _sample_rows(m, tag, per_block=6):
    r = rng(tag)
    rows = {0, m - 1}
    for b0 in range(0, m, 256):
        hi = min(m, b0 + 256)
        rows.update(int(v) for v in r.integers(b0, hi, size=min(per_block, hi - b0)))
    return np.array(sorted(rows))


def _plan_matches(uh, lw, x, y, cfg, persistent=True, **kw):
    p = lw.plan(x, y, mode=uh.ACT_FP8_PER_TOKEN, **kw)
    assert p.kernel == uh.KERNEL_GEMM_LDS, p.kernel
    bm, bn = (int(v) for v in cfg.split("x"))
    assert (p.block_m, p.block_n) == (bm, bn), (p.block_m, p.block_n)
    if persistent:
        assert p.tiles > p.grid, (p.tiles, p.grid)   # several tiles each
    return p


def _fp8_weight(uh, orc, n, k, tag, gpu, gated=False):
    """Quantize on the GPU (bit-exact with the oracle; checked elsewhere) and
    read the canonical encoding back for the oracle."""
    w = torch.randn((n, k), generator=torch.Generator().manual_seed(tag)) * 0.02
    lw = uh.LinearWeight.quantize(w.to(gpu), uh.ENCODING_FP8_E4M3_ROW, gated=gated)
    q, s = lw.export()
    return lw, q, s


@pytest.mark.parametrize("cfg,m,n,k,persistent", CASES)
def test_persistent_gemm_no_epilogue(uh, orc, gpu, cfg, m, n, k, persistent):
    lw, q, s = _fp8_weight(uh, orc, n, k, tag=m + n, gpu=gpu)
    xb = activations_bf16(orc, m, k, tag=m + 1)
    xq, xs = orc.act_quantize(xb)
    rows = _sample_rows(m, tag=m)
    ref = orc.fp8_gemm(xq[rows], xs[rows], q, s)[0]
    x = to_torch_bf16(xb, gpu)
    yb = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    _plan_matches(uh, lw, x, yb, cfg, persistent)
    lw.forward(x, yb, mode=uh.ACT_FP8_PER_TOKEN)           # staged bf16 stores
    y32 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(yb[rows]), ref, bf16_out=True,
                 what=f"{cfg} bf16 {m}x{n}x{k}")
    assert_close(y32[rows].cpu().numpy(), ref, what=f"{cfg} f32 {m}x{n}x{k}")
    # pre-quantized activations take the same launch
    xq_t = torch.from_numpy(xq).to(gpu)
    xs_t = torch.from_numpy(xs).to(gpu)
    y2 = lw.forward(xq_t, x_scales=xs_t)
    assert_close(bf16_tensor_to_f32(y2[rows]), ref, bf16_out=True,
                 what=f"{cfg} pre-quantized {m}x{n}x{k}")


@pytest.mark.parametrize("cfg,m,n,k,persistent", CASES)
def test_persistent_gemm_silu_mul(uh, orc, gpu, cfg, m, n, k, persistent):
    lw, q, s = _fp8_weight(uh, orc, n, k, tag=m + n + 1, gpu=gpu, gated=True)
    f = n // 2
    xb = activations_bf16(orc, m, k, tag=m + 2)
    xq, xs = orc.act_quantize(xb)
    rows = _sample_rows(m, tag=m + 1)
    ref = orc.silu_mul(orc.fp8_gemm(xq[rows], xs[rows], q, s)[0])
    x = to_torch_bf16(xb, gpu)
    yb = torch.empty((m, f), dtype=torch.bfloat16, device=gpu)
    _plan_matches(uh, lw, x, yb, cfg, persistent)
    lw.forward(x, yb, mode=uh.ACT_FP8_PER_TOKEN)
    y32 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(yb[rows]), ref, bf16_out=True,
                 what=f"{cfg} silu bf16")
    assert_close(y32[rows].cpu().numpy(), ref, what=f"{cfg} silu f32")


@pytest.mark.parametrize("cfg,m,n,k,persistent", CASES)
def test_persistent_gemm_residual(uh, orc, gpu, cfg, m, n, k, persistent):
    lw, q, s = _fp8_weight(uh, orc, n, k, tag=m + n + 2, gpu=gpu)
    xb = activations_bf16(orc, m, k, tag=m + 3)
    rb = activations_bf16(orc, m, n, tag=m + 4)
    xq, xs = orc.act_quantize(xb)
    rows = _sample_rows(m, tag=m + 2)
    ref = orc.fp8_gemm(xq[rows], xs[rows], q, s)[0] + orc.bf16_to_f32(rb[rows])
    x = to_torch_bf16(xb, gpu)
    y = to_torch_bf16(rb, gpu)
    _plan_matches(uh, lw, x, y, cfg, persistent, residual=y)
    y32 = lw.forward(x, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN,
                     residual=y.float())                    # f32 scalar epilogue
    lw.forward(x, y, residual=y, mode=uh.ACT_FP8_PER_TOKEN)  # in place, staged bf16
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(y[rows]), ref, bf16_out=True,
                 what=f"{cfg} residual bf16")
    assert_close(y32[rows].cpu().numpy(), ref, what=f"{cfg} residual f32")


def test_prefill_gemm_full_config(uh, orc, gpu):
    """The benchmarked prefill shape: M=2048, K=4096, N=28672, weights
    ~N(0, 0.02) quantized per row, bf16 activations ~N(0, 1) quantized per
    token inside the call, bf16 output (256 x 224 blocks, 1024 tiles)."""
    m, n, k = 2048, 28672, 4096
    lw, q, s = _fp8_weight(uh, orc, n, k, tag=4, gpu=gpu)
    xb = activations_bf16(orc, m, k, tag=5)
    xq, xs = orc.act_quantize(xb)
    rows = _sample_rows(m, tag=6, per_block=5)
    ref = orc.fp8_gemm(xq[rows], xs[rows], q, s)[0]
    x = to_torch_bf16(xb, gpu)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    p = _plan_matches(uh, lw, x, y, "256x224")
    assert p.tiles == 1024
    lw.forward(x, y, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert_close(bf16_tensor_to_f32(y[rows]), ref, bf16_out=True,
                 what="prefill 2048x28672x4096")
    # every row is finite and the device's own quantized activations match
    assert bool(torch.isfinite(y.float()).all())
    xq_d, xs_d = uh.quantize_activations(x)
    assert np.array_equal(xq_d.cpu().numpy(), xq)
    assert np.array_equal(xs_d.cpu().numpy().view(np.uint32), xs.view(np.uint32))

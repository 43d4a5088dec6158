"""GPU parity of split-K decode launches (9 <= M <= 32, few stripes, long K):
workgroups streaming different K parts of a stripe group write fp32 partial
sums and the last to arrive adds them.  Checks against the oracle (1e-2 x
RMS), with the epilogues, through the library's scratch and through a
caller workspace (counters zero on entry and left zero: two calls in a row
agree bit for bit), and that a launch is deterministic."""
import numpy as np
import pytest
import torch

from helpers import (activations_bf16, assert_close, bf16_tensor_to_f32,
                     to_torch_bf16, weights)

pytestmark = pytest.mark.gpu


def _setup(uh, orc, enc, m, n, k, tag):
    w = weights(n, k, tag=tag)
    if enc == "fp8":
        parts = orc.fp8_quantize_rows(w)
        lw = uh.LinearWeight.from_fp8(*parts)
        ref_fn = orc.fp8_gemv
    else:
        parts = orc.aq4_quantize(w)
        lw = uh.LinearWeight.from_aq4(*parts)
        ref_fn = orc.aq4_gemv
    xb = activations_bf16(orc, m, k, tag=tag + 1)
    return lw, parts, ref_fn, xb


@pytest.mark.parametrize("m,n,k", [(16, 4096, 14336), (32, 4096, 14336),
                                   (17, 1000, 12288), (9, 300, 16384)])
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_split_k_parity(uh, orc, gpu, enc, m, n, k):
    lw, parts, ref_fn, xb = _setup(uh, orc, enc, m, n, k, tag=m + n)
    assert lw.workspace_size(m) > 0, "this shape is expected to split K"
    ref = ref_fn(xb, *parts)[0]
    x = to_torch_bf16(xb, gpu)
    y1 = lw.forward(x, out_dtype=torch.float32)
    y2 = lw.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "split-K launches must be deterministic"
    assert_close(y1.cpu().numpy(), ref, what=f"{enc} split {m}x{n}x{k}")
    yb = lw.forward(x)
    assert_close(bf16_tensor_to_f32(yb), ref, bf16_out=True, what=f"{enc} split bf16")


@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_split_k_caller_workspace(uh, orc, gpu, enc):
    m, n, k = 24, 2000, 14336
    lw, parts, ref_fn, xb = _setup(uh, orc, enc, m, n, k, tag=91)
    need = lw.workspace_size(m)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    x = to_torch_bf16(xb, gpu)
    ya = lw.forward(x, out_dtype=torch.float32, workspace=ws)
    yb = lw.forward(x, out_dtype=torch.float32, workspace=ws)     # counters reset
    yc = lw.forward(x, out_dtype=torch.float32)                   # library scratch
    torch.cuda.synchronize()
    assert torch.equal(ya, yb) and torch.equal(ya, yc)
    assert_close(ya.cpu().numpy(), ref_fn(xb, *parts)[0], what=f"{enc} split workspace")
    too_small = torch.zeros(need - 1, dtype=torch.uint8, device=gpu)
    with pytest.raises(uh.HipError) as e:
        lw.forward(x, workspace=too_small)
    assert e.value.status == uh.Status.BUFFER_TOO_SMALL


def test_split_k_with_epilogues(uh, orc, gpu):
    m, f, k = 16, 600, 14336
    w = weights(2 * f, k, tag=93)
    parts = orc.aq4_quantize(w)
    g = uh.LinearWeight.from_aq4(*parts, gated=True)
    xb = activations_bf16(orc, m, k, tag=94)
    ref = orc.silu_mul(orc.aq4_gemv(xb, *parts)[0])
    assert g.workspace_size(m) > 0
    y = g.forward(to_torch_bf16(xb, gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), ref, what="split silu_mul")
    lw, parts2, ref_fn, xb2 = _setup(uh, orc, "fp8", m, 1200, k, tag=95)
    r = torch.randn(m, 1200, device=gpu)
    y2 = lw.forward(to_torch_bf16(xb2, gpu), out_dtype=torch.float32, residual=r)
    torch.cuda.synchronize()
    assert_close(y2.cpu().numpy(), ref_fn(xb2, *parts2)[0] + r.cpu().numpy(),
                 what="split residual")


def test_split_k_shapes_share_workspace(uh, orc, gpu):
    """Split launches of different stripe counts one after another through
    the same scratch (the library's, then one caller workspace): a launch
    with few stripes leaves partial sums where a launch with more stripes
    keeps counters unless the counter region has one size for all, which
    showed as wrong, run-to-run varying results of the second launch."""
    cases = [("fp8", 17, 1000, 12288), ("aq4", 16, 4096, 14336),
             ("fp8", 9, 300, 16384), ("aq4", 32, 4096, 14336), ("fp8", 16, 4096, 14336)]
    setups = [(_setup(uh, orc, enc, m, n, k, tag=m + n + 7), m) for enc, m, n, k in cases]
    refs = [ref_fn(xb, *parts)[0] for (lw, parts, ref_fn, xb), m in setups]
    need = max(lw.workspace_size(m) for (lw, _, _, _), m in setups)
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    for workspace in (None, ws):
        for rep in range(2):
            for ((lw, parts, ref_fn, xb), m), ref in zip(setups, refs):
                x = to_torch_bf16(xb, gpu)
                y = lw.forward(x, out_dtype=torch.float32, workspace=workspace)
                torch.cuda.synchronize()
                assert_close(y.cpu().numpy(), ref,
                             what=f"shared scratch {m}x{lw.n} rep {rep} ws {workspace is not None}")

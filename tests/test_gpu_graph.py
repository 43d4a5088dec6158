"""GPU: forwards captured in a HIP graph (how bench.py times them) give the
eager result on every replay.

Each case runs the forward eagerly, captures the same call into a
torch.cuda.CUDAGraph, then replays it several times with unrelated eager work
and synchronizations in between, comparing every replay with the eager output
bit for bit (the kernels are deterministic).  Covers each decode kernel
family, the fused epilogues, the prefill GEMM with a caller workspace (no
allocation may happen under capture) and one step of a small decode stack.
"""
import numpy as np
import pytest
import torch

from helpers import weights

pytestmark = pytest.mark.gpu


def _replays_match(fn, out, reps=4):
    fn()
    torch.cuda.synchronize()
    ref = out.clone()
    out.zero_()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                               # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    for i in range(reps):
        out.fill_(float("nan") if out.is_floating_point() else 0)
        junk = torch.randn(1 << 16, device=out.device).sum()   # eager work between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i} differs from the eager result"
        del junk


@pytest.mark.parametrize("enc", ["fp8", "aq4"])
@pytest.mark.parametrize("m,n,k", [(1, 14336, 4096), (8, 28672, 4096), (8, 4096, 14336),
                                   (3, 1000, 512), (17, 6200, 1024),
                                   (24, 2000, 14336)])   # split K: counters reset
def test_decode_forward_under_graph(uh, gpu, enc, m, n, k):
    code = uh.ENCODING_FP8_E4M3_ROW if enc == "fp8" else uh.ENCODING_AQ4_G128
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(n, k, tag=m)).to(gpu), code)
    x = torch.randn(m, k, device=gpu).bfloat16()
    y = torch.empty(m, n, device=gpu, dtype=torch.bfloat16)
    _replays_match(lambda: lw.forward(x, y), y)


def test_epilogues_under_graph(uh, gpu):
    g = uh.LinearWeight.quantize(torch.from_numpy(weights(2 * 1024, 1024, tag=5)).to(gpu),
                                 uh.ENCODING_AQ4_G128, gated=True)
    x = torch.randn(8, 1024, device=gpu).bfloat16()
    a = torch.empty(8, 1024, device=gpu, dtype=torch.bfloat16)
    _replays_match(lambda: g.forward(x, a), a)
    d = uh.LinearWeight.quantize(torch.from_numpy(weights(512, 1024, tag=6)).to(gpu),
                                 uh.ENCODING_AQ4_G128)
    r = torch.randn(8, 512, device=gpu)
    y = torch.empty(8, 512, device=gpu)
    _replays_match(lambda: d.forward(x, y, residual=r), y)


def test_prefill_gemm_under_graph_with_caller_workspace(uh, gpu):
    m, n, k = 512, 2048, 1024
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(n, k, tag=7)).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW)
    x = torch.randn(m, k, device=gpu).bfloat16()
    # the first 1 KiB (split-K counters: this grid splits K) starts at zero
    ws = torch.zeros(lw.workspace_size(m, mode=uh.ACT_FP8_PER_TOKEN), dtype=torch.uint8,
                     device=gpu)
    y = torch.empty(m, n, device=gpu, dtype=torch.bfloat16)
    _replays_match(lambda: lw.forward(x, y, mode=uh.ACT_FP8_PER_TOKEN, workspace=ws), y)


def test_small_stack_step_under_graph(uh, gpu):
    import stack
    st = stack.DecodeStack(uh, torch, gpu, batch=8, layers=2, hidden=512, qkv=768,
                           ffn=1024, vocab=2000)
    st.h0.copy_(torch.randn(st.h0.shape, device=gpu))
    _replays_match(lambda: st.step(), st.logits)
    assert torch.isfinite(st.logits.float()).all()
    st.destroy()


def test_library_workspace_outgrown_after_capture(uh, gpu):
    """A graph captured with the library-owned prefill workspace replays
    correctly after a larger call on the same stream has grown that
    workspace (the outgrown buffer stays allocated)."""
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(512, 1024, tag=21)).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW)
    xs = torch.randn(256, 1024, device=gpu).bfloat16()
    ys = torch.empty(256, 512, device=gpu, dtype=torch.bfloat16)
    xb = torch.randn(2048, 1024, device=gpu).bfloat16()
    yb = torch.empty(2048, 512, device=gpu, dtype=torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lw.forward(xs, ys, mode=uh.ACT_FP8_PER_TOKEN)   # allocates for M = 256
    s.synchronize()
    ref = ys.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        lw.forward(xs, ys, mode=uh.ACT_FP8_PER_TOKEN)
    with torch.cuda.stream(s):
        lw.forward(xb, yb, mode=uh.ACT_FP8_PER_TOKEN)   # grows the buffer
    s.synchronize()
    for i in range(3):
        ys.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, ref), f"replay {i} after the workspace grew"


def test_library_workspace_per_stream(uh, gpu):
    """Prefill calls on two streams at once use separate library-owned
    workspaces: each matches its result computed alone."""
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(2048, 2048, tag=22)).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW)
    xa = torch.randn(1024, 2048, device=gpu).bfloat16()
    xb = torch.randn(1024, 2048, device=gpu).bfloat16()
    ra = lw.forward(xa, mode=uh.ACT_FP8_PER_TOKEN)
    rb = lw.forward(xb, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ya = torch.empty_like(ra)
    yb = torch.empty_like(rb)
    for _ in range(2):                       # first round allocates
        sa.wait_stream(torch.cuda.current_stream())
        sb.wait_stream(torch.cuda.current_stream())
        for _ in range(4):
            lw.forward(xa, ya, mode=uh.ACT_FP8_PER_TOKEN, stream=sa)
            lw.forward(xb, yb, mode=uh.ACT_FP8_PER_TOKEN, stream=sb)
        torch.cuda.synchronize()
        assert torch.equal(ya, ra)
        assert torch.equal(yb, rb)

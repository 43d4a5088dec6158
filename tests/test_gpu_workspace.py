"""Library-owned forward workspaces and the forward-plan query, on the GPU.

* The first split-K decode call on a freshly created non-blocking stream
  (whose library workspace is allocated and zeroed by that call) matches the
  oracle: the zeroing is ordered before the kernel on the call's own stream.
* ullm_linear_release_workspaces frees the library buffers; later calls
  allocate anew and still match.
* A call that would have to grow a library workspace under stream capture is
  refused (allocation is not allowed there) instead of allocating.
* ullm_linear_forward_plan reports the decode GEMV with its split-K parts and
  the prefill GEMM's block, tiles and grid.
"""
import numpy as np
import pytest
import torch

from helpers import activations_bf16, assert_close, to_torch_bf16, weights

pytestmark = pytest.mark.gpu


def _split_k_weight(uh, orc, gpu, tag):
    n, k = 4096, 14336
    w = weights(n, k, tag=tag)
    q, s = orc.fp8_quantize_rows(w)
    return uh.LinearWeight.from_fp8(q, s), q, s, n, k


def test_first_split_k_call_on_fresh_nonblocking_stream(uh, orc, gpu):
    lw, q, s, n, k = _split_k_weight(uh, orc, gpu, tag=71)
    m = 16
    xb = activations_bf16(orc, m, k, tag=72)
    ref, _ = orc.fp8_gemv(xb, q, s)
    x = to_torch_bf16(xb, gpu)
    y = torch.empty((m, n), dtype=torch.float32, device=gpu)
    assert lw.plan(x, y).split_k > 1
    # Keep the null stream busy so that an unordered memset would race.
    busy = torch.randn((4096, 4096), device=gpu)
    stream = torch.cuda.Stream(device=gpu)   # non-blocking, default priority
    torch.cuda.synchronize()
    for _ in range(4):
        busy = busy @ busy * 1e-3
    with torch.cuda.stream(stream):
        lw.forward(x, y, stream=stream)
    stream.synchronize()
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), ref, what="split-K on a fresh stream")


def test_release_workspaces_then_forward_again(uh, orc, gpu):
    lw, q, s, n, k = _split_k_weight(uh, orc, gpu, tag=73)
    xb = activations_bf16(orc, 12, k, tag=74)
    ref, _ = orc.fp8_gemv(xb, q, s)
    x = to_torch_bf16(xb, gpu)
    y1 = lw.forward(x, out_dtype=torch.float32)
    fq = uh.LinearWeight.from_fp8(*orc.fp8_quantize_rows(weights(64, 512, tag=75)))
    xp = to_torch_bf16(activations_bf16(orc, 300, 512, tag=76), gpu)
    p1 = fq.forward(xp, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    uh.release_workspaces(0)
    y2 = lw.forward(x, out_dtype=torch.float32)
    p2 = fq.forward(xp, out_dtype=torch.float32, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(p1, p2)
    assert_close(y2.cpu().numpy(), ref, what="after release")
    uh.release_workspaces(0)  # twice in a row is fine
    with pytest.raises(uh.HipError) as e:
        uh.release_workspaces(99)
    assert e.value.status == uh.Status.INVALID_ARGUMENT


# The refused call records nothing, so torch warns that the graph is empty.
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_growth_under_capture_is_refused(uh, orc, gpu):
    fq = uh.LinearWeight.from_fp8(*orc.fp8_quantize_rows(weights(64, 1024, tag=77)))
    uh.release_workspaces(0)
    x = to_torch_bf16(activations_bf16(orc, 500, 1024, tag=78), gpu)
    y = torch.empty((500, 64), dtype=torch.bfloat16, device=gpu)
    s = torch.cuda.Stream(device=gpu)
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.stream(s):
        try:
            with torch.cuda.graph(g, stream=s):
                try:
                    fq.forward(x, y, mode=uh.ACT_FP8_PER_TOKEN, stream=s)
                except uh.HipError as exc:   # refused inside the capture
                    err = exc
        except RuntimeError:
            pass  # the (empty) capture itself may be rejected; the call was refused
    torch.cuda.synchronize()
    assert err is not None and err.status == uh.Status.INVALID_ARGUMENT
    assert "capture" in err.message
    # outside capture the same call allocates and works
    fq.forward(x, y, mode=uh.ACT_FP8_PER_TOKEN)
    torch.cuda.synchronize()


def test_plan_reports_launches(uh, orc, gpu):
    lw = uh.LinearWeight.from_fp8(*orc.fp8_quantize_rows(weights(4096, 4096, tag=79)))
    x1 = torch.zeros((1, 4096), dtype=torch.bfloat16, device=gpu)
    y1 = torch.empty((1, 4096), dtype=torch.bfloat16, device=gpu)
    p = lw.plan(x1, y1)
    assert p.kernel == uh.KERNEL_GEMV and p.split_k == 1 and p.tiles == 0
    x = torch.zeros((2048, 4096), dtype=torch.bfloat16, device=gpu)
    y = torch.empty((2048, 4096), dtype=torch.bfloat16, device=gpu)
    p = lw.plan(x, y, mode=uh.ACT_FP8_PER_TOKEN)
    assert p.kernel == uh.KERNEL_GEMM_LDS
    # one round of 256 x 128 ping-pong blocks on a 256-CU device
    assert (p.block_m, p.block_n) == (256, 128) and p.tiles == 256
    # unaligned pre-quantized activations take the direct kernel
    xq = torch.zeros((64, 4096 + 3), dtype=torch.uint8, device=gpu)[:, 3:]
    xs = torch.ones((64,), dtype=torch.float32, device=gpu)
    p = lw.plan(xq, y[:64], x_scales=xs)
    assert p.kernel == uh.KERNEL_GEMM_DIRECT
    empty = torch.zeros((0, 4096), dtype=torch.bfloat16, device=gpu)
    assert lw.plan(empty, y[:0]).kernel == 0

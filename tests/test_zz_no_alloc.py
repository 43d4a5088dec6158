"""ullm_linear_forward_noalloc against ullm_linear_forward, through the C ABI.

The allocation-free entry point runs the same kernels as the ordinary one,
with its scratch (split-K counters and partials, quantized prefill
activations) in the library's fixed per-device array, so its outputs must be
bit-identical to the ordinary entry point's on the same inputs.  Each case
makes two calls in a row, the second with a smaller input, so the second
runs over what the first left in the shared array.
"""
import numpy as np
import pytest
import torch

from helpers import activations_bf16, to_torch_bf16, weights

pytestmark = pytest.mark.gpu


def _pair(uh, lw, x, **kw):
    ref = lw.forward(x, **kw)
    got = lw.forward(x, noalloc=True, **kw)
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_split_k_decode_two_calls(uh, orc, gpu, enc):
    # N = 4096, K = 14336, 9 <= M <= 32: the decode GEMV splits K and uses
    # counters and partials in the scratch.
    n, k = 4096, 14336
    w = torch.from_numpy(weights(n, k, tag=61)).to(gpu)
    lw = uh.LinearWeight.quantize(w, uh.ENCODING_FP8_E4M3_ROW if enc == "fp8"
                                  else uh.ENCODING_AQ4_G128)
    for m in (32, 16):
        x = to_torch_bf16(activations_bf16(orc, m, k, tag=m + 62), gpu)
        assert lw.plan(x, torch.empty((m, n), dtype=torch.bfloat16, device=gpu)).split_k > 1
        ref, got = _pair(uh, lw, x, out_dtype=torch.float32)
        assert torch.equal(ref, got), (enc, m)
        ref, got = _pair(uh, lw, x)
        assert torch.equal(ref, got), (enc, m)


def test_prefill_quantized_activations_two_calls(uh, orc, gpu):
    n, k = 1000, 4096
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(n, k, tag=63)).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW)
    for m in (2048, 300):
        x = to_torch_bf16(activations_bf16(orc, m, k, tag=m + 64), gpu)
        ref, got = _pair(uh, lw, x, mode=uh.ACT_FP8_PER_TOKEN)
        assert torch.equal(ref, got), m
        r = to_torch_bf16(activations_bf16(orc, m, n, tag=m + 65), gpu)
        ref, got = _pair(uh, lw, x, mode=uh.ACT_FP8_PER_TOKEN, residual=r,
                         out_dtype=torch.float32)
        assert torch.equal(ref, got), m


def test_decode_without_scratch_and_gated(uh, orc, gpu):
    f, k = 700, 4096
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(2 * f, k, tag=66)).to(gpu),
                                  uh.ENCODING_AQ4_G128, gated=True)
    for m in (8, 1):
        x = to_torch_bf16(activations_bf16(orc, m, k, tag=m + 67), gpu)
        ref, got = _pair(uh, lw, x)
        assert torch.equal(ref, got), m


def test_limits_and_workspace_rejected(uh, orc, gpu):
    # 4096 x 16384 activations need 64 MiB of quantized scratch: refused.
    n, k = 16, 16384
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(n, k, tag=68)).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW)
    x = torch.zeros((4096, k), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(uh.HipError) as e:
        lw.forward(x, mode=uh.ACT_FP8_PER_TOKEN, noalloc=True)
    assert e.value.status == uh.Status.UNSUPPORTED
    ws = torch.empty((1 << 20,), dtype=torch.uint8, device=gpu)
    with pytest.raises(uh.HipError) as e:
        lw.forward(x[:8], mode=uh.ACT_FP8_PER_TOKEN, noalloc=True, workspace=ws)
    assert e.value.status == uh.Status.INVALID_ARGUMENT
    # an accepted call after the refusals still matches
    ref, got = _pair(uh, lw, x[:64].normal_(), mode=uh.ACT_FP8_PER_TOKEN)
    assert torch.equal(ref, got)


def test_graph_replays(uh, orc, gpu):
    """Captured after one eager call, replayed three times with eager work
    between the replays; every replay equals the eager result."""
    n, k, m = 4096, 14336, 16
    lw = uh.LinearWeight.quantize(torch.from_numpy(weights(n, k, tag=69)).to(gpu),
                                  uh.ENCODING_FP8_E4M3_ROW)
    x = to_torch_bf16(activations_bf16(orc, m, k, tag=70), gpu)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        lw.forward(x, y, noalloc=True, stream=s)
        s.synchronize()
        eager = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            lw.forward(x, y, noalloc=True, stream=s)
    for i in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        other = lw.forward(x[:9], noalloc=True)   # eager use of the same scratch
        torch.cuda.synchronize()
        assert other.shape == (9, n)

"""Fused add + per-token activation quantization on the GPU, bit-exact
against the oracle (bf16_add, then act_quantize): the sum, the E4M3 codes and
the fp32 scales.  Covers the vectorized kernel (aligned rows, K % 8 == 0)
and the generic one, strided rows, the sum written in place over either
input or not at all, and rows with infinities, NaN, zeros and ties."""
import numpy as np
import pytest
import torch

from helpers import activations_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _check(orc, a_bits, b_bits, xq, xs, s=None):
    q_ref, s_ref, sum_ref = orc.add_act_quantize(a_bits, b_bits)
    assert np.array_equal(xq.cpu().numpy(), q_ref)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    if s is not None:
        got = _bits(s)
        nan = (sum_ref & 0x7FFF) > 0x7F80
        assert np.array_equal(got[~nan], sum_ref[~nan])
        assert np.all((got[nan] & 0x7FFF) > 0x7F80)


# 512-thread vector path: one, four and eight chunks per thread; K = 1001
# takes the scalar kernel
@pytest.mark.parametrize("m,k", [(2048, 4096), (7, 14336), (2, 32768), (5, 1001), (3, 24)])
def test_add_quantize_parity(uh, orc, gpu, m, k):
    a_bits = activations_bf16(orc, m, k, tag=m + 700)
    b_bits = activations_bf16(orc, m, k, tag=m + 701)
    a, b = to_torch_bf16(a_bits, gpu), to_torch_bf16(b_bits, gpu)
    out = torch.empty_like(a)
    xq, xs = uh.add_quantize_activations(a, b, out)
    torch.cuda.synchronize()
    _check(orc, a_bits, b_bits, xq, xs, out)
    xq2, xs2 = uh.add_quantize_activations(a, b)  # no sum output
    torch.cuda.synchronize()
    assert torch.equal(xq, xq2) and torch.equal(xs, xs2)


def test_add_quantize_in_place_and_strided(uh, orc, gpu):
    m, k = 9, 4096
    a_bits = activations_bf16(orc, m, k, tag=710)
    b_bits = activations_bf16(orc, m, k, tag=711)
    for target in ("a", "b"):
        wide_a = torch.zeros((m, k + 64), dtype=torch.bfloat16, device=gpu)
        wide_b = torch.zeros((m, k + 128), dtype=torch.bfloat16, device=gpu)
        a, b = wide_a[:, :k], wide_b[:, :k]
        a.copy_(to_torch_bf16(a_bits, gpu))
        b.copy_(to_torch_bf16(b_bits, gpu))
        out = a if target == "a" else b
        xq, xs = uh.add_quantize_activations(a, b, out)
        torch.cuda.synchronize()
        _check(orc, a_bits, b_bits, xq, xs, out)


def test_add_quantize_special_rows(uh, orc, gpu):
    k = 512
    rs = np.random.default_rng(712)
    a = rs.standard_normal((6, k)).astype(np.float32)
    b = rs.standard_normal((6, k)).astype(np.float32)
    a[0, 3], b[0, 3] = np.inf, 1.0           # inf in the sum
    a[1, 5], b[1, 5] = np.inf, -np.inf       # NaN in the sum
    a[2] = 0.0
    b[2] = 0.0                               # all-zero row: scale 0, codes 0
    a[3] = -b[3]                             # exact cancellation
    a[4], b[4] = 1.0, 2.0 ** -8              # every element a tie (1 + 2^-8)
    b[5, 7] = 3.0e38
    a[5, 7] = 3.0e38                         # overflows to inf in bf16
    a_bits = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    b_bits = torch.from_numpy(b).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ta, tb = to_torch_bf16(a_bits, gpu), to_torch_bf16(b_bits, gpu)
    out = torch.empty_like(ta)
    xq, xs = uh.add_quantize_activations(ta, tb, out)
    torch.cuda.synchronize()
    _check(orc, a_bits, b_bits, xq, xs, out)

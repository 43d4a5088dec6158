"""Shared helpers for the parity tests: seeded inputs and tolerance checks.

Tolerance (north star): max |Y_gpu - Y_ref| <= 1e-2 * RMS(Y_ref), where Y_ref
is the oracle's fp32-accumulated output from the same quantized weights and
the same bf16 activations.  For bf16 outputs the reference value itself must
be rounded to bf16, so half a bf16 ulp of |Y_ref| is added per element.
"""
import numpy as np

REL_TOL = 1e-2
SEED = 20260803


def rng(tag: int = 0):
    return np.random.default_rng(SEED + tag)


def weights(n, k, tag=0, std=0.02):
    return (rng(tag).standard_normal((n, k)) * std).astype(np.float32)


def activations_bf16(orc, m, k, tag=1):
    return orc.bf16_from_f32(rng(tag).standard_normal((m, k)).astype(np.float32))


def to_torch_bf16(bits, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(
        torch.bfloat16).to(device)


def bf16_tensor_to_f32(t):
    import torch
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def bf16_half_ulp(v):
    a = np.abs(v.astype(np.float64))
    a = np.where(a == 0, np.finfo(np.float32).tiny, a)
    return np.exp2(np.floor(np.log2(a)) - 8)


def assert_close(y, y_ref, bf16_out=False, rel=REL_TOL, what=""):
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    assert y.shape == y_ref.shape, (y.shape, y_ref.shape)
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    rms = float(np.sqrt(np.mean(y_ref ** 2))) if y_ref.size else 0.0
    err = np.abs(y - y_ref)
    bound = rel * rms + (bf16_half_ulp(y_ref) if bf16_out else 0.0)
    worst = float(np.max(err - bound)) if err.size else 0.0
    assert worst <= 0.0, (
        f"{what}: max|d|={float(err.max()):.3e} rms={rms:.3e} "
        f"outliers={int(np.sum(err > bound))}")
    return float(err.max()) / rms if rms else 0.0


GEMV_VARIANTS = {1: "single", 2: "single_lds", 3: "multi", 4: "rs", 5: "split"}


def check_gemv_plan(lw, x, y, expect):
    """The decode launch ullm_linear_forward_plan reports for (x, y) is
    `expect` = (variant, waves, stripes per group, row classes).  The
    expectations were read on a 256-CU MI355X; the launcher's grid tiers
    depend on the CU count, so other devices skip the check."""
    import torch
    if torch.cuda.get_device_properties(x.device).multi_processor_count != 256:
        return
    p = lw.plan(x, y)
    got = (GEMV_VARIANTS.get(p.gemv_variant, p.gemv_variant), p.gemv_waves,
           p.gemv_stripes, p.gemv_row_classes)
    assert got == tuple(expect), f"plan {got}, expected {tuple(expect)}"

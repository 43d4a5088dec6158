"""The algorithmic byte and flop counts behind every roofline figure that
bench.py reports, checked against the per-configuration table of the
benchmark specification (bytes = weights + scales/zeros + activations in +
outputs out, compulsory traffic only).  The table's values were worked out
independently of bench.py's formulas, so a dropped term or a wrong operand
(K for N, a scale per group counted per row) fails here."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "ullm-project_amd"))

import bench  # noqa: E402
import stack  # noqa: E402


def test_headline_and_config1_bytes():
    assert bench.aq4_bytes(1, 14336, 4096) == 31_232_000
    assert bench.fp8_bytes(1, 4096, 4096) == 16_809_984


@pytest.mark.parametrize("k,n,m1,m32", [
    (4096, 6144, 25_210_880, 25_845_760),       # qkv
    (4096, 4096, 16_809_984, 17_317_888),       # o
    (4096, 28672, 117_620_736, 119_652_352),    # gate_up
    (14336, 4096, 58_773_504, 59_916_288),      # down
])
def test_fp8_sweep_bytes(k, n, m1, m32):
    assert bench.fp8_bytes(1, n, k) == m1
    assert bench.fp8_bytes(32, n, k) == m32


def test_stack_step_bytes():
    # 32 layers of qkv, o, gate_up and down plus the lm_head, AQ4, batch 8
    assert stack.step_bytes() == 4_024_619_008


def test_gemm_flops_and_peaks():
    assert 2 * 2048 * 28672 * 4096 == 481_036_337_152
    # dense FP8: 256 CUs x 2.4 GHz x 8192 flop per clock per CU = 5033 TF,
    # quoted as 5.03 PF
    assert abs(bench.FP8_PEAK_TFLOPS / (256 * 2.4e9 * 8192 / 1e12) - 1) < 1e-3
    assert bench.HBM_PEAK_GBS == 8000.0

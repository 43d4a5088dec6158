"""The per-token activation quantizer divides by the row scale through the
row's reciprocal and one fused residual step (act_quant_vec_kernel in
ullm-project_amd/src/weights.hip).  This checks, exhaustively over every
finite bf16 row maximum and every bf16 element it bounds (1,065,402,238
pairs), that the E4M3 codes equal those of the correctly rounded quotient,
so the kernel keeps the oracle's definition XA = e4m3(x / a) bit-exactly.
The GPU tests compare the kernel's codes with the oracle's directly."""
import os
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_reciprocal_division_gives_the_exact_codes(tmp_path):
    exe = tmp_path / "act_quant_division_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-std=c11",
                    f"-I{ROOT / 'oracle'}", str(ROOT / "tests" / "act_quant_division_check.c"),
                    str(ROOT / "oracle" / "ullm_oracle.c"), "-lm", "-o", str(exe)], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    words = r.stdout.split()
    counts = dict(zip(words[::2], map(int, words[1::2])))
    assert r.returncode == 0 and counts["code_diff"] == 0, r.stdout + r.stderr
    assert counts["pairs"] == 1065402238, r.stdout
    # the fast quotient does differ in fp32 on some pairs: the check has teeth
    assert counts["fp32_diff"] > 0, r.stdout

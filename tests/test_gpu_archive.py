"""The static archive the reference's FFI crate links (CMake target
ullm_hip_stub), exercised on the GPU: tests/archive_check.c, linked against
the archive with amdhip64 and stdc++ as cargo links ullm-hip-sys, creates an
FP8 and an AQ4 weight, runs a forward and checks it against the library's
own dequantized weights in double precision (1e-2 x RMS).  The numerics are
pinned against the oracle by the other GPU tests; this one checks that the
kernels in the static archive register and run."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent.parent / "ullm-project_amd" / "lib" / "ullm_archive_check"


def test_static_archive_forward(gpu):
    if not EXE.exists():
        pytest.fail(f"{EXE} is missing: build it with __graft_entry__.build()")
    print("archive check: FP8 and AQ4, M=2 N=48 K=256", flush=True)
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=90)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr

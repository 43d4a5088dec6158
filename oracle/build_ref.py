"""Build recipe for oracle/_ref: the reference's own ABI v1 host stub.

Compiles, with g++ straight from where they lie:
  * /root/reference/native/hip/src/hip_stub.cpp (the reference implementation
    of ullm_get_abi_version, ullm_query_version, ullm_backend_probe and
    ullm_context_probe, reference include/ullm/hip.h:106-121) into
    oracle/_ref/libullm_ref_stub.so;
  * /root/reference/native/hip/src/hip_evidence_stub.cpp (the reference's
    host stub of the evidence ABI, native/hip/src/evidence_abi.h:48-60: its
    argument validation, then "HIP unavailable") into
    oracle/_ref/libullm_ref_evidence_stub.so.
TEST INFRASTRUCTURE ONLY: tests compare this library's v1 entry points with
it.  Nothing is copied from the reference tree; when the tree is absent (the
GPU box) this does nothing and the tests that need it skip.

The reference's quantized linear path does not exist, so there is nothing
else of the reference to build.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "_ref" / "libullm_ref_stub.so"
OUT_EVIDENCE = OUT.parent / "libullm_ref_evidence_stub.so"


def _gxx(src: Path, out: Path) -> None:
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared",
           "-Wall", "-Wextra", "-Wpedantic", "-Werror",
           f"-I{REF / 'include'}", f"-I{src.parent}", str(src), "-o", str(out)]
    subprocess.run(cmd, check=True)


def build() -> Path | None:
    src = REF / "native" / "hip" / "src" / "hip_stub.cpp"
    if not src.exists():
        return None
    OUT.parent.mkdir(exist_ok=True)
    _gxx(src, OUT)
    ev = REF / "native" / "hip" / "src" / "hip_evidence_stub.cpp"
    if ev.exists():
        _gxx(ev, OUT_EVIDENCE)
    return OUT


if __name__ == "__main__":
    print(build())

"""Build recipe for oracle/_ref: the reference's own ABI v1 host stub.

Compiles /root/reference/native/hip/src/hip_stub.cpp (the reference
implementation of ullm_get_abi_version, ullm_query_version,
ullm_backend_probe and ullm_context_probe, reference include/ullm/hip.h:106-121)
with g++ straight from where it lies, into oracle/_ref/libullm_ref_stub.so.
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


def build() -> Path | None:
    src = REF / "native" / "hip" / "src" / "hip_stub.cpp"
    if not src.exists():
        return None
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared",
           "-Wall", "-Wextra", "-Wpedantic", "-Werror",
           f"-I{REF / 'include'}", str(src), "-o", str(OUT)]
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build())

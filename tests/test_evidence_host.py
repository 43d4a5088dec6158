"""The evidence ABI without a GPU (include/ullm/hip_evidence.h).

* Struct layouts equal the reference's (native/hip/src/evidence_abi.h:62-118
  asserts 40 and 72 bytes and every field offset), checked through a C probe
  of this repo's header and the ctypes mirror.
* Every call the reference rejects before touching a device gets the same
  status, message length and message from this library as from the
  reference's own host stub (native/hip/src/hip_evidence_stub.cpp, compiled
  from its sources into oracle/_ref; skipped where the tree is absent).
* Handles that are not live are ULLM_STATUS_HIP_INVALID_HANDLE with the
  runtime's diagnostic (native/hip/src/hip_evidence_runtime.hip.cpp:715-720,
  771-774), and a valid submit with no GPU visible fails as a HIP runtime
  error, never as a silent CPU result.
"""
import ctypes
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_EV = ROOT / "oracle" / "_ref" / "libullm_ref_evidence_stub.so"

PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "ullm/hip_evidence.h"
#define S(T) printf("%s size %zu\n", #T, sizeof(T));
#define F(T, f) printf("%s.%s %zu\n", #T, #f, offsetof(T, f));
int main(void) {
  S(ullm_hip_evidence_request_t) F(ullm_hip_evidence_request_t, struct_size)
  F(ullm_hip_evidence_request_t, abi_version) F(ullm_hip_evidence_request_t, input)
  F(ullm_hip_evidence_request_t, input_size) F(ullm_hip_evidence_request_t, reserved)
  S(ullm_hip_evidence_result_t) F(ullm_hip_evidence_result_t, output_size)
  F(ullm_hip_evidence_result_t, allocation_count) F(ullm_hip_evidence_result_t, copy_count)
  F(ullm_hip_evidence_result_t, dispatch_count) F(ullm_hip_evidence_result_t, selected_backend)
  F(ullm_hip_evidence_result_t, fallback_used) F(ullm_hip_evidence_result_t, terminal)
  F(ullm_hip_evidence_result_t, reserved)
  return 0;
}
"""

# The reference's static_asserts (evidence_abi.h:62-99).
REFERENCE_LAYOUT = {
    "ullm_hip_evidence_request_t size": 40,
    "ullm_hip_evidence_request_t.struct_size": 0,
    "ullm_hip_evidence_request_t.abi_version": 4,
    "ullm_hip_evidence_request_t.input": 8,
    "ullm_hip_evidence_request_t.input_size": 16,
    "ullm_hip_evidence_request_t.reserved": 24,
    "ullm_hip_evidence_result_t size": 72,
    "ullm_hip_evidence_result_t.output_size": 8,
    "ullm_hip_evidence_result_t.allocation_count": 16,
    "ullm_hip_evidence_result_t.copy_count": 24,
    "ullm_hip_evidence_result_t.dispatch_count": 32,
    "ullm_hip_evidence_result_t.selected_backend": 40,
    "ullm_hip_evidence_result_t.fallback_used": 44,
    "ullm_hip_evidence_result_t.terminal": 48,
    "ullm_hip_evidence_result_t.reserved": 52,
}


def test_evidence_layout(uh, tmp_path):
    src = tmp_path / "p.c"
    src.write_text(PROBE)
    exe = tmp_path / "p"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Wpedantic", "-Werror",
                    f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    types = {"ullm_hip_evidence_request_t": uh.EvidenceRequest,
             "ullm_hip_evidence_result_t": uh.EvidenceResult}
    seen = 0
    for line in out.splitlines():
        key, value = line.rsplit(" ", 1)
        if key in REFERENCE_LAYOUT:
            assert REFERENCE_LAYOUT[key] == int(value), line
            seen += 1
        if key.endswith(" size"):
            assert ctypes.sizeof(types[key[:-5]]) == int(value), line
        else:
            t, f = key.split(".")
            assert getattr(types[t], f).offset == int(value), line
    assert seen == len(REFERENCE_LAYOUT)


def _sink(uh, capacity=256, **over):
    buf = ctypes.create_string_buffer(max(capacity, 1))
    s = uh.new(uh.ErrorSink, message=ctypes.cast(buf, ctypes.c_char_p),
               message_capacity=capacity)
    for k, v in over.items():
        if k == "reserved":
            s.reserved[0] = v
        else:
            setattr(s, k, v)
    return s, buf


def _bind(lib, uh):
    for n in ("ullm_hip_evidence_submit", "ullm_hip_evidence_wait",
              "ullm_hip_evidence_destroy"):
        fn = getattr(lib, n)
        fn.argtypes = uh._SIGNATURES[n]
        fn.restype = ctypes.c_uint32
    return lib


def rejected_before_device(uh, lib):
    """(case, status, message_length, message) of calls that fail validation."""
    data = ctypes.create_string_buffer(b"abc", 3)
    res = []

    def submit(case, req, out=True, **sink):
        s, buf = _sink(uh, **sink)
        h = ctypes.c_void_p(0x77)
        st = lib.ullm_hip_evidence_submit(None if req is None else ctypes.byref(req),
                                          ctypes.byref(h) if out else None,
                                          ctypes.byref(s))
        res.append((case, st, s.message_length, buf.value))

    good = dict(input=ctypes.cast(data, ctypes.c_void_p), input_size=3)
    submit("null request", None)
    submit("short request", uh.evidence_new(uh.EvidenceRequest, struct_size=32, **good))
    submit("abi 2", uh.evidence_new(uh.EvidenceRequest, abi_version=2, **good))
    r = uh.evidence_new(uh.EvidenceRequest, **good)
    r.reserved[3] = 1
    submit("reserved", r)
    submit("null input", uh.evidence_new(uh.EvidenceRequest, input=None, input_size=3))
    submit("empty input", uh.evidence_new(uh.EvidenceRequest,
                                          input=ctypes.cast(data, ctypes.c_void_p),
                                          input_size=0))
    submit("null completion", uh.evidence_new(uh.EvidenceRequest, **good), out=False)
    submit("truncated message", None, capacity=8)
    submit("zero-capacity sink", None, capacity=0)
    for field, val in (("struct_size", 40), ("abi_version", 3), ("reserved", 1)):
        submit(f"bad sink {field}", uh.evidence_new(uh.EvidenceRequest, **good),
               **{field: val})
        s, buf = _sink(uh, **{field: val})
        res.append((f"wait bad sink {field}",
                    lib.ullm_hip_evidence_wait(None, 0, None, 0, None, ctypes.byref(s)),
                    s.message_length, buf.value))
        s, buf = _sink(uh, **{field: val})
        res.append((f"destroy bad sink {field}",
                    lib.ullm_hip_evidence_destroy(None, ctypes.byref(s)),
                    s.message_length, buf.value))
    s, buf = _sink(uh)
    res.append(("destroy null", lib.ullm_hip_evidence_destroy(None, ctypes.byref(s)),
                s.message_length, buf.value))
    return res


def test_validation_matches_reference_stub(uh):
    if not REF_EV.exists():
        pytest.skip("reference evidence stub not built here (reference tree absent)")
    mine = rejected_before_device(uh, uh.lib())
    ref = rejected_before_device(uh, _bind(ctypes.CDLL(str(REF_EV)), uh))
    assert len(mine) == len(ref)
    for a, b in zip(mine, ref):
        assert a == b, (a, b)


def test_validation_statuses(uh):
    cases = {c[0]: c for c in rejected_before_device(uh, uh.lib())}
    S = uh.Status
    assert cases["null request"][1] == S.INVALID_ARGUMENT
    assert cases["null request"][3] == b"evidence request is null"
    assert cases["short request"][1] == S.INVALID_ARGUMENT
    assert cases["abi 2"][1] == S.INVALID_ABI_VERSION
    assert cases["reserved"][1] == S.RESERVED_NONZERO
    assert cases["null input"][1] == S.INVALID_ARGUMENT
    assert cases["empty input"][1] == S.INVALID_ARGUMENT
    assert cases["null completion"][1] == S.INVALID_ARGUMENT
    assert cases["truncated message"][1] == S.BUFFER_TOO_SMALL
    assert cases["truncated message"][2] == len("evidence request is null")
    assert cases["bad sink struct_size"][1] == S.INVALID_ARGUMENT
    assert cases["bad sink abi_version"][1] == S.INVALID_ABI_VERSION
    assert cases["bad sink reserved"][1] == S.RESERVED_NONZERO
    assert cases["destroy null"][1] == S.INVALID_ARGUMENT


def test_handles_that_are_not_live(uh):
    lib = uh.lib()
    res = uh.evidence_new(uh.EvidenceResult)
    out = ctypes.create_string_buffer(8)
    for h in (None, 0x1234, 1, 2 ** 40):
        s, buf = _sink(uh)
        st = lib.ullm_hip_evidence_wait(h, 0, ctypes.cast(out, ctypes.c_void_p), 8,
                                        ctypes.byref(res), ctypes.byref(s))
        assert st == uh.Status.HIP_INVALID_HANDLE
        assert buf.value == b"evidence completion handle is not live"
        hh = ctypes.c_void_p(h)
        s, buf = _sink(uh)
        assert lib.ullm_hip_evidence_destroy(ctypes.byref(hh), ctypes.byref(s)) \
            == uh.Status.HIP_INVALID_HANDLE
        assert buf.value == b"evidence completion handle is not live"
        assert hh.value == h


def test_submit_without_gpu_is_a_runtime_error(uh):
    if uh.backend_probe()[0]:
        pytest.skip("a GPU is visible")
    with pytest.raises(uh.HipError) as e:
        uh.submit_evidence(b"\x01\x02\x03")
    assert e.value.status == uh.Status.HIP_RUNTIME_ERROR
    # the raw call leaves the completion null
    data = ctypes.create_string_buffer(b"x", 1)
    req = uh.evidence_new(uh.EvidenceRequest, input=ctypes.cast(data, ctypes.c_void_p),
                          input_size=1)
    h = ctypes.c_void_p(0x55)
    assert uh.lib().ullm_hip_evidence_submit(ctypes.byref(req), ctypes.byref(h), None) \
        == uh.Status.HIP_RUNTIME_ERROR
    assert not h.value

"""The evidence ABI on the GPU, through the C ABI (include/ullm/hip_evidence.h).

Contract (reference native/hip/src/hip_evidence_runtime.hip.cpp:539-789 and
crates/ullm-hip/src/lib.rs:408-441): the output is the input XOR 0x5a byte
for byte; a successful wait reports 2 device allocations, 2 copies, 1
dispatch, backend HIP, no fallback, terminal; wait consumes the handle on
every outcome; destroy consumes a live handle and nulls it; stale handles are
ULLM_STATUS_HIP_INVALID_HANDLE; at most two completions are outstanding.
"""
import ctypes
import threading
import time

import pytest

pytestmark = pytest.mark.gpu


def _pattern(n, seed=7):
    return bytes((i * 131 + seed * 17 + (i >> 8)) & 0xFF for i in range(n))


@pytest.mark.parametrize("size", [1, 3, 15, 16, 17, 255, 256, 257, 4101,
                                  (1 << 20) + 3, 64 << 20])
def test_evidence_byte_exact(uh, gpu, size):
    data = _pattern(size, seed=size % 251)
    out, rep = uh.run_evidence(data, timeout_ms=20000)
    assert out == uh.expected_evidence_output(data)
    assert rep == {"output_size": size, "allocation_count": 2, "copy_count": 2,
                   "dispatch_count": 1, "selected_backend": uh.BACKEND_HIP,
                   "fallback_used": False, "terminal": True}


def _raw_submit(uh, data):
    src = ctypes.create_string_buffer(bytes(data), len(data))
    req = uh.evidence_new(uh.EvidenceRequest, input=ctypes.cast(src, ctypes.c_void_p),
                          input_size=len(data))
    h = ctypes.c_void_p()
    st = uh.lib().ullm_hip_evidence_submit(ctypes.byref(req), ctypes.byref(h), None)
    return st, h, src


def _raw_wait(uh, h, n, timeout_ms=20000, result=None, cap=None):
    out = ctypes.create_string_buffer(max(n, 1))
    res = result if result is not None else uh.evidence_new(uh.EvidenceResult)
    st = uh.lib().ullm_hip_evidence_wait(h, timeout_ms, ctypes.cast(out, ctypes.c_void_p),
                                         n if cap is None else cap,
                                         ctypes.byref(res), None)
    return st, out.raw[:n], res


def test_input_is_copied_at_submit(uh, gpu):
    data = _pattern(4096)
    st, h, src = _raw_submit(uh, data)
    assert st == uh.Status.OK
    ctypes.memset(src, 0, len(data))     # the caller reuses its buffer at once
    st, out, _ = _raw_wait(uh, h, len(data))
    assert st == uh.Status.OK and out == uh.expected_evidence_output(data)


def test_wait_consumes_the_handle(uh, gpu):
    data = _pattern(300)
    # timeout 0: one poll; either finished or timed out, consumed either way
    st, h, _ = _raw_submit(uh, data)
    assert st == uh.Status.OK
    st, out, _ = _raw_wait(uh, h, len(data), timeout_ms=0)
    assert st in (uh.Status.OK, uh.Status.HIP_TIMEOUT)
    if st == uh.Status.OK:
        assert out == uh.expected_evidence_output(data)
    assert _raw_wait(uh, h, len(data))[0] == uh.Status.HIP_INVALID_HANDLE
    hh = ctypes.c_void_p(h.value)
    assert uh.lib().ullm_hip_evidence_destroy(ctypes.byref(hh), None) \
        == uh.Status.HIP_INVALID_HANDLE
    # a malformed result or a short output also consumes it
    st, h, _ = _raw_submit(uh, data)
    bad = uh.evidence_new(uh.EvidenceResult, struct_size=64)
    assert _raw_wait(uh, h, len(data), result=bad)[0] == uh.Status.INVALID_ARGUMENT
    assert _raw_wait(uh, h, len(data))[0] == uh.Status.HIP_INVALID_HANDLE
    st, h, _ = _raw_submit(uh, data)
    assert _raw_wait(uh, h, len(data), cap=len(data) - 1)[0] == uh.Status.INVALID_ARGUMENT
    assert _raw_wait(uh, h, len(data))[0] == uh.Status.HIP_INVALID_HANDLE
    bad = uh.evidence_new(uh.EvidenceResult)
    bad.reserved[2] = 1
    st, h, _ = _raw_submit(uh, data)
    assert _raw_wait(uh, h, len(data), result=bad)[0] == uh.Status.RESERVED_NONZERO


def test_destroy_and_double_destroy(uh, gpu):
    st, h, _ = _raw_submit(uh, _pattern(1000))
    assert st == uh.Status.OK and h.value
    raw = h.value
    assert uh.lib().ullm_hip_evidence_destroy(ctypes.byref(h), None) == uh.Status.OK
    assert h.value is None
    again = ctypes.c_void_p(raw)
    assert uh.lib().ullm_hip_evidence_destroy(ctypes.byref(again), None) \
        == uh.Status.HIP_INVALID_HANDLE
    assert _raw_wait(uh, again, 1000)[0] == uh.Status.HIP_INVALID_HANDLE


def _submit_when_free(uh, data, seconds=5.0):
    deadline = time.monotonic() + seconds
    while True:
        st, h, src = _raw_submit(uh, data)
        if st != uh.Status.INTERNAL_ERROR or time.monotonic() > deadline:
            return st, h, src
        time.sleep(0.001)


def test_two_outstanding_completions_at_most(uh, gpu):
    a = _pattern(512, 1)
    b = _pattern(700, 2)
    st1, h1, _ = _submit_when_free(uh, a)
    st2, h2, _ = _submit_when_free(uh, b)
    assert st1 == uh.Status.OK and st2 == uh.Status.OK
    st3, h3, _ = _raw_submit(uh, b"z")
    assert st3 == uh.Status.INTERNAL_ERROR and not h3.value
    # results are per handle, in any order
    st, out, _ = _raw_wait(uh, h2, len(b))
    assert st == uh.Status.OK and out == uh.expected_evidence_output(b)
    st, h4, _ = _raw_submit(uh, b"q")          # the waited slot is free again
    assert st == uh.Status.OK
    st, out, _ = _raw_wait(uh, h1, len(a))
    assert st == uh.Status.OK and out == uh.expected_evidence_output(a)
    assert uh.lib().ullm_hip_evidence_destroy(ctypes.byref(h4), None) == uh.Status.OK
    # a destroyed completion's slot is reclaimed once its work has finished
    st, h5, _ = _submit_when_free(uh, b"r")
    assert st == uh.Status.OK
    assert _raw_wait(uh, h5, 1)[1] == bytes([ord("r") ^ 0x5A])


def test_two_threads(uh, gpu):
    errors = []

    def worker(seed):
        try:
            for i in range(25):
                data = _pattern(1 + (seed * 977 + i * 131) % 70000, seed + i)
                out, rep = uh.run_evidence(data, timeout_ms=20000)
                assert out == uh.expected_evidence_output(data)
        except Exception as exc:  # reported below
            errors.append(exc)

    ts = [threading.Thread(target=worker, args=(s,)) for s in (1, 2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(120)
    assert not errors, errors

"""C-ABI checks that need no GPU.

* libullm_hip.so loads and exports every function include/ullm/*.h declares.
* The headers compile as strict C99 and C++17, and a C layout probe built with
  gcc agrees with the ctypes structs of the Python host mirror (the check the
  reference's ullm-hip-sys build.rs:330-408 makes between C and Rust).
* Error-sink, struct-header and reserved-word validation follow the reference
  ABI v1 (native/hip/src/hip_stub.cpp:10-98); the four v1 functions are
  compared case by case with the reference's own stub compiled from its
  sources into oracle/_ref (skipped where the reference tree is absent).
* Linear-layer entry points reject malformed descriptors before touching a
  device, and report ULLM_STATUS_HIP_UNAVAILABLE when no GPU is visible.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include" / "ullm").glob("*.h"))
REF_LIB = ROOT / "oracle" / "_ref" / "libullm_ref_stub.so"


def declared_functions():
    names = set()
    for h in HEADERS:
        text = h.read_text()
        names |= set(re.findall(r"ULLM_HIP_API\s+ullm_status_t\s*\n?\s*(ullm_\w+)\s*\(", text))
    return names


def test_exports_every_declared_function(uh):
    names = declared_functions()
    assert len(names) >= 12
    out = subprocess.run(["nm", "-D", "--defined-only", str(uh.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert names <= exported, names - exported
    lib = uh.lib()
    for n in names:
        assert getattr(lib, n) is not None


LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "ullm/ullm.h"
#define S(T) printf("%s size %zu\n", #T, sizeof(T));
#define F(T, f) printf("%s.%s %zu\n", #T, #f, offsetof(T, f));
int main(void) {
  S(ullm_error_sink_t) F(ullm_error_sink_t, message) F(ullm_error_sink_t, message_length) F(ullm_error_sink_t, reserved)
  S(ullm_version_info_t) F(ullm_version_info_t, patch) F(ullm_version_info_t, reserved)
  S(ullm_backend_probe_result_t) F(ullm_backend_probe_result_t, hip_runtime_present)
  S(ullm_context_probe_result_t) F(ullm_context_probe_result_t, reserved)
  S(ullm_linear_weight_desc_t) F(ullm_linear_weight_desc_t, n) F(ullm_linear_weight_desc_t, memory)
  F(ullm_linear_weight_desc_t, values) F(ullm_linear_weight_desc_t, stream) F(ullm_linear_weight_desc_t, layout)
  F(ullm_linear_weight_desc_t, reserved0) F(ullm_linear_weight_desc_t, reserved)
  S(ullm_linear_weight_info_t) F(ullm_linear_weight_info_t, device_bytes) F(ullm_linear_weight_info_t, layout)
  F(ullm_linear_weight_info_t, reserved)
  S(ullm_linear_forward_desc_t) F(ullm_linear_forward_desc_t, m) F(ullm_linear_forward_desc_t, x_scales)
  F(ullm_linear_forward_desc_t, y_row_stride) F(ullm_linear_forward_desc_t, x_dtype) F(ullm_linear_forward_desc_t, alpha)
  F(ullm_linear_forward_desc_t, stream) F(ullm_linear_forward_desc_t, workspace_size) F(ullm_linear_forward_desc_t, epilogue)
  F(ullm_linear_forward_desc_t, residual_dtype) F(ullm_linear_forward_desc_t, residual)
  F(ullm_linear_forward_desc_t, residual_row_stride) F(ullm_linear_forward_desc_t, reserved)
  S(ullm_linear_act_quant_desc_t) F(ullm_linear_act_quant_desc_t, xq) F(ullm_linear_act_quant_desc_t, reserved)
  S(ullm_linear_add_act_quant_desc_t) F(ullm_linear_add_act_quant_desc_t, b)
  F(ullm_linear_add_act_quant_desc_t, sum_row_stride) F(ullm_linear_add_act_quant_desc_t, x_scales)
  F(ullm_linear_add_act_quant_desc_t, reserved)
  S(ullm_linear_plan_t) F(ullm_linear_plan_t, kernel) F(ullm_linear_plan_t, grid) F(ullm_linear_plan_t, split_k)
  F(ullm_linear_plan_t, gemv_variant) F(ullm_linear_plan_t, gemv_row_classes)
  F(ullm_linear_plan_t, reserved)
  S(ullm_linear_weight_export_desc_t) F(ullm_linear_weight_export_desc_t, values) F(ullm_linear_weight_export_desc_t, reserved)
  S(ullm_safetensors_open_desc_t) F(ullm_safetensors_open_desc_t, expected_sha256) F(ullm_safetensors_open_desc_t, reserved)
  S(ullm_safetensors_tensor_info_t) F(ullm_safetensors_tensor_info_t, shape) F(ullm_safetensors_tensor_info_t, offset)
  F(ullm_safetensors_tensor_info_t, reserved)
  S(ullm_linear_weight_load_desc_t) F(ullm_linear_weight_load_desc_t, values) F(ullm_linear_weight_load_desc_t, value_parts)
  F(ullm_linear_weight_load_desc_t, device) F(ullm_linear_weight_load_desc_t, scales) F(ullm_linear_weight_load_desc_t, stream)
  F(ullm_linear_weight_load_desc_t, reserved)
  S(ullm_linear_weights_save_desc_t) F(ullm_linear_weights_save_desc_t, weights) F(ullm_linear_weights_save_desc_t, metadata_count)
  F(ullm_linear_weights_save_desc_t, reserved)
  return 0;
}
"""


def test_python_constants_mirror_header_macros(uh):
    """Every ULLM_LINEAR_* value macro of linear.h has the same value under
    its unprefixed name in ullm_hip (the module hard-codes them)."""
    text = (ROOT / "include" / "ullm" / "linear.h").read_text()
    macros = re.findall(r"#define ULLM_LINEAR_(\w+) UINT32_C\((\d+)\)", text)
    assert len(macros) >= 20
    for name, value in macros:
        assert getattr(uh, name) == int(value), name


def test_headers_compile_and_layout_matches_ctypes(uh, tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(LAYOUT_PROBE)
    flags = ["-Wall", "-Wextra", "-Wpedantic", "-Werror", f"-I{ROOT / 'include'}"]
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", *flags, str(src), "-o", str(exe)], check=True)
    cpp = tmp_path / "probe.cpp"
    cpp.write_text(LAYOUT_PROBE)
    subprocess.run(["g++", "-std=c++17", "-Wconversion", "-Wshadow", *flags, "-c",
                    str(cpp), "-o", str(tmp_path / "probe.o")], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    types = {
        "ullm_error_sink_t": uh.ErrorSink, "ullm_version_info_t": uh.VersionInfo,
        "ullm_backend_probe_result_t": uh.BackendProbeResult,
        "ullm_context_probe_result_t": uh.ContextProbeResult,
        "ullm_linear_weight_desc_t": uh.WeightDesc, "ullm_linear_weight_info_t": uh.WeightInfo,
        "ullm_linear_forward_desc_t": uh.ForwardDesc,
        "ullm_linear_act_quant_desc_t": uh.ActQuantDesc,
        "ullm_linear_add_act_quant_desc_t": uh.AddActQuantDesc,
        "ullm_linear_plan_t": uh.Plan,
        "ullm_linear_weight_export_desc_t": uh.ExportDesc,
        "ullm_safetensors_open_desc_t": uh.StOpenDesc,
        "ullm_safetensors_tensor_info_t": uh.StTensorInfo,
        "ullm_linear_weight_load_desc_t": uh.WeightLoadDesc,
        "ullm_linear_weights_save_desc_t": uh.WeightsSaveDesc,
    }
    for line in out.splitlines():
        key, value = line.rsplit(" ", 1)
        if key.endswith(" size"):
            t = key[:-5]
            assert ctypes.sizeof(types[t]) == int(value), line
        else:
            t, f = key.split(".")
            assert getattr(types[t], f).offset == int(value), line
    # v1 layouts are those of the reference ABI (sink 48 B, probes 32 B)
    assert ctypes.sizeof(uh.ErrorSink) == 48
    assert ctypes.sizeof(uh.VersionInfo) == 32
    assert ctypes.sizeof(uh.BackendProbeResult) == 32
    assert ctypes.sizeof(uh.ContextProbeResult) == 32


# -------------------------------------------------------------- sink rules

def make_sink(uh, capacity=256, **over):
    buf = ctypes.create_string_buffer(max(capacity, 1))
    s = uh.new(uh.ErrorSink, message=ctypes.cast(buf, ctypes.c_char_p),
               message_capacity=capacity)
    for k, v in over.items():
        setattr(s, k, v)
    return s, buf


def run_cases(uh, lib):
    """Status and message bookkeeping of the v1 functions over edge cases."""
    res = []
    U32 = ctypes.c_uint32
    for cap in (0, 1, 8, 256):
        s, buf = make_sink(uh, cap)
        st = lib.ullm_get_abi_version(None, ctypes.byref(s))
        res.append(("abi-null-out", cap, st, s.message_length, buf.raw[:1]))
    for field, val in (("struct_size", 47), ("abi_version", 2), ("reserved", (1, 0))):
        s, _ = make_sink(uh)
        if field == "reserved":
            s.reserved[0] = 1
        else:
            setattr(s, field, val)
        v = U32()
        res.append(("bad-sink", field, lib.ullm_get_abi_version(ctypes.byref(v), ctypes.byref(s))))
    s, _ = make_sink(uh, 16)
    s.message = None
    res.append(("cap-null-msg", lib.ullm_get_abi_version(ctypes.byref(U32()), ctypes.byref(s))))
    v = U32()
    res.append(("abi-ok", lib.ullm_get_abi_version(ctypes.byref(v), None), v.value))
    for size, ver, resv in ((32, 1, 0), (31, 1, 0), (64, 1, 0), (32, 2, 0), (32, 1, 1)):
        info = uh.VersionInfo(struct_size=size, abi_version=ver)
        info.reserved[2] = resv
        s, _ = make_sink(uh)
        res.append(("version", size, ver, resv,
                    lib.ullm_query_version(ctypes.byref(info), ctypes.byref(s))))
    res.append(("version-null", lib.ullm_query_version(None, None)))
    for backend in (0, 1, 7):
        for size, resv in ((32, 0), (16, 0), (32, 5)):
            r = uh.BackendProbeResult(struct_size=size, abi_version=1)
            r.reserved[1] = resv
            s, _ = make_sink(uh)
            st = lib.ullm_backend_probe(backend, ctypes.byref(r), ctypes.byref(s))
            res.append(("probe", backend, size, resv, st, r.available))
    for size, resv in ((32, 0), (8, 0), (32, 3)):
        r = uh.ContextProbeResult(struct_size=size, abi_version=1)
        r.reserved[3] = resv
        s, _ = make_sink(uh)
        st = lib.ullm_context_probe(ctypes.c_void_p(0x10), ctypes.byref(r), ctypes.byref(s))
        res.append(("ctx", size, resv, st, r.context_present, r.hip_available))
    return res


def _bind(path, uh):
    lib = ctypes.CDLL(str(path))
    for n in ("ullm_get_abi_version", "ullm_query_version", "ullm_backend_probe",
              "ullm_context_probe"):
        fn = getattr(lib, n)
        fn.argtypes = uh._SIGNATURES[n]
        fn.restype = ctypes.c_uint32
    return lib


def test_sink_truncation_semantics(uh):
    lib = uh.lib()
    s, buf = make_sink(uh, 8)
    st = lib.ullm_get_abi_version(None, ctypes.byref(s))
    assert st == uh.Status.BUFFER_TOO_SMALL
    assert s.message_length == len("abi_version output is null")
    assert buf.raw[:8] == b"abi_vers"[:7] + b"\0"
    s, buf = make_sink(uh, 0)
    assert lib.ullm_get_abi_version(None, ctypes.byref(s)) == uh.Status.BUFFER_TOO_SMALL
    s, buf = make_sink(uh, 256)
    assert lib.ullm_get_abi_version(None, ctypes.byref(s)) == uh.Status.INVALID_ARGUMENT
    assert buf.value == b"abi_version output is null"


def test_v1_functions_match_reference_stub(uh):
    if not REF_LIB.exists():
        pytest.skip("reference stub not built here (reference tree absent)")
    mine = run_cases(uh, uh.lib())
    ref = run_cases(uh, _bind(REF_LIB, uh))
    assert len(mine) == len(ref)
    for a, b in zip(mine, ref):
        assert a == b, (a, b)


def test_v1_status_values(uh):
    _no_gpu(uh)
    cases = run_cases(uh, uh.lib())
    abi_ok = [c for c in cases if c[0] == "abi-ok"][0]
    assert abi_ok[1] == 0 and abi_ok[2] == 1
    probe_ok = [c for c in cases if c[0] == "probe" and c[1] == 1
                and c[2] == 32 and c[3] == 0][0]
    # no GPU in this container: unavailable, never a silent success
    assert probe_ok[4] == uh.Status.HIP_UNAVAILABLE and probe_ok[5] == 0
    assert uh.abi_version() == 1
    assert uh.version()[0] == 0


# ------------------------------------------------------ linear descriptors

def _no_gpu(uh):
    if uh.backend_probe()[0]:
        pytest.skip("a GPU is visible: the no-device statuses do not apply")


def _wdesc(uh, **kw):
    base = dict(encoding=uh.ENCODING_FP8_E4M3_ROW, source=uh.SOURCE_F32, n=16, k=64,
                memory=uh.MEMORY_HOST, device=0, values=0x1000)
    base.update(kw)
    return uh.new(uh.WeightDesc, **base)


@pytest.mark.parametrize("change,status", [
    (dict(struct_size=8), "INVALID_ARGUMENT"),
    (dict(abi_version=7), "INVALID_ABI_VERSION"),
    (dict(reserved=(0, 0, 1)), "RESERVED_NONZERO"),
    (dict(reserved0=1), "RESERVED_NONZERO"),
    (dict(layout=7), "INVALID_ARGUMENT"),
    (dict(layout=1, n=15), "INVALID_ARGUMENT"),     # gated pair needs even N
    (dict(encoding=9), "UNSUPPORTED"),
    (dict(source=0), "INVALID_ARGUMENT"),
    (dict(memory=5), "INVALID_ARGUMENT"),
    (dict(n=0), "INVALID_ARGUMENT"),
    (dict(k=0), "INVALID_ARGUMENT"),
    (dict(n=1 << 31), "UNSUPPORTED"),
    (dict(encoding=2, k=200), "INVALID_ARGUMENT"),
    (dict(values=None), "INVALID_ARGUMENT"),
    (dict(source=2), "INVALID_ARGUMENT"),           # encoded without scales
    (dict(source=2, encoding=2, k=128, scales=0x10), "INVALID_ARGUMENT"),  # no zeros
    (dict(), "HIP_UNAVAILABLE"),                    # valid, but no GPU here
])
def test_weight_create_validation(uh, change, status):
    if status == "HIP_UNAVAILABLE":
        _no_gpu(uh)
    d = _wdesc(uh)
    for k, v in change.items():
        if k == "reserved":
            for i, x in enumerate(v):
                d.reserved[i] = x
        else:
            setattr(d, k, v)
    h = ctypes.c_void_p(0xdead)
    s, buf = make_sink(uh)
    st = uh.lib().ullm_linear_weight_create(ctypes.byref(d), ctypes.byref(h), ctypes.byref(s))
    assert st == getattr(uh.Status, status), (st, buf.value)
    assert s.message_length > 0


def test_linear_entry_points_reject_bad_handles(uh):
    lib = uh.lib()
    s, _ = make_sink(uh)
    bogus = ctypes.c_void_p(0x1234)
    fwd = uh.new(uh.ForwardDesc, weight=bogus, m=1, x=0x10, y=0x20, alpha=1.0)
    assert lib.ullm_linear_forward(ctypes.byref(fwd), ctypes.byref(s)) == uh.Status.HIP_INVALID_HANDLE
    fwd.weight = None
    assert lib.ullm_linear_forward(ctypes.byref(fwd), None) == uh.Status.INVALID_ARGUMENT
    assert lib.ullm_linear_forward(None, None) == uh.Status.INVALID_ARGUMENT
    fwd = uh.new(uh.ForwardDesc, weight=bogus)
    fwd.reserved[0] = 1
    assert lib.ullm_linear_forward(ctypes.byref(fwd), None) == uh.Status.RESERVED_NONZERO
    h = ctypes.c_void_p(0x1234)
    assert lib.ullm_linear_weight_destroy(ctypes.byref(h), None) == uh.Status.HIP_INVALID_HANDLE
    assert lib.ullm_linear_weight_destroy(None, None) == uh.Status.INVALID_ARGUMENT
    info = uh.new(uh.WeightInfo)
    assert lib.ullm_linear_weight_query(bogus, ctypes.byref(info), None) == uh.Status.HIP_INVALID_HANDLE
    assert lib.ullm_linear_weight_dequantize(bogus, 0x10, None, None) == uh.Status.HIP_INVALID_HANDLE
    exp = uh.new(uh.ExportDesc, memory=1, values=0x10, scales=0x10)
    assert lib.ullm_linear_weight_export(bogus, ctypes.byref(exp), None) == uh.Status.HIP_INVALID_HANDLE
    n = ctypes.c_uint64()
    fwd = uh.new(uh.ForwardDesc, weight=bogus)
    assert lib.ullm_linear_workspace_size(ctypes.byref(fwd), ctypes.byref(n), None) \
        == uh.Status.HIP_INVALID_HANDLE


def test_activation_quant_validation(uh):
    lib = uh.lib()
    d = uh.new(uh.ActQuantDesc, m=0, k=64)
    assert lib.ullm_linear_quantize_activations(ctypes.byref(d), None) == uh.Status.OK
    d = uh.new(uh.ActQuantDesc, m=4, k=0)
    assert lib.ullm_linear_quantize_activations(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT
    d = uh.new(uh.ActQuantDesc, m=4, k=64, x_row_stride=32)
    assert lib.ullm_linear_quantize_activations(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT
    d = uh.new(uh.ActQuantDesc, m=4, k=64)
    assert lib.ullm_linear_quantize_activations(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT
    d.struct_size = 16
    assert lib.ullm_linear_quantize_activations(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT


def test_add_activation_quant_validation(uh):
    lib = uh.lib()
    f = lib.ullm_linear_add_quantize_activations
    assert ctypes.sizeof(uh.AddActQuantDesc) == 128
    d = uh.new(uh.AddActQuantDesc, m=0, k=64)
    assert f(ctypes.byref(d), None) == uh.Status.OK
    d = uh.new(uh.AddActQuantDesc, m=4, k=0)
    assert f(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT
    for field in ("a_row_stride", "b_row_stride", "sum_row_stride"):
        d = uh.new(uh.AddActQuantDesc, m=4, k=64, **{field: 32})
        assert f(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT, field
    d = uh.new(uh.AddActQuantDesc, m=4, k=64)  # null pointers
    assert f(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT
    # an in-place sum with another stride than the input it replaces
    d = uh.new(uh.AddActQuantDesc, m=4, k=64, a=0x1000, b=0x2000, sum=0x1000,
               a_row_stride=64, sum_row_stride=128, xq=0x3000, x_scales=0x4000)
    assert f(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT
    d = uh.new(uh.AddActQuantDesc, m=4, k=64)
    d.reserved[2] = 1
    assert f(ctypes.byref(d), None) == uh.Status.RESERVED_NONZERO
    d = uh.new(uh.AddActQuantDesc, m=4, k=64)
    d.struct_size = 16
    assert f(ctypes.byref(d), None) == uh.Status.INVALID_ARGUMENT


def test_python_mirror_raises_without_gpu(uh):
    _no_gpu(uh)
    available, present, diag = uh.backend_probe()
    assert not available and present and "unavailable" in diag
    import numpy as np
    with pytest.raises(uh.HipError) as e:
        uh.LinearWeight.from_fp8(np.zeros((16, 64), np.uint8), np.ones(16, np.float32))
    assert e.value.status == uh.Status.HIP_UNAVAILABLE


def test_plan_release_and_noalloc_entry_points_validate(uh):
    """ullm_linear_forward_plan, ullm_linear_forward_noalloc and
    ullm_linear_release_workspaces reject malformed calls before touching a
    device, with the same statuses as ullm_linear_forward."""
    lib = uh.lib()
    bogus = ctypes.c_void_p(0x1234)
    fwd = uh.new(uh.ForwardDesc, weight=bogus, m=1, x=0x10, y=0x20, alpha=1.0)
    plan = uh.new(uh.Plan)
    assert lib.ullm_linear_forward_plan(ctypes.byref(fwd), ctypes.byref(plan), None) \
        == uh.Status.HIP_INVALID_HANDLE
    assert lib.ullm_linear_forward_noalloc(ctypes.byref(fwd), None) \
        == uh.Status.HIP_INVALID_HANDLE
    assert lib.ullm_linear_forward_plan(None, ctypes.byref(plan), None) \
        == uh.Status.INVALID_ARGUMENT
    assert lib.ullm_linear_forward_noalloc(None, None) == uh.Status.INVALID_ARGUMENT
    fwd.reserved[0] = 1
    assert lib.ullm_linear_forward_noalloc(ctypes.byref(fwd), None) \
        == uh.Status.RESERVED_NONZERO
    s, buf = make_sink(uh, 256, abi_version=3)
    assert lib.ullm_linear_forward_plan(ctypes.byref(fwd), ctypes.byref(plan),
                                        ctypes.byref(s)) == uh.Status.INVALID_ABI_VERSION
    if not uh.backend_probe()[0]:
        s, buf = make_sink(uh)
        assert lib.ullm_linear_release_workspaces(0, ctypes.byref(s)) \
            == uh.Status.HIP_UNAVAILABLE
        assert s.message_length > 0
    assert ctypes.sizeof(uh.Plan) == 64

"""Python host mirror of the uLLM HIP backend over its C ABI.

Mirrors the reference's Rust layering:
  * the ``ullm_*`` ctypes declarations play the part of ``ullm-hip-sys``
    (reference crates/ullm-hip-sys/src/bindings.rs:1-119);
  * ``Status``, ``HipError``, ``abi_version``, ``version``, ``backend_probe``,
    ``context_probe`` mirror ``ullm-hip`` (reference
    crates/ullm-hip/src/lib.rs:20-76 Status, :78-113 HipError, :189-268
    probes) with the same 256-byte diagnostic buffers (lib.rs:18,154-170);
  * ``LinearWeight`` / ``linear_forward`` / ``quantize_activations`` wrap the
    linear-layer extension of include/ullm/linear.h, the calls a future
    ``HipBackend::execute`` (reference crates/ullm-hip/src/lib.rs:487-513)
    would make for a Matmul with a quantized weight.

PyTorch is used only to hold device memory and to name streams.  There is no
fallback: if the native library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import enum
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libullm_hip.so"
ERROR_CAPACITY = 256
ABI_VERSION = 1

# ------------------------------------------------------------------ statuses


class Status(enum.IntEnum):
    OK = 0
    INVALID_ARGUMENT = 1
    BUFFER_TOO_SMALL = 2
    UNSUPPORTED = 3
    HIP_UNAVAILABLE = 4
    INVALID_ABI_VERSION = 5
    RESERVED_NONZERO = 6
    INTERNAL_ERROR = 7
    HIP_TIMEOUT = 8
    HIP_INVALID_HANDLE = 9
    HIP_ZERO_DISPATCH = 10
    HIP_RUNTIME_ERROR = 11
    HIP_DISPATCH_CONTRACT = 12
    OUT_OF_MEMORY = 13


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        try:
            self.status = Status(status)
        except ValueError:
            self.status = status
        self.message = message
        super().__init__(f"{getattr(self.status, 'name', status)}: {message}")


ENCODING_FP8_E4M3_ROW = 1
ENCODING_AQ4_G128 = 2
SOURCE_F32 = 1
SOURCE_ENCODED = 2
MEMORY_HOST = 1
MEMORY_DEVICE = 2
DTYPE_BF16 = 1
DTYPE_F32 = 2
DTYPE_F8E4M3FN = 3
ACT_EXACT = 0
ACT_FP8_PER_TOKEN = 1
LAYOUT_PLAIN = 0
LAYOUT_GATED_PAIRS = 1
EPILOGUE_NONE = 0
EPILOGUE_SILU_MUL = 1
EPILOGUE_RESIDUAL_ADD = 2
KERNEL_GEMV = 1
KERNEL_GEMM_DIRECT = 2
KERNEL_GEMM_LDS = 3
GEMV_SINGLE = 1
GEMV_SINGLE_LDS = 2
GEMV_MULTI_STRIPE = 3
GEMV_REGISTER_STAGED = 4
GEMV_SPLIT_K = 5
BACKEND_HIP = 1

# ------------------------------------------------------------------- structs
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_vp = ctypes.c_void_p


class ErrorSink(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32),
                ("message", ctypes.c_char_p), ("message_capacity", _u64),
                ("message_length", _u64), ("reserved", _u64 * 2)]


class VersionInfo(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("major", _u32),
                ("minor", _u32), ("patch", _u32), ("reserved", _u32 * 3)]


class BackendProbeResult(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("backend", _u32),
                ("available", _u32), ("hip_runtime_present", _u32),
                ("reserved", _u32 * 3)]


class ContextProbeResult(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32),
                ("context_present", _u32), ("hip_available", _u32),
                ("reserved", _u32 * 4)]


class WeightDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32),
                ("encoding", _u32), ("source", _u32), ("n", _u64), ("k", _u64),
                ("memory", _u32), ("device", _i32), ("values", _vp),
                ("scales", _vp), ("zeros", _vp), ("stream", _vp),
                ("layout", _u32), ("reserved0", _u32), ("reserved", _u64 * 3)]


class WeightInfo(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32),
                ("encoding", _u32), ("device", _i32), ("n", _u64), ("k", _u64),
                ("device_bytes", _u64), ("layout", _u32), ("reserved0", _u32),
                ("reserved", _u64 * 3)]


class ForwardDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("weight", _vp),
                ("m", _u64), ("x", _vp), ("x_row_stride", _u64),
                ("x_scales", _vp), ("y", _vp), ("y_row_stride", _u64),
                ("x_dtype", _u32), ("y_dtype", _u32), ("activation_mode", _u32),
                ("alpha", ctypes.c_float), ("stream", _vp), ("workspace", _vp),
                ("workspace_size", _u64), ("epilogue", _u32),
                ("residual_dtype", _u32), ("residual", _vp),
                ("residual_row_stride", _u64), ("reserved", _u64 * 1)]


class Plan(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("kernel", _u32),
                ("block_m", _u32), ("block_n", _u32), ("tiles", _u32),
                ("grid", _u32), ("split_k", _u32), ("gemv_variant", _u32),
                ("gemv_waves", _u32), ("gemv_stripes", _u32),
                ("gemv_row_classes", _u32), ("reserved", _u64 * 2)]


class EvidenceRequest(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32),
                ("input", ctypes.c_void_p), ("input_size", _u64),
                ("reserved", _u32 * 4)]


class EvidenceResult(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32),
                ("output_size", _u64), ("allocation_count", _u64),
                ("copy_count", _u64), ("dispatch_count", _u64),
                ("selected_backend", _u32), ("fallback_used", _u32),
                ("terminal", _u32), ("reserved", _u32 * 4)]


class ActQuantDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("m", _u64),
                ("k", _u64), ("x", _vp), ("x_row_stride", _u64), ("xq", _vp),
                ("x_scales", _vp), ("stream", _vp), ("reserved", _u64 * 4)]


class AddActQuantDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("m", _u64),
                ("k", _u64), ("a", _vp), ("a_row_stride", _u64), ("b", _vp),
                ("b_row_stride", _u64), ("sum", _vp), ("sum_row_stride", _u64),
                ("xq", _vp), ("x_scales", _vp), ("stream", _vp),
                ("reserved", _u64 * 4)]


class ExportDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("memory", _u32),
                ("reserved0", _u32), ("values", _vp), ("scales", _vp),
                ("zeros", _vp), ("stream", _vp), ("reserved", _u64 * 4)]


class StOpenDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("path", ctypes.c_char_p),
                ("expected_sha256", _vp), ("expected_size", _u64),
                ("reserved", _u64 * 4)]


class StTensorInfo(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("dtype", _u32),
                ("rank", _u32), ("shape", _u64 * 8), ("offset", _u64),
                ("bytes", _u64), ("reserved", _u64 * 4)]


class WeightLoadDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("file", _vp),
                ("encoding", _u32), ("layout", _u32),
                ("values", ctypes.POINTER(ctypes.c_char_p)), ("value_parts", _u32),
                ("device", _i32), ("scales", ctypes.c_char_p), ("zeros", ctypes.c_char_p),
                ("stream", _vp), ("reserved", _u64 * 4)]


class WeightsSaveDesc(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("abi_version", _u32), ("path", ctypes.c_char_p),
                ("names", ctypes.POINTER(ctypes.c_char_p)),
                ("weights", ctypes.POINTER(_vp)), ("count", _u64),
                ("metadata_keys", ctypes.POINTER(ctypes.c_char_p)),
                ("metadata_values", ctypes.POINTER(ctypes.c_char_p)),
                ("metadata_count", _u64), ("reserved", _u64 * 4)]


# safetensors dtype strings by ULLM_ST_DTYPE_* value
ST_DTYPES = {1: "BOOL", 2: "U8", 3: "I8", 4: "F8_E4M3", 5: "F8_E5M2", 6: "U16",
             7: "I16", 8: "F16", 9: "BF16", 10: "U32", 11: "I32", 12: "F32",
             13: "U64", 14: "I64", 15: "F64"}


def new(struct_type, **fields):
    """A struct with its {struct_size, abi_version} header filled in."""
    s = struct_type()
    s.struct_size = ctypes.sizeof(struct_type)
    s.abi_version = ABI_VERSION
    for k, v in fields.items():
        setattr(s, k, v)
    return s


# --------------------------------------------------------------- the library
_SIGNATURES = {
    "ullm_get_abi_version": [ctypes.POINTER(_u32), ctypes.POINTER(ErrorSink)],
    "ullm_query_version": [ctypes.POINTER(VersionInfo), ctypes.POINTER(ErrorSink)],
    "ullm_backend_probe": [_u32, ctypes.POINTER(BackendProbeResult),
                           ctypes.POINTER(ErrorSink)],
    "ullm_context_probe": [_vp, ctypes.POINTER(ContextProbeResult),
                           ctypes.POINTER(ErrorSink)],
    "ullm_linear_weight_create": [ctypes.POINTER(WeightDesc), ctypes.POINTER(_vp),
                                  ctypes.POINTER(ErrorSink)],
    "ullm_linear_weight_destroy": [ctypes.POINTER(_vp), ctypes.POINTER(ErrorSink)],
    "ullm_linear_weight_query": [_vp, ctypes.POINTER(WeightInfo),
                                 ctypes.POINTER(ErrorSink)],
    "ullm_linear_weight_export": [_vp, ctypes.POINTER(ExportDesc),
                                  ctypes.POINTER(ErrorSink)],
    "ullm_linear_weight_dequantize": [_vp, _vp, _vp, ctypes.POINTER(ErrorSink)],
    "ullm_linear_forward": [ctypes.POINTER(ForwardDesc), ctypes.POINTER(ErrorSink)],
    "ullm_linear_workspace_size": [ctypes.POINTER(ForwardDesc), ctypes.POINTER(_u64),
                                   ctypes.POINTER(ErrorSink)],
    "ullm_linear_quantize_activations": [ctypes.POINTER(ActQuantDesc),
                                         ctypes.POINTER(ErrorSink)],
    "ullm_linear_add_quantize_activations": [ctypes.POINTER(AddActQuantDesc),
                                             ctypes.POINTER(ErrorSink)],
    "ullm_linear_forward_plan": [ctypes.POINTER(ForwardDesc), ctypes.POINTER(Plan),
                                 ctypes.POINTER(ErrorSink)],
    "ullm_linear_release_workspaces": [_i32, ctypes.POINTER(ErrorSink)],
    "ullm_linear_forward_noalloc": [ctypes.POINTER(ForwardDesc), ctypes.POINTER(ErrorSink)],
    "ullm_hip_evidence_submit": [ctypes.POINTER(EvidenceRequest), ctypes.POINTER(_vp),
                                 ctypes.POINTER(ErrorSink)],
    "ullm_hip_evidence_wait": [_vp, _u32, _vp, _u64, ctypes.POINTER(EvidenceResult),
                               ctypes.POINTER(ErrorSink)],
    "ullm_hip_evidence_destroy": [ctypes.POINTER(_vp), ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_open": [ctypes.POINTER(StOpenDesc), ctypes.POINTER(_vp),
                              ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_close": [ctypes.POINTER(_vp), ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_tensor_count": [_vp, ctypes.POINTER(_u64), ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_tensor_name": [_vp, _u64, ctypes.c_char_p, _u64,
                                     ctypes.POINTER(_u64), ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_tensor_info": [_vp, ctypes.c_char_p, ctypes.POINTER(StTensorInfo),
                                     ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_metadata": [_vp, ctypes.c_char_p, ctypes.c_char_p, _u64,
                                  ctypes.POINTER(_u64), ctypes.POINTER(ErrorSink)],
    "ullm_safetensors_file_sha256": [_vp, ctypes.c_char_p, ctypes.POINTER(ErrorSink)],
    "ullm_linear_weight_load": [ctypes.POINTER(WeightLoadDesc), ctypes.POINTER(_vp),
                                ctypes.POINTER(ErrorSink)],
    "ullm_linear_weights_save": [ctypes.POINTER(WeightsSaveDesc), ctypes.c_char_p,
                                 ctypes.POINTER(ErrorSink)],
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libullm_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with ullm-project_amd/build.py")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _u32
        _lib = L
    return _lib


class _Sink:
    def __init__(self, capacity: int = ERROR_CAPACITY):
        self.buf = ctypes.create_string_buffer(capacity)
        self.sink = new(ErrorSink, message=ctypes.cast(self.buf, ctypes.c_char_p),
                        message_capacity=capacity)

    @property
    def ref(self):
        return ctypes.byref(self.sink)

    def text(self) -> str:
        n = min(self.sink.message_length, len(self.buf) - 1)
        return self.buf.raw[:n].decode(errors="replace")


def _check(status: int, sink: _Sink):
    if status != Status.OK:
        raise HipError(status, sink.text())


# ------------------------------------------------------------- v1 functions

def abi_version() -> int:
    s = _Sink()
    v = _u32()
    _check(lib().ullm_get_abi_version(ctypes.byref(v), s.ref), s)
    return v.value


def version() -> tuple:
    s = _Sink()
    info = new(VersionInfo)
    _check(lib().ullm_query_version(ctypes.byref(info), s.ref), s)
    return (info.major, info.minor, info.patch)


def backend_probe():
    """(available, hip_runtime_present, diagnostic) like ullm_hip::backend_probe."""
    s = _Sink()
    r = new(BackendProbeResult)
    st = lib().ullm_backend_probe(BACKEND_HIP, ctypes.byref(r), s.ref)
    if st not in (Status.OK, Status.HIP_UNAVAILABLE):
        raise HipError(st, s.text())
    return bool(r.available), bool(r.hip_runtime_present), s.text()


def context_probe():
    s = _Sink()
    r = new(ContextProbeResult)
    st = lib().ullm_context_probe(None, ctypes.byref(r), s.ref)
    if st not in (Status.OK, Status.HIP_UNAVAILABLE):
        raise HipError(st, s.text())
    return bool(r.context_present), bool(r.hip_available), s.text()


# ------------------------------------------------------------ linear layer

def _ptr(t) -> int | None:
    return None if t is None else int(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


class LinearWeight:
    """A device-resident quantized weight W[N][K] (opaque native handle).

    ``gated=True`` (ULLM_LINEAR_LAYOUT_GATED_PAIRS) marks a fused gate/up
    projection whose N = 2F rows are the F gate rows followed by the F up
    rows; its forward applies SiLU(gate) * up and returns F columns."""

    def __init__(self, handle: int, encoding: int, n: int, k: int, device: int,
                 gated: bool = False):
        self.handle = handle
        self.encoding = encoding
        self.n = n
        self.k = k
        self.device = device
        self.gated = gated

    @property
    def n_out(self) -> int:
        """Output columns of a forward: F = N / 2 for a gated pair, else N."""
        return self.n // 2 if self.gated else self.n

    # -- construction -----------------------------------------------------
    @classmethod
    def _create(cls, encoding, source, n, k, memory, device, values, scales=None,
                zeros=None, stream=None, gated=False):
        s = _Sink()
        d = new(WeightDesc, encoding=encoding, source=source, n=n, k=k,
                memory=memory, device=device, values=values, scales=scales,
                zeros=zeros, stream=stream,
                layout=LAYOUT_GATED_PAIRS if gated else LAYOUT_PLAIN)
        h = _vp()
        _check(lib().ullm_linear_weight_create(ctypes.byref(d), ctypes.byref(h),
                                               s.ref), s)
        return cls(h.value, encoding, n, k, device, gated)

    @classmethod
    def quantize(cls, w, encoding: int, stream=None, gated=False):
        """Quantize an f32 weight tensor [N][K] (CUDA or CPU) on the GPU."""
        import torch
        assert w.dtype == torch.float32 and w.dim() == 2
        w = w.contiguous()
        n, k = w.shape
        if w.is_cuda:
            return cls._create(encoding, SOURCE_F32, n, k, MEMORY_DEVICE,
                               w.device.index, _ptr(w), stream=_stream(stream),
                               gated=gated)
        return cls._create(encoding, SOURCE_F32, n, k, MEMORY_HOST, 0, _ptr(w),
                           stream=None, gated=gated)

    @classmethod
    def from_fp8(cls, q, s, device=0, stream=None, gated=False):
        """Upload canonical E4M3 codes q uint8 [N][K] and f32 scales [N]."""
        n, k = q.shape
        mem = MEMORY_DEVICE if getattr(q, "is_cuda", False) else MEMORY_HOST
        return cls._create(ENCODING_FP8_E4M3_ROW, SOURCE_ENCODED, n, k, mem,
                           device, _addr(q), _addr(s), None,
                           _stream(stream) if mem == MEMORY_DEVICE else None,
                           gated=gated)

    @classmethod
    def from_aq4(cls, packed, scales, zeros, device=0, stream=None, gated=False):
        """Upload canonical AQ4: u32 [N][K/8], f16 bits [N][K/128] x 2."""
        n = packed.shape[0]
        k = packed.shape[1] * 8
        mem = MEMORY_DEVICE if getattr(packed, "is_cuda", False) else MEMORY_HOST
        return cls._create(ENCODING_AQ4_G128, SOURCE_ENCODED, n, k, mem, device,
                           _addr(packed), _addr(scales), _addr(zeros),
                           _stream(stream) if mem == MEMORY_DEVICE else None,
                           gated=gated)

    # -- lifetime ----------------------------------------------------------
    def destroy(self):
        if self.handle:
            s = _Sink()
            h = _vp(self.handle)
            self.handle = None
            _check(lib().ullm_linear_weight_destroy(ctypes.byref(h), s.ref), s)

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def info(self) -> WeightInfo:
        s = _Sink()
        i = new(WeightInfo)
        _check(lib().ullm_linear_weight_query(self.handle, ctypes.byref(i), s.ref), s)
        return i

    # -- debug / parity ----------------------------------------------------
    def export(self):
        """Canonical encoded buffers as numpy arrays (host)."""
        import numpy as np
        n, k = self.n, self.k
        if self.encoding == ENCODING_FP8_E4M3_ROW:
            v = np.empty((n, k), np.uint8)
            sc = np.empty(n, np.float32)
            z = None
        else:
            v = np.empty((n, k // 8), np.uint32)
            sc = np.empty((n, k // 128), np.uint16)
            z = np.empty((n, k // 128), np.uint16)
        s = _Sink()
        d = new(ExportDesc, memory=MEMORY_HOST, values=v.ctypes.data,
                scales=sc.ctypes.data, zeros=None if z is None else z.ctypes.data)
        _check(lib().ullm_linear_weight_export(self.handle, ctypes.byref(d), s.ref), s)
        return (v, sc) if z is None else (v, sc, z)

    def dequantize(self, stream=None):
        import torch
        out = torch.empty((self.n, self.k), dtype=torch.float32,
                          device=f"cuda:{self.device}")
        s = _Sink()
        _check(lib().ullm_linear_weight_dequantize(self.handle, _ptr(out),
                                                   _stream(stream), s.ref), s)
        return out

    # -- compute -----------------------------------------------------------
    def workspace_size(self, m, *, mode=ACT_EXACT, x_dtype=DTYPE_BF16):
        """Bytes of caller workspace a forward of m rows needs
        (ullm_linear_workspace_size); 0 when it needs none."""
        import torch
        probe = torch.empty((1,), dtype=torch.uint8)  # any non-null address
        d = new(ForwardDesc, weight=self.handle, m=m, x=_ptr(probe),
                x_row_stride=0, x_scales=_ptr(probe), y=_ptr(probe),
                y_row_stride=0, x_dtype=x_dtype, y_dtype=DTYPE_BF16,
                activation_mode=mode, alpha=1.0,
                epilogue=EPILOGUE_SILU_MUL if self.gated else EPILOGUE_NONE)
        out = _u64(0)
        s = _Sink()
        _check(lib().ullm_linear_workspace_size(ctypes.byref(d), ctypes.byref(out),
                                                s.ref), s)
        return int(out.value)

    def _forward_desc(self, x, y, *, x_scales, alpha, mode, stream, workspace,
                      residual):
        import torch
        x_dtype = DTYPE_F8E4M3FN if x.dtype in (torch.uint8, torch.float8_e4m3fn) \
            else DTYPE_BF16
        epi = EPILOGUE_SILU_MUL if self.gated else EPILOGUE_NONE
        res = {}
        if residual is not None:
            epi = EPILOGUE_RESIDUAL_ADD
            res = dict(residual=_ptr(residual),
                       residual_row_stride=residual.stride(0),
                       residual_dtype=DTYPE_F32 if residual.dtype == torch.float32
                       else DTYPE_BF16)
        return new(ForwardDesc, weight=self.handle, m=x.shape[0], x=_ptr(x),
                   x_row_stride=x.stride(0) if x.dim() == 2 else 0,
                   x_scales=_ptr(x_scales), y=_ptr(y), y_row_stride=y.stride(0),
                   x_dtype=x_dtype,
                   y_dtype=DTYPE_F32 if y.dtype == torch.float32 else DTYPE_BF16,
                   activation_mode=mode, alpha=alpha, stream=_stream(stream),
                   workspace=_ptr(workspace),
                   workspace_size=0 if workspace is None
                   else workspace.numel() * workspace.element_size(),
                   epilogue=epi, **res)

    def forward(self, x, y=None, *, x_scales=None, out_dtype=None, alpha=1.0,
                mode=ACT_EXACT, stream=None, workspace=None, residual=None,
                noalloc=False):
        """y = alpha * x @ W^T for x bf16 [M][>=K] (row stride honoured) or
        pre-quantized e4m3 (uint8) with x_scales.  A gated-pair weight returns
        silu(gate) * up (F columns); ``residual`` (bf16 or f32 [M][>=N], may
        be ``y`` itself) is added to the product (ULLM_LINEAR_EPILOGUE_*).
        ``noalloc`` calls ullm_linear_forward_noalloc (scratch from the
        library's fixed per-device array; ``workspace`` must be None)."""
        import torch
        m = x.shape[0]
        if y is None:
            dt = out_dtype or torch.bfloat16
            y = torch.empty((m, self.n_out), dtype=dt, device=x.device)
        d = self._forward_desc(x, y, x_scales=x_scales, alpha=alpha, mode=mode,
                               stream=stream, workspace=workspace,
                               residual=residual)
        s = _Sink()
        fn = lib().ullm_linear_forward_noalloc if noalloc else lib().ullm_linear_forward
        _check(fn(ctypes.byref(d), s.ref), s)
        return y

    def plan(self, x, y, *, x_scales=None, alpha=1.0, mode=ACT_EXACT,
             stream=None, workspace=None, residual=None) -> Plan:
        """The launch forward() would make with these arguments
        (ullm_linear_forward_plan); launches nothing."""
        d = self._forward_desc(x, y, x_scales=x_scales, alpha=alpha, mode=mode,
                               stream=stream, workspace=workspace,
                               residual=residual)
        out = new(Plan)
        s = _Sink()
        _check(lib().ullm_linear_forward_plan(ctypes.byref(d), ctypes.byref(out),
                                              s.ref), s)
        return out


def release_workspaces(device: int = 0) -> None:
    """Free the library-owned forward workspaces of a device
    (ullm_linear_release_workspaces)."""
    s = _Sink()
    _check(lib().ullm_linear_release_workspaces(device, s.ref), s)


# ------------------------------------------------------------------ evidence
EVIDENCE_ABI_VERSION = 1
EVIDENCE_XOR = 0x5A


def evidence_new(struct_type, **fields):
    """An evidence struct with its {struct_size, abi_version} header."""
    s = struct_type()
    s.struct_size = ctypes.sizeof(struct_type)
    s.abi_version = EVIDENCE_ABI_VERSION
    for k, v in fields.items():
        setattr(s, k, v)
    return s


class EvidenceCompletion:
    """A submitted evidence transform (reference crates/ullm-hip/src/
    lib.rs:293-375): wait() consumes it; dropping it destroys it."""

    def __init__(self, handle: int, size: int):
        self.handle = handle
        self.size = size

    def wait(self, output: bytearray, timeout_ms: int) -> dict:
        if self.handle is None:
            raise HipError(Status.HIP_INVALID_HANDLE,
                           "evidence completion was already consumed")
        handle, self.handle = self.handle, None
        buf = (ctypes.c_uint8 * len(output)).from_buffer(output) if len(output) else None
        res = evidence_new(EvidenceResult)
        s = _Sink()
        _check(lib().ullm_hip_evidence_wait(handle, min(int(timeout_ms), 2 ** 32 - 1),
                                            ctypes.cast(buf, _vp) if buf is not None else None,
                                            len(output), ctypes.byref(res), s.ref), s)
        return {"output_size": res.output_size,
                "allocation_count": res.allocation_count,
                "copy_count": res.copy_count,
                "dispatch_count": res.dispatch_count,
                "selected_backend": res.selected_backend,
                "fallback_used": bool(res.fallback_used),
                "terminal": bool(res.terminal)}

    def destroy(self):
        if self.handle is None:
            return
        h = _vp(self.handle)
        self.handle = None
        lib().ullm_hip_evidence_destroy(ctypes.byref(h), None)

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def submit_evidence(data: bytes) -> EvidenceCompletion:
    """Queue the XOR-0x5a evidence transform of ``data`` on the GPU
    (reference lib.rs:377-406)."""
    if len(data) == 0:
        raise HipError(Status.INVALID_ARGUMENT, "evidence input must not be empty")
    src = ctypes.create_string_buffer(bytes(data), len(data))
    req = evidence_new(EvidenceRequest, input=ctypes.cast(src, _vp),
                       input_size=len(data))
    h = _vp()
    s = _Sink()
    _check(lib().ullm_hip_evidence_submit(ctypes.byref(req), ctypes.byref(h), s.ref), s)
    if not h.value:
        raise HipError(Status.INTERNAL_ERROR,
                       "native evidence submit returned a null completion")
    return EvidenceCompletion(h.value, len(data))


def expected_evidence_output(data: bytes) -> bytes:
    return bytes(b ^ EVIDENCE_XOR for b in data)


def run_evidence(data: bytes, timeout_ms: int = 10000):
    """Submit, wait and check the exact no-fallback byte contract
    (reference lib.rs:408-441)."""
    c = submit_evidence(data)
    out = bytearray(len(data))
    rep = c.wait(out, timeout_ms)
    if rep["dispatch_count"] == 0:
        raise HipError(Status.HIP_ZERO_DISPATCH,
                       "evidence result contains zero kernel dispatches")
    if (rep["selected_backend"] != BACKEND_HIP or rep["fallback_used"]
            or not rep["terminal"] or rep["output_size"] != len(data)
            or rep["allocation_count"] != 2 or rep["copy_count"] != 2
            or rep["dispatch_count"] != 1
            or bytes(out) != expected_evidence_output(data)):
        raise HipError(Status.HIP_DISPATCH_CONTRACT,
                       "evidence result failed the exact no-fallback byte contract")
    return bytes(out), rep


def _addr(a):
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return int(a.data_ptr())
    return int(a.ctypes.data)


# ------------------------------------------------------------ weight files

def _cstrs(items):
    arr = (ctypes.c_char_p * len(items))()
    for i, v in enumerate(items):
        arr[i] = v.encode() if isinstance(v, str) else v
    return arr


def _string_call(fn, *args):
    """Call a string-returning entry point, growing the buffer on demand."""
    cap = 256
    while True:
        buf = ctypes.create_string_buffer(cap)
        n = _u64(0)
        s = _Sink()
        st = fn(*args, buf, cap, ctypes.byref(n), s.ref)
        if st == Status.BUFFER_TOO_SMALL and n.value + 1 > cap:
            cap = n.value + 1
            continue
        _check(st, s)
        return buf.raw[:n.value].decode()


class SafetensorsFile:
    """An open, validated safetensors file (ullm_safetensors_open).

    ``sha256`` (hex string or 32 bytes) and ``size`` make the open check the
    file's content against a model lock's record before anything is read."""

    def __init__(self, path, sha256=None, size=None):
        digest = None
        if sha256 is not None:
            digest = bytes.fromhex(sha256) if isinstance(sha256, str) else bytes(sha256)
            assert len(digest) == 32
        self._digest = ctypes.create_string_buffer(digest, 32) if digest else None
        d = new(StOpenDesc, path=str(path).encode(),
                expected_sha256=ctypes.cast(self._digest, _vp) if digest else None,
                expected_size=size or 0)
        h = _vp()
        s = _Sink()
        _check(lib().ullm_safetensors_open(ctypes.byref(d), ctypes.byref(h), s.ref), s)
        self.handle = h.value
        self.path = str(path)

    def close(self):
        if self.handle:
            h = _vp(self.handle)
            self.handle = None
            s = _Sink()
            _check(lib().ullm_safetensors_close(ctypes.byref(h), s.ref), s)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self):
        n = _u64(0)
        s = _Sink()
        _check(lib().ullm_safetensors_tensor_count(self.handle, ctypes.byref(n), s.ref), s)
        return [_string_call(lib().ullm_safetensors_tensor_name, self.handle, i)
                for i in range(n.value)]

    def info(self, name):
        """(dtype string, shape tuple, byte offset in the file, byte count)."""
        i = new(StTensorInfo)
        s = _Sink()
        _check(lib().ullm_safetensors_tensor_info(self.handle, name.encode(),
                                                  ctypes.byref(i), s.ref), s)
        return ST_DTYPES[i.dtype], tuple(i.shape[:i.rank]), i.offset, i.bytes

    def metadata(self, key):
        return _string_call(lib().ullm_safetensors_metadata, self.handle, key.encode())

    def sha256(self) -> str:
        out = ctypes.create_string_buffer(32)
        s = _Sink()
        _check(lib().ullm_safetensors_file_sha256(self.handle, out, s.ref), s)
        return out.raw.hex()


def load_weight(file, values, encoding, *, scales=None, zeros=None, gated=False,
                device=0, stream=None):
    """A LinearWeight from tensors of an open SafetensorsFile
    (ullm_linear_weight_load).  ``values``: one tensor name, or a list of float
    tensors stacked along N (e.g. [gate, up] for a gated pair)."""
    parts = [values] if isinstance(values, str) else list(values)
    arr = _cstrs(parts)
    d = new(WeightLoadDesc, file=file.handle, encoding=encoding,
            layout=LAYOUT_GATED_PAIRS if gated else LAYOUT_PLAIN,
            values=arr, value_parts=len(parts), device=device,
            scales=scales.encode() if scales else None,
            zeros=zeros.encode() if zeros else None,
            stream=_stream(stream) if stream is not None else None)
    h = _vp()
    s = _Sink()
    _check(lib().ullm_linear_weight_load(ctypes.byref(d), ctypes.byref(h), s.ref), s)
    w = LinearWeight(h.value, encoding, 0, 0, device, gated)
    info = w.info()
    w.n, w.k = int(info.n), int(info.k)
    return w


def load_saved_weight(file, name, device=0, stream=None):
    """A weight written by save_weights, by its name (encoding and layout from
    the file's metadata)."""
    enc = file.metadata(f"{name}.encoding")
    gated = file.metadata(f"{name}.layout") == "gated_pairs"
    if enc == "fp8_e4m3_row":
        return load_weight(file, f"{name}.weight", ENCODING_FP8_E4M3_ROW,
                           scales=f"{name}.weight_scale", gated=gated, device=device,
                           stream=stream)
    if enc == "aq4_g128":
        return load_weight(file, f"{name}.qweight", ENCODING_AQ4_G128,
                           scales=f"{name}.scales", zeros=f"{name}.zeros", gated=gated,
                           device=device, stream=stream)
    raise ValueError(f"unknown encoding {enc!r} for {name}")


def save_weights(path, weights, metadata=None) -> str:
    """Write {name: LinearWeight} in canonical encodings (ullm_linear_weights_save);
    returns the file's SHA-256 (hex)."""
    names = list(weights)
    harr = (_vp * len(names))(*[weights[n].handle for n in names])
    meta = dict(metadata or {})
    d = new(WeightsSaveDesc, path=str(path).encode(), names=_cstrs(names),
            weights=harr, count=len(names), metadata_keys=_cstrs(list(meta)),
            metadata_values=_cstrs(list(meta.values())), metadata_count=len(meta))
    out = ctypes.create_string_buffer(32)
    s = _Sink()
    _check(lib().ullm_linear_weights_save(ctypes.byref(d), out, s.ref), s)
    return out.raw.hex()


def add_quantize_activations(a, b, out=None, stream=None):
    """Per-token E4M3 quantization of a + b (bf16 [M][K] each, rounded
    to bf16 first): returns (xq uint8 [M][K], scales f32 [M]).  ``out``
    (bf16 [M][>=K], may be ``a`` or ``b``) receives the sum when given."""
    import torch
    m, k = a.shape
    if tuple(b.shape) != (m, k) or (out is not None and tuple(out.shape) != (m, k)):
        raise ValueError("a, b and out must have the same shape")
    xq = torch.empty((m, k), dtype=torch.uint8, device=a.device)
    xs = torch.empty((m,), dtype=torch.float32, device=a.device)
    d = new(AddActQuantDesc, m=m, k=k, a=_ptr(a), a_row_stride=a.stride(0),
            b=_ptr(b), b_row_stride=b.stride(0),
            sum=_ptr(out) if out is not None else None,
            sum_row_stride=out.stride(0) if out is not None else 0,
            xq=_ptr(xq), x_scales=_ptr(xs), stream=_stream(stream))
    s = _Sink()
    _check(lib().ullm_linear_add_quantize_activations(ctypes.byref(d), s.ref), s)
    return xq, xs


def quantize_activations(x, xq=None, xs=None, stream=None):
    """Per-token E4M3 quantization: returns (xq uint8 [M][K], scales f32 [M]),
    into the given contiguous outputs when passed."""
    import torch
    m, k = x.shape
    if xq is None:
        xq = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    if xs is None:
        xs = torch.empty((m,), dtype=torch.float32, device=x.device)
    if xq.shape != (m, k) or not xq.is_contiguous() or xq.dtype != torch.uint8:
        raise ValueError("xq must be a contiguous uint8 [M][K] tensor")
    if xs.shape != (m,) or xs.dtype != torch.float32:
        raise ValueError("xs must be a float32 [M] tensor")
    d = new(ActQuantDesc, m=m, k=k, x=_ptr(x), x_row_stride=x.stride(0),
            xq=_ptr(xq), x_scales=_ptr(xs), stream=_stream(stream))
    s = _Sink()
    _check(lib().ullm_linear_quantize_activations(ctypes.byref(d), s.ref), s)
    return xq, xs

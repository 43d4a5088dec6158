"""ctypes wrapper over the C oracle (oracle/ullm_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by ``__graft_entry__.smoke()``
and by bench.py's ``cpu_baseline`` leg, always as the checker or the timed CPU
restatement, never as part of the product path.  The numeric definitions are
stated in oracle/ullm_oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
SOURCES = [HERE / "ullm_oracle.c"]
CFLAGS = [
    "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math",
    "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra",
]


def build(force: bool = False) -> Path:
    """Compile the oracle shared library with gcc (plain C, OpenMP)."""
    if force or not LIB_PATH.exists() or any(
            s.stat().st_mtime > LIB_PATH.stat().st_mtime for s in SOURCES):
        tmp = LIB_PATH.with_suffix(".so.tmp")
        cmd = ["gcc", *CFLAGS, *map(str, SOURCES), "-o", str(tmp), "-lm"]
        subprocess.run(cmd, check=True)
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_native(out_dir: Path) -> Path:
    """Compile the same source with ``-march=native`` for the machine this runs
    on (the CPU-baseline timing copy; built where it is timed, since the
    container that builds the tree and the GPU box have different CPUs)."""
    out = Path(out_dir) / "liboracle_native.so"
    flags = [f for f in CFLAGS if not f.startswith("-march=")] + ["-march=native"]
    subprocess.run(["gcc", *flags, *map(str, SOURCES), "-o", str(out), "-lm"], check=True)
    return out


def use_library(path: Path) -> None:
    """Route every oracle call through the library at ``path`` (a build of the
    same source, e.g. build_native's)."""
    global _lib
    _lib = _load(Path(path))


_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = _load(LIB_PATH)
    return _lib


def _load(path: Path) -> ctypes.CDLL:
    L = ctypes.CDLL(str(path))
    sig = {
        "orc_e4m3_from_f32": (ctypes.c_uint8, [_F]),
        "orc_e4m3_to_f32": (_F, [ctypes.c_uint8]),
        "orc_bf16_from_f32": (ctypes.c_uint16, [_F]),
        "orc_bf16_to_f32": (_F, [ctypes.c_uint16]),
        "orc_f16_from_f32": (ctypes.c_uint16, [_F]),
        "orc_f16_to_f32": (_F, [ctypes.c_uint16]),
        "orc_e4m3_from_f32_n": (None, [_P, _P, _I]),
        "orc_bf16_from_f32_n": (None, [_P, _P, _I]),
        "orc_f16_from_f32_n": (None, [_P, _P, _I]),
        "orc_fp8_quantize_rows": (None, [_P, _I, _I, _P, _P]),
        "orc_fp8_dequantize": (None, [_P, _P, _I, _I, _P]),
        "orc_aq4_quantize": (None, [_P, _I, _I, _P, _P, _P]),
        "orc_aq4_dequantize": (None, [_P, _P, _P, _I, _I, _P]),
        "orc_fp8_gemv": (None, [_I, _I, _I, _P, _I, _P, _P, _F, _P, _P, ctypes.c_int]),
        "orc_aq4_gemv": (None, [_I, _I, _I, _P, _I, _P, _P, _P, _F, _P, _P, ctypes.c_int]),
        "orc_act_quantize": (None, [_I, _I, _P, _I, _P, _P]),
        "orc_bf16_add": (None, [_I, _P, _P, _P]),
        "orc_fp8_gemm": (None, [_I, _I, _I, _P, _P, _P, _P, _F, _P, _P, ctypes.c_int]),
        "orc_silu_mul": (None, [_I, _I, _P, _P]),
        "orc_max_threads": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- scalar formats -------------------------------------------------------

def e4m3_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_from_f32_n(_p(x), _p(out), x.size)
    return out


def e4m3_to_f32(codes) -> np.ndarray:
    table = np.array([lib().orc_e4m3_to_f32(i) for i in range(256)], np.float32)
    return table[np.asarray(codes, dtype=np.uint8)]


def bf16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_from_f32_n(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f16_from_f32_n(_p(x), _p(out), x.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---- weights --------------------------------------------------------------

def fp8_quantize_rows(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.uint8)
    s = np.empty(n, np.float32)
    lib().orc_fp8_quantize_rows(_p(w), n, k, _p(q), _p(s))
    return q, s


def fp8_dequantize(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    lib().orc_fp8_dequantize(_p(q), _p(s), n, k, _p(out))
    return out


def aq4_quantize(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 128 == 0
    p = np.empty((n, k // 8), np.uint32)
    s = np.empty((n, k // 128), np.uint16)
    z = np.empty((n, k // 128), np.uint16)
    lib().orc_aq4_quantize(_p(w), n, k, _p(p), _p(s), _p(z))
    return p, s, z


def aq4_dequantize(p, s, z) -> np.ndarray:
    p = np.ascontiguousarray(p, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    z = np.ascontiguousarray(z, np.uint16)
    n = p.shape[0]
    k = p.shape[1] * 8
    out = np.empty((n, k), np.float32)
    lib().orc_aq4_dequantize(_p(p), _p(s), _p(z), n, k, _p(out))
    return out


# ---- contractions ---------------------------------------------------------

def fp8_gemv(x_bf16, q, s, alpha=1.0, want64=False, threads=0):
    """x_bf16: uint16 [m][ldx>=k]; returns (y32 [m][n], y64 or None)."""
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    m, ldx = x_bf16.shape
    n, k = q.shape
    y32 = np.empty((m, n), np.float32)
    y64 = np.empty((m, n), np.float64) if want64 else None
    lib().orc_fp8_gemv(m, n, k, _p(x_bf16), ldx, _p(q), _p(s), alpha,
                       _p(y32), _p(y64), threads)
    return y32, y64


def aq4_gemv(x_bf16, p, s, z, alpha=1.0, want64=False, threads=0):
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    p = np.ascontiguousarray(p, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    z = np.ascontiguousarray(z, np.uint16)
    m, ldx = x_bf16.shape
    n = p.shape[0]
    k = p.shape[1] * 8
    y32 = np.empty((m, n), np.float32)
    y64 = np.empty((m, n), np.float64) if want64 else None
    lib().orc_aq4_gemv(m, n, k, _p(x_bf16), ldx, _p(p), _p(s), _p(z), alpha,
                       _p(y32), _p(y64), threads)
    return y32, y64


def act_quantize(x_bf16):
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    m, k = x_bf16.shape
    xq = np.empty((m, k), np.uint8)
    xs = np.empty(m, np.float32)
    lib().orc_act_quantize(m, k, _p(x_bf16), k, _p(xq), _p(xs))
    return xq, xs


def bf16_add(a_bf16, b_bf16):
    """Elementwise bf16 add: the fp32 sum rounded to bf16 (RNE)."""
    a = np.ascontiguousarray(a_bf16, np.uint16)
    b = np.ascontiguousarray(b_bf16, np.uint16)
    assert a.shape == b.shape
    out = np.empty(a.shape, np.uint16)
    lib().orc_bf16_add(a.size, _p(a), _p(b), _p(out))
    return out


def add_act_quantize(a_bf16, b_bf16):
    """Per-token quantization of a + b: returns (codes, scales, sum)."""
    s = bf16_add(a_bf16, b_bf16)
    xq, xs = act_quantize(s)
    return xq, xs, s


def fp8_gemm(xq, xs, q, s, alpha=1.0, want64=False, threads=0):
    xq = np.ascontiguousarray(xq, np.uint8)
    xs = np.ascontiguousarray(xs, np.float32)
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    m, k = xq.shape
    n = q.shape[0]
    y32 = np.empty((m, n), np.float32)
    y64 = np.empty((m, n), np.float64) if want64 else None
    lib().orc_fp8_gemm(m, n, k, _p(xq), _p(xs), _p(q), _p(s), alpha,
                       _p(y32), _p(y64), threads)
    return y32, y64


def silu_mul(gu):
    """SiLU-gate epilogue of an fp32 gate/up product gu [m][2F] -> [m][F]."""
    gu = np.ascontiguousarray(gu, np.float32)
    m, f2 = gu.shape
    assert f2 % 2 == 0
    out = np.empty((m, f2 // 2), np.float32)
    lib().orc_silu_mul(m, f2 // 2, _p(gu), _p(out))
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())

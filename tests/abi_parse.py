"""Small parsers of the C headers (include/ullm/*.h) and of the checked-in Rust
bindings (rust/ullm-hip-sys/src/*.rs), and a repr(C) layout calculator, so
that the CPU tests can compare constants, struct layouts and function
signatures across the two languages without a Rust toolchain.

Types are normalised to a common form:
  scalars      'u8' 'u32' 'i32' 'u64' 'f32' 'char' 'void' 'ullm_status_t' ...
  pointers     ('ptr', 'const'|'mut', <pointee>)
  arrays       ('array', <element>, <length>)
Opaque and named struct types keep their names.
"""
from __future__ import annotations

import re
from pathlib import Path

C_SCALARS = {
    "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "int16_t": "i16",
    "uint32_t": "u32", "int32_t": "i32", "uint64_t": "u64", "int64_t": "i64",
    "float": "f32", "double": "f64", "char": "char", "void": "void",
}
RUST_SCALARS = {"c_char": "char", "c_void": "void"}

SIZES = {"u8": 1, "i8": 1, "char": 1, "u16": 2, "i16": 2, "u32": 4, "i32": 4,
         "f32": 4, "u64": 8, "i64": 8, "f64": 8, "ullm_status_t": 4}


def _strip_c_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _strip_rust_comments(text: str) -> str:
    return re.sub(r"//[^\n]*", " ", text)


# ----------------------------------------------------------------- C side
def c_constants(text: str) -> dict[str, int]:
    out = {}
    text = _strip_c_comments(text)
    for m in re.finditer(r"^\s*#define\s+(ULLM_\w+)\s+(?:UINT\d+_C\()?(0x[0-9a-fA-F]+|\d+)\)?\s*$",
                         text, flags=re.M):
        out[m.group(1)] = int(m.group(2), 0)
    return out


def _c_decl(text: str, consts: dict[str, int]):
    """'const char *const *values' -> (name, type)"""
    text = " ".join(text.split())
    m = re.match(r"^(.*?)(\w+)\s*(?:\[(\w+)\])?$", text)
    assert m, text
    typ, name, arr = m.group(1), m.group(2), m.group(3)
    t = _c_pointer_type(typ)
    if arr is not None:
        n = int(arr) if arr.isdigit() else consts[arr]
        t = ("array", t, n)
    return name, t


def _c_pointer_type(typ: str):
    tokens = re.findall(r"\*|const|[A-Za-z_]\w*", typ)
    base = None
    const = False
    i = 0
    while i < len(tokens) and tokens[i] != "*":
        if tokens[i] == "const":
            const = True
        else:
            base = tokens[i]
        i += 1
    t = C_SCALARS.get(base, base)
    pointee_const = const
    while i < len(tokens):
        assert tokens[i] == "*", typ
        t = ("ptr", "const" if pointee_const else "mut", t)
        i += 1
        pointee_const = False
        if i < len(tokens) and tokens[i] == "const":
            pointee_const = True
            i += 1
    return t


def c_structs(text: str, consts: dict[str, int]) -> dict[str, list]:
    body = _strip_c_comments(text)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", body, flags=re.S):
        name = m.group(3)
        fields = []
        for decl in m.group(2).split(";"):
            if decl.strip():
                fields.append(_c_decl(decl, consts))
        out[name] = fields
    return out


def c_functions(text: str) -> dict[str, tuple]:
    body = _strip_c_comments(text)
    out = {}
    for m in re.finditer(r"ULLM_HIP_API\s+(\w+)\s+(\w+)\s*\((.*?)\)\s*;", body, flags=re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        args = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p and p != "void":
                pname, ptype = _c_decl(p, {})
                if isinstance(ptype, tuple) and ptype[0] == "array":
                    ptype = ("ptr", "mut", ptype[1])  # an array parameter is a pointer
                args.append((pname, ptype))
        out[name] = (C_SCALARS.get(ret, ret), args)
    return out


# -------------------------------------------------------------- Rust side
def _rust_type(t: str):
    t = " ".join(t.split())
    m = re.match(r"^\*(const|mut) (.*)$", t)
    if m:
        return ("ptr", m.group(1), _rust_type(m.group(2)))
    m = re.match(r"^\[(.*); (\w+)\]$", t)
    if m:
        return ("array", _rust_type(m.group(1)), int(m.group(2)))
    return RUST_SCALARS.get(t, t)


def rust_constants(text: str) -> dict[str, int]:
    out = {}
    for m in re.finditer(r"pub const (ULLM_\w+): \w+ = (0x[0-9a-fA-F]+|\d+);", text):
        out[m.group(1)] = int(m.group(2), 0)
    return out


def rust_structs(text: str) -> dict[str, list]:
    body = _strip_rust_comments(text)
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\](?:\s*#\[[^\]]*\])*\s*pub struct (\w+) \{(.*?)\n\}", body, flags=re.S):
        fields = []
        for line in m.group(2).split("\n"):
            fm = re.match(r"\s*(?:pub )?(\w+): (.*?),\s*$", line)
            if fm:
                fields.append((fm.group(1), _rust_type(fm.group(2))))
        out[m.group(1)] = fields
    return out


def rust_functions(text: str) -> dict[str, tuple]:
    body = _strip_rust_comments(text)
    out = {}
    for block in re.findall(r'extern "C" \{(.*?)\n\}', body, flags=re.S):
        for m in re.finditer(r"pub fn (\w+)\((.*?)\)\s*->\s*(\w+);", block, flags=re.S):
            args = []
            for p in m.group(2).split(","):
                p = " ".join(p.split())
                if p:
                    n, t = p.split(": ", 1)
                    args.append((n, _rust_type(t)))
            out[m.group(1)] = (m.group(3), args)
    return out


# ---------------------------------------------------------- repr(C) layout
def size_align(t, structs: dict[str, list]) -> tuple[int, int]:
    if isinstance(t, tuple) and t[0] == "ptr":
        return 8, 8
    if isinstance(t, tuple) and t[0] == "array":
        s, a = size_align(t[1], structs)
        return s * t[2], a
    if t in SIZES:
        return SIZES[t], SIZES[t]
    if t in structs:
        lay = layout(t, structs)
        return lay["size"], lay["align"]
    raise KeyError(t)


def layout(name: str, structs: dict[str, list]) -> dict:
    off = 0
    align = 1
    offsets = []
    for fname, ftype in structs[name]:
        s, a = size_align(ftype, structs)
        off = (off + a - 1) // a * a
        offsets.append((fname, off))
        off += s
        align = max(align, a)
    size = (off + align - 1) // align * align
    return {"size": size, "align": align, "offsets": offsets}


def layout_line(name: str, structs: dict[str, list]) -> str:
    lay = layout(name, structs)
    fields = " ".join(f"{f}={o}" for f, o in lay["offsets"])
    return f"layout {name} size={lay['size']} align={lay['align']} {fields}"


def read(path: Path) -> str:
    return Path(path).read_text()

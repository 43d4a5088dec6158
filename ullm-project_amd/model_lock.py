"""Model-lock checks for the weight files the linear layer loads.

Follows the reference's lock format (reference docs/models/model-lock.md):

* every consumed file is recorded with its path, ``size_bytes`` and
  ``sha256`` ("Required lock contents"), and loading rejects a missing file
  or a content mismatch ("Resolution procedure", step 7);
* the lock fingerprint is ``sha256:<hex>`` of the RFC 8785 (JSON
  Canonicalization Scheme) serialization of ``{"schema_version": ...,
  "model": ...}`` and of nothing else ("Fingerprint").

Safetensors files are verified by the native loader itself
(``ullm_safetensors_open`` with the recorded digest and size), so the bytes
that are checked are the bytes that are then parsed; other files are hashed
here.  The canonicalization implements RFC 8785 for the value types a lock
holds (objects, arrays, strings, integers, booleans, null); a non-integral
number is rejected rather than serialized approximately.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import ullm_hip


def _jcs_string(s: str) -> str:
    # RFC 8785 3.2.2.2: JSON string escaping with the shortest forms, other
    # characters (including non-ASCII) as themselves.
    out = ['"']
    for ch in s:
        o = ord(ch)
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif ch == "\b":
            out.append("\\b")
        elif ch == "\f":
            out.append("\\f")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif o < 0x20:
            out.append(f"\\u{o:04x}")
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def _utf16_key(s: str):
    # RFC 8785 3.2.3: members sorted by their names as UTF-16 code units.
    return s.encode("utf-16-be")


def canonical_json(value) -> str:
    """RFC 8785 serialization of a lock value."""
    if value is None:
        return "null"
    if value is True:
        return "true"
    if value is False:
        return "false"
    if isinstance(value, int):
        if abs(value) > 2 ** 53:
            raise ValueError("integer outside the IEEE-754 double exact range")
        return str(value)
    if isinstance(value, float):
        if value.is_integer() and abs(value) <= 2 ** 53:
            return str(int(value))
        raise ValueError("non-integral numbers are not expected in a model lock")
    if isinstance(value, str):
        return _jcs_string(value)
    if isinstance(value, (list, tuple)):
        return "[" + ",".join(canonical_json(v) for v in value) + "]"
    if isinstance(value, dict):
        for k in value:
            if not isinstance(k, str):
                raise ValueError("object keys must be strings")
        items = sorted(value.items(), key=lambda kv: _utf16_key(kv[0]))
        return "{" + ",".join(_jcs_string(k) + ":" + canonical_json(v)
                              for k, v in items) + "}"
    raise ValueError(f"unsupported JSON value {type(value).__name__}")


def fingerprint(lock: dict) -> str:
    """``sha256:<hex>`` over the JCS form of {schema_version, model}."""
    body = {"schema_version": lock["schema_version"], "model": lock["model"]}
    return "sha256:" + hashlib.sha256(canonical_json(body).encode("utf-8")).hexdigest()


def load_lock(path) -> dict:
    """A lock file as authored: JSON, or YAML read with the safe loader."""
    text = Path(path).read_text(encoding="utf-8")
    if str(path).endswith((".yaml", ".yml")):
        import yaml
        return yaml.safe_load(text)
    return json.loads(text)


class LockError(RuntimeError):
    pass


def _records(lock: dict):
    model = lock["model"]
    for key in ("files", "evidence_files"):
        for rec in model.get(key) or []:
            yield rec


def verify(lock: dict, root, expected_fingerprint: str | None = None):
    """Check every recorded file under ``root`` (size and SHA-256) and,
    when given, the lock's fingerprint.  Returns {path: SafetensorsFile} for
    the safetensors files, opened and verified by the native loader; the
    caller closes them.  Raises LockError on any mismatch or missing file."""
    if expected_fingerprint is not None and fingerprint(lock) != expected_fingerprint:
        raise LockError("lock fingerprint mismatch")
    root = Path(root)
    opened = {}
    try:
        for rec in _records(lock):
            path = root / rec["path"]
            if not path.is_file():
                raise LockError(f"missing locked file {rec['path']}")
            size, digest = int(rec["size_bytes"]), rec["sha256"]
            if rec["path"].endswith(".safetensors"):
                try:
                    opened[rec["path"]] = ullm_hip.SafetensorsFile(path, sha256=digest,
                                                                   size=size)
                except ullm_hip.HipError as e:
                    raise LockError(f"{rec['path']}: {e.message}") from e
                continue
            if path.stat().st_size != size:
                raise LockError(f"{rec['path']}: size mismatch")
            h = hashlib.sha256()
            with open(path, "rb") as f:
                for chunk in iter(lambda: f.read(1 << 20), b""):
                    h.update(chunk)
            if h.hexdigest() != digest:
                raise LockError(f"{rec['path']}: SHA-256 mismatch")
    except Exception:
        for f in opened.values():
            f.close()
        raise
    return opened

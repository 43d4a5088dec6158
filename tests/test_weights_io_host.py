"""Weight files on the CPU: the native safetensors reader/writer of
include/ullm/weights_io.h and the model-lock checks of model_lock.py.

Independent checkers: files written by the ``safetensors`` library (a
separate implementation of the format), Python's ``hashlib`` for SHA-256, and
the RFC 8785 examples for the lock fingerprint's canonical JSON.  No GPU is
needed: opening, validating, hashing and the argument checks of the weight
loader all run before any device is touched.
"""
import ctypes
import hashlib
import json
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file


def _file_sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def _raw_file(path, header, data=b""):
    h = json.dumps(header).encode() if not isinstance(header, bytes) else header
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)
    return path


def test_sha256_matches_hashlib_on_many_lengths(uh, tmp_path):
    rng = np.random.default_rng(1)
    for n in list(range(0, 140)) + [1000, 4096 + 7, 65536 + 13, (1 << 20) + 3]:
        p = tmp_path / f"f{n}.safetensors"
        save_file({"x": torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8))}, str(p))
        with uh.SafetensorsFile(p) as f:
            assert f.sha256() == _file_sha(p), n


def test_sha256_known_answers():
    # FIPS 180-4 examples, through the same code path via a helper file is not
    # possible for arbitrary bytes; hashlib itself is pinned by them here and
    # the native digest is compared with hashlib above.
    assert hashlib.sha256(b"abc").hexdigest() == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert hashlib.sha256(b"").hexdigest() == \
        "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


def test_open_checks_expected_digest_and_size(uh, tmp_path):
    p = tmp_path / "w.safetensors"
    save_file({"w": torch.arange(64, dtype=torch.float32).reshape(8, 8)}, str(p))
    good = _file_sha(p)
    size = p.stat().st_size
    with uh.SafetensorsFile(p, sha256=good, size=size) as f:
        assert f.sha256() == good
    bad = ("0" if good[0] != "0" else "1") + good[1:]
    with pytest.raises(uh.HipError) as e:
        uh.SafetensorsFile(p, sha256=bad)
    assert e.value.status == uh.Status.INVALID_ARGUMENT and "SHA-256" in e.value.message
    with pytest.raises(uh.HipError) as e:
        uh.SafetensorsFile(p, size=size + 1)
    assert "size" in e.value.message


def test_reader_agrees_with_the_safetensors_library(uh, tmp_path):
    tensors = {
        "a.weight": torch.randn(5, 7),
        "b": torch.randn(3, 2, 4).to(torch.float16),
        "c": torch.randn(6, 16).to(torch.bfloat16),
        "d": torch.randn(4, 32).to(torch.float8_e4m3fn),
        "e": torch.arange(12, dtype=torch.int32).reshape(3, 4),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 9),
        "u": torch.arange(10, dtype=torch.uint8),
    }
    p = tmp_path / "m.safetensors"
    save_file(tensors, str(p), metadata={"format": "pt", "note": "héllo \"q\"\n"})
    raw = p.read_bytes()
    hlen = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + hlen])
    with uh.SafetensorsFile(p) as f, safe_open(str(p), "pt") as ref:
        assert f.names() == sorted(ref.keys())
        assert f.metadata("note") == "héllo \"q\"\n"
        assert f.metadata("format") == "pt"
        for name in ref.keys():
            dtype, shape, offset, nbytes = f.info(name)
            t = ref.get_tensor(name)
            assert shape == tuple(t.shape), name
            assert dtype == header[name]["dtype"], name
            b, e = header[name]["data_offsets"]
            assert offset == 8 + hlen + b and nbytes == e - b, name
            assert raw[offset:offset + nbytes] == t.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()
        with pytest.raises(uh.HipError):
            f.info("missing")
        with pytest.raises(uh.HipError):
            f.metadata("missing")


@pytest.mark.parametrize("header,data,what", [
    ({"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 7, "out of range"),
    ({"x": {"dtype": "F33", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 8, "unknown dtype"),
    ({"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8, "does not match"),
    ({"x": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]},
      "y": {"dtype": "U8", "shape": [4], "data_offsets": [2, 6]}}, b"\0" * 8, "overlap"),
    ({"x": {"dtype": "U8", "shape": [4], "data_offsets": [4, 8]}}, b"\0" * 8, "gap"),
    ({"x": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}, b"\0" * 6, "end of the file"),
    ({"x": {"dtype": "U8", "shape": [4.0], "data_offsets": [0, 4]}}, b"\0" * 4, "integers"),
    ({"x": {"dtype": "U8", "shape": [-4], "data_offsets": [0, 4]}}, b"\0" * 4, "shape entry"),
    ({"x": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4], "z": 1}}, b"\0" * 4, "exactly"),
    ({"__metadata__": {"k": 3}}, b"", "not a string"),
    ([1, 2], b"", "start with"),
])
def test_malformed_files_are_rejected(uh, tmp_path, header, data, what):
    p = _raw_file(tmp_path / "bad.safetensors", header, data)
    with pytest.raises(uh.HipError) as e:
        uh.SafetensorsFile(p)
    assert e.value.status == uh.Status.INVALID_ARGUMENT
    assert what in e.value.message, e.value.message


def test_malformed_headers_raw(uh, tmp_path):
    dup = b'{"x":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},' \
          b'"x":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}'
    for hdr, data, what in [
        (dup, b"\0", "duplicate"),
        (b'{"x":', b"", "unexpected end"),
        (b'{"x":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}} x', b"\0", "trailing"),
        (b'{"a\\ud800":1}', b"", "surrogate"),
    ]:
        p = _raw_file(tmp_path / "raw.safetensors", hdr, data)
        with pytest.raises(uh.HipError) as e:
            uh.SafetensorsFile(p)
        assert what in e.value.message, (what, e.value.message)
    # header length beyond the file, a file shorter than 8 bytes
    p = tmp_path / "short.safetensors"
    p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(uh.HipError):
        uh.SafetensorsFile(p)
    p.write_bytes(b"\1\2")
    with pytest.raises(uh.HipError):
        uh.SafetensorsFile(p)
    with pytest.raises(uh.HipError):
        uh.SafetensorsFile(tmp_path / "does-not-exist.safetensors")


def test_handles_and_strings(uh, tmp_path):
    p = tmp_path / "n.safetensors"
    long_name = "layer." + "x" * 400
    save_file({long_name: torch.zeros(2), "b": torch.zeros(1)}, str(p))
    f = uh.SafetensorsFile(p)
    assert f.names() == sorted([long_name, "b"])
    # explicit small buffer: BUFFER_TOO_SMALL with the full length reported
    buf = ctypes.create_string_buffer(8)
    n = ctypes.c_uint64()
    st = uh.lib().ullm_safetensors_tensor_name(f.handle, 1, buf, 8, ctypes.byref(n), None)
    assert st == uh.Status.BUFFER_TOO_SMALL and n.value == len(long_name)
    assert buf.value == long_name[:7].encode()
    h = f.handle
    f.close()
    i = uh.new(uh.StTensorInfo)
    assert uh.lib().ullm_safetensors_tensor_info(h, b"b", ctypes.byref(i), None) == \
        uh.Status.HIP_INVALID_HANDLE
    hv = ctypes.c_void_p(h)
    assert uh.lib().ullm_safetensors_close(ctypes.byref(hv), None) == uh.Status.HIP_INVALID_HANDLE
    d = uh.new(uh.StOpenDesc, path=str(p).encode())
    d.reserved[1] = 1
    out = ctypes.c_void_p()
    assert uh.lib().ullm_safetensors_open(ctypes.byref(d), ctypes.byref(out), None) == \
        uh.Status.RESERVED_NONZERO


def test_weight_load_argument_checks_before_the_device(uh, tmp_path):
    p = tmp_path / "w.safetensors"
    save_file({"w16": torch.randn(16, 128).to(torch.float16),
               "wk": torch.randn(16, 64), "w16k": torch.randn(4, 64).to(torch.float16),
               "q": torch.randn(16, 128).to(torch.float8_e4m3fn),
               "s": torch.ones(16), "s_bad": torch.ones(3),
               "p": torch.zeros(16, 16, dtype=torch.int32)}, str(p))
    with uh.SafetensorsFile(p) as f:
        def load(*a, **k):
            with pytest.raises(uh.HipError) as e:
                uh.load_weight(f, *a, **k)
            return e.value
        assert load("nope", uh.ENCODING_AQ4_G128).status == uh.Status.INVALID_ARGUMENT
        assert "disagree on K" in load(["w16", "w16k"], uh.ENCODING_FP8_E4M3_ROW).message
        assert "dtype" in load(["w16", "wk"], uh.ENCODING_FP8_E4M3_ROW).message
        assert "no scales" in load("w16", uh.ENCODING_FP8_E4M3_ROW, scales="s").message
        assert "shape" in load("q", uh.ENCODING_FP8_E4M3_ROW, scales="s_bad").message
        assert "U32" in load("p", uh.ENCODING_AQ4_G128, scales="s", zeros="s").message
        # valid requests reach the device check: no GPU in this container
        if not uh.backend_probe()[0]:
            assert load("w16", uh.ENCODING_AQ4_G128).status == uh.Status.HIP_UNAVAILABLE
            assert load("q", uh.ENCODING_FP8_E4M3_ROW, scales="s").status == \
                uh.Status.HIP_UNAVAILABLE


# ------------------------------------------------------------- model lock

def test_jcs_rfc8785_examples():
    import model_lock as ml
    # RFC 8785 section 3.2.3: member order by UTF-16 code units (the emoji's
    # surrogates sort before U+FB33 although its code point is larger)
    obj = {"€": "Euro Sign", "\r": "Carriage Return",
           "דּ": "Hebrew Letter Dalet With Dagesh", "1": "One",
           "\U0001F600": "Emoji: Grinning Face", "\u0080": "Control",
           "ö": "Latin Small Letter O With Diaeresis"}
    order = [k for k in json.loads(ml.canonical_json(obj))]
    assert order == ["\r", "1", "\u0080", "ö", "€", "\U0001F600", "דּ"]
    # section 3.2.2.2: shortest escapes, other characters as themselves
    s = "\u20ac$\u000f\u000aA'\u0042\u0022\u005c\\\"/"
    want = '"\u20ac$' + "\\u000f" + "\\n" + "A'B" + '\\"' + "\\\\" * 2 + '\\"' + '/"'
    assert ml.canonical_json(s) == want
    assert ml.canonical_json({"string": s, "literals": [None, True, False]}) == \
        '{"literals":[null,true,false],"string":' + want + "}"
    assert ml.canonical_json({"b": [1, {"z": 0, "a": -3}], "a": {}}) == \
        '{"a":{},"b":[1,{"a":-3,"z":0}]}'
    with pytest.raises(ValueError):
        ml.canonical_json({"x": 0.5})


def _lock(tmp_path, uh):
    (tmp_path / "config.json").write_text('{"hidden_size": 64}')
    save_file({"w": torch.randn(4, 4)}, str(tmp_path / "model.safetensors"))
    files = []
    for name in ("config.json", "model.safetensors"):
        p = tmp_path / name
        files.append({"path": name, "size_bytes": p.stat().st_size,
                      "sha256": _file_sha(p), "git_blob": None, "lfs_oid": None,
                      "source_page_url": None, "download_url": None})
    return {"schema_version": 1, "generated_at": "2026-01-01T00:00:00Z",
            "aliases": ["tiny"],
            "model": {"repo_id": "local/tiny", "repo_type": "model",
                      "requested_revision": "main", "resolved_revision": "0" * 40,
                      "license": {"id": None}, "base_models": [],
                      "evidence_files": [], "files": files, "derivation": None}}


def test_lock_fingerprint_and_verify(uh, tmp_path):
    import model_lock as ml
    lock = _lock(tmp_path, uh)
    fp = ml.fingerprint(lock)
    assert fp.startswith("sha256:") and len(fp) == 71
    # bookkeeping members are outside the fingerprint; key order is irrelevant
    other = json.loads(json.dumps(lock))
    other["generated_at"] = "later"
    other["aliases"] = []
    other["model"] = dict(reversed(list(other["model"].items())))
    assert ml.fingerprint(other) == fp
    other["model"]["files"][0]["size_bytes"] += 1
    assert ml.fingerprint(other) != fp
    opened = ml.verify(lock, tmp_path, expected_fingerprint=fp)
    assert list(opened) == ["model.safetensors"]
    assert opened["model.safetensors"].names() == ["w"]
    for f in opened.values():
        f.close()
    with pytest.raises(ml.LockError):
        ml.verify(lock, tmp_path, expected_fingerprint="sha256:" + "0" * 64)
    # one flipped byte in the weights, then a missing file
    p = tmp_path / "model.safetensors"
    raw = bytearray(p.read_bytes())
    raw[-1] ^= 1
    p.write_bytes(bytes(raw))
    with pytest.raises(ml.LockError) as e:
        ml.verify(lock, tmp_path)
    assert "SHA-256" in str(e.value)
    p.unlink()
    with pytest.raises(ml.LockError):
        ml.verify(lock, tmp_path)
    (tmp_path / "config.json").write_text('{"hidden_size": 65}')
    with pytest.raises(ml.LockError):
        ml.verify({"schema_version": 1, "model": {"files": lock["model"]["files"][:1]}},
                  tmp_path)


def test_lock_yaml_is_read_with_the_safe_loader(tmp_path):
    import model_lock as ml
    p = tmp_path / "lock.yaml"
    p.write_text("schema_version: 1\nmodel:\n  repo_id: a/b\n  files: []\n")
    lock = ml.load_lock(p)
    assert lock["model"]["repo_id"] == "a/b"
    p.write_text("schema_version: !!python/object/apply:os.system ['true']\nmodel: {}\n")
    import yaml
    with pytest.raises(yaml.YAMLError):
        ml.load_lock(p)

"""The C-ABI library on the CPU: it loads without a GPU, exports every entry point include/sdhip.h
declares, and its host-only parts (the pointer head of src/head.rs) match the oracle.  No GPU
compute is called here."""
import ctypes
import json
import os
import re
import struct

import numpy as np
import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "sdhip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(sd_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(sdamd):
    lib = ctypes.CDLL(sdamd.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 14
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert sorted(sdamd.SYMBOLS) == names, "the Python binding and the header disagree"


def test_missing_library_fails_loudly(sdamd, monkeypatch):
    monkeypatch.setattr(sdamd, "LIB_PATH", "/nonexistent/libsdhip.so")
    monkeypatch.setattr(sdamd, "_lib", None)
    with pytest.raises(sdamd.EngineError, match="missing"):
        sdamd.lib()


def test_head_matches_oracle(sdamd, oracle, tiny_model):
    """src/head.rs:55-77 in f64 on the host: product vs oracle on the tiny model's head."""
    with open(os.path.join(tiny_model, "head.safetensors"), "rb") as f:
        raw = f.read()
    head = sdamd.Head.load(raw)
    t = oracle.read_safetensors(os.path.join(tiny_model, "head.safetensors"))
    d = t["norm.weight"].shape[0]
    rng = np.random.default_rng(0)
    for n_opts, temp in [(2, 1.0), (5, 0.3), (3, 0.0)]:
        hidden = rng.standard_normal((n_opts + 1, d)).astype(np.float32)
        got = head.probs(hidden, d, temp)
        want = oracle.head_probs(t, hidden, temp)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)
        assert abs(got.sum() - 1) < 1e-12


def _safetensors(entries, data=b""):
    h = json.dumps(entries).encode()
    return struct.pack("<Q", len(h)) + h + data


def test_head_load_errors(sdamd):
    """The reference's messages (src/head.rs:26-48)."""
    with pytest.raises(sdamd.EngineError, match="malformed"):
        sdamd.Head.load(b"\x01\x02")
    with pytest.raises(sdamd.EngineError, match="malformed"):
        sdamd.Head.load(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(sdamd.EngineError, match="malformed"):
        sdamd.Head.load(_safetensors({"x": {"dtype": "F32"}}))
    with pytest.raises(sdamd.EngineError, match="head tensor x is F16, expected F32"):
        sdamd.Head.load(_safetensors({"x": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4))
    with pytest.raises(sdamd.EngineError, match="head.safetensors: no norm.weight"):
        sdamd.Head.load(_safetensors({"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4))


def test_head_rejects_too_few_rows(sdamd, tiny_model):
    with open(os.path.join(tiny_model, "head.safetensors"), "rb") as f:
        head = sdamd.Head.load(f.read())
    with pytest.raises(sdamd.EngineError, match="at least one option"):
        head.probs(np.zeros((1, 512), np.float32), 512, 1.0)
    with pytest.raises(sdamd.EngineError, match="do not match hidden size"):
        head.probs(np.zeros((3, 256), np.float32), 256, 1.0)


def test_decode_scale_codes_matches_oracle(sdamd, oracle):
    """The engine's load-time decode of 8-bit scale codes (sd_decode_scale_codes, C++, host only)
    against the oracle's restatement of src/model.rs:217-236: bit for bit, over rows with many
    exponents, every code and both signs."""
    rng = np.random.default_rng(21)
    n, g = 300, 64
    head = np.zeros((n, 2), np.uint16)
    head[:, 0] = rng.uniform(1e-4, 8.0, n).astype(np.float16).view(np.uint16)
    head[:, 1] = rng.integers(0, 4096, n)
    head[:4, 1] = [0, 1, 4096, 65535]
    codes = rng.integers(0, 256, (n, g)).astype(np.uint8)
    codes[0] = np.arange(g)
    src = np.concatenate([head.view(np.uint8).reshape(-1), codes.reshape(-1)]).tobytes()
    got = sdamd.decode_scale_codes(src, n, g)
    want = oracle.decode_scale_codes(src, n, g)
    assert np.array_equal(got, want)


def test_decode_scale_codes_checks_lengths(sdamd):
    """sd_decode_scale_codes refuses buffers shorter than n rows of g codes need (and decodes again
    afterwards): a short source would otherwise be read past its end."""
    import ctypes as C
    n, g = 2, 8
    src = np.zeros(n * (4 + g), np.uint8)
    out = np.zeros(n * g, np.uint16)
    L = sdamd.lib()
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)
    with pytest.raises(sdamd.EngineError, match="source bytes"):
        sdamd._call(L.sd_decode_scale_codes, ptr(src), src.size - 1, n, g, ptr(out), out.size)
    with pytest.raises(sdamd.EngineError, match="destination"):
        sdamd._call(L.sd_decode_scale_codes, ptr(src), src.size, n, g, ptr(out), out.size - 1)
    assert sdamd.decode_scale_codes(src.tobytes(), n, g).shape == (n, g)


def test_peak_library_exports_every_declared_symbol(sdamd):
    """libsdpeak.so (the achievable-peak microbenchmarks bench.py reports beside the published
    peaks) loads without a GPU and exports every entry point include/sdpeak.h declares."""
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "sdpeak.h").read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(sd_[a-z_0-9]+)\s*\(", text)))
    assert names == sorted(sdamd.PEAK_SYMBOLS)
    lib = ctypes.CDLL(sdamd.PEAK_LIB_PATH)
    assert all(hasattr(lib, n) for n in names)
    sdamd.peak_lib()

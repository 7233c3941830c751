"""Python host binding of the MI355X engine (libsdhip.so, C ABI in include/sdhip.h).

Mirrors the reference crate's engine API (src/engine.rs): `Engine.load(dir)` (Engine::load,
175-303), `hidden_size` (305-307), `adapter`, `forward(ids, rows, cache, keep, timed)` -> `Output`
(529-662), `profile(ids)` (668-711) and `Snapshot` (81-87); the pointer head `Head` (src/head.rs)
and `ask_ids`, the engine half of `Decider::run` (src/lib.rs:183-199).  It is the same binding a
Rust `engine.rs` shim makes over the C ABI, used here by the tests and bench.py.

There is no fallback: if libsdhip.so is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import math
import threading
import os
from dataclasses import dataclass

import numpy as np

from . import model as _model

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsdhip.so")
CONTEXT = 4096

SYMBOLS = [
    "sd_engine_load", "sd_engine_free", "sd_engine_hidden_size", "sd_engine_adapter", "sd_engine_forward",
    "sd_snapshot_len", "sd_snapshot_free", "sd_engine_profile", "sd_head_load", "sd_head_free", "sd_head_probs",
    "sd_ask_ids", "sd_op_matmul", "sd_op_gdn", "sd_engine_forward_batch", "sd_engine_ask_batch",
    "sd_op_repack_w4", "sd_decode_scale_codes", "sd_op_matmul_fmt", "sd_op_matmul_split", "sd_op_gate_up_silu",
    "sd_op_embed", "sd_op_add_norm", "sd_op_silu_mul", "sd_op_add_bias", "sd_op_conv", "sd_op_gnorm",
    "sd_op_attention", "sd_engine_trace", "sd_op_matmul_noalloc",
]
VOID_SYMBOLS = ("sd_engine_free", "sd_snapshot_free", "sd_head_free", "sd_engine_hidden_size", "sd_engine_adapter",
                "sd_snapshot_len")


class EngineError(RuntimeError):
    """The reference's `crate::Error` (src/lib.rs:23-30)."""


class sd_config(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_size_t), ("intermediate_size", C.c_size_t), ("n_layers", C.c_size_t),
        ("layer_types", C.POINTER(C.c_uint8)),
        ("num_attention_heads", C.c_size_t), ("num_key_value_heads", C.c_size_t), ("head_dim", C.c_size_t),
        ("rotary_dim", C.c_size_t), ("linear_num_key_heads", C.c_size_t), ("linear_key_head_dim", C.c_size_t),
        ("linear_value_head_dim", C.c_size_t), ("rope_theta", C.c_double), ("unrotate", C.POINTER(C.c_double)),
    ]


class sd_tensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p), ("offset", C.c_uint64), ("bytes", C.c_uint64), ("N", C.c_uint32), ("K", C.c_uint32),
        ("bits", C.c_uint32), ("group", C.c_uint32), ("asym", C.c_uint32), ("had", C.c_int32),
    ]


class sd_embed(C.Structure):
    _fields_ = [
        ("rows_path", C.c_char_p), ("vocab", C.c_uint64), ("row_bytes", C.c_uint64), ("n_parts", C.c_size_t),
        ("part_names", C.POINTER(C.c_char_p)), ("part_bytes", C.POINTER(C.c_uint64)),
        ("wire_row_bytes", C.c_uint64), ("u8", C.c_int32),
    ]


_lib = None


def lib():
    """The loaded libsdhip.so; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EngineError(f"{LIB_PATH} is missing: build it with `make -C strands-decider-rs_amd` "
                              "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        vp, sz, i32, err = C.c_void_p, C.c_size_t, C.c_int, C.c_char_p
        L.sd_engine_load.argtypes = [C.POINTER(sd_config), C.POINTER(sd_tensor), sz, C.POINTER(C.c_char_p),
                                     C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), sz, C.POINTER(sd_embed),
                                     C.POINTER(vp), err, sz]
        L.sd_engine_free.argtypes = [vp]
        L.sd_engine_hidden_size.argtypes = [vp]
        L.sd_engine_hidden_size.restype = sz
        L.sd_engine_adapter.argtypes = [vp]
        L.sd_engine_adapter.restype = C.c_char_p
        L.sd_engine_forward.argtypes = [vp, vp, sz, vp, sz, vp, i32, i32, vp, C.POINTER(C.c_double), C.POINTER(vp),
                                        err, sz]
        L.sd_engine_forward_batch.argtypes = [vp, vp, vp, sz, vp, sz, vp, i32, vp, C.POINTER(C.c_double), err, sz]
        L.sd_engine_ask_batch.argtypes = [vp, vp, vp, sz, C.POINTER(vp), vp, C.POINTER(vp), vp, vp, i32, vp,
                                          C.POINTER(C.c_double), err, sz]
        L.sd_snapshot_len.argtypes = [vp]
        L.sd_snapshot_len.restype = sz
        L.sd_snapshot_free.argtypes = [vp]
        L.sd_engine_profile.argtypes = [vp, vp, sz, C.POINTER(C.c_char_p), C.POINTER(C.c_double), sz,
                                        C.POINTER(sz), err, sz]
        L.sd_head_load.argtypes = [vp, sz, C.POINTER(vp), err, sz]
        L.sd_head_free.argtypes = [vp]
        L.sd_head_probs.argtypes = [vp, vp, sz, sz, C.c_double, vp, err, sz]
        L.sd_ask_ids.argtypes = [vp, vp, vp, sz, sz, C.POINTER(vp), vp, C.POINTER(vp), vp, vp, vp, err, sz]
        L.sd_op_matmul.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, err, sz]
        L.sd_op_repack_w4.argtypes = [vp, vp, i32, i32, vp, err, sz]
        L.sd_op_gdn.argtypes = [vp, vp, i32, i32, i32, vp, vp, i32, i32, i32, i32, vp, i32, vp, vp, err, sz]
        L.sd_decode_scale_codes.argtypes = [vp, sz, sz, sz, vp, sz, err, sz]
        L.sd_op_matmul_fmt.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, err, sz]
        L.sd_op_matmul_split.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, err, sz]
        L.sd_op_gate_up_silu.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, err, sz]
        L.sd_op_embed.argtypes = [vp, i32, vp, vp, vp, i32, i32, i32, i32, vp, vp, err, sz]
        L.sd_op_add_norm.argtypes = [vp, vp, vp, i32, vp, i32, vp, vp, vp, err, sz]
        L.sd_op_silu_mul.argtypes = [vp, i32, i32, vp, vp, err, sz]
        L.sd_op_add_bias.argtypes = [vp, i32, i32, vp, vp, err, sz]
        L.sd_op_conv.argtypes = [vp, i32, i32, i32, vp, vp, vp, vp, err, sz]
        L.sd_op_gnorm.argtypes = [vp, vp, i32, i32, vp, i32, i32, i32, vp, vp, err, sz]
        L.sd_op_attention.argtypes = [vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, i32, vp, vp, err, sz]
        L.sd_engine_trace.argtypes = [vp, vp, sz, vp, vp, sz, vp, vp, sz, C.POINTER(sz), err, sz]
        L.sd_op_matmul_noalloc.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, vp, err, sz]
        for name in SYMBOLS:
            if name not in VOID_SYMBOLS:
                getattr(L, name).restype = i32
        _lib = L
    return _lib


_tls = threading.local()


def _call(fn, *args):
    # one error buffer per thread, reused (a call's message is read before the thread's next call)
    buf = getattr(_tls, "err", None)
    if buf is None:
        buf = _tls.err = C.create_string_buffer(1024)
    rc = fn(*args, buf, 1024)
    if rc != 0:
        raise EngineError(buf.value.decode(errors="replace"))


def _ptr(a):
    # the address as an int: the c_void_p argument types take it as it is (data_as builds a
    # ctypes object per call)
    return None if a is None else a.ctypes.data


class Snapshot:
    """The torso state after a prefix (src/engine.rs:81-87); continue with Engine.forward(cache=)."""

    def __init__(self, handle, engine):
        self._h, self._engine = handle, engine

    @property
    def len(self) -> int:
        return lib().sd_snapshot_len(self._h)

    def free(self):
        if self._h:
            lib().sd_snapshot_free(self._h)
            self._h = None

    def __del__(self):
        # A snapshot must be freed before its engine; the engine keeps a reference to live ones.
        try:
            self.free()
        except Exception:
            pass


@dataclass
class Output:
    """src/engine.rs:89-96."""
    hidden: np.ndarray  # [len(rows), d] f32
    d: int
    gpu_ms: float | None
    snapshot: Snapshot | None


class Engine:
    def __init__(self, handle, manifest):
        self._h = handle
        self.manifest = manifest
        self._snaps = []

    @staticmethod
    def load(model_dir: str, manifest: _model.Manifest | None = None) -> "Engine":
        """src/engine.rs:175-303: read the manifest, upload shards and the embedding."""
        m = manifest or _model.read_manifest(model_dir)
        c = m.config
        kinds = []
        for k in c.layer_types:
            if k not in _model.LAYER_KIND:
                raise EngineError(f"unsupported layer type {k}")
            kinds.append(_model.LAYER_KIND[k])
        lt = (C.c_uint8 * len(kinds))(*kinds)
        unrot = (C.c_double * len(c.unrotate))(*c.unrotate) if c.unrotate else None
        cfg = sd_config(c.hidden_size, c.intermediate_size, len(kinds), lt, c.num_attention_heads,
                        c.num_key_value_heads, c.head_dim, c.rotary_dim, c.linear_num_key_heads,
                        c.linear_key_head_dim, c.linear_value_head_dim, c.rope_theta, unrot)
        names = list(m.tensors)
        ts = (sd_tensor * len(names))()
        keep = []
        for i, n in enumerate(names):
            t = m.tensors[n]
            b = n.encode()
            keep.append(b)
            ts[i] = sd_tensor(b, t.offset, t.bytes, t.N, t.K, t.bits, t.group, int(t.asym),
                              -1 if t.had is None else int(t.had))
        for s in m.shards:
            if s.wire is not None:
                raise EngineError(f"{s.path}: packed (wire) shards are a download format; convert them first")
        paths = [os.path.join(model_dir, _model.shard_file(i)).encode() for i in range(len(m.shards))]
        cpaths = (C.c_char_p * len(paths))(*paths)
        starts = (C.c_uint64 * len(m.shards))(*[s.start for s in m.shards])
        sizes = (C.c_uint64 * len(m.shards))(*[s.bytes for s in m.shards])
        e = m.embed
        if e is None:
            raise EngineError("manifest has no embedding")
        pn = [p[0].encode() for p in e.parts]
        emb = sd_embed(os.path.join(model_dir, e.rows).encode(), e.vocab, e.row_bytes, len(pn),
                       (C.c_char_p * len(pn))(*pn), (C.c_uint64 * len(pn))(*[p[1] for p in e.parts]),
                       e.wire_row_bytes or 0, int(bool(e.u8)))
        h = C.c_void_p()
        _call(lib().sd_engine_load, C.byref(cfg), ts, len(names), cpaths, starts, sizes, len(m.shards),
              C.byref(emb), C.byref(h))
        return Engine(h, m)

    def hidden_size(self) -> int:
        return lib().sd_engine_hidden_size(self._h)

    @property
    def adapter(self) -> str:
        return lib().sd_engine_adapter(self._h).decode()

    def forward(self, ids, rows, cache: Snapshot | None = None, keep: bool = False, timed: bool = False) -> Output:
        """src/engine.rs:529-662."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        rows_a = np.ascontiguousarray(rows, dtype=np.uintp)
        d = self.hidden_size()
        hidden = np.empty((len(rows_a), d), np.float32)
        ms = C.c_double(math.nan)
        snap = C.c_void_p()
        _call(lib().sd_engine_forward, self._h, _ptr(ids), len(ids), _ptr(rows_a), len(rows_a),
              cache._h if cache is not None else None, int(keep), int(timed), _ptr(hidden), C.byref(ms),
              C.byref(snap) if keep else None)
        s = None
        if keep:
            s = Snapshot(snap, self)
            self._snaps.append(s)
        return Output(hidden, d, ms.value if timed else None, s)

    def forward_batch(self, seqs, rows, cache: Snapshot | None = None, timed: bool = False):
        """Several independent sequences in one forward, each continuing from `cache` as its own
        forward would (no counterpart in the reference's Engine; it replaces the per-question
        forwards of Decider::ask_all, src/lib.rs:192-198).  rows[q] indexes sequence q.
        Returns ([hidden rows of sequence q], gpu_ms)."""
        seqs = [np.ascontiguousarray(q, dtype=np.uint32) for q in seqs]
        ids = np.ascontiguousarray(np.concatenate(seqs) if seqs else np.zeros(0, np.uint32), dtype=np.uint32)
        lens = np.array([len(q) for q in seqs], dtype=np.uintp)
        flat, base, spans = [], 0, []
        for q, r in zip(seqs, rows):
            spans.append((len(flat), len(r)))
            flat.extend(base + int(i) for i in r)
            base += len(q)
        rows_a = np.ascontiguousarray(flat, dtype=np.uintp)
        d = self.hidden_size()
        hidden = np.empty((len(rows_a), d), np.float32)
        ms = C.c_double(math.nan)
        _call(lib().sd_engine_forward_batch, self._h, _ptr(ids), _ptr(lens), len(lens), _ptr(rows_a), len(rows_a),
              cache._h if cache is not None else None, int(timed), _ptr(hidden), C.byref(ms))
        return [hidden[a:a + n] for a, n in spans], (ms.value if timed else None)

    def ask_batch(self, head: "Head", questions, options, temperatures, cache: Snapshot | None = None,
                  timed: bool = False):
        """The question half of Decider::ask_all (src/lib.rs:192-198) with the pointer head on the
        device: question i continues from `cache`; options[i] index its option rows (its last token
        is the answer row).  Returns ([option probabilities of question i], gpu_ms)."""
        qs = [np.ascontiguousarray(q, dtype=np.uint32) for q in questions]
        ops = [np.ascontiguousarray(o, dtype=np.uintp) for o in options]
        nq = len(qs)
        qptr = (C.c_void_p * nq)(*[q.ctypes.data for q in qs])
        qlen = np.array([len(q) for q in qs], np.uintp)
        optr = (C.c_void_p * nq)(*[o.ctypes.data for o in ops])
        nopt = np.array([len(o) for o in ops], np.uintp)
        temps = np.ascontiguousarray(temperatures, dtype=np.float64)
        out = np.empty(int(nopt.sum()), np.float64)
        ms = C.c_double(math.nan)
        _call(lib().sd_engine_ask_batch, self._h, head._h, cache._h if cache is not None else None, nq, qptr,
              _ptr(qlen), optr, _ptr(nopt), _ptr(temps), int(timed), _ptr(out), C.byref(ms))
        res, o = [], 0
        for n in nopt:
            res.append(out[o:o + n])
            o += n
        return res, (ms.value if timed else None)

    def profile(self, ids):
        """src/engine.rs:668-711: [(label, ms)], slowest first."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        cap = 64
        labels = (C.c_char_p * cap)()
        ms = (C.c_double * cap)()
        n = C.c_size_t()
        _call(lib().sd_engine_profile, self._h, _ptr(ids), len(ids), labels, ms, cap, C.byref(n))
        return [(labels[i].decode(), ms[i]) for i in range(min(n.value, cap))]

    def trace(self, ids, rows, cache: Snapshot | None = None, cap: int = 256):
        """Per-layer activations (a test hook, no counterpart in the reference): after every residual
        add + RMSNorm of the layers, the residual x [len(rows), d] f32 and the normalized h (f16) of
        the given rows.  Returns [(x, h)] in plan order."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        rows_a = np.ascontiguousarray(rows, dtype=np.uintp)
        d = self.hidden_size()
        x = np.empty((cap, len(rows_a), d), np.float32)
        h = np.empty((cap, len(rows_a), d), np.uint16)
        n = C.c_size_t()
        _call(lib().sd_engine_trace, self._h, _ptr(ids), len(ids), cache._h if cache is not None else None,
              _ptr(rows_a), len(rows_a), _ptr(x), _ptr(h), cap, C.byref(n))
        k = min(n.value, cap)
        return [(x[i], h[i].view(np.float16).astype(np.float32)) for i in range(k)]

    def free(self):
        if self._h:
            for s in self._snaps:
                s.free()
            self._snaps = []
            lib().sd_engine_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Head:
    """src/head.rs: the pointer head, CPU f64."""

    def __init__(self, handle):
        self._h = handle

    @staticmethod
    def load(data: bytes) -> "Head":
        h = C.c_void_p()
        buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
        _call(lib().sd_head_load, buf, len(data), C.byref(h))
        return Head(h)

    def probs(self, hidden: np.ndarray, d: int, temperature: float) -> np.ndarray:
        hidden = np.ascontiguousarray(hidden, dtype=np.float32)
        n = hidden.size // d
        out = np.empty(n - 1, np.float64)
        _call(lib().sd_head_probs, self._h, _ptr(hidden), n, d, float(temperature), _ptr(out))
        return out

    def __del__(self):
        try:
            if self._h:
                lib().sd_head_free(self._h)
                self._h = None
        except Exception:
            pass


def ask_ids(engine: Engine, head: Head, state, questions, options, temperatures):
    """The engine half of Decider::run (src/lib.rs:183-199) over token ids: one list of option
    probabilities per question."""
    st = np.ascontiguousarray(state, dtype=np.uint32)
    qs = [np.ascontiguousarray(q, dtype=np.uint32) for q in questions]
    ops = [np.ascontiguousarray(o, dtype=np.uintp) for o in options]
    nq = len(qs)
    qptr = (C.c_void_p * nq)(*[q.ctypes.data for q in qs])
    qlen = np.array([len(q) for q in qs], np.uintp)
    optr = (C.c_void_p * nq)(*[o.ctypes.data for o in ops])
    nopt = np.array([len(o) for o in ops], np.uintp)
    temps = np.ascontiguousarray(temperatures, dtype=np.float64)
    out = np.empty(int(nopt.sum()), np.float64)
    _call(lib().sd_ask_ids, engine._h, head._h, _ptr(st), len(st), nq, qptr, _ptr(qlen), optr, _ptr(nopt),
          _ptr(temps), _ptr(out))
    res, o = [], 0
    for n in nopt:
        res.append(out[o:o + n])
        o += n
    return res


def load_decider(model_dir: str):
    """Engine + Head + decider settings of a model directory (the engine half of Decider::load,
    src/lib.rs:120-134; tokenizer and prompt rendering stay with the caller)."""
    import json
    eng = Engine.load(model_dir)
    with open(os.path.join(model_dir, "head.safetensors"), "rb") as f:
        head = Head.load(f.read())
    with open(os.path.join(model_dir, "hobson_config.json")) as f:
        cfg = json.load(f)
    return eng, head, cfg


# ---- kernel-level entry points (device pointers as ints; stream handle as int or None) ----------

def op_matmul(A, Wq, Sc, Y, M, N, K, exact=False, cfg=-1, packed=False, stream=None):
    """sd_op_matmul on device pointers; packed: Wq and Sc already went through op_repack_w4."""
    _call(lib().sd_op_matmul, C.c_void_p(A), C.c_void_p(Wq), C.c_void_p(Sc), C.c_void_p(Y), M, N, K, int(exact), cfg,
          int(packed), C.c_void_p(stream) if stream else None)


def op_repack_w4(Wq, Sc, N, K, stream=None):
    """sd_op_repack_w4: rewrites an N x K matrix's words and scales in place into what the GEMM
    kernels read (the engine nibble order, and 32-column x 64-k tiles where the shape allows)."""
    _call(lib().sd_op_repack_w4, C.c_void_p(Wq), C.c_void_p(Sc), N, K, C.c_void_p(stream) if stream else None)


def op_gdn(qkv, big, stride, a_off, b_off, negA, dtb, L, H, dk, dv, state, load_state, o, stream=None):
    _call(lib().sd_op_gdn, C.c_void_p(qkv), C.c_void_p(big), stride, a_off, b_off, C.c_void_p(negA), C.c_void_p(dtb),
          L, H, dk, dv, C.c_void_p(state), int(load_state), C.c_void_p(o), C.c_void_p(stream) if stream else None)


def decode_scale_codes(src: bytes, n: int, g: int) -> np.ndarray:
    """sd_decode_scale_codes (src/model.rs:217-236): n rows of g 8-bit scale codes -> f16 bits [n, g]."""
    buf = np.frombuffer(bytes(src), np.uint8).copy()
    out = np.empty((n, g), np.uint16)
    _call(lib().sd_decode_scale_codes, _ptr(buf), buf.size, n, g, _ptr(out), out.size)
    return out


def _sp(stream):
    return C.c_void_p(stream) if stream else None


def op_matmul_fmt(A, Wq, Sc, Bi, Y, M, N, K, bits, group, asym, stream=None):
    """sd_op_matmul_fmt: the reference GEMV for any weight format (model layout, f32 dequant)."""
    _call(lib().sd_op_matmul_fmt, C.c_void_p(A), C.c_void_p(Wq), C.c_void_p(Sc), C.c_void_p(Bi) if Bi else None,
          C.c_void_p(Y), M, N, K, bits, group, int(asym), _sp(stream))


def op_matmul_split(A, Wq, Sc, part, M, N, K, exact, cfg, ks, packed=False, stream=None):
    _call(lib().sd_op_matmul_split, C.c_void_p(A), C.c_void_p(Wq), C.c_void_p(Sc), C.c_void_p(part), M, N, K,
          int(exact), cfg, ks, int(packed), _sp(stream))


def op_gate_up_silu(A, Wq, Sc, mid, M, N, K, exact, cfg=-1, stream=None):
    _call(lib().sd_op_gate_up_silu, C.c_void_p(A), C.c_void_p(Wq), C.c_void_p(Sc), C.c_void_p(mid), M, N, K,
          int(exact), cfg, _sp(stream))


def op_embed(ids, L, Q, S, Bi, d, bits, group, asym, x, stream=None):
    _call(lib().sd_op_embed, C.c_void_p(ids), L, C.c_void_p(Q), C.c_void_p(S), C.c_void_p(Bi) if Bi else None, d, bits,
          group, int(asym), C.c_void_p(x), _sp(stream))


def op_add_norm(x, y, w, d, rows, nrows, h16=None, h32=None, stream=None):
    _call(lib().sd_op_add_norm, C.c_void_p(x), C.c_void_p(y) if y else None, C.c_void_p(w), d,
          C.c_void_p(rows) if rows else None, nrows, C.c_void_p(h16) if h16 else None, C.c_void_p(h32) if h32 else None,
          _sp(stream))


def op_silu_mul(big, L, I_, mid, stream=None):
    _call(lib().sd_op_silu_mul, C.c_void_p(big), L, I_, C.c_void_p(mid), _sp(stream))


def op_add_bias(y, L, N, c, stream=None):
    _call(lib().sd_op_add_bias, C.c_void_p(y), L, N, C.c_void_p(c), _sp(stream))


def op_conv(big, stride, L, Cn, w, hist, out, stream=None):
    _call(lib().sd_op_conv, C.c_void_p(big), stride, L, Cn, C.c_void_p(w), C.c_void_p(hist), C.c_void_p(out), _sp(stream))


def op_gnorm(o, big, stride, z_off, w, L, H, DV, out, stream=None):
    _call(lib().sd_op_gnorm, C.c_void_p(o), C.c_void_p(big), stride, z_off, C.c_void_p(w), L, H, DV, C.c_void_p(out),
          _sp(stream))


def op_attention(big, stride, qw, kw, rope, L, P, HQ, HK, HD, RD, Q, Kc, Vt, ctx, out, stream=None):
    _call(lib().sd_op_attention, C.c_void_p(big), stride, C.c_void_p(qw), C.c_void_p(kw), C.c_void_p(rope), L, P, HQ, HK,
          HD, RD, C.c_void_p(Q), C.c_void_p(Kc), C.c_void_p(Vt), ctx, C.c_void_p(out), _sp(stream))


def op_matmul_noalloc(A, Wq, Sc, Y, M, N, K, exact=False, stream=None):
    """sd_op_matmul_noalloc: sd_op_matmul (engine plan, pre-packed weights) with no device allocation."""
    _call(lib().sd_op_matmul_noalloc, C.c_void_p(A), C.c_void_p(Wq), C.c_void_p(Sc), C.c_void_p(Y), M, N, K,
          int(exact), _sp(stream))


# ---- achievable-peak microbenchmarks (libsdpeak.so, include/sdpeak.h; used by bench.py) ----------

PEAK_LIB_PATH = os.path.join(HERE, "libsdpeak.so")
PEAK_SYMBOLS = ["sd_peak_mfma", "sd_peak_hbm"]
_peak = None


def peak_lib():
    """The loaded libsdpeak.so; raises if it is not built."""
    global _peak
    if _peak is None:
        if not os.path.exists(PEAK_LIB_PATH):
            raise EngineError(f"{PEAK_LIB_PATH} is missing: build it with `make -C strands-decider-rs_amd`")
        L = C.CDLL(PEAK_LIB_PATH)
        vp, sz, i32, err = C.c_void_p, C.c_size_t, C.c_int, C.c_char_p
        L.sd_peak_mfma.argtypes = [i32, i32, i32, i32, vp, vp, err, sz]
        L.sd_peak_hbm.argtypes = [i32, sz, i32, vp, vp, err, sz]
        for name in PEAK_SYMBOLS:
            getattr(L, name).restype = i32
        _peak = L
    return _peak


def peak_mfma(variant: int, wg_per_cu: int, iters: int, launches: int, stream=None) -> dict:
    """sd_peak_mfma: 0 MFMA alone, 1 the (2,1) GEMM loop mix, 2 the (4,1) mix; 3, 4, 5 the same on
    random operands (include/sdpeak.h)."""
    out = np.zeros(4, np.float64)
    _call(peak_lib().sd_peak_mfma, variant, wg_per_cu, iters, launches, _sp(stream), _ptr(out))
    return {"ms": float(out[0]), "tflops": float(out[1]), "clock_ghz": float(out[2]), "cus": int(out[3])}


def peak_hbm(variant: int, nbytes: int, launches: int, stream=None) -> dict:
    """sd_peak_hbm: 0 streaming read, 1 copy (read + write counted) over nbytes."""
    out = np.zeros(4, np.float64)
    _call(peak_lib().sd_peak_hbm, variant, nbytes, launches, _sp(stream), _ptr(out))
    return {"ms": float(out[0]), "gbps": float(out[1]), "clock_ghz": float(out[2]), "cus": int(out[3])}

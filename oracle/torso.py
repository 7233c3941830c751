"""CPU oracle of the whole torso forward, with prefix snapshots.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (or the timed CPU baseline).  The product never imports it.

It composes the C restatements in oracle.c exactly as the reference's plan wires the kernels
(src/engine.rs:396-524), with the reference's buffer precisions (x f32, h/y/big/mid/o f16, qkvc
and GDN output f32), the matmul tile table that decides f16 vs f32 dequantization
(src/engine.rs:414-444: M <= 20 or a non-default format or N % 64 != 0 -> GEMV with f32 dequant,
else the tiled kernel with f16 dequant), the restore/snapshot semantics of `forward`
(src/engine.rs:529-662) and the pointer head (src/head.rs:55-77).  It reads the model directory
on its own (plain JSON + numpy) so that it shares no loader code with the product.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CONTEXT = 4096  # src/engine.rs:16

_lib = None


def lib():
    """The compiled oracle (oracle/liboracle.so, built by oracle/Makefile)."""
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run `make -C oracle`")
        _lib = ctypes.CDLL(path)
    return _lib


def P(a):
    """Pointer to a numpy array's data (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


I = ctypes.c_int


# ---- thin wrappers over oracle.c ------------------------------------------------------------

def f2h(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f2h_n(P(x), P(out), ctypes.c_int64(x.size))
    return out


def h2f(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_h2f_n(P(h), P(out), ctypes.c_int64(h.size))
    return out


def matmul(A16, Wq, Sc, N, K, f16_deq, bits=4, group=32, asym=False, Bi=None):
    """Y[M,N] f16 bits = A[M,K] (f16 bits) . deq(W)^T (src/kernels.rs:590-709)."""
    A16 = np.ascontiguousarray(A16, dtype=np.uint16)
    M = A16.size // K
    Y = np.empty((M, N), np.uint16)
    lib().or_matmul(P(A16), P(np.ascontiguousarray(Wq)), P(np.ascontiguousarray(Sc)), P(Bi), I(M), I(N), I(K),
                    I(bits), I(group), I(int(asym)), I(int(f16_deq)), P(Y))
    return Y


def dequant(Wq, Sc, N, K, f16_deq, bits=4, group=32, asym=False, Bi=None):
    """deq(W)[N,K] as f32: the tiled kernel's f16 dequant or the GEMV's f32 dequant."""
    out = np.empty((N, K), np.float32)
    lib().or_dequant(P(np.ascontiguousarray(Wq)), P(np.ascontiguousarray(Sc)), P(Bi), I(N), I(K), I(bits), I(group),
                     I(int(asym)), I(int(f16_deq)), P(out))
    return out


def add_norm(x, y16, w, rows=None, out_f32=False):
    """x += y (if y16 is not None), then RMSNorm of the given rows (src/kernels.rs:93-120)."""
    L, d = x.shape
    rows = np.arange(L, dtype=np.uint32) if rows is None else np.ascontiguousarray(rows, dtype=np.uint32)
    if out_f32:
        out = np.empty((len(rows), d), np.float32)
        lib().or_add_norm(P(x), P(y16), P(w), I(d), P(rows), I(len(rows)), None, P(out))
    else:
        out = np.empty((len(rows), d), np.uint16)
        lib().or_add_norm(P(x), P(y16), P(w), I(d), P(rows), I(len(rows)), P(out), None)
    return out


def embed(ids, Q, S, d, bits=4, group=32, asym=False, Bi=None):
    """x[L, d] f32 = the dequantized table rows ids (src/kernels.rs:63-89)."""
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    x = np.empty((len(ids), d), np.float32)
    lib().or_embed(P(ids), I(len(ids)), P(np.ascontiguousarray(Q, dtype=np.uint32)),
                   P(np.ascontiguousarray(S, dtype=np.uint16)),
                   P(None if Bi is None else np.ascontiguousarray(Bi, dtype=np.uint16)), I(d), I(bits), I(group),
                   I(int(asym)), P(x))
    return x


def add_bias(y16, c):
    """y[t, j] = f16(f32(y) + c[j]) on f16 bits (src/kernels.rs:138-149)."""
    y = np.ascontiguousarray(y16, dtype=np.uint16).copy()
    L, N = y.shape
    lib().or_add_bias(P(y), I(L), I(N), P(np.ascontiguousarray(c, dtype=np.float32)))
    return y


def decode_scale_codes(src, n, g):
    """8-bit scale codes -> f16 bits [n, g] (src/model.rs:217-236): each of the n rows has a 4-byte
    header (m as f16 bits, j as u16, little-endian), then the n*g codes follow, sign << 7 | k each;
    |scale| = f16(f32(m * 2^(-k j / 4096))) with the power and product in f64, and the code's sign
    bit becomes the f16 sign bit."""
    src = np.frombuffer(bytes(src), np.uint8)
    return decode_scale_rows(src[:4 * n].reshape(n, 4), src[4 * n:4 * n + n * g].reshape(n, g))


def decode_scale_rows(head, codes):
    """decode_scale_codes with the headers [n, 4] and codes [n, g] (u8) given apart."""
    h = np.ascontiguousarray(head, dtype=np.uint8).view(np.uint16).reshape(-1, 2)
    c = np.asarray(codes, dtype=np.uint16)
    m = h[:, 0].view(np.float16).astype(np.float64)[:, None]
    j = h[:, 1].astype(np.float64)[:, None]
    k = (c & 127).astype(np.float64)
    mag = (m * np.power(2.0, -(k * j) / 4096.0)).astype(np.float32).astype(np.float16).view(np.uint16)
    return mag | ((c & 128) << 8).astype(np.uint16)


def rope_table(rd, theta, ctx=CONTEXT):
    t = np.empty((ctx, rd), np.float32)
    lib().or_rope_table(I(ctx), I(rd), ctypes.c_double(theta), P(t))
    return t


def fwht(x):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().or_fwht(P(x), I(x.size))
    return x


# ---- model ------------------------------------------------------------------------------------

class Snapshot:
    """The prefix state after a forward (src/engine.rs:81-87): GDN state and conv history per
    linear layer, compact K/V rows [hk][len][hd] per attention layer."""

    def __init__(self, length, state, hist, k, v):
        self.len, self.state, self.hist, self.k, self.v = length, state, hist, k, v


class OracleModel:
    def __init__(self, model_dir):
        with open(os.path.join(model_dir, "manifest.json")) as f:
            m = json.load(f)
        self.cfg = c = m["config"]
        self.tensors = m["tensors"]
        self.shards = []
        for i, s in enumerate(m["shards"]):
            data = np.fromfile(os.path.join(model_dir, f"weights.{i}.bin"), dtype=np.uint8)
            self.shards.append((s["start"], s["bytes"], data))
        e = m["embed"]
        # embedding rows in token-id order, parts back to back; with `u8` the row stores the scale
        # part as 8-bit codes (4-byte header + one code per scale) and is wire_row_bytes long
        # (src/model.rs:260-283)
        u8 = bool(e.get("u8", False))
        rb = e.get("wire_row_bytes") or e["row_bytes"]
        rows = np.fromfile(os.path.join(model_dir, e["rows"]), dtype=np.uint8).reshape(e["vocab"], rb)
        self.embed, off = {}, 0
        for name, b in e["parts"]:
            if u8 and name == "embed.s":
                g = b // 2
                part = decode_scale_rows(rows[:, off:off + 4], rows[:, off + 4:off + 4 + g])
                self.embed[name] = np.ascontiguousarray(part).view(np.uint8).reshape(-1)
                off += 4 + g
            else:
                self.embed[name] = np.ascontiguousarray(rows[:, off:off + b]).reshape(-1)
                off += b
        self.d = c["hidden_size"]
        self.I = c["intermediate_size"]
        self.H, self.DK, self.DV = c["linear_num_key_heads"], c["linear_key_head_dim"], c["linear_value_head_dim"]
        self.HQ, self.HK, self.HD = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        self.RD = c["rotary_dim"]
        self.kinds = c["layer_types"]
        self.linear = [i for i, k in enumerate(self.kinds) if k == "linear_attention"]
        self.full = [i for i, k in enumerate(self.kinds) if k == "full_attention"]
        self.rope = rope_table(self.RD, c["rope_theta"])
        self.C = 2 * self.H * self.DK + self.H * self.DV
        self.state = {i: np.zeros((self.H, self.DK, self.DV), np.float32) for i in self.linear}
        self.hist = {i: np.zeros((3, self.C), np.uint16) for i in self.linear}
        self.kc = {i: np.zeros((self.HK, CONTEXT, self.HD), np.uint16) for i in self.full}
        self.vc = {i: np.zeros((self.HK, CONTEXT, self.HD), np.uint16) for i in self.full}
        self.unrotate = c.get("unrotate")
        hp = os.path.join(model_dir, "head.safetensors")
        self.head = read_safetensors(hp) if os.path.exists(hp) else None

    def raw(self, name, dtype):
        if name in self.embed:
            return self.embed[name].view(dtype)
        t = self.tensors[name]
        for start, n, data in self.shards:
            if start <= t["offset"] < start + n:
                o = t["offset"] - start
                return data[o:o + t["bytes"]].view(dtype)
        raise KeyError(name)

    def f32(self, name):
        return self.raw(name, np.float32)

    def mm(self, a16, name, L):
        t = self.tensors[name + ".q"]
        N, K = t["N"], t["K"]
        bits, group, asym = t.get("bits", 4), t.get("group", 32), t.get("asym", False)
        default = bits == 4 and group == 32 and not asym
        f16_deq = L > 20 and default and N % 64 == 0
        Bi = self.raw(name + ".b", np.uint16) if asym else None
        return matmul(a16, self.raw(name + ".q", np.uint32), self.raw(name + ".s", np.uint16), N, K, f16_deq,
                      bits, group, asym, Bi)

    def forward(self, ids, rows, cache=None, keep=False, trace=None, taps=None, tap_rows=None):
        """Hidden rows [len(rows), d] f32 (and a Snapshot when keep); src/engine.rs:529-662.
        `trace`, when a list, receives (label, array) per sublayer output for per-layer checks.
        `taps`, when a list, receives (x, h) after every residual add + RMSNorm of the layers (in
        plan order: each layer's in_norm, then its post_norm): the residual stream x (f32) and the
        normalized activations h (f16 bits) that feed the next sublayer, of the rows tap_rows (all
        rows when None)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        L = len(ids)
        Pn = cache.len if cache else 0
        if L == 0 or Pn + L > CONTEXT:
            raise ValueError(f"context of {Pn + L} tokens: must be 1 to {CONTEXT}")
        if any(r >= L for r in rows):
            raise ValueError("row out of range")
        o = lib()
        d, H, DK, DV, C = self.d, self.H, self.DK, self.DV, self.C
        if cache:
            for i in self.linear:
                self.state[i][...] = cache.state[i]
                self.hist[i][...] = cache.hist[i]
            for i in self.full:
                self.kc[i][:, :Pn] = cache.k[i]
                self.vc[i][:, :Pn] = cache.v[i]
        else:
            for i in self.linear:
                self.hist[i][...] = 0
        ef = self.tensors["embed.q"]
        x = np.empty((L, d), np.float32)
        o.or_embed(P(ids), I(L), P(self.raw("embed.q", np.uint32)), P(self.raw("embed.s", np.uint16)),
                   P(self.raw("embed.b", np.uint16) if ef.get("asym") else None), I(d), I(ef.get("bits", 4)),
                   I(ef.get("group", 32)), I(int(ef.get("asym", False))), P(x))
        y = None
        sel = slice(None) if tap_rows is None else np.asarray(tap_rows)

        def tap(h):
            if taps is not None:
                taps.append((x[sel].copy(), h[sel].copy()))
            return h

        for i, kind in enumerate(self.kinds):
            p = f"layers.{i}."
            h = tap(add_norm(x, y if i > 0 else None, self.f32(p + "in_norm")))
            if kind == "adapter":
                y = self.mm(h, p + "proj", L)
                o.or_add_bias(P(y), I(L), I(d), P(self.f32(p + "bias")))
                if trace is not None:
                    trace.append((f"{i}.proj", y.copy()))
                continue
            if kind == "linear_attention":
                big = self.mm(h, p + "in_proj", L)
                n = big.shape[1]
                qkvc = np.empty((L, C), np.float32)
                o.or_conv(P(big), I(n), I(L), I(C), P(self.f32(p + "conv")), P(self.hist[i]), P(qkvc))
                o.or_hist_update(P(big), I(n), I(L), I(C), P(self.hist[i]))
                of = np.empty((L, H * DV), np.float32)
                o.or_gdn(P(qkvc), P(big), I(n), I(C + H * DV), I(C + H * DV + H), P(self.f32(p + "neg_exp_A")),
                         P(self.f32(p + "dt_bias")), I(L), I(H), I(DK), I(DV), P(self.state[i]), I(int(cache is not None)), P(of))
                og = np.empty((L, H * DV), np.uint16)
                o.or_gnorm(P(of), P(big), I(n), I(C), P(self.f32(p + "gnorm")), I(L), I(H), I(DV), P(og))
                y = self.mm(og, p + "out_proj", L)
                if trace is not None:
                    trace.append((f"{i}.gdn", of.copy()))
            else:
                big = self.mm(h, p + "qkv", L)
                n = big.shape[1]
                Q = np.empty((self.HQ, L, self.HD), np.uint16)
                o.or_qk_prep(P(big), I(n), P(self.f32(p + "q_norm")), P(self.f32(p + "k_norm")), P(self.rope),
                             I(L), I(Pn), I(CONTEXT), I(self.HQ), I(self.HK), I(self.HD), I(self.RD), P(Q),
                             P(self.kc[i]), P(self.vc[i]))
                att = np.empty((L, self.HQ * self.HD), np.uint16)
                o.or_attn(P(Q), P(self.kc[i]), P(self.vc[i]), P(big), I(n), I(L), I(Pn), I(CONTEXT), I(self.HQ),
                          I(self.HK), I(self.HD), P(att))
                y = self.mm(att, p + "o_proj", L)
                if trace is not None:
                    trace.append((f"{i}.attn", att.copy()))
            if trace is not None:
                trace.append((f"{i}.mixer", y.copy()))
            h = tap(add_norm(x, y, self.f32(p + "post_norm")))
            big = self.mm(h, p + "gate_up", L)
            mid = np.empty((L, self.I), np.uint16)
            o.or_silu_mul(P(big), I(L), I(self.I), P(mid))
            y = self.mm(mid, p + "down", L)
            if trace is not None:
                trace.append((f"{i}.mlp", y.copy()))
                trace.append((f"{i}.x", x.copy()))
        hidden = np.zeros((0, d), np.float32)
        if len(rows):
            hidden = add_norm(x, y, self.f32("final_norm"), rows=rows, out_f32=True)
            if self.unrotate is not None:
                u = np.asarray(self.unrotate, np.float64)
                hidden = np.stack([(fwht(r).astype(np.float64) * u).astype(np.float32) for r in hidden])
        snap = None
        if keep:
            t = Pn + L
            snap = Snapshot(t, {i: self.state[i].copy() for i in self.linear}, {i: self.hist[i].copy() for i in self.linear},
                            {i: self.kc[i][:, :t].copy() for i in self.full}, {i: self.vc[i][:, :t].copy() for i in self.full})
        return hidden, snap

    def probs(self, hidden, temperature=1.0):
        return head_probs(self.head, hidden, temperature)


def read_safetensors(path):
    """F32 tensors of a safetensors file (header JSON + raw little-endian data)."""
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + n])
    data = raw[8 + n:]
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        a, b = e["data_offsets"]
        out[name] = np.frombuffer(data[a:b], dtype=np.float32).reshape(e["shape"])
    return out


def head_probs(t, hidden, temperature):
    """src/head.rs:55-77: LayerNorm (eps 1e-5) in f64, q from the last row, k per option row,
    logits = k.q * dim^-0.5 / max(T, 1e-6), softmax."""
    def project(which, x):
        x = x.astype(np.float64)
        mean = x.mean()
        var = ((x - mean) ** 2).mean()
        xn = (x - mean) / np.sqrt(var + 1e-5) * t["norm.weight"].astype(np.float64) + t["norm.bias"].astype(np.float64)
        return t[f"{which}.bias"].astype(np.float64) + t[f"{which}.weight"].astype(np.float64) @ xn
    dim = t["q.weight"].shape[0]
    q = project("q", hidden[-1])
    scale = dim ** -0.5 / max(temperature, 1e-6)
    logits = np.array([project("k", r) @ q * scale for r in hidden[:-1]])
    e = np.exp(logits - logits.max())
    return e / e.sum()

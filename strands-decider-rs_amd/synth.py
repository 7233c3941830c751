"""Seeded random-init models in the reference's model-directory format.

Writes `manifest.json`, `weights.0.bin` (GPU layout), the embedding rows file, `head.safetensors`
and `hobson_config.json` the way the reference reads them (src/model.rs:22-103, src/head.rs:25-52,
src/lib.rs:89-98), so the same directory loads in the reference wherever it can run.

Layouts written (the reference's, src/kernels.rs:550-586, 640-709; src/engine.rs:473-518):
  * quantized matrix `name.q`: [N][K/32] blocks of 4 u32; element e of a block is in word e/8 at
    bits 4*(e%8); value (q - 8) * scale with `name.s` = [N][K/32] fp16 scales;
  * GDN in_proj rows: [q (H*dk) | k (H*dk) | v (H*dv) | z (H*dv) | a (H) | b (H) | pad to 64];
  * attention qkv rows: [q head s (hd) | gate head s (hd)] for each q head, then K heads, V heads;
  * gate_up rows: [gate (I) | up (I)].

Value distributions (seeded per tensor name): uniform nibbles with code 0 remapped to 8 (values -7..7,
zero mean); scales uniform in
[0.5, 1] * s0 / sqrt(K) (s0 chosen so a sublayer's output has roughly unit scale); norm weights
1 + 0.1 N(0,1) (the reference bakes "1 + w" into the file); conv taps N(0, 0.5); A_log-style decay
negA = -U(0, 16) and dt_bias = 1 (Qwen's initialisation); head projections N(0, 1/d).
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import zlib

import numpy as np

VOCAB_2B = 151936

# The 2B hybrid of the benchmark: 24 layers, [GDN, GDN, GDN, attention] x 6.
CONFIG_2B = dict(
    hidden_size=2048, intermediate_size=6144,
    layer_types=(["linear_attention"] * 3 + ["full_attention"]) * 6,
    num_attention_heads=8, num_key_value_heads=2, head_dim=256,
    linear_num_key_heads=16, linear_key_head_dim=128, linear_value_head_dim=128,
    rms_norm_eps=1e-6, rope_theta=10000000.0, rotary_dim=64,
)

# A small model of the same family for fast parity tests (same head shapes, fewer of them).
CONFIG_TINY = dict(
    hidden_size=512, intermediate_size=1024,
    layer_types=(["linear_attention"] * 3 + ["full_attention"]) * 2,
    num_attention_heads=4, num_key_value_heads=2, head_dim=256,
    linear_num_key_heads=4, linear_key_head_dim=128, linear_value_head_dim=128,
    rms_norm_eps=1e-6, rope_theta=10000000.0, rotary_dim=64,
)

S0 = 0.22  # with scale ~ U(0.5, 1) S0 / sqrt(K), y = h W^T has std ~ 3.5 S0 for unit-scale h


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def in_proj_rows(cfg) -> int:
    h, dk, dv = cfg["linear_num_key_heads"], cfg["linear_key_head_dim"], cfg["linear_value_head_dim"]
    n = 2 * h * dk + 2 * h * dv + 2 * h
    return (n + 63) // 64 * 64


def qkv_rows(cfg) -> int:
    return 2 * cfg["num_attention_heads"] * cfg["head_dim"] + 2 * cfg["num_key_value_heads"] * cfg["head_dim"]


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """Codes [..., K] (0..15) -> [..., K/32, 4] u32, element e of a block in word e/8 at bits 4(e%8)."""
    q = q.astype(np.uint32).reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    w = np.zeros(q.shape[:-1], np.uint32)
    for j in range(8):
        w |= q[..., j] << np.uint32(4 * j)
    return w.reshape(*q.shape[:-2], q.shape[-2] // 4, 4)


# byte -> byte with each zero nibble replaced by 8
_NIB_FIX = np.array([((b & 15) or 8) | (((b >> 4) or 8) << 4) for b in range(256)], np.uint8)


def quant(rng: np.random.Generator, n: int, k: int, s0: float = S0):
    """int4 g32 codes [N][K/32][4] u32 and fp16 scales [N][K/32].  Codes are uniform nibbles with
    code 0 (value -8) replaced by code 8 (value 0): values -7..7, zero mean, so a 24-layer residual
    stream stays bounded."""
    b = rng.integers(0, np.iinfo(np.uint64).max, size=n * k // 16, dtype=np.uint64, endpoint=True).view(np.uint8)
    codes = _NIB_FIX[b].view(np.uint32).reshape(n, k // 32, 4)
    scales = (rng.uniform(0.5, 1.0, size=(n, k // 32)) * (s0 / np.sqrt(k))).astype(np.float16)
    return codes, scales


def _norm(rng, n):
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def layer_tensors(cfg, i: int, kind: str, seed: int):
    """(name, array) pairs of layer i in file order."""
    d, inter = cfg["hidden_size"], cfg["intermediate_size"]
    p = f"layers.{i}."
    out = []

    def mat(name, n, k):
        q, s = quant(_rng(seed, p + name), n, k)
        out.append((p + name + ".q", q))
        out.append((p + name + ".s", s))

    out.append((p + "in_norm", _norm(_rng(seed, p + "in_norm"), d)))
    if kind == "linear_attention":
        h, dk, dv = cfg["linear_num_key_heads"], cfg["linear_key_head_dim"], cfg["linear_value_head_dim"]
        c = 2 * h * dk + h * dv
        mat("in_proj", in_proj_rows(cfg), d)
        out.append((p + "conv", (0.5 * _rng(seed, p + "conv").standard_normal((c, 4))).astype(np.float32)))
        out.append((p + "neg_exp_A", (-_rng(seed, p + "A").uniform(0.0, 16.0, h)).astype(np.float32)))
        out.append((p + "dt_bias", np.ones(h, np.float32)))
        out.append((p + "gnorm", _norm(_rng(seed, p + "gnorm"), dv)))
        mat("out_proj", d, h * dv)
    elif kind == "full_attention":
        hd, hq = cfg["head_dim"], cfg["num_attention_heads"]
        mat("qkv", qkv_rows(cfg), d)
        out.append((p + "q_norm", _norm(_rng(seed, p + "q_norm"), hd)))
        out.append((p + "k_norm", _norm(_rng(seed, p + "k_norm"), hd)))
        mat("o_proj", d, hq * hd)
    elif kind == "adapter":
        mat("proj", d, d)
        out.append((p + "bias", (0.1 * _rng(seed, p + "bias").standard_normal(d)).astype(np.float32)))
        return out
    out.append((p + "post_norm", _norm(_rng(seed, p + "post_norm"), d)))
    mat("gate_up", 2 * inter, d)
    mat("down", d, inter)
    return out


def _safetensors(tensors: dict) -> bytes:
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, dtype=np.float32)
        header[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def write_model(out_dir: str, cfg: dict | None = None, vocab: int = 4096, seed: int = 0,
                head_dim_out: int = 256, temperature: float = 1.0) -> str:
    """Writes a seeded model directory; returns it.  Skips the work if the same model is there."""
    cfg = dict(CONFIG_TINY if cfg is None else cfg)
    key = hashlib.sha1(json.dumps([cfg, vocab, seed, head_dim_out, temperature, 5], sort_keys=True).encode()).hexdigest()
    stamp = os.path.join(out_dir, ".synth")
    if os.path.exists(stamp) and open(stamp).read() == key:
        return out_dir
    os.makedirs(out_dir, exist_ok=True)
    d = cfg["hidden_size"]

    tensors, offset = {}, 0
    with open(os.path.join(out_dir, "weights.0.bin.tmp"), "wb") as f:
        def put(name, a, **meta):
            nonlocal offset
            pad = (-offset) % 256
            f.write(b"\0" * pad)
            offset += pad
            raw = np.ascontiguousarray(a).tobytes()
            f.write(raw)
            tensors[name] = dict(offset=offset, bytes=len(raw), shape=list(a.shape), **meta)
            offset += len(raw)

        for i, kind in enumerate(cfg["layer_types"]):
            for name, a in layer_tensors(cfg, i, kind, seed):
                if name.endswith(".q"):
                    n, nb, _ = a.shape
                    put(name, a, N=n, K=nb * 32, bits=4, group=32, asym=False)
                else:
                    put(name, a)
        put("final_norm", _norm(_rng(seed, "final_norm"), d))
    os.replace(os.path.join(out_dir, "weights.0.bin.tmp"), os.path.join(out_dir, "weights.0.bin"))

    # Embedding rows: per token id, the q part then the s part (src/model.rs:260-283).
    eq, es = quant(_rng(seed, "embed"), vocab, d, s0=0.27 * np.sqrt(d))
    rows = np.concatenate([eq.view(np.uint8).reshape(vocab, -1), es.view(np.uint8).reshape(vocab, -1)], axis=1)
    rows.tofile(os.path.join(out_dir, "embed.bin"))
    tensors["embed.q"] = dict(shape=[vocab, d // 32, 4], N=vocab, K=d, bits=4, group=32, asym=False)
    tensors["embed.s"] = dict(shape=[vocab, d // 32])

    manifest = dict(
        config=cfg,
        shards=[dict(path="weights.0.bin", start=0, bytes=offset)],
        tensors=tensors,
        embed=dict(rows="embed.bin", vocab=vocab, row_bytes=rows.shape[1],
                   parts=[["embed.q", d // 2], ["embed.s", d // 16]]),
    )
    with open(os.path.join(out_dir, "manifest.json"), "w") as f:
        json.dump(manifest, f)

    r = _rng(seed, "head")
    head = {
        "norm.weight": _norm(r, d), "norm.bias": 0.1 * r.standard_normal(d),
        "q.weight": r.standard_normal((head_dim_out, d)) / np.sqrt(d), "q.bias": np.zeros(head_dim_out),
        "k.weight": r.standard_normal((head_dim_out, d)) / np.sqrt(d), "k.bias": np.zeros(head_dim_out),
    }
    with open(os.path.join(out_dir, "head.safetensors"), "wb") as f:
        f.write(_safetensors(head))
    with open(os.path.join(out_dir, "hobson_config.json"), "w") as f:
        json.dump(dict(max_length=4096, temperature=temperature, temperature_by_kind={}, ordinal_smoothing=0.0), f)
    with open(stamp, "w") as f:
        f.write(key)
    return out_dir

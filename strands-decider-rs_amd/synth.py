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


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Codes [N][K] (0 .. 2^bits - 1) -> u32 words [N][K/32][bits] in the reference's block layout
    (src/kernels.rs:550-576): int4 element e of a 32-block in word e/8 at bits 4(e%8); int2 in word
    e/16 at bits 2(e%16); int3 as int2 (its low two bits) plus a third word holding bit 2 of element
    e at bit e."""
    n, k = codes.shape
    c = codes.astype(np.uint32).reshape(n, k // 32, 32)
    if bits == 4:
        return pack_nibbles(codes)
    words = np.zeros((n, k // 32, bits), np.uint32)
    for e in range(32):
        words[:, :, e // 16] |= (c[:, :, e] & np.uint32(3)) << np.uint32(2 * (e % 16))
        if bits == 3:
            words[:, :, 2] |= ((c[:, :, e] >> np.uint32(2)) & np.uint32(1)) << np.uint32(e)
    return words


# standard deviation of the dequantized code values per format (int4 without code 0: -7..7)
_CODE_STD = {4: np.sqrt((15 ** 2 - 1) / 12), 3: np.sqrt((8 ** 2 - 1) / 12), 2: np.sqrt((4 ** 2 - 1) / 12)}


def quant_fmt(rng: np.random.Generator, n: int, k: int, bits: int, group: int, asym: bool, s0: float = S0):
    """A matrix in any of the reference's formats (src/kernels.rs:550-576): words [N][K/32][bits],
    f16 scales [N][K/group] and, asymmetric, f16 biases [N][K/group].  Symmetric values are
    (q - 2^(bits-1)) s; asymmetric ones q s + b with b centring the codes.  The scales keep the
    output scale of `quant`."""
    codes = rng.integers(0, 1 << bits, size=(n, k), dtype=np.uint32)
    if bits == 4 and not asym:
        codes[codes == 0] = 8
    ng = k // group
    scales = (rng.uniform(0.5, 1.0, size=(n, ng)) * (s0 / np.sqrt(k)) * (_CODE_STD[4] / _CODE_STD[bits]))
    scales = scales.astype(np.float16)
    bias = None
    if asym:
        centre = ((1 << bits) - 1) / 2.0
        bias = (-centre * scales.astype(np.float64) * rng.uniform(0.9, 1.1, size=(n, ng))).astype(np.float16)
    return pack_codes(codes, bits), scales, bias


def encode_scale_codes(scales: np.ndarray, rng: np.random.Generator):
    """f16 scales [n, g] -> the 8-bit scale codes of the download format (src/model.rs:217-236),
    one row each: a 4-byte header (m as f16 bits, j as u16) then g codes sign << 7 | k with
    |scale| ~ m 2^(-k j / 4096).  Returns (row bytes [n, 4 + g] u8, the f16 scales the codes decode
    to).  m is the row's largest magnitude, j the step that spans its range in 127 codes."""
    a = np.abs(scales.astype(np.float64))
    n, g = a.shape
    m = np.maximum(a.max(1), 1e-4).astype(np.float16).astype(np.float64)
    lo = np.maximum(a.min(1), 1e-6)
    j = np.clip(np.ceil(-4096 * np.log2(lo / m) / 127), 1, 4095).astype(np.uint16)
    k = np.clip(np.rint(-4096 * np.log2(np.maximum(a, 1e-30) / m[:, None]) / j[:, None]), 0, 127).astype(np.uint8)
    # one code in ten carries a flipped sign (a negative scale), so the sign bit is exercised
    sign = (np.signbit(scales.astype(np.float32)) ^ (rng.random((n, g)) < 0.1)).astype(np.uint8)
    codes = (sign << 7) | k
    head = np.zeros((n, 2), np.uint16)
    head[:, 0] = m.astype(np.float16).view(np.uint16)
    head[:, 1] = j
    rows = np.concatenate([head.view(np.uint8).reshape(n, 4), codes], axis=1)
    mag = (m[:, None] * np.power(2.0, -(k.astype(np.float64) * j[:, None]) / 4096.0))
    dec = mag.astype(np.float32).astype(np.float16)
    dec = np.where(sign.astype(bool), -dec, dec).astype(np.float16)
    return rows, dec


def _norm(rng, n):
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def layer_tensors(cfg, i: int, kind: str, seed: int, mat_fmt=None):
    """(name, array, format) triples of layer i in file order; format (bits, group, asym) for the
    quantized words, None otherwise.  mat_fmt maps a matrix name (e.g. "down", or "3.down" for one
    layer only) to a non-default format."""
    d, inter = cfg["hidden_size"], cfg["intermediate_size"]
    p = f"layers.{i}."
    out = []
    mat_fmt = mat_fmt or {}

    def mat(name, n, k):
        fmt = mat_fmt.get(f"{i}.{name}", mat_fmt.get(name))
        if fmt is None or tuple(fmt) == (4, 32, False):
            q, s = quant(_rng(seed, p + name), n, k)
            out.append((p + name + ".q", q, (4, 32, False)))
            out.append((p + name + ".s", s, None))
            return
        bits, group, asym = fmt
        q, s, b = quant_fmt(_rng(seed, p + name), n, k, bits, group, asym)
        out.append((p + name + ".q", q, (bits, group, asym)))
        out.append((p + name + ".s", s, None))
        if asym:
            out.append((p + name + ".b", b, None))

    out.append((p + "in_norm", _norm(_rng(seed, p + "in_norm"), d), None))
    if kind == "linear_attention":
        h, dk, dv = cfg["linear_num_key_heads"], cfg["linear_key_head_dim"], cfg["linear_value_head_dim"]
        c = 2 * h * dk + h * dv
        mat("in_proj", in_proj_rows(cfg), d)
        out.append((p + "conv", (0.5 * _rng(seed, p + "conv").standard_normal((c, 4))).astype(np.float32), None))
        out.append((p + "neg_exp_A", (-_rng(seed, p + "A").uniform(0.0, 16.0, h)).astype(np.float32), None))
        out.append((p + "dt_bias", np.ones(h, np.float32), None))
        out.append((p + "gnorm", _norm(_rng(seed, p + "gnorm"), dv), None))
        mat("out_proj", d, h * dv)
    elif kind == "full_attention":
        hd, hq = cfg["head_dim"], cfg["num_attention_heads"]
        mat("qkv", qkv_rows(cfg), d)
        out.append((p + "q_norm", _norm(_rng(seed, p + "q_norm"), hd), None))
        out.append((p + "k_norm", _norm(_rng(seed, p + "k_norm"), hd), None))
        mat("o_proj", d, hq * hd)
    elif kind == "adapter":
        mat("proj", d, d)
        out.append((p + "bias", (0.1 * _rng(seed, p + "bias").standard_normal(d)).astype(np.float32), None))
        return out
    out.append((p + "post_norm", _norm(_rng(seed, p + "post_norm"), d), None))
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
                head_dim_out: int = 256, temperature: float = 1.0, embed_fmt=(4, 32, False), u8_embed: bool = False,
                mat_fmt=None) -> str:
    """Writes a seeded model directory; returns it.  Skips the work if the same model is there.
    embed_fmt: (bits, group, asym) of the embedding table; u8_embed: its rows in the download
    format with 8-bit scale codes (the hosted model's, src/model.rs:260-283); mat_fmt: matrices in
    non-default formats (see layer_tensors)."""
    cfg = dict(CONFIG_TINY if cfg is None else cfg)
    embed_fmt = tuple(embed_fmt)
    mat_fmt = {k: list(v) for k, v in (mat_fmt or {}).items()}
    key = hashlib.sha1(json.dumps([cfg, vocab, seed, head_dim_out, temperature, 6, list(embed_fmt), u8_embed, mat_fmt],
                                  sort_keys=True).encode()).hexdigest()
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
            for name, a, fmt in layer_tensors(cfg, i, kind, seed, mat_fmt):
                if fmt is not None:
                    n, nb, _ = a.shape
                    put(name, a, N=n, K=nb * 32, bits=fmt[0], group=fmt[1], asym=bool(fmt[2]))
                else:
                    put(name, a)
        put("final_norm", _norm(_rng(seed, "final_norm"), d))
    os.replace(os.path.join(out_dir, "weights.0.bin.tmp"), os.path.join(out_dir, "weights.0.bin"))

    # Embedding rows: per token id, the q part, the s part, then (asym) the b part
    # (src/model.rs:260-283).  With u8_embed the s part is stored as 8-bit scale codes: a 4-byte
    # header and one code per scale (the download format the reference decodes at load).
    ebits, egroup, easym = embed_fmt
    if (ebits, egroup, easym) == (4, 32, False):
        eq, es = quant(_rng(seed, "embed"), vocab, d, s0=0.27 * np.sqrt(d))
        eb = None
    else:
        eq, es, eb = quant_fmt(_rng(seed, "embed"), vocab, d, ebits, egroup, easym, s0=0.27 * np.sqrt(d))
    g = d // egroup
    qb, sb = eq.view(np.uint8).reshape(vocab, -1), es.view(np.uint8).reshape(vocab, -1)
    parts = [["embed.q", qb.shape[1]], ["embed.s", sb.shape[1]]]
    row_parts = [qb]
    if u8_embed:
        codes, _ = encode_scale_codes(es, _rng(seed, "embed.codes"))
        row_parts.append(codes)
    else:
        row_parts.append(sb)
    if easym:
        bb = eb.view(np.uint8).reshape(vocab, -1)
        parts.append(["embed.b", bb.shape[1]])
        row_parts.append(bb)
    rows = np.concatenate(row_parts, axis=1)
    rows.tofile(os.path.join(out_dir, "embed.bin"))
    tensors["embed.q"] = dict(shape=[vocab, d // 32, ebits], N=vocab, K=d, bits=ebits, group=egroup, asym=bool(easym))
    tensors["embed.s"] = dict(shape=[vocab, g], u8=bool(u8_embed))
    if easym:
        tensors["embed.b"] = dict(shape=[vocab, g])
    emb = dict(rows="embed.bin", vocab=vocab, row_bytes=sum(b for _, b in parts), parts=parts)
    if u8_embed:
        emb["wire_row_bytes"] = rows.shape[1]
        emb["u8"] = True

    manifest = dict(
        config=cfg,
        shards=[dict(path="weights.0.bin", start=0, bytes=offset)],
        tensors=tensors,
        embed=emb,
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

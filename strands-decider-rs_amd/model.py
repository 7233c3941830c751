"""Model directory reader: the manifest and the files the engine loads.

Mirrors the reference's model-file types (src/model.rs:22-103: `Manifest`, `Config`, `Shard`,
`Tensor`, `Embed`) and `embed_parts` (src/model.rs:260-283).  Only the on-disk GPU layout is read;
the packed "wire" download format and its 8-bit scale codes (src/model.rs:204-257) are a
download-time conversion and are rejected here with an error.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

LINEAR = "linear_attention"
FULL = "full_attention"
ADAPTER = "adapter"
LAYER_KIND = {LINEAR: 0, FULL: 1, ADAPTER: 2}


@dataclass
class Config:
    """src/model.rs:31-47."""
    hidden_size: int
    intermediate_size: int
    layer_types: list
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    linear_num_key_heads: int
    linear_key_head_dim: int
    linear_value_head_dim: int
    rms_norm_eps: float
    rope_theta: float
    rotary_dim: int
    unrotate: list | None = None


@dataclass
class Tensor:
    """src/model.rs:58-83 (defaults: bits 4, group 32, symmetric)."""
    offset: int = 0
    bytes: int = 0
    shape: list = field(default_factory=list)
    N: int = 0
    K: int = 0
    bits: int = 4
    group: int = 32
    asym: bool = False
    had: int | None = None
    u8: bool = False
    wire: int | None = None


@dataclass
class Shard:
    path: str
    start: int
    bytes: int
    wire: int | None = None


@dataclass
class Embed:
    """src/model.rs:92-103."""
    rows: str
    vocab: int
    row_bytes: int
    parts: list
    wire_row_bytes: int | None = None
    u8: bool = False


@dataclass
class Manifest:
    config: Config
    shards: list
    tensors: dict
    embed: Embed | None
    tokenizer: str | None = None


def shard_file(i: int) -> str:
    """src/model.rs:110-112."""
    return f"weights.{i}.bin"


def read_manifest(d: str) -> Manifest:
    """src/model.rs:105-108."""
    path = os.path.join(d, "manifest.json")
    try:
        with open(path) as f:
            m = json.load(f)
    except OSError as e:
        raise RuntimeError(f"{path}: {e}") from None
    c = m["config"]
    cfg = Config(**{k: c[k] for k in Config.__dataclass_fields__ if k in c})
    tensors = {}
    for name, t in m["tensors"].items():
        tensors[name] = Tensor(**{k: t[k] for k in Tensor.__dataclass_fields__ if k in t})
    shards = [Shard(**{k: s[k] for k in Shard.__dataclass_fields__ if k in s}) for s in m["shards"]]
    embed = None
    if m.get("embed"):
        e = m["embed"]
        embed = Embed(**{k: e[k] for k in Embed.__dataclass_fields__ if k in e})
    return Manifest(cfg, shards, tensors, embed, m.get("tokenizer"))


def embed_parts(d: str, e: Embed, decode=None) -> list:
    """The embedding table, one array per part, all rows (src/model.rs:260-283).  Rows stored with
    8-bit scale codes (`u8`) have their "embed.s" part decoded by `decode(src, n, g)` (the engine's
    own, sd_decode_scale_codes, when None)."""
    data = np.fromfile(os.path.join(d, e.rows), dtype=np.uint8)
    rb = e.wire_row_bytes or e.row_bytes
    if data.size != e.vocab * rb:
        raise RuntimeError(f"{e.rows}: {data.size} bytes, expected {e.vocab} rows of {rb}")
    rows = data.reshape(e.vocab, rb)
    out, off = [], 0
    for name, b in e.parts:
        if e.u8 and name == "embed.s":
            if decode is None:
                from . import decode_scale_codes as decode
            g = b // 2
            part = np.empty((e.vocab, g), np.uint16)
            for r in range(e.vocab):
                part[r] = decode(rows[r, off:off + 4 + g].tobytes(), 1, g)[0]
            out.append((name, part.view(np.uint8).reshape(-1)))
            off += 4 + g
        else:
            out.append((name, np.ascontiguousarray(rows[:, off:off + b]).reshape(-1)))
            off += b
    return out

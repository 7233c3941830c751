"""Host-side model format: the synthetic writer produces the reference's model-directory layout
(src/model.rs:22-103, src/kernels.rs:550-586) and the manifest reader accepts it."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import cases  # noqa: E402


def test_pack_nibbles_layout(synth):
    """Element e of a 32-block sits in word e/8 at bits 4(e%8); two independent packers agree."""
    codes = (np.arange(64, dtype=np.uint32) % 16).reshape(1, 64)
    w = synth.pack_nibbles(codes)
    assert w.shape == (1, 2, 4)
    assert w[0, 0, 0] == 0x76543210 and w[0, 0, 1] == 0xFEDCBA98
    rng = np.random.default_rng(0)
    c = rng.integers(0, 16, size=(7, 96), dtype=np.uint32)
    assert np.array_equal(synth.pack_nibbles(c).reshape(7, -1), cases.pack_codes(c, 4).reshape(7, -1))


def test_quant_codes_are_zero_mean(synth):
    codes, scales = synth.quant(np.random.default_rng(1), 64, 256)
    nib = np.stack([(codes >> (4 * j)) & 15 for j in range(8)], -1)
    assert nib.min() >= 1 and nib.max() <= 15  # code 0 (value -8) never appears
    assert abs(nib.astype(np.float64).mean() - 8) < 0.05
    assert scales.dtype == np.float16 and scales.shape == (64, 8)


def test_row_layouts(synth):
    cfg = synth.CONFIG_2B
    assert synth.in_proj_rows(cfg) == 8256  # 8224 padded to 64
    assert synth.qkv_rows(cfg) == 5120


def test_tiny_model_directory(sdamd, synth, tiny_model):
    m = sdamd.model.read_manifest(tiny_model)
    c = synth.CONFIG_TINY
    assert m.config.hidden_size == c["hidden_size"]
    assert len(m.config.layer_types) == len(c["layer_types"])
    t = m.tensors["layers.0.in_proj.q"]
    assert (t.N, t.K, t.bits, t.group) == (synth.in_proj_rows(c), c["hidden_size"], 4, 32)
    assert t.bytes == t.N * t.K // 2
    parts = sdamd.model.embed_parts(tiny_model, m.embed)
    assert [p[0] for p in parts] == ["embed.q", "embed.s"]
    assert parts[0][1].size == 4096 * c["hidden_size"] // 2
    with open(os.path.join(tiny_model, "manifest.json")) as f:
        raw = json.load(f)
    offs = sorted((v["offset"], v["bytes"]) for k, v in raw["tensors"].items() if "offset" in v)
    for (o1, b1), (o2, _) in zip(offs, offs[1:]):
        assert o1 % 256 == 0 and o1 + b1 <= o2  # aligned, non-overlapping


def test_embedding_rows_with_scale_codes(sdamd, synth, oracle, tmp_path):
    """An int3 embedding whose rows store 8-bit scale codes (the hosted model's download format,
    src/model.rs:260-283): the product's reader (the engine's C++ decode) and the oracle's decode
    give the same f16 scales, and the codes do encode the writer's scales closely."""
    d = synth.write_model(str(tmp_path / "u8"), synth.CONFIG_TINY, vocab=300, seed=4, embed_fmt=(3, 32, False),
                          u8_embed=True)
    m = sdamd.model.read_manifest(d)
    assert m.embed.u8 and m.embed.wire_row_bytes == 512 * 3 // 8 + 4 + 512 // 32
    parts = dict(sdamd.model.embed_parts(d, m.embed))
    om = oracle.OracleModel(d)
    assert np.array_equal(parts["embed.s"], om.embed["embed.s"])
    assert np.array_equal(parts["embed.q"], om.embed["embed.q"])
    assert m.tensors["embed.q"].bits == 3 and parts["embed.q"].size == 300 * 512 * 3 // 8


def test_wire_row_size_is_checked(sdamd, tiny_model):
    m = sdamd.model.read_manifest(tiny_model)
    e = m.embed
    e.wire_row_bytes = 10
    with pytest.raises(RuntimeError, match="expected"):
        sdamd.model.embed_parts(tiny_model, e)


def test_other_formats_are_written(sdamd, synth, tmp_path):
    """Adapter layers and matrices in non-default formats land in the manifest as the reference
    describes them (src/model.rs:58-83)."""
    cfg = dict(synth.CONFIG_TINY, layer_types=["linear_attention", "adapter", "full_attention", "adapter"])
    d = synth.write_model(str(tmp_path / "fmt"), cfg, vocab=64, seed=5,
                          mat_fmt={"proj": (3, 64, True), "1.proj": (2, 128, False), "down": (4, 64, False)})
    m = sdamd.model.read_manifest(d)
    t = m.tensors
    assert (t["layers.1.proj.q"].bits, t["layers.1.proj.q"].group, t["layers.1.proj.q"].asym) == (2, 128, False)
    assert (t["layers.3.proj.q"].bits, t["layers.3.proj.q"].group, t["layers.3.proj.q"].asym) == (3, 64, True)
    assert t["layers.3.proj.b"].bytes == 512 * 512 // 64 * 2
    assert t["layers.0.down.q"].group == 64 and t["layers.0.down.s"].bytes == 512 * 1024 // 64 * 2
    assert t["layers.0.in_proj.q"].group == 32


def test_manifest_missing_is_an_error(sdamd, tmp_path):
    with pytest.raises(RuntimeError, match="manifest.json"):
        sdamd.model.read_manifest(str(tmp_path))

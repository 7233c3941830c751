"""Engine-level parity for the hosted model's format pieces on the GPU (the reference's
src/model.rs:260-283, src/engine.rs:434-472, src/kernels.rs:63-89, 138-149, 590-635): an int3
embedding whose rows store 8-bit scale codes, a vocabulary past 2^16 (the hosted one has about
248k ids), adapter layers (first and last layer too) and matrices in non-default formats, which the
reference sends to its f32-dequant GEMV at every length.  Forwards, a snapshot continuation and
ask_ids against the oracle's own forwards of the same model directory."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN_TOL = 2e-2
PROB_TOL = 2e-3
VOCAB = 248320
LAYERS = ["adapter", "linear_attention", "linear_attention", "full_attention", "adapter", "linear_attention",
          "full_attention", "adapter"]
MAT_FMT = {
    "proj": (3, 64, True),        # adapters: int3, group 64, asymmetric
    "4.proj": (2, 128, False),    # one adapter in int2, group 128
    "5.down": (4, 64, False),     # int4 with group 64
    "3.o_proj": (3, 32, False),   # an attention projection in int3
    "1.gate_up": (4, 32, True),   # an asymmetric gate_up (no fused silu * mul for any layer then)
}


@pytest.fixture(scope="module")
def hosted(sdamd, synth, oracle, tmp_path_factory):
    cfg = dict(synth.CONFIG_TINY, layer_types=LAYERS)
    path = synth.write_model(str(tmp_path_factory.mktemp("hosted")), cfg, vocab=VOCAB, seed=7,
                             embed_fmt=(3, 32, False), u8_embed=True, mat_fmt=MAT_FMT)
    eng, head, _ = sdamd.load_decider(path)
    om = oracle.OracleModel(path)
    yield eng, head, om
    eng.free()


def ids_for(seed, n):
    ids = np.random.default_rng(seed).integers(0, VOCAB, n).astype(np.uint32)
    ids[0] = VOCAB - 1  # the last row of the table
    if n > 2:
        ids[1] = 248069  # the hosted tokenizer's largest id in the reference's fixtures
    return ids


@pytest.mark.parametrize("L", [1, 7, 20, 21, 64, 130])
def test_hosted_format_forward_matches_oracle(hosted, L):
    eng, head, om = hosted
    ids = ids_for(L, L)
    rows = sorted({0, L // 2, L - 1})
    got = eng.forward(ids, rows).hidden
    want, _ = om.forward(ids, rows)
    err = np.abs(got - want).max()
    print(f"hosted-format model, L={L}: max |dh| {err:.3g}", flush=True)
    assert err < HIDDEN_TOL, f"L={L}: max |dh| {err}"


def test_hosted_format_continuation_and_ask(hosted, sdamd):
    eng, head, om = hosted
    state = ids_for(100, 90)
    qs = [ids_for(101, 12), ids_for(102, 33)]
    options = [[1, 4, 9], [2, 20, 30]]
    prefix = eng.forward(state, [], keep=True).snapshot
    _, osnap = om.forward(state, [], keep=True)
    for q, o in zip(qs, options):
        rows = list(o) + [len(q) - 1]
        got = eng.forward(q, rows, cache=prefix).hidden
        want, _ = om.forward(q, rows, cache=osnap)
        assert np.abs(got - want).max() < HIDDEN_TOL
    probs = sdamd.ask_ids(eng, head, state, qs, options, [1.0, 0.8])
    for q, o, t, g in zip(qs, options, [1.0, 0.8], probs):
        h, _ = om.forward(q, list(o) + [len(q) - 1], cache=osnap)
        want = om.probs(h, t)
        assert np.abs(g - want).max() < PROB_TOL
        assert int(np.argmax(g)) == int(np.argmax(want))
    prefix.free()

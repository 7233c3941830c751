"""The benchmark's own workload on the GPU against the oracle: the 2B hybrid (24 layers, hidden 2048,
seeded random weights), a 512-token state forwarded with a snapshot, then 3 x 40-token questions as
one batched forward from it with the pointer head on the device (Decider::ask_all, src/lib.rs:192-198;
the parity property of tests/engine_parity.rs:58-85 at the benchmark's shapes).  These shapes take
the prefill GEMM tiles, the fused SiLU * mul epilogue and the recurrent GDN path that the small
model's tests reach only at other sizes.  The per-layer test compares the residual stream and the
normalized activations after every add + RMSNorm of the 24 layers (48 taps)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN_TOL = 2e-2   # hidden rows and per-layer activations, absolute
PROB_TOL = 2e-3     # answer probabilities, absolute

STATE_LEN, Q_LEN = 512, 40
OPTIONS = [[5, 17], [3, 20, 33], [1, 8, 15, 22, 30]]  # option token indices per question
TAP_ROWS = [0, 1, 255, 256, STATE_LEN - 1]


@pytest.fixture(scope="module")
def two_b(sdamd, model_2b, oracle):
    eng, head, cfg = sdamd.load_decider(model_2b)
    om = oracle.OracleModel(model_2b)
    yield eng, head, cfg, om
    eng.free()


def state_and_questions(synth):
    rng = np.random.default_rng(2026)
    state = rng.integers(0, synth.VOCAB_2B, STATE_LEN).astype(np.uint32)
    questions = [rng.integers(0, synth.VOCAB_2B, Q_LEN).astype(np.uint32) for _ in OPTIONS]
    return state, questions


@pytest.mark.timeout(600)
def test_2b_state_and_batched_questions_match_oracle(two_b, synth):
    eng, head, cfg, om = two_b
    temp = float(cfg["temperature"])
    state, questions = state_and_questions(synth)
    rows = [0, 255, STATE_LEN - 1]

    out = eng.forward(state, rows, keep=True)
    want, osnap = om.forward(state, rows, keep=True)
    err = np.abs(out.hidden - want).max()
    print(f"2B prefill of {STATE_LEN}: max |dh| {err:.3g}", flush=True)
    assert err < HIDDEN_TOL, f"prefill hidden rows: max |dh| {err}"

    probs, _ = eng.ask_batch(head, questions, OPTIONS, [temp] * len(OPTIONS), cache=out.snapshot)
    hid, _ = eng.forward_batch(questions, [list(o) + [Q_LEN - 1] for o in OPTIONS], cache=out.snapshot)
    for i, (q, opts) in enumerate(zip(questions, OPTIONS)):
        ohid, _ = om.forward(q, list(opts) + [Q_LEN - 1], cache=osnap)
        herr = np.abs(hid[i] - ohid).max()
        op = om.probs(ohid, temp)
        perr = np.abs(np.asarray(probs[i]) - op).max()
        print(f"question {i}: max |dh| {herr:.3g}, probs {np.round(probs[i], 5)} oracle {np.round(op, 5)}", flush=True)
        assert herr < HIDDEN_TOL, f"question {i}: max |dh| {herr}"
        assert perr < PROB_TOL, f"question {i}: max |dp| {perr}"
        assert int(np.argmax(probs[i])) == int(np.argmax(op)), f"question {i}: answer differs from the oracle's"
    out.snapshot.free()


@pytest.mark.timeout(600)
def test_2b_per_layer_activations_match_oracle(two_b, oracle, synth):
    """After every residual add + RMSNorm of the 512-token prefill: the residual x (f32) and the
    normalized activations h (f16) that feed the next sublayer, within 2e-2 absolute, layer by
    layer, on rows at the start, middle and end of the sequence."""
    eng, head, cfg, om = two_b
    state, _ = state_and_questions(synth)
    got = eng.trace(state, TAP_ROWS)
    taps = []
    om.forward(state, [], taps=taps, tap_rows=TAP_ROWS)
    assert len(got) == len(taps) == 48
    worst = (0.0, 0.0)
    for i, ((gx, gh), (wx, wh)) in enumerate(zip(got, taps)):
        ex = float(np.abs(gx - wx).max())
        eh = float(np.abs(gh - oracle.h2f(wh)).max())
        worst = (max(worst[0], ex), max(worst[1], eh))
        assert ex < HIDDEN_TOL and eh < HIDDEN_TOL, f"tap {i} (layer {i // 2}): max |dx| {ex}, max |dh| {eh}"
    print(f"2B per-layer taps: max |dx| {worst[0]:.3g}, max |dh| {worst[1]:.3g} over 48 taps", flush=True)

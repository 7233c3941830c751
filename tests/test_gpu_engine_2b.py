"""The benchmark's own workload on the GPU against the oracle: the 2B hybrid (24 layers, hidden 2048,
seeded random weights), a 512-token state forwarded with a snapshot, then 3 x 40-token questions as
one batched forward from it with the pointer head on the device (Decider::ask_all, src/lib.rs:192-198;
the parity property of tests/engine_parity.rs:58-85 at the benchmark's shapes).  These shapes take
the prefill GEMM tiles, the fused SiLU * mul epilogue and the recurrent GDN path that the small
model's tests reach only at other sizes."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN_TOL = 2e-2   # hidden rows, absolute
PROB_TOL = 2e-3     # answer probabilities, absolute

STATE_LEN, Q_LEN = 512, 40
OPTIONS = [[5, 17], [3, 20, 33], [1, 8, 15, 22, 30]]  # option token indices per question


def test_2b_state_and_batched_questions_match_oracle(sdamd, synth, model_2b, oracle):
    eng, head, cfg = sdamd.load_decider(model_2b)
    try:
        om = oracle.OracleModel(model_2b)
        temp = float(cfg["temperature"])
        rng = np.random.default_rng(2026)
        state = rng.integers(0, synth.VOCAB_2B, STATE_LEN).astype(np.uint32)
        questions = [rng.integers(0, synth.VOCAB_2B, Q_LEN).astype(np.uint32) for _ in OPTIONS]
        rows = [0, 255, STATE_LEN - 1]

        out = eng.forward(state, rows, keep=True)
        want, osnap = om.forward(state, rows, keep=True)
        err = np.abs(out.hidden - want).max()
        print(f"2B prefill of {STATE_LEN}: max |dh| {err:.3g}", flush=True)
        assert err < HIDDEN_TOL, f"prefill hidden rows: max |dh| {err}"

        probs, _ = eng.ask_batch(head, questions, OPTIONS, [temp] * len(OPTIONS), cache=out.snapshot)
        for i, (q, opts) in enumerate(zip(questions, OPTIONS)):
            ohid, _ = om.forward(q, list(opts) + [Q_LEN - 1], cache=osnap)
            op = om.probs(ohid, temp)
            perr = np.abs(np.asarray(probs[i]) - op).max()
            print(f"question {i}: probs {np.round(probs[i], 5)} oracle {np.round(op, 5)}", flush=True)
            assert perr < PROB_TOL, f"question {i}: max |dp| {perr}"
        out.snapshot.free()
    finally:
        eng.free()

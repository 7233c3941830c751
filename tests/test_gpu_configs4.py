"""BASELINE configs[4] on the GPU against the oracle, at the top of its range: the 2B hybrid encodes a
2048-token state (the longest configs[4] draws: the M > 1024 GEMM plan, a gated-delta-net scan of 32
chunks, attention over up to 2048 keys), then 8 questions of 64 tokens (the longest it draws) are
answered from its snapshot as one batched forward of 8 sequences (512 rows, each question attending
over 2048 + 64 keys) with the device head, and again as one forward of the state with the 8
questions as its branches (2560 rows).  Each question is compared with the
oracle's own forward of that question from its snapshot: hidden rows within 2e-2, probabilities
within 2e-3, the same answer (tests/engine_parity.rs:58-85 at the sweep's shapes)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN_TOL = 2e-2
PROB_TOL = 2e-3
STATE_LEN, N_Q, Q_LEN = 2048, 8, 64


@pytest.mark.timeout(900)
def test_configs4_long_state_and_eight_questions(sdamd, synth, model_2b, oracle):
    eng, head, cfg = sdamd.load_decider(model_2b)
    try:
        om = oracle.OracleModel(model_2b)
        temp = float(cfg["temperature"])
        rng = np.random.default_rng(404)
        state = rng.integers(0, synth.VOCAB_2B, STATE_LEN).astype(np.uint32)
        qs = [rng.integers(0, synth.VOCAB_2B, Q_LEN).astype(np.uint32) for _ in range(N_Q)]
        opts = [sorted(rng.choice(len(q) - 1, int(rng.integers(2, 6)), replace=False).tolist()) for q in qs]
        rows = [0, STATE_LEN // 2 - 1, STATE_LEN - 1]

        out = eng.forward(state, rows, keep=True)
        print(f"configs[4]: GPU prefill of {STATE_LEN} done; oracle prefill (one to two minutes on the host)", flush=True)
        want, osnap = om.forward(state, rows, keep=True)
        err = np.abs(out.hidden - want).max()
        print(f"configs[4] prefill of {STATE_LEN}: max |dh| {err:.3g}", flush=True)
        assert err < HIDDEN_TOL

        probs, _ = eng.ask_batch(head, qs, opts, [temp] * N_Q, cache=out.snapshot)
        hid, _ = eng.forward_batch(qs, [list(o) + [len(q) - 1] for q, o in zip(qs, opts)], cache=out.snapshot)
        # ask_all as sd_ask_ids serves it: one forward of the state with the 8 questions as its
        # branches (2560 rows)
        tree = sdamd.ask_ids(eng, head, state, qs, opts, [temp] * N_Q)
        for i, (q, o) in enumerate(zip(qs, opts)):
            ohid, _ = om.forward(q, list(o) + [len(q) - 1], cache=osnap)
            op = om.probs(ohid, temp)
            herr = np.abs(hid[i] - ohid).max()
            perr = np.abs(np.asarray(probs[i]) - op).max()
            print(f"question {i} ({len(q)} tokens, {len(o)} options): max |dh| {herr:.3g}, max |dp| {perr:.3g}",
                  flush=True)
            assert herr < HIDDEN_TOL, f"question {i}: max |dh| {herr}"
            assert perr < PROB_TOL, f"question {i}: max |dp| {perr}"
            assert int(np.argmax(probs[i])) == int(np.argmax(op)), f"question {i}: answer differs from the oracle's"
            terr = np.abs(np.asarray(tree[i]) - op).max()
            print(f"question {i} in the one-forward ask_all: max |dp| {terr:.3g}", flush=True)
            assert terr < PROB_TOL, f"question {i} (one-forward ask_all): max |dp| {terr}"
            assert int(np.argmax(tree[i])) == int(np.argmax(op)), f"question {i} (one-forward ask_all): answer differs"
        out.snapshot.free()
    finally:
        eng.free()

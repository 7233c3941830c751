"""Engine-level parity on the GPU through the C ABI: forward vs the oracle's forward on the same
seeded model, snapshot continuation vs a full forward (tests/engine_parity.rs:58-85), ask_all
probabilities, error paths of Engine::forward (src/engine.rs:530-537)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN_TOL = 2e-2   # per-row activations / hidden states, absolute
PROB_TOL = 2e-3     # answer probabilities, absolute


@pytest.fixture(scope="module")
def tiny(sdamd, tiny_model, oracle):
    eng, head, cfg = sdamd.load_decider(tiny_model)
    om = oracle.OracleModel(tiny_model)
    yield eng, head, om
    eng.free()


def ids_for(seed, n, vocab=4096):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.uint32)


@pytest.mark.parametrize("L", [1, 7, 20, 21, 64, 100, 300])
def test_forward_matches_oracle(tiny, L):
    eng, head, om = tiny
    ids = ids_for(L, L)
    rows = sorted({0, L // 2, L - 1})
    got = eng.forward(ids, rows).hidden
    want, _ = om.forward(ids, rows)
    err = np.abs(got - want).max()
    assert err < HIDDEN_TOL, f"L={L}: max |dh| {err}"


def test_snapshot_continuation_matches_full_forward(tiny, oracle):
    eng, head, om = tiny
    state, q = ids_for(1, 150), ids_for(2, 40)
    opts = [3, 10, 20]
    rows = opts + [len(q) - 1]
    prefix = eng.forward(state, [], keep=True).snapshot
    assert prefix.len == 150
    cached = eng.forward(q, rows, cache=prefix).hidden
    full = eng.forward(np.concatenate([state, q]), [150 + r for r in rows]).hidden
    assert np.abs(cached - full).max() < HIDDEN_TOL
    pa, pb = head.probs(cached, cached.shape[1], 1.0), head.probs(full, full.shape[1], 1.0)
    assert np.abs(pa - pb).max() < PROB_TOL
    # the same snapshot twice in a row (the K/V prefix is not restored the second time)
    again = eng.forward(q, rows, cache=prefix).hidden
    np.testing.assert_array_equal(again, cached)
    # the oracle's own continuation agrees with the GPU's
    _, osnap = om.forward(state, [], keep=True)
    ocached, _ = om.forward(q, rows, cache=osnap)
    assert np.abs(cached - ocached).max() < HIDDEN_TOL
    prefix.free()


def test_ask_ids_matches_oracle(tiny, sdamd):
    eng, head, om = tiny
    state = ids_for(3, 120)
    qs = [ids_for(10 + i, 30 + 5 * i) for i in range(3)]
    options = [[2, 5], [1, 4, 9], [3, 6, 12, 18, 25]]
    temps = [1.0, 0.7, 1.3]
    got = sdamd.ask_ids(eng, head, state, qs, options, temps)
    _, snap = om.forward(state, [], keep=True)
    for q, o, t, g in zip(qs, options, temps, got):
        rows = list(o) + [len(q) - 1]
        h, _ = om.forward(q, rows, cache=snap)
        want = om.probs(h, t)
        assert np.abs(g - want).max() < PROB_TOL
        # the answer must match exactly (these seeds' top-two margins are 0.076 to 0.87, far above PROB_TOL)
        assert int(np.argmax(g)) == int(np.argmax(want))
    # one question: a single forward of state ++ question
    one = sdamd.ask_ids(eng, head, state, qs[:1], options[:1], temps[:1])[0]
    assert np.abs(one - got[0]).max() < PROB_TOL


# (state tokens, question lengths): states shorter than the conv window (1-3 tokens: the branches'
# conv reads the history the state's scan leaves), one whole chunk, 8 mixed lengths, and 31
# questions (state + 31 branches = the 32 sequences a forward holds)
TREE_CASES = [(1, [21, 40]), (2, [64, 23]), (3, [30, 64, 22]), (64, [65, 21]),
              (130, [24, 33, 64, 21, 50, 41, 29, 60]), (200, [21] * 31)]


@pytest.mark.parametrize("case", range(len(TREE_CASES)))
def test_ask_ids_tree_matches_snapshot_path(tiny, sdamd, case):
    """ask_ids with every question longer than 20 tokens runs one forward of the state with every
    question as a branch of it (the branches attend the state's rows and their own; their delta rule
    continues from the state's final state and history).  Each question's probabilities match the
    snapshot path's (the state's forward with keep, then the questions from the snapshot,
    src/lib.rs:192-198) and the oracle's forward of that question from the state's snapshot."""
    eng, head, om = tiny
    ns, lens = TREE_CASES[case]
    state = ids_for(900 + case, ns)
    qs = [ids_for(1000 + 50 * case + i, L) for i, L in enumerate(lens)]
    options = [sorted(np.random.default_rng(2000 + 50 * case + i).choice(L - 1, 3, replace=False).tolist())
               for i, L in enumerate(lens)]
    temps = [1.0] * len(lens)
    snap = eng.forward(state, [], keep=True).snapshot
    via_snap, _ = eng.ask_batch(head, qs, options, temps, cache=snap)
    got = sdamd.ask_ids(eng, head, state, qs, options, temps)
    # the tree forward rewrote the live K/V rows and states: the same snapshot continuation again
    # restores its prefix and gives the same bits
    again, _ = eng.ask_batch(head, qs, options, temps, cache=snap)
    snap.free()
    for i in range(len(qs)):
        np.testing.assert_array_equal(again[i], via_snap[i])
    _, osnap = om.forward(state, [], keep=True)
    for i, (q, o) in enumerate(zip(qs, options)):
        h, _ = om.forward(q, list(o) + [len(q) - 1], cache=osnap)
        want = om.probs(h, 1.0)
        top = np.sort(want)
        # these seeds' top-two margins are 0.0054 to 0.50: an argmax flip is a real error
        assert top[-1] - top[-2] > 2 * PROB_TOL
        assert np.abs(got[i] - via_snap[i]).max() < PROB_TOL, f"question {i}"
        assert np.abs(got[i] - want).max() < PROB_TOL, f"question {i}"
        assert int(np.argmax(got[i])) == int(np.argmax(want)), f"question {i}"


@pytest.mark.parametrize("last", ["full_attention", "linear_attention"])
def test_cache_only_forward_leaves_the_same_snapshot(sdamd, synth, tmp_path_factory, last):
    """A forward that reads no hidden row runs only the cache-writing steps of its last layer (qkv and
    qk_prep, or in_proj and the delta rule): its snapshot continues exactly as that of a forward of
    the same tokens that reads rows (the steps writing the cache are the same kernels on the same
    inputs; an attention layer's K/V-only GEMM runs the full qkv GEMM's configuration on fewer
    columns), for a last layer of either kind, at state lengths on the short-input and the prefill
    GEMM plans."""
    cfg = dict(synth.CONFIG_TINY)
    if last == "linear_attention":
        cfg["layer_types"] = (["full_attention"] + ["linear_attention"] * 3) * 2
    path = synth.write_model(str(tmp_path_factory.mktemp("co")), cfg, vocab=4096, seed=3)
    eng, head, _ = sdamd.load_decider(path)
    try:
        for n_state in (90, 150, 300, 700):
            state, q = ids_for(60 + n_state, n_state), ids_for(61, 37)
            rows = [2, 11, 36]
            bare = eng.forward(state, [], keep=True).snapshot
            read = eng.forward(state, [0, n_state - 1], keep=True).snapshot
            a = eng.forward(q, rows, cache=bare).hidden
            b = eng.forward(q, rows, cache=read).hidden
            np.testing.assert_array_equal(a, b)
            bare.free()
            read.free()
    finally:
        eng.free()


@pytest.mark.parametrize("last", ["full_attention", "linear_attention"])
def test_compact_last_layer_matches_the_full_tail(sdamd, synth, oracle, tmp_path_factory, last):
    """A forward reading at most half its rows runs its last layer's tail (o_proj or out_proj, the
    residual add + norm, the MLP) on those rows only, gathered after the token mixer.  Rows read in
    any order, repeated, and single: the same hidden rows (within the tolerance: the tail's matmuls
    then have another M) as a forward reading every row, and, without the repeat, as the oracle.
    (A repeated row is a race in the reference's final norm, which adds the sublayer output to the
    residual row in place once per read; the oracle adds it twice, the compact tail once.)"""
    cfg = dict(synth.CONFIG_TINY)
    if last == "linear_attention":
        cfg["layer_types"] = (["full_attention"] + ["linear_attention"] * 3) * 2
    path = synth.write_model(str(tmp_path_factory.mktemp("ct")), cfg, vocab=4096, seed=4)
    eng, head, _ = sdamd.load_decider(path)
    om = oracle.OracleModel(path)
    try:
        for L, rows in ((100, [77, 3, 99, 3, 50]), (130, [129]), (41, [0, 40, 20])):
            ids = ids_for(70 + L, L)
            every = eng.forward(ids, list(range(L))).hidden
            got = eng.forward(ids, rows).hidden
            assert np.abs(got - every[rows]).max() < HIDDEN_TOL
            uniq = list(dict.fromkeys(rows))
            want, _ = om.forward(ids, uniq)
            assert np.abs(eng.forward(ids, uniq).hidden - want).max() < HIDDEN_TOL
    finally:
        eng.free()


def test_forward_errors(tiny, sdamd):
    eng, head, om = tiny
    with pytest.raises(sdamd.EngineError, match="must be 1 to 4096"):
        eng.forward(np.zeros(0, np.uint32), [])
    with pytest.raises(sdamd.EngineError, match="out of range"):
        eng.forward(ids_for(4, 5), [5])
    with pytest.raises(sdamd.EngineError, match="must be 1 to 4096"):
        eng.forward(ids_for(5, 4097), [0])
    snap = eng.forward(ids_for(6, 4000), [], keep=True).snapshot
    with pytest.raises(sdamd.EngineError, match="context of 4100"):
        eng.forward(ids_for(7, 100), [0], cache=snap)
    snap.free()
    # the engine still works after the errors
    h = eng.forward(ids_for(8, 10), [9]).hidden
    assert np.isfinite(h).all()


def test_profile_labels(tiny):
    eng, _, _ = tiny
    prof = eng.profile(ids_for(9, 64))
    labels = {k for k, _ in prof}
    assert {"embed", "norm", "in_proj", "conv", "gdn", "gnorm", "out_proj", "qkv", "qk_prep", "attn", "o_proj",
            "gate_up", "silu", "down"} <= labels
    assert all(ms >= 0 for _, ms in prof)


@pytest.mark.parametrize("lens", [(40, 25, 70, 64, 129), (5, 12, 20), (33,), (100, 24, 30)])
def test_forward_batch_matches_separate_forwards(tiny, lens):
    """Independent sequences in one forward == each sequence's own forward from the snapshot
    (conv history, GDN state, RoPE positions and attention masks per sequence).  Batches of at most
    64 tokens per sequence on average take the token-by-token delta rule with the conv inside it;
    (100, 24, 30) gives it a sequence of two 64-token blocks, whose second block's conv reads the
    first block's rows."""
    eng, head, om = tiny
    state = ids_for(20, 150)
    seqs = [ids_for(30 + i, n) for i, n in enumerate(lens)]
    rows = [sorted({0, n // 3, n - 1}) for n in lens]
    prefix = eng.forward(state, [], keep=True).snapshot
    got, _ = eng.forward_batch(seqs, rows, cache=prefix)
    for q, r, g in zip(seqs, rows, got):
        want = eng.forward(q, r, cache=prefix).hidden
        err = np.abs(g - want).max()
        assert err < HIDDEN_TOL, f"lens {lens}: max |dh| {err} vs the separate forward"
    # and against the oracle's continuation, for the longest sequence
    _, osnap = om.forward(state, [], keep=True)
    k = int(np.argmax(lens))
    owant, _ = om.forward(seqs[k], rows[k], cache=osnap)
    assert np.abs(got[k] - owant).max() < HIDDEN_TOL
    # the prefix is intact afterwards: a plain continuation still matches
    again = eng.forward(seqs[0], rows[0], cache=prefix).hidden
    assert np.abs(again - got[0]).max() < HIDDEN_TOL
    prefix.free()


def test_forward_batch_random_mixes(tiny):
    """Seeded random batches (1 to 6 sequences of 21 to 90 tokens, or of 1 to 20) from one snapshot
    against each sequence's own forward.  The batch and its parts run different plans: the chunked or
    the token-by-token delta rule (with the conv inside it) by average length, the question-size or
    prefill GEMM tiles by total rows, the short-row GEMV below 21 rows."""
    eng, head, om = tiny
    rng = np.random.default_rng(77)
    prefix = eng.forward(ids_for(60, 90), [], keep=True).snapshot
    for case in range(8):
        nseq = int(rng.integers(1, 7))
        lo, hi = (1, 21) if case == 7 else (21, 91)
        lens = [int(rng.integers(lo, hi)) for _ in range(nseq)]
        seqs = [ids_for(1000 + 10 * case + i, n) for i, n in enumerate(lens)]
        rows = [sorted({0, n // 2, n - 1}) for n in lens]
        got, _ = eng.forward_batch(seqs, rows, cache=prefix)
        for q, r, g in zip(seqs, rows, got):
            want = eng.forward(q, r, cache=prefix).hidden
            err = np.abs(g - want).max()
            assert err < HIDDEN_TOL, f"case {case}, lens {lens}: max |dh| {err} vs the separate forward"
    prefix.free()


def test_forward_batch_without_prefix(tiny):
    eng, head, om = tiny
    seqs = [ids_for(40, 50), ids_for(41, 90)]
    rows = [[0, 49], [10, 89]]
    got, _ = eng.forward_batch(seqs, rows)
    for q, r, g in zip(seqs, rows, got):
        want, _ = om.forward(q, r)
        assert np.abs(g - want).max() < HIDDEN_TOL


def test_forward_batch_errors(tiny, sdamd):
    eng, head, om = tiny
    with pytest.raises(sdamd.EngineError, match="mixes sequences"):
        eng.forward_batch([ids_for(50, 10), ids_for(51, 30)], [[0], [0]])
    with pytest.raises(sdamd.EngineError, match="1 to 32 sequences"):
        eng.forward_batch([ids_for(52 + i, 30) for i in range(33)], [[0]] * 33)
    with pytest.raises(sdamd.EngineError, match="has no tokens"):
        eng.forward_batch([ids_for(53, 30), np.zeros(0, np.uint32)], [[0], []])
    snap = eng.forward(ids_for(54, 4000), [], keep=True).snapshot
    with pytest.raises(sdamd.EngineError, match="at most 4096"):
        eng.forward_batch([ids_for(55, 60), ids_for(56, 60)], [[0], [0]], cache=snap)
    snap.free()
    h = eng.forward(ids_for(57, 10), [9]).hidden
    assert np.isfinite(h).all()


def test_ask_ids_mixed_lengths(tiny, sdamd):
    """Questions of <= 20 tokens and longer ones go to separate batches; every answer matches the
    oracle's own forward of that question from the prefix."""
    eng, head, om = tiny
    state = ids_for(60, 90)
    qs = [ids_for(61, 10), ids_for(62, 45), ids_for(63, 18), ids_for(64, 70)]
    options = [[1, 4], [2, 9, 30], [0, 5, 11], [3, 50]]
    temps = [1.0, 1.0, 0.5, 2.0]
    got = sdamd.ask_ids(eng, head, state, qs, options, temps)
    _, snap = om.forward(state, [], keep=True)
    for q, o, t, g in zip(qs, options, temps, got):
        h, _ = om.forward(q, list(o) + [len(q) - 1], cache=snap)
        assert np.abs(g - om.probs(h, t)).max() < PROB_TOL


def test_ask_batch_device_head_matches_host_head(tiny, sdamd):
    """The pointer head on the device (f64) against Head::probs on the host (src/head.rs:66-77) on the
    same hidden rows: the torso is deterministic, so only the f64 summation order differs."""
    eng, head, om = tiny
    state = ids_for(70, 100)
    qs = [ids_for(71, 33), ids_for(72, 47), ids_for(73, 25)]
    options = [[1, 5, 20], [2, 40], [0, 3, 7, 11, 24]]
    temps = [1.0, 0.8, 1e-9]  # the last one exercises the max(T, 1e-6) floor
    prefix = eng.forward(state, [], keep=True).snapshot
    got, ms = eng.ask_batch(head, qs, options, temps, cache=prefix, timed=True)
    assert ms is not None and ms > 0
    hid, _ = eng.forward_batch(qs, [list(o) + [len(q) - 1] for q, o in zip(qs, options)], cache=prefix)
    for g, h, t in zip(got, hid, temps):
        want = head.probs(h, h.shape[1], t)
        assert g.shape == want.shape
        assert np.abs(g - want).max() < 1e-9
        assert abs(g.sum() - 1.0) < 1e-12
    # without a prefix: each question is a whole sequence
    got0, _ = eng.ask_batch(head, qs[:2], options[:2], temps[:2])
    hid0, _ = eng.forward_batch(qs[:2], [list(o) + [len(q) - 1] for q, o in zip(qs[:2], options[:2])])
    for g, h, t in zip(got0, hid0, temps):
        assert np.abs(g - head.probs(h, h.shape[1], t)).max() < 1e-9
    with pytest.raises(sdamd.EngineError, match="out of range"):
        eng.ask_batch(head, qs[:1], [[33]], [1.0], cache=prefix)
    with pytest.raises(sdamd.EngineError, match="no options"):
        eng.ask_batch(head, qs[:1], [[]], [1.0], cache=prefix)
    prefix.free()


def test_rotated_torso_unrotate_on_device(sdamd, synth, oracle, tmp_path_factory):
    """A rotated torso (src/engine.rs:652-660): hidden rows are unrotate * FWHT(row).  forward applies
    it on the host, ask_ids on the device before the head; both match the oracle."""
    cfg = dict(synth.CONFIG_TINY)
    d = cfg["hidden_size"]
    cfg["unrotate"] = [float(x) for x in np.random.default_rng(9).choice([-1.0, 1.0], d) / np.sqrt(d)]
    path = synth.write_model(str(tmp_path_factory.mktemp("rot")), cfg, vocab=4096, seed=1)
    eng, head, _ = sdamd.load_decider(path)
    om = oracle.OracleModel(path)
    try:
        state, q = ids_for(80, 60), ids_for(81, 30)
        rows = [4, 12, 29]
        got = eng.forward(np.concatenate([state, q]), [60 + r for r in rows]).hidden
        want, _ = om.forward(np.concatenate([state, q]), [60 + r for r in rows])
        assert np.abs(got - want).max() < HIDDEN_TOL
        qs = [q, ids_for(82, 26)]
        options = [[4, 12], [3, 9, 20]]
        probs = sdamd.ask_ids(eng, head, state, qs, options, [1.0, 1.0])
        _, snap = om.forward(state, [], keep=True)
        for qq, o, g in zip(qs, options, probs):
            h, _ = om.forward(qq, list(o) + [len(qq) - 1], cache=snap)
            assert np.abs(g - om.probs(h, 1.0)).max() < PROB_TOL
    finally:
        eng.free()


@pytest.mark.parametrize("rd", [32, 12])
def test_other_rotary_dims_forward_and_questions(sdamd, synth, oracle, tmp_path_factory, rd):
    """rotary_dim 32 and 12: the attention reads the queries qk_prep wrote (with rotary_dim 64, the
    tiny and 2B configs' value, it normalizes and rotates them itself; 12 is not a multiple of 8, so
    qk_prep reads the rotate-half partners back from LDS); a forward and a one-forward ask_ids
    against the oracle."""
    cfg = dict(synth.CONFIG_TINY, rotary_dim=rd)
    path = synth.write_model(str(tmp_path_factory.mktemp(f"rd{rd}")), cfg, vocab=4096, seed=2)
    eng, head, _ = sdamd.load_decider(path)
    om = oracle.OracleModel(path)
    try:
        state, q = ids_for(90, 70), ids_for(91, 33)
        rows = [0, 17, 32]
        got = eng.forward(np.concatenate([state, q]), [70 + r for r in rows]).hidden
        want, _ = om.forward(np.concatenate([state, q]), [70 + r for r in rows])
        assert np.abs(got - want).max() < HIDDEN_TOL
        qs = [q, ids_for(92, 25), ids_for(93, 41)]
        options = [[4, 12], [3, 9, 20], [1, 30]]
        probs = sdamd.ask_ids(eng, head, state, qs, options, [1.0, 1.0, 1.0])
        _, snap = om.forward(state, [], keep=True)
        for qq, o, g in zip(qs, options, probs):
            h, _ = om.forward(qq, list(o) + [len(qq) - 1], cache=snap)
            assert np.abs(g - om.probs(h, 1.0)).max() < PROB_TOL
    finally:
        eng.free()


def test_interleaved_snapshots_read_in_place(tiny, sdamd):
    """Question forwards read each snapshot's GDN states and conv histories in place (no restore
    copy).  Alternating between two snapshots, batching from one, and chaining a keep-forward from a
    snapshot must each continue their own prefix, as the oracle's copies do."""
    eng, head, om = tiny
    s1, s2 = ids_for(90, 70), ids_for(91, 45)
    q1, q2, q3 = ids_for(92, 30), ids_for(93, 2), ids_for(94, 25)
    rows1, rows2, rows3 = [0, 14, 29], [0, 1], [3, 24]
    a = eng.forward(s1, [], keep=True).snapshot
    b = eng.forward(s2, [], keep=True).snapshot
    _, oa = om.forward(s1, [], keep=True)
    _, ob = om.forward(s2, [], keep=True)
    for snap, osnap, q, r in [(a, oa, q1, rows1), (b, ob, q2, rows2), (a, oa, q2, rows2), (b, ob, q1, rows1)]:
        got = eng.forward(q, r, cache=snap).hidden
        want, _ = om.forward(q, r, cache=osnap)
        assert np.abs(got - want).max() < HIDDEN_TOL
    got, _ = eng.forward_batch([q1, q3], [rows1, rows3], cache=b)
    for g, q, r in zip(got, [q1, q3], [rows1, rows3]):
        want, _ = om.forward(q, r, cache=ob)
        assert np.abs(g - want).max() < HIDDEN_TOL
    # a keep-forward from snapshot a, then a question from the new snapshot (a + q3)
    c = eng.forward(q3, [], cache=a, keep=True).snapshot
    _, oc = om.forward(q3, [], cache=oa, keep=True)
    assert c.len == len(s1) + len(q3)
    got = eng.forward(q1, rows1, cache=c).hidden
    want, _ = om.forward(q1, rows1, cache=oc)
    assert np.abs(got - want).max() < HIDDEN_TOL
    # the snapshots are unchanged by all of it
    again = eng.forward(q2, rows2, cache=b).hidden
    want, _ = om.forward(q2, rows2, cache=ob)
    assert np.abs(again - want).max() < HIDDEN_TOL
    for s in (a, b, c):
        s.free()


@pytest.mark.parametrize("rd", [13, 0, 258])
def test_rotary_dim_checked_at_load(sdamd, synth, tmp_path, rd):
    """Rotate-half pairs dim d with d + rotary_dim / 2 over a table of rotary_dim / 2 (cos, sin)
    pairs per position: an odd rotary_dim, none, or one past head_dim fails at load instead of
    giving wrong Q/K."""
    cfg = dict(synth.CONFIG_TINY, rotary_dim=rd)
    d = synth.write_model(str(tmp_path / f"rd{rd}"), cfg, vocab=512, seed=5)
    with pytest.raises(sdamd.EngineError, match="rotary_dim must be even, from 2 to head_dim"):
        sdamd.Engine.load(d)


def test_plan_cache_evicts_and_recaptures(tiny):
    """More distinct lengths than the plan cache holds: the least recently used plans are evicted,
    and a length whose plan was evicted is captured again with the same result, bit for bit."""
    eng, head, om = tiny
    first = eng.forward(ids_for(11, 23), [0, 22]).hidden
    # longest first, so the pool grows once (which drops every plan) and then only evictions follow
    for L in range(640, 640 - 530, -1):
        eng.forward(ids_for(L, L), [L - 1])
    again = eng.forward(ids_for(11, 23), [0, 22]).hidden
    assert np.array_equal(first, again)
    # the cache holds at most 512 plans: the lengths used first were evicted and are captured again
    h = eng.forward(ids_for(640, 640), [639]).hidden
    assert np.isfinite(h).all()


def test_load_rejects_matrices_sharing_memory_with_other_shapes(sdamd, tiny_model, tmp_path):
    """Two manifest matrices at the same offset with different shapes are refused at load: the
    rewrite into the engine layout happens once per memory, so a GEMM would otherwise read one of
    them in the wrong bit order.  Same-shaped aliases still load."""
    import json
    import os
    import shutil
    d = tmp_path / "alias"
    shutil.copytree(tiny_model, d)
    with open(d / "manifest.json") as f:
        man = json.load(f)
    t = man["tensors"]
    a, b = "layers.0.in_proj", "layers.0.gate_up"
    assert (t[a + ".q"]["N"], t[a + ".q"]["K"]) != (t[b + ".q"]["N"], t[b + ".q"]["K"])
    bad = json.loads(json.dumps(man))
    for part in (".q", ".s"):  # point in_proj at gate_up's larger words and scales
        bad["tensors"][a + part]["offset"] = t[b + part]["offset"]
    with open(d / "manifest.json", "w") as f:
        json.dump(bad, f)
    with pytest.raises(sdamd.EngineError, match="share memory with different shapes"):
        sdamd.Engine.load(str(d))
    # an alias of the same shape and format loads, and the shared matrix is rewritten once
    same = json.loads(json.dumps(man))
    for part in (".q", ".s"):
        same["tensors"]["layers.4.gate_up" + part]["offset"] = t[b + part]["offset"]
    assert (t["layers.4.gate_up.q"]["N"], t["layers.4.gate_up.q"]["K"]) == (t[b + ".q"]["N"], t[b + ".q"]["K"])
    with open(d / "manifest.json", "w") as f:
        json.dump(same, f)
    eng = sdamd.Engine.load(str(d))
    try:
        h = eng.forward(ids_for(11, 30), [29]).hidden
        assert np.isfinite(h).all()
    finally:
        eng.free()


def test_checked_mode(sdamd, tiny_model, tmp_path, monkeypatch):
    """STRANDS_DECIDER_CHECKED=1 (the reference's runtime-check switch, src/engine.rs:283, 335-338):
    every step runs eagerly and is synchronized.  Results are bit-identical to the captured graphs',
    and a residual stream gone non-finite is reported with the step that produced it (forced from
    the host: one layer's out_proj scales set to f16 infinity), where the unchecked engine returns
    the non-finite rows silently."""
    import json
    import os
    import shutil
    eng = sdamd.Engine.load(tiny_model)
    monkeypatch.setenv("STRANDS_DECIDER_CHECKED", "1")
    chk = sdamd.Engine.load(tiny_model)
    monkeypatch.delenv("STRANDS_DECIDER_CHECKED")
    try:
        for L in (7, 100):
            ids = ids_for(70 + L, L)
            np.testing.assert_array_equal(chk.forward(ids, [0, L - 1]).hidden, eng.forward(ids, [0, L - 1]).hidden)
    finally:
        chk.free()
        eng.free()
    d = tmp_path / "inf"
    shutil.copytree(tiny_model, d)
    with open(d / "manifest.json") as f:
        man = json.load(f)
    t = man["tensors"]["layers.1.out_proj.s"]
    sh = next(s for s in man["shards"] if s["start"] <= t["offset"] < s["start"] + s["bytes"])
    path = d / sdamd.model.shard_file(man["shards"].index(sh))
    raw = bytearray(path.read_bytes())
    off = t["offset"] - sh["start"]
    raw[off:off + t["bytes"]] = np.full(t["bytes"] // 2, 0x7C00, np.uint16).tobytes()
    path.write_bytes(bytes(raw))
    bad = sdamd.Engine.load(str(d))
    try:
        h = bad.forward(ids_for(80, 30), [29]).hidden
        assert not np.isfinite(h).all()
    finally:
        bad.free()
    monkeypatch.setenv("STRANDS_DECIDER_CHECKED", "1")
    bad = sdamd.Engine.load(str(d))
    monkeypatch.delenv("STRANDS_DECIDER_CHECKED")
    try:
        with pytest.raises(sdamd.EngineError, match=r"step \d+ \(norm\).*non-finite"):
            bad.forward(ids_for(80, 30), [29])
        # the error is raised before the rows are read back; the engine still works afterwards
        with pytest.raises(sdamd.EngineError, match="non-finite"):
            bad.forward(ids_for(81, 5), [4])
    finally:
        bad.free()

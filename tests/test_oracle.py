"""Pins the CPU oracle (oracle/oracle.c, oracle/torso.py) before it is trusted as the checker of
the HIP path.  Every restated function is checked against something that does not share its code:
numpy's IEEE f16 conversion, the golden fixtures written by tests/golden/make_golden.py from
float64 brute force, transformers' gated-delta-rule and torch attention, closed forms in float64,
scipy's Hadamard matrix, and the model-level prefix/continuation invariant.

The reference itself (Rust + wgpu) cannot be built or run here, and its own fixtures
(tests/fixtures/browser.json, expected.json) need the hosted weights and tokenizer, which are not
available offline; they pin nothing for a random-init model.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

from conftest import f16_ulp

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import cases  # noqa: E402

I = ctypes.c_int


def golden(name):
    return np.load(os.path.join(HERE, "golden", name + ".npz"))


def within_ulp(got, want, ulps=1.0, extra=0.0):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    err = np.abs(got - want)
    tol = ulps * f16_ulp(want) * 1.001 + extra
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} beyond {ulps} f16 ulp; max err {err.max()}"


# ---- f16 conversions --------------------------------------------------------------------------

def test_h2f_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.h2f(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_round_to_nearest_even(oracle):
    rng = np.random.default_rng(0)
    # every f16 value, the exact midpoints between neighbours (ties), and one f32 ulp either side
    h = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    near = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0001,
                        2.0**-14, 2.0**-14 * (1 - 2.0**-11), np.inf, -np.inf, np.nan], np.float32)
    x = np.concatenate([h.astype(np.float32), near, -near, bits, special]).astype(np.float32)
    got = oracle.f2h(x)
    want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)


# ---- quantized matmul -------------------------------------------------------------------------

def _mm_args(c):
    return (c["W"], c["S"].view(np.uint16), c["N"], c["K"])


@pytest.mark.parametrize("name", list(cases.MATMUL_CASES))
def test_dequant_bit_exact(oracle, name):
    c = cases.matmul_inputs(name)
    g = golden("matmul")
    assert str(g[f"{name}.digest"]) == cases.digest(c["A"], c["W"], c["S"], c["B"]), "input generator drifted"
    Bi = c["B"].view(np.uint16) if c["asym"] else None
    kw = dict(bits=c["bits"], group=c["group"], asym=c["asym"], Bi=Bi)
    d32 = oracle.dequant(*_mm_args(c), f16_deq=False, **kw)
    d16 = oracle.dequant(*_mm_args(c), f16_deq=True, **kw)
    assert cases.digest(d32) == str(g[f"{name}.deq32"])
    assert cases.digest(d16) == str(g[f"{name}.deq16"])
    if name == "m_int4_small":  # the two dequant modes really differ on these scales
        assert (d32 != d16).mean() > 0.3


def test_dequant_known_answer(oracle):
    """One 32-block per format with scale 2, bias 0.5: the values follow from the code table."""
    codes = np.tile(np.arange(16, dtype=np.uint32), 2)[None, :]
    one16 = np.array([2.0], np.float16).view(np.uint16)
    d = oracle.dequant(cases.pack_codes(codes, 4), one16, 1, 32, False)
    assert np.array_equal(d[0], (codes[0].astype(np.float32) - 8) * 2)
    # int4 word layout: element e in word e/8 at bits 4(e%8)
    assert cases.pack_codes(np.arange(32, dtype=np.uint32)[None, :] % 16, 4)[0, 0, 0] == 0x76543210
    c3 = (np.arange(32, dtype=np.uint32) % 8)[None, :]
    b = np.array([0.5], np.float16).view(np.uint16)
    d = oracle.dequant(cases.pack_codes(c3, 3), one16, 1, 32, False, bits=3, group=32, asym=True, Bi=b)
    assert np.array_equal(d[0], c3[0] * 2.0 + 0.5)
    c2 = (np.arange(32, dtype=np.uint32) % 4)[None, :]
    d = oracle.dequant(cases.pack_codes(c2, 2), one16, 1, 32, False, bits=2, group=32)
    assert np.array_equal(d[0], (c2[0].astype(np.float32) - 2) * 2)


@pytest.mark.parametrize("name", list(cases.MATMUL_CASES))
@pytest.mark.parametrize("f16_deq", [False, True])
def test_matmul_matches_brute_force(oracle, name, f16_deq):
    """f32 accumulation vs the float64 brute force: within one f16 rounding of the output."""
    c = cases.matmul_inputs(name)
    g = golden("matmul")
    Bi = c["B"].view(np.uint16) if c["asym"] else None
    Y = oracle.matmul(c["A"].view(np.uint16), *_mm_args(c), f16_deq, bits=c["bits"], group=c["group"],
                      asym=c["asym"], Bi=Bi)
    within_ulp(oracle.h2f(Y), g[f"{name}.{'y16' if f16_deq else 'y32'}"].astype(np.float32), extra=1e-6)


# ---- embedding and the hosted model's scale codes ---------------------------------------------

EMBED_FORMATS = [(4, 32, False), (3, 32, False), (3, 64, True), (2, 128, False), (4, 64, True), (2, 32, True)]


@pytest.mark.parametrize("bits,group,asym", EMBED_FORMATS)
def test_embed_matches_independent_decode(oracle, bits, group, asym):
    """or_embed (src/kernels.rs:63-89) against the float64 decode of tests/golden/make_golden.py,
    written from the format description: (q - 2^(bits-1)) s is exact in f32, and q s + b rounds once
    in both, so the rows agree bit for bit.  Codes, scales and biases are independent draws; the
    ids repeat and go out of order."""
    import make_golden
    rng = np.random.default_rng(bits * 100 + group + asym)
    vocab, d = 37, 256
    codes = rng.integers(0, 1 << bits, size=(vocab, d), dtype=np.uint32)
    Q = cases.pack_codes(codes, bits)
    S = rng.uniform(-0.05, 0.05, size=vocab * d // group).astype(np.float16)
    B = rng.uniform(-0.3, 0.3, size=vocab * d // group).astype(np.float16) if asym else None
    ids = rng.integers(0, vocab, 50).astype(np.uint32)
    ids[:3] = [vocab - 1, 0, vocab - 1]
    x = oracle.embed(ids, Q, S.view(np.uint16), d, bits, group, asym, None if B is None else B.view(np.uint16))
    want = make_golden.decode(codes, S, B, vocab, d, bits, group, asym)[ids].astype(np.float32)
    assert np.array_equal(x.view(np.uint32), want.view(np.uint32))


def test_add_bias_closed_form(oracle):
    """or_add_bias (src/kernels.rs:138-149): one f32 add of the f16 value and the f32 bias, rounded
    to f16 (numpy's IEEE arithmetic)."""
    rng = np.random.default_rng(13)
    y = (4 * rng.standard_normal((9, 48))).astype(np.float16)
    c = rng.standard_normal(48).astype(np.float32)
    c[:4] = [0.0, 65504.0, 1e-8, -3.0]
    got = oracle.add_bias(y.view(np.uint16), c)
    want = (y.astype(np.float32) + c[None, :]).astype(np.float16)
    assert np.array_equal(got, want.view(np.uint16))


def _scale_rows(m, j, codes):
    head = np.zeros((len(m), 2), np.uint16)
    head[:, 0] = np.asarray(m, np.float16).view(np.uint16)
    head[:, 1] = j
    return head.view(np.uint8).reshape(len(m), 4), np.asarray(codes, np.uint8)


def test_decode_scale_codes_known_answers(oracle):
    """src/model.rs:217-236 at the exponents whose power of two is exact: k j = 0, 4096, 8192 and
    12288 give m, m/2, m/4, m/8; the code's top bit is the sign; j = 0 gives m for every k."""
    m = [0.01, 3.5, 1e-3, 65504.0]
    j = [4096, 2048, 1024, 0]
    codes = [[0, 1, 2, 3, 128, 129], [0, 2, 4, 6, 130, 132], [0, 4, 8, 12, 128 | 8, 128 | 12],
             [0, 17, 127, 128, 128 | 5, 255]]
    h, c = _scale_rows(m, j, codes)
    got = oracle.decode_scale_rows(h, c).view(np.float16).astype(np.float64)
    m16 = np.asarray(m, np.float16).astype(np.float64)
    want = np.array([[1, 1 / 2, 1 / 4, 1 / 8, -1, -1 / 2], [1, 1 / 2, 1 / 4, 1 / 8, -1 / 2, -1 / 4],
                     [1, 1 / 2, 1 / 4, 1 / 8, -1 / 4, -1 / 8], [1, 1, 1, -1, -1, -1]]) * m16[:, None]
    assert np.array_equal(got, want)
    # the packed form (headers first, then all codes) reads the same values
    flat = np.concatenate([h.reshape(-1), c.reshape(-1)]).tobytes()
    assert np.array_equal(oracle.decode_scale_codes(flat, 4, 6), oracle.decode_scale_rows(h, c))


def test_decode_scale_codes_random(oracle):
    """Random headers and codes against exp2 in float64 (a different routine from the oracle's
    power), within one f16 rounding of the magnitude."""
    rng = np.random.default_rng(14)
    n, g = 40, 64
    m = rng.uniform(1e-3, 2.0, n)
    j = rng.integers(0, 400, n)
    c = rng.integers(0, 256, (n, g))
    h, cc = _scale_rows(m, j, c)
    got = oracle.decode_scale_rows(h, cc).view(np.float16).astype(np.float32)
    m16 = np.asarray(m, np.float16).astype(np.float64)
    mag = m16[:, None] * np.exp2(-(c & 127) * j[:, None] / 4096.0)
    want = np.where(c >= 128, -mag, mag).astype(np.float32)
    within_ulp(got, want, ulps=0.5, extra=0.0)


# ---- row and elementwise kernels --------------------------------------------------------------

def test_add_norm_closed_form(oracle):
    rng = np.random.default_rng(3)
    L, d = 7, 512
    x = rng.standard_normal((L, d)).astype(np.float32)
    y = rng.standard_normal((L, d)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    x0 = x.copy()
    h = oracle.add_norm(x, y.view(np.uint16), w)
    xs = x0 + y.astype(np.float32)
    assert np.array_equal(x, xs)  # residual update is one f32 add
    r = xs.astype(np.float64)
    want = r / np.sqrt((r * r).mean(1, keepdims=True) + 1e-6) * w
    within_ulp(oracle.h2f(h), want.astype(np.float32), extra=1e-6)
    rows = np.array([5, 0, 6], np.uint32)
    h32 = oracle.add_norm(x, None, w, rows=rows, out_f32=True)
    np.testing.assert_allclose(h32, want[rows], rtol=2e-6, atol=1e-6)


def test_silu_mul_closed_form(oracle):
    rng = np.random.default_rng(4)
    L, I_ = 5, 64
    big = (3 * rng.standard_normal((L, 2 * I_))).astype(np.float16)
    mid = np.empty((L, I_), np.uint16)
    oracle.lib().or_silu_mul(oracle.P(big.view(np.uint16)), I(L), I(I_), oracle.P(mid))
    g, u = big[:, :I_].astype(np.float64), big[:, I_:].astype(np.float64)
    within_ulp(oracle.h2f(mid), (g / (1 + np.exp(-g)) * u).astype(np.float32), extra=1e-7)


@pytest.mark.parametrize("L", [1, 2, 5])
def test_conv_and_history(oracle, L):
    """Depthwise causal conv over (3 history rows ++ this call's rows), SiLU; the history keeps the
    last 3 pre-conv rows of that concatenation."""
    rng = np.random.default_rng(L)
    C, stride = 16, 24
    big = rng.standard_normal((L, stride)).astype(np.float16)
    hist = rng.standard_normal((3, C)).astype(np.float16)
    w = rng.standard_normal((C, 4)).astype(np.float32)
    out = np.empty((L, C), np.float32)
    h = hist.view(np.uint16).copy()
    oracle.lib().or_conv(oracle.P(big.view(np.uint16)), I(stride), I(L), I(C), oracle.P(w), oracle.P(h), oracle.P(out))
    seq = np.concatenate([hist, big[:, :C]]).astype(np.float64)  # [3 + L, C]
    s = sum(w[:, j].astype(np.float64) * seq[j:j + L] for j in range(4))
    np.testing.assert_allclose(out, s / (1 + np.exp(-s)), rtol=1e-5, atol=1e-6)
    oracle.lib().or_hist_update(oracle.P(big.view(np.uint16)), I(stride), I(L), I(C), oracle.P(h))
    assert np.array_equal(h, np.concatenate([hist, big[:, :C]])[-3:].view(np.uint16))


def test_gnorm_closed_form(oracle):
    rng = np.random.default_rng(5)
    L, H, DV, z_off = 3, 2, 64, 10
    o = rng.standard_normal((L, H * DV)).astype(np.float32)
    stride = z_off + H * DV + 6
    big = rng.standard_normal((L, stride)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(DV)).astype(np.float32)
    out = np.empty((L, H * DV), np.uint16)
    oracle.lib().or_gnorm(oracle.P(o), oracle.P(big.view(np.uint16)), I(stride), I(z_off), oracle.P(w), I(L), I(H),
                          I(DV), oracle.P(out))
    o3 = o.reshape(L, H, DV).astype(np.float64)
    z = big[:, z_off:z_off + H * DV].reshape(L, H, DV).astype(np.float64)
    want = w * o3 / np.sqrt((o3 ** 2).mean(-1, keepdims=True) + 1e-6) * z / (1 + np.exp(-z))
    within_ulp(oracle.h2f(out), want.reshape(L, -1).astype(np.float32), extra=1e-7)


# ---- gated delta rule -------------------------------------------------------------------------

def run_gdn(oracle, c, qkv=None, big=None, negA=None):
    qkv = c["qkv"] if qkv is None else qkv
    big = c["big"] if big is None else big
    negA = c["negA"] if negA is None else negA
    L, H, dk, dv = c["L"], c["H"], c["dk"], c["dv"]
    st = c["state0"].copy()
    o = np.empty((L, H * dv), np.float32)
    oracle.lib().or_gdn(oracle.P(qkv), oracle.P(big.view(np.uint16)), I(c["stride"]), I(c["a_off"]), I(c["b_off"]),
                        oracle.P(negA), oracle.P(c["dtb"]), I(L), I(H), I(dk), I(dv), oracle.P(st),
                        I(int(c["load"])), oracle.P(o))
    return o, st


@pytest.mark.parametrize("name", list(cases.GDN_CASES))
def test_gdn_matches_transformers(oracle, name):
    c = cases.gdn_inputs(name)
    g = golden("gdn")
    assert str(g[f"{name}.digest"]) == cases.digest(c["qkv"], c["big"], c["negA"], c["dtb"], c["state0"])
    o, st = run_gdn(oracle, c)
    np.testing.assert_allclose(o, g[f"{name}.o"], rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(st[:, ::cases.STATE_ROW_STEP], g[f"{name}.state"], rtol=1e-4, atol=2e-5)


def test_gdn_zero_beta_only_decays(oracle):
    """beta = sigmoid(-30) ~ 1e-13: no writes, S_t = e^(g_1 + .. + g_t) S_0 and o_t = S_t^T qn_t."""
    c = cases.gdn_inputs("g_l33_h2_rect")
    big = c["big"].copy()
    big[:, c["H"]:] = -30.0
    o, st = run_gdn(oracle, c, big=big)
    H, dk, dv, L = c["H"], c["dk"], c["dv"], c["L"]
    a = big[:, :H].astype(np.float64) + c["dtb"]
    gsum = np.cumsum(c["negA"] * np.where(a > 20, a, np.log1p(np.exp(a))), axis=0)  # [L, H]
    q = c["qkv"][:, :H * dk].reshape(L, H, dk).astype(np.float64)
    qn = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(dk)
    want = np.exp(gsum)[:, :, None] * np.einsum("hkv,lhk->lhv", c["state0"].astype(np.float64), qn)
    np.testing.assert_allclose(o, want.reshape(L, -1), rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(st, np.exp(gsum[-1])[:, None, None] * c["state0"], rtol=1e-4, atol=1e-7)


def test_gdn_softplus_passes_large_inputs_through(oracle):
    """softplus(x) = x above 20 (src/kernels.rs:286): a = 100 decays by e^(negA * 100) per token
    instead of overflowing exp."""
    c = cases.gdn_inputs("g_l5_h1_state")
    big = c["big"].copy()
    big[:, 0] = 100.0
    big[:, 1] = -30.0  # beta ~ 0: the state only decays
    negA = np.array([-0.005], np.float32)
    _, st = run_gdn(oracle, c, big=big, negA=negA)
    np.testing.assert_allclose(st, np.exp(-0.5 * c["L"]) * c["state0"], rtol=1e-5, atol=1e-8)


def test_gdn_orthonormal_keys_retrieve_values(oracle):
    """No decay (negA = 0), beta = 1 and orthonormal keys: the state is sum_i k_i v_i^T, so a query
    equal to an earlier key k_j reads back v_j / sqrt(dk)."""
    rng = np.random.default_rng(9)
    L, H, dk, dv = 12, 1, 32, 16
    keys = np.linalg.qr(rng.standard_normal((dk, dk)))[0][:L].astype(np.float32)  # orthonormal rows
    vals = rng.standard_normal((L, dv)).astype(np.float32)
    qidx = rng.integers(0, np.arange(L) + 1)  # query t asks for key qidx[t] <= t
    qkv = np.concatenate([keys[qidx] * 3.0, keys, vals], axis=1).astype(np.float32)  # |q| is normalized away
    big = np.zeros((L, 2), np.float16)
    big[:, 1] = 30.0
    c = dict(L=L, H=H, dk=dk, dv=dv, load=False, qkv=qkv, big=big, stride=2, a_off=0, b_off=1,
             negA=np.zeros(1, np.float32), dtb=np.zeros(1, np.float32), state0=np.zeros((H, dk, dv), np.float32))
    o, st = run_gdn(oracle, c)
    np.testing.assert_allclose(o, vals[qidx] / np.sqrt(dk), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(st[0], keys.T @ vals, rtol=1e-5, atol=1e-5)


# ---- attention ----------------------------------------------------------------------------------

def test_rope_table_f64(oracle):
    rd, theta = 64, 1e7
    t = oracle.rope_table(rd, theta, ctx=4096)
    pos = np.arange(4096, dtype=np.float64)[:, None]
    ang = pos / theta ** (np.arange(0, rd, 2, dtype=np.float64) / rd)
    np.testing.assert_allclose(t[:, 0::2], np.cos(ang).astype(np.float32), atol=1e-7, rtol=0)
    np.testing.assert_allclose(t[:, 1::2], np.sin(ang).astype(np.float32), atol=1e-7, rtol=0)


def test_qk_prep_closed_form(oracle):
    """RMSNorm (eps 1e-6) then rotate-half RoPE on the first rd dims at position P + t; V copied."""
    rng = np.random.default_rng(11)
    HQ, HK, HD, RD, L, P, LT = 2, 1, 64, 16, 4, 5, 12
    stride = 2 * HQ * HD + 2 * HK * HD
    big = rng.standard_normal((L, stride)).astype(np.float16)
    qw = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    rope = oracle.rope_table(RD, 1e4, ctx=LT)
    Q = np.empty((HQ, L, HD), np.uint16)
    K = np.zeros((HK, LT, HD), np.uint16)
    V = np.zeros((HK, LT, HD), np.uint16)
    oracle.lib().or_qk_prep(oracle.P(big.view(np.uint16)), I(stride), oracle.P(qw), oracle.P(kw), oracle.P(rope),
                            I(L), I(P), I(LT), I(HQ), I(HK), I(HD), I(RD), oracle.P(Q), oracle.P(K), oracle.P(V))

    def want(x, w, pos):
        x = x.astype(np.float64)
        n = x / np.sqrt((x * x).mean() + 1e-6) * w
        ang = pos / 1e4 ** (np.arange(0, RD, 2) / RD)
        c, s = np.cos(ang), np.sin(ang)
        r = n.copy()
        h = RD // 2
        r[:h] = n[:h] * c - n[h:RD] * s
        r[h:RD] = n[h:RD] * c + n[:h] * s
        return r

    for t in range(L):
        for hq in range(HQ):
            within_ulp(oracle.h2f(Q[hq, t]), want(big[t, hq * 2 * HD:hq * 2 * HD + HD], qw, P + t), extra=1e-6)
        k_off = 2 * HQ * HD
        within_ulp(oracle.h2f(K[0, P + t]), want(big[t, k_off:k_off + HD], kw, P + t), extra=1e-6)
        assert np.array_equal(V[0, P + t], big[t, k_off + HK * HD:k_off + 2 * HK * HD].view(np.uint16))
    assert not K[:, :P].any() and not K[:, P + L:].any()


@pytest.mark.parametrize("name", list(cases.ATTN_CASES))
def test_attention_matches_torch(oracle, name):
    c = cases.attn_inputs(name)
    g = golden("attn")
    assert str(g[f"{name}.digest"]) == cases.digest(c["Q"], c["K"], c["V"], c["big"])
    out = np.empty((c["L"], c["HQ"] * c["HD"]), np.uint16)
    oracle.lib().or_attn(oracle.P(c["Q"].view(np.uint16)), oracle.P(c["K"].view(np.uint16)),
                         oracle.P(c["V"].view(np.uint16)), oracle.P(c["big"].view(np.uint16)), I(c["stride"]),
                         I(c["L"]), I(c["P"]), I(c["LT"]), I(c["HQ"]), I(c["HK"]), I(c["HD"]), oracle.P(out))
    within_ulp(oracle.h2f(out), g[f"{name}.out"].astype(np.float32), extra=1e-6)


def test_attention_single_key_is_gated_value(oracle):
    c = cases.attn_inputs("a_first_token")
    out = np.empty((1, c["HQ"] * c["HD"]), np.uint16)
    oracle.lib().or_attn(oracle.P(c["Q"].view(np.uint16)), oracle.P(c["K"].view(np.uint16)),
                         oracle.P(c["V"].view(np.uint16)), oracle.P(c["big"].view(np.uint16)), I(c["stride"]),
                         I(1), I(0), I(c["LT"]), I(c["HQ"]), I(c["HK"]), I(c["HD"]), oracle.P(out))
    HD = c["HD"]
    for h in range(c["HQ"]):
        gate = c["big"][0, h * 2 * HD + HD:(h + 1) * 2 * HD].astype(np.float64)
        within_ulp(oracle.h2f(out[0, h * HD:(h + 1) * HD]), c["V"][0, 0].astype(np.float64) / (1 + np.exp(-gate)),
                   extra=1e-7)


# ---- unrotate and head ----------------------------------------------------------------------

def test_fwht_is_sylvester_hadamard(oracle):
    from scipy.linalg import hadamard
    x = np.random.default_rng(2).standard_normal(256).astype(np.float32)
    np.testing.assert_allclose(oracle.fwht(x), hadamard(256) @ x.astype(np.float64), rtol=1e-5, atol=1e-4)


def test_head_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    d, do = 64, 32
    t = {"norm.weight": rng.standard_normal(d), "norm.bias": rng.standard_normal(d),
         "q.weight": rng.standard_normal((do, d)), "q.bias": rng.standard_normal(do),
         "k.weight": rng.standard_normal((do, d)), "k.bias": rng.standard_normal(do)}
    t = {k: v.astype(np.float32) for k, v in t.items()}
    hidden = rng.standard_normal((4, d)).astype(np.float32)
    p = oracle.head_probs(t, hidden, 0.7)
    T = {k: torch.from_numpy(v).double() for k, v in t.items()}
    x = torch.nn.functional.layer_norm(torch.from_numpy(hidden).double(), (d,), T["norm.weight"], T["norm.bias"], 1e-5)
    q = torch.nn.functional.linear(x[-1], T["q.weight"], T["q.bias"])
    k = torch.nn.functional.linear(x[:-1], T["k.weight"], T["k.bias"])
    want = torch.softmax(k @ q / np.sqrt(do) / 0.7, 0).numpy()
    np.testing.assert_allclose(p, want, rtol=1e-12, atol=1e-14)


# ---- the whole torso ------------------------------------------------------------------------

def test_oracle_prefix_then_question_equals_full_forward(oracle, tiny_model):
    """src/engine.rs:552-614 semantics: a forward from a snapshot continues the full sequence
    (only the matmul dequant mode differs between a short and a long forward)."""
    m = oracle.OracleModel(tiny_model)
    rng = np.random.default_rng(12)
    ids = rng.integers(0, 4096, size=40).astype(np.uint32)
    rows_full = [31, 35, 39]
    full, _ = m.forward(ids, rows_full)
    _, snap = m.forward(ids[:30], [], keep=True)
    assert snap.len == 30
    part, _ = m.forward(ids[30:], [r - 30 for r in rows_full], cache=snap)
    np.testing.assert_allclose(part, full, atol=2e-2, rtol=0)
    np.testing.assert_allclose(m.probs(part), m.probs(full), atol=2e-3, rtol=0)
    # the snapshot is unchanged by later forwards: a second continuation gives the same rows
    again, _ = m.forward(ids[30:], [r - 30 for r in rows_full], cache=snap)
    assert np.array_equal(again, part)

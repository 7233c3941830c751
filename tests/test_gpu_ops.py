"""Kernel-level parity of the row kernels and attention on the GPU, through the C ABI, against the C
oracle on the same seeded inputs: embed (every weight format), add_norm, silu_mul, add_bias, conv,
gnorm (src/kernels.rs:63-190, 377-396), and qk_prep + attention at the 2B's head shape (hd 256,
8 q heads, 2 kv heads, rotary 64; src/kernels.rs:400-541), including the key-split path of a short
suffix over a long cached prefix."""
import ctypes
import os
import sys

import numpy as np
import pytest

from conftest import f16_ulp

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import cases  # noqa: E402

I = ctypes.c_int


def dev(a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def empty(nbytes):
    return torch.zeros(max(nbytes, 16), dtype=torch.uint8, device="cuda")


def host(t, dtype, shape):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype)[:int(np.prod(shape))].reshape(shape)


def within(got, want, ulps=1.0, extra=0.0, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    err = np.abs(got - want)
    tol = ulps * f16_ulp(want) * 1.001 + extra
    bad = err > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond tolerance; max err {err.max()}"


@pytest.mark.parametrize("bits,group,asym", [(4, 32, False), (3, 32, False), (3, 64, True), (2, 128, False),
                                             (4, 64, True), (2, 32, True)])
def test_embed_formats(sdamd, oracle, bits, group, asym):
    """k_embed for int4/int3/int2, symmetric and asymmetric, groups 32-128: bit-exact rows (the
    values are exact in f32, or one f32 rounding of q s + b in both)."""
    rng = np.random.default_rng(bits * 10 + group + asym)
    vocab, d = 1000, 2048
    codes = rng.integers(0, 1 << bits, size=(vocab, d), dtype=np.uint32)
    Q = cases.pack_codes(codes, bits)
    S = rng.uniform(-0.05, 0.05, size=vocab * d // group).astype(np.float16)
    B = rng.uniform(-0.3, 0.3, size=vocab * d // group).astype(np.float16) if asym else None
    ids = rng.integers(0, vocab, 77).astype(np.uint32)
    ids[:2] = [vocab - 1, 0]
    dQ, dS, dids = dev(Q), dev(S), dev(ids)
    dB = dev(B) if asym else None
    dx = empty(len(ids) * d * 4)
    sdamd.op_embed(dids.data_ptr(), len(ids), dQ.data_ptr(), dS.data_ptr(), dB.data_ptr() if asym else None, d, bits,
                   group, asym, dx.data_ptr())
    got = host(dx, np.float32, (len(ids), d))
    want = oracle.embed(ids, Q, S.view(np.uint16), d, bits, group, asym, None if B is None else B.view(np.uint16))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("d,with_y,gather", [(2048, True, False), (2048, False, False), (512, True, True),
                                             (3072, True, False)])
def test_add_norm(sdamd, oracle, d, with_y, gather):
    """x += y (one f32 add, bit-exact) and the RMSNorm to f16 within one f16 ulp (f32 sums in a
    different order), or to f32 for the final norm's gathered rows."""
    rng = np.random.default_rng(d + with_y)
    L = 37
    x = (3 * rng.standard_normal((L, d))).astype(np.float32)
    y = rng.standard_normal((L, d)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    rows = np.array([36, 0, 5, 20], np.uint32) if gather else None
    n = len(rows) if gather else L
    dx, dy, dw = dev(x), dev(y), dev(w)
    drows = dev(rows) if gather else None
    dh = empty(n * d * 4)
    if gather:
        sdamd.op_add_norm(dx.data_ptr(), dy.data_ptr() if with_y else None, dw.data_ptr(), d, drows.data_ptr(), n,
                          h32=dh.data_ptr())
    else:
        sdamd.op_add_norm(dx.data_ptr(), dy.data_ptr() if with_y else None, dw.data_ptr(), d, None, n,
                          h16=dh.data_ptr())
    xo = x.copy()
    want = oracle.add_norm(xo, y.view(np.uint16) if with_y else None, w, rows=rows, out_f32=gather)
    if gather:
        got = host(dh, np.float32, (n, d))
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)
        return
    got = host(dh, np.float16, (n, d)).astype(np.float32)
    assert np.array_equal(host(dx, np.float32, (L, d)), xo)
    within(got, oracle.h2f(want), what="h")


def test_silu_mul(sdamd, oracle):
    rng = np.random.default_rng(3)
    L, I_ = 29, 6144
    big = (3 * rng.standard_normal((L, 2 * I_))).astype(np.float16)
    dbig, dmid = dev(big), empty(L * I_ * 2)
    sdamd.op_silu_mul(dbig.data_ptr(), L, I_, dmid.data_ptr())
    mid = np.empty((L, I_), np.uint16)
    oracle.lib().or_silu_mul(oracle.P(big.view(np.uint16)), I(L), I(I_), oracle.P(mid))
    within(host(dmid, np.float16, (L, I_)), oracle.h2f(mid), what="mid")


def test_add_bias(sdamd, oracle):
    """One f32 add of the f16 value and the f32 bias, rounded to f16: bit-exact."""
    rng = np.random.default_rng(4)
    L, N = 21, 2048
    y = (2 * rng.standard_normal((L, N))).astype(np.float16)
    c = rng.standard_normal(N).astype(np.float32)
    dy, dc = dev(y), dev(c)
    sdamd.op_add_bias(dy.data_ptr(), L, N, dc.data_ptr())
    assert np.array_equal(host(dy, np.uint16, (L, N)), oracle.add_bias(y.view(np.uint16), c))


@pytest.mark.parametrize("L", [1, 2, 3, 50, 513])
def test_conv(sdamd, oracle, L):
    """Depthwise causal conv + SiLU with the 3 history rows in front (f32 within 1e-5 relative)."""
    rng = np.random.default_rng(L)
    C, stride = 6144, 8256
    big = rng.standard_normal((L, stride)).astype(np.float16)
    hist = rng.standard_normal((3, C)).astype(np.float16)
    w = (0.5 * rng.standard_normal((C, 4))).astype(np.float32)
    dbig, dh, dw, dout = dev(big), dev(hist), dev(w), empty(L * C * 4)
    sdamd.op_conv(dbig.data_ptr(), stride, L, C, dw.data_ptr(), dh.data_ptr(), dout.data_ptr())
    want = np.empty((L, C), np.float32)
    oracle.lib().or_conv(oracle.P(big.view(np.uint16)), I(stride), I(L), I(C), oracle.P(w),
                         oracle.P(hist.view(np.uint16).copy()), oracle.P(want))
    np.testing.assert_allclose(host(dout, np.float32, (L, C)), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("z_off,stride", [(6144, 8256), (6142, 8250)])
def test_gnorm(sdamd, oracle, z_off, stride):
    """Gated RMSNorm: 16 lanes per row with 16-byte accesses where the gate offsets allow (multiples
    of 8), one wave per row otherwise; within one f16 ulp of the oracle."""
    rng = np.random.default_rng(6)
    L, H, DV = 45, 16, 128
    o = (2 * rng.standard_normal((L, H * DV))).astype(np.float32)
    big = rng.standard_normal((L, stride)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(DV)).astype(np.float32)
    do_, dbig, dw, dout = dev(o), dev(big), dev(w), empty(L * H * DV * 2)
    sdamd.op_gnorm(do_.data_ptr(), dbig.data_ptr(), stride, z_off, dw.data_ptr(), L, H, DV, dout.data_ptr())
    want = np.empty((L, H * DV), np.uint16)
    oracle.lib().or_gnorm(oracle.P(o), oracle.P(big.view(np.uint16)), I(stride), I(z_off), oracle.P(w), I(L), I(H),
                          I(DV), oracle.P(want))
    within(host(dout, np.float16, (L, H * DV)), oracle.h2f(want), what="gnorm")


# ---- qk_prep + attention at the 2B's head shape ----------------------------------------------------

HQ, HK, HD, RD, CTX = 8, 2, 256, 64, 4096


class AttnCase:
    """A cache shared by successive calls (a prefix, then a suffix continuing it), on the GPU and in
    the oracle's layout."""

    def __init__(self, sdamd, oracle, seed, rd=RD):
        self.sdamd, self.oracle, self.rd = sdamd, oracle, rd
        self.rng = np.random.default_rng(seed)
        self.qw = (1 + 0.1 * self.rng.standard_normal(HD)).astype(np.float32)
        self.kw = (1 + 0.1 * self.rng.standard_normal(HD)).astype(np.float32)
        self.rope = oracle.rope_table(rd, 1e7)
        self.dqw, self.dkw, self.drope = dev(self.qw), dev(self.kw), dev(self.rope)
        self.dK, self.dV = empty(HK * CTX * HD * 2), empty(HK * CTX * HD * 2)
        self.oK = np.zeros((HK, CTX, HD), np.uint16)
        self.oV = np.zeros((HK, CTX, HD), np.uint16)
        self.stride = 2 * HQ * HD + 2 * HK * HD

    def run(self, L, P):
        big = self.rng.standard_normal((L, self.stride)).astype(np.float16)
        dbig, dQ, dout = dev(big), empty(HQ * L * HD * 2), empty(L * HQ * HD * 2)
        self.sdamd.op_attention(dbig.data_ptr(), self.stride, self.dqw.data_ptr(), self.dkw.data_ptr(),
                                self.drope.data_ptr(), L, P, HQ, HK, HD, self.rd, dQ.data_ptr(), self.dK.data_ptr(),
                                self.dV.data_ptr(), CTX, dout.data_ptr())
        o = self.oracle
        Q = np.empty((HQ, L, HD), np.uint16)
        o.lib().or_qk_prep(o.P(big.view(np.uint16)), I(self.stride), o.P(self.qw), o.P(self.kw), o.P(self.rope), I(L),
                           I(P), I(CTX), I(HQ), I(HK), I(HD), I(self.rd), o.P(Q), o.P(self.oK), o.P(self.oV))
        out = np.empty((L, HQ * HD), np.uint16)
        o.lib().or_attn(o.P(Q), o.P(self.oK), o.P(self.oV), o.P(big.view(np.uint16)), I(self.stride), I(L), I(P),
                        I(CTX), I(HQ), I(HK), I(HD), o.P(out))
        gotQ = host(dQ, np.float16, (HQ, L, HD))
        # K in blocks of 32 rows: [HK][CTX/32][HD/32][32 rows][32 dims] -> [HK][CTX][HD]
        gotK = host(self.dK, np.float16, (HK, CTX // 32, HD // 32, 32, 32)).transpose(0, 1, 3, 2, 4).reshape(HK, CTX, HD)[:, P:P + L]
        # V^T in blocks of 32 rows: [HK][CTX/32][HD][32] -> [HK][HD][CTX]
        gotVt = host(self.dV, np.float16, (HK, CTX // 32, HD, 32)).transpose(0, 2, 1, 3).reshape(HK, HD, CTX)[:, :, P:P + L]
        # q/k norm + RoPE: f32 math rounded to f16, within one f16 ulp; rotate-half can cancel terms
        # of size ~1 down to ~1e-4, where f32 rounding of the terms (a few 1e-7 either side) is
        # several f16 ulps of the result, hence the absolute allowance
        within(gotQ, o.h2f(Q), extra=1e-6, what="Q")
        within(gotK, o.h2f(self.oK[:, P:P + L]), extra=1e-6, what="K cache rows")
        # V is copied unchanged, transposed
        assert np.array_equal(gotVt.transpose(0, 2, 1).astype(np.float16).view(np.uint16), self.oV[:, P:P + L])
        got = host(dout, np.float16, (L, HQ * HD)).astype(np.float32)
        want = o.h2f(out)
        # scores, softmax and P.V in f32 against the oracle's f64 softmax: within 2 f16 ulp + 1e-3
        within(got, want, ulps=2.0, extra=1e-3, what=f"attention out L={L} P={P}")
        return np.abs(got - want).max()


def test_attention_prefill_512(sdamd, oracle):
    """L = 512 queries from an empty cache: 32 query blocks x 8 heads, no key split."""
    c = AttnCase(sdamd, oracle, 1)
    err = c.run(512, 0)
    print(f"attention L=512 P=0: max |d out| {err:.3g}", flush=True)


def test_attention_suffix_over_prefix(sdamd, oracle):
    """A 40-token suffix over the 512-token prefix the first call wrote: 3 query blocks x 8 heads
    split the 552 keys over 8 workgroups each and merge them in k_attn_combine."""
    c = AttnCase(sdamd, oracle, 2)
    c.run(512, 0)
    err = c.run(40, 512)
    print(f"attention L=40 P=512 (key split): max |d out| {err:.3g}", flush=True)
    err = c.run(1, 552)  # a single query at the end of the cache
    print(f"attention L=1 P=552: max |d out| {err:.3g}", flush=True)


def test_attention_long_prefix_ragged(sdamd, oracle):
    """Query blocks that straddle 16-row and 32-key boundaries over a longer prefix (keys up to 1148)."""
    c = AttnCase(sdamd, oracle, 3)
    c.run(1101, 0)
    c.run(47, 1101)


@pytest.mark.parametrize("rd", [32, 12, 2])
def test_attention_other_rotary_dims(sdamd, oracle, rd):
    """rotary_dim other than 64: the attention reads the queries qk_prep wrote (with rotary_dim 64,
    the case of the other tests, it normalizes and rotates them itself).  32 pairs rotate-half
    partners with a lane shuffle; 12 and 2 (not multiples of 8) read them back from LDS.  A prefill
    and a key-split suffix."""
    c = AttnCase(sdamd, oracle, 4 + rd, rd=rd)
    c.run(512, 0)
    err = c.run(40, 512)
    print(f"attention rotary {rd}, L=40 P=512: max |d out| {err:.3g}", flush=True)

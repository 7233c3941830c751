"""Kernel-level parity on the GPU: the int4 GEMM (BASELINE configs 0 and 1) and the gated delta
rule (config 2), through the C ABI (sd_op_matmul / sd_op_gdn), against the C oracle."""
import os
import sys

import numpy as np
import pytest

from conftest import f16_ulp

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import cases as gcases  # noqa: E402

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    """numpy array -> device bytes (torch is only the allocator here)."""
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def host(t, dtype, shape):
    return t.cpu().numpy().view(dtype).reshape(shape)


def gemm_case(synth, rng, M, N, K, lo=0, smin=0.005, smax=0.02):
    A = rng.standard_normal((M, K)).astype(np.float16)
    W = synth.pack_nibbles(rng.integers(lo, 16, size=(N, K), dtype=np.uint32))
    S = rng.uniform(smin, smax, size=(N, K // 32)).astype(np.float16)
    return A, W, S


def run_gemm(sdamd, A, W, S, M, N, K, exact, cfg=-1):
    dA, dW, dS = dev(A), dev(W), dev(S)
    dY = torch.empty(M * N * 2, dtype=torch.uint8, device="cuda")
    sdamd.op_matmul(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dY.data_ptr(), M, N, K, exact, cfg)
    torch.cuda.synchronize()
    return host(dY, np.float16, (M, N))


def check_gemm(oracle, A, W, S, Y, N, K, exact):
    want = oracle.h2f(oracle.matmul(A.view(np.uint16), W, S.view(np.uint16), N, K, f16_deq=not exact))
    got = Y.astype(np.float32)
    err = np.abs(got - want)
    tol = 1.01 * f16_ulp(want) + 2e-5
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside 1 f16 ulp; max err {err.max()} at {np.argmax(err)}"


# M <= 20 uses the reference GEMV's f32 dequant (exact), larger M the tiled kernel's f16 dequant.
@pytest.mark.parametrize("M,N,K", [
    (128, 6144, 2048),
    (1, 64, 128), (5, 320, 256), (17, 200, 384), (40, 2048, 2048), (64, 8256, 2048),
    (100, 1000, 512), (512, 2048, 6144), (300, 5120, 2048),
    (1100, 640, 512), (2100, 384, 256),  # long prefill: (3,1) with k halves, (4,1)
])
def test_gemm_matches_oracle(sdamd, synth, oracle, M, N, K):
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    A, W, S = gemm_case(synth, rng, M, N, K)
    exact = M <= 20
    Y = run_gemm(sdamd, A, W, S, M, N, K, exact)
    check_gemm(oracle, A, W, S, Y, N, K, exact)


def test_gemm_every_config(sdamd, synth, oracle):
    """Each kernel configuration (tile shape, dequant mode) on ragged shapes, in the plain weight
    layout (N not a multiple of 32) and the tiled one (N = 352, 96: column tiles past N)."""
    rng = np.random.default_rng(5)
    cfg, ran = 0, 0
    while True:
        for (M, N, K) in [(3, 100, 256), (37, 330, 640), (130, 72, 1024), (37, 352, 640), (130, 96, 1024)]:
            A, W, S = gemm_case(synth, rng, M, N, K)
            for exact in (False, True):
                try:
                    Y = run_gemm(sdamd, A, W, S, M, N, K, exact, cfg)
                except sdamd.EngineError as e:
                    if "no configuration" in str(e):
                        assert cfg >= 2 and ran > 0
                        return
                    # f16-dequant configuration asked for f32 dequant (or the reverse), a
                    # 64-wide-step configuration given K / ks not a multiple of 256, or a
                    # three-steps-ahead one given K / ks not a multiple of 512
                    assert "does not match" in str(e) or "multiple of 256" in str(e) or "multiple of 512" in str(e)
                    continue
                check_gemm(oracle, A, W, S, Y, N, K, exact)
                ran += 1
        cfg += 1


@pytest.mark.parametrize("M", [512, 8])
def test_layer_gemm_set(sdamd, synth, oracle, M):
    """q, k, v, o, gate, up, down of a 2048-wide layer at M = 512 and 8."""
    rng = np.random.default_rng(M)
    for (N, K) in [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (6144, 2048), (6144, 2048), (2048, 6144)]:
        A, W, S = gemm_case(synth, rng, M, N, K)
        exact = M <= 20
        Y = run_gemm(sdamd, A, W, S, M, N, K, exact)
        check_gemm(oracle, A, W, S, Y, N, K, exact)


def gdn_case(rng, L, H, dk=128, dv=128, negA=-1.0, dtb=0.0, a_scale=1.0):
    C = 2 * H * dk + H * dv
    qkv = rng.standard_normal((L, C)).astype(np.float32)
    stride = 2 * H
    big = np.zeros((L, stride), np.float16)
    big[:, :H] = (a_scale * rng.standard_normal((L, H))).astype(np.float16)  # a (decay input)
    big[:, H:] = rng.standard_normal((L, H)).astype(np.float16)  # b (beta logit)
    nA = np.full(H, negA, np.float32)
    db = np.full(H, dtb, np.float32)
    return qkv, big, stride, nA, db


def run_gdn(sdamd, qkv, big, stride, nA, db, L, H, state0, load):
    dq, db_, dn, dd = dev(qkv), dev(big), dev(nA), dev(db)
    dst = dev(state0)
    do = torch.empty(L * H * 128 * 4, dtype=torch.uint8, device="cuda")
    sdamd.op_gdn(dq.data_ptr(), db_.data_ptr(), stride, 0, H, dn.data_ptr(), dd.data_ptr(), L, H, 128, 128,
                 dst.data_ptr(), load, do.data_ptr())
    torch.cuda.synchronize()
    return host(do, np.float32, (L, H * 128)), host(dst, np.float32, state0.shape)


def oracle_gdn(oracle, qkv, big, stride, nA, db, L, H, state0, load):
    import ctypes
    st = state0.copy()
    o = np.empty((L, H * 128), np.float32)
    I = ctypes.c_int
    oracle.lib().or_gdn(oracle.P(qkv), oracle.P(big.view(np.uint16)), I(stride), I(0), I(H), oracle.P(nA),
                        oracle.P(db), I(L), I(H), I(128), I(128), oracle.P(st), I(int(load)), oracle.P(o))
    return o, st


@pytest.mark.parametrize("L,H,load,negA,a_scale", [
    (512, 16, False, -1.0, 1.0),
    (1, 2, False, -1.0, 1.0), (3, 2, True, -1.0, 1.0), (63, 2, False, -1.0, 1.0), (64, 2, True, -1.0, 1.0),
    (65, 2, False, -1.0, 1.0), (130, 4, True, -1.0, 1.0), (200, 2, True, -16.0, 3.0),
])
def test_gdn_matches_sequential_oracle(sdamd, oracle, L, H, load, negA, a_scale):
    """The chunked recurrence equals the reference's token-by-token recurrence (fp32)."""
    rng = np.random.default_rng(L * 131 + H)
    qkv, big, stride, nA, db = gdn_case(rng, L, H, negA=negA, a_scale=a_scale)
    state0 = (0.1 * rng.standard_normal((H, 128, 128))).astype(np.float32)
    o, st = run_gdn(sdamd, qkv, big, stride, nA, db, L, H, state0, load)
    wo, wst = oracle_gdn(oracle, qkv, big, stride, nA, db, L, H, state0, load)
    np.testing.assert_allclose(o, wo, rtol=2e-4, atol=2e-4)
    np.testing.assert_allclose(st, wst, rtol=2e-4, atol=2e-4)


def test_gemm_prepacked_weights(sdamd, synth):
    """sd_op_repack_w4 once + sd_op_matmul(packed=1) gives the very same output as the per-call
    rewrite of sd_op_matmul(packed=0), for shapes with the tiled layout (N a multiple of 32) and
    without it (N = 336 + 8)."""
    rng = np.random.default_rng(11)
    for (M, N, K, exact) in [(96, 640, 1024, False), (512, 256, 2048, False), (7, 320, 512, True),
                             (40, 344, 512, False), (5, 344, 256, True)]:
        A, W, S = gemm_case(synth, rng, M, N, K)
        Y0 = run_gemm(sdamd, A, W, S, M, N, K, exact)
        dA, dW, dS = dev(A), dev(W), dev(S)
        sdamd.op_repack_w4(dW.data_ptr(), dS.data_ptr(), N, K)
        dY = torch.empty(M * N * 2, dtype=torch.uint8, device="cuda")
        sdamd.op_matmul(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dY.data_ptr(), M, N, K, exact, -1, True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(dY, np.float16, (M, N)), Y0)
        if N % 32 == 0:  # tiled: words and scales were rewritten
            assert not np.array_equal(host(dW, np.uint32, W.shape), W)
            assert not np.array_equal(host(dS, np.float16, S.shape), S)
        else:  # the model's layout is what the GEMV reads for this shape
            assert np.array_equal(host(dW, np.uint32, W.shape), W)


# ---- the f32-dequant GEMV (short inputs, non-default formats) ---------------------------------------

GEMV_FORMATS = [(4, 32, False), (4, 64, True), (3, 32, False), (3, 64, True), (2, 128, False), (2, 32, True)]


GEMV_SHAPES = [(1, 64, 128), (8, 2048, 2048), (17, 200, 384), (20, 96, 4096), (40, 330, 640), (130, 512, 1024),
               (5, 100, 160)]


# every format at every shape whose K its group divides (a format's groups must tile K)
@pytest.mark.parametrize("bits,group,asym,M,N,K", [f + s for f in GEMV_FORMATS for s in GEMV_SHAPES if s[2] % f[1] == 0])
def test_gemv_formats(sdamd, oracle, bits, group, asym, M, N, K):
    """The reference's matmul_gemv(f) for every format (src/kernels.rs:590-635) in the model's layout:
    f32 dequant, f32 accumulation, within one f16 ulp of the oracle.  Ragged N, K not a multiple of
    128, and M past the 32 rows of one workgroup."""
    rng = np.random.default_rng(bits * 1000 + group + M + N + K + asym)
    A = rng.standard_normal((M, K)).astype(np.float16)
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint32)
    W = gcases.pack_codes(codes, bits)
    S = rng.uniform(0.005, 0.03, size=N * K // group).astype(np.float16)
    B = rng.uniform(-0.1, 0.1, size=N * K // group).astype(np.float16) if asym else None
    dA, dW, dS = dev(A), dev(W), dev(S)
    dB = dev(B) if asym else None
    dY = torch.empty(M * N * 2, dtype=torch.uint8, device="cuda")
    sdamd.op_matmul_fmt(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dB.data_ptr() if asym else None, dY.data_ptr(),
                        M, N, K, bits, group, asym)
    torch.cuda.synchronize()
    got = host(dY, np.float16, (M, N))
    want = oracle.h2f(oracle.matmul(A.view(np.uint16), W, S.view(np.uint16), N, K, False, bits=bits, group=group,
                                    asym=asym, Bi=None if B is None else B.view(np.uint16)))
    err = np.abs(got.astype(np.float32) - want)
    assert (err <= 1.01 * f16_ulp(want) + 2e-5).all(), f"max err {err.max()}"


@pytest.mark.parametrize("M", [1, 3, 8, 16, 17, 20])
@pytest.mark.parametrize("N,K", [(8256, 2048), (5120, 2048), (12288, 2048), (2048, 6144), (96, 512), (344, 256)])
def test_gemv_short_rows(sdamd, synth, oracle, M, N, K):
    """The engine's GEMV rows (M <= 20) on the 2B's shapes in the tiled layout, and untileable ones in
    the model's layout: the reference GEMV's f32 dequant within one f16 ulp."""
    rng = np.random.default_rng(M * 7 + N + K)
    A, W, S = gemm_case(synth, rng, M, N, K)
    Y = run_gemm(sdamd, A, W, S, M, N, K, True)
    check_gemm(oracle, A, W, S, Y, N, K, True)


def split_sum(part, ks, M, N):
    """The consumer's sum of the split-K slots: slot order in f32, then one rounding to f16."""
    p = part.reshape(ks, M, N)
    s = p[0].copy()
    for z in range(1, ks):
        s += p[z]
    return s.astype(np.float16)


@pytest.mark.parametrize("M,N,K,exact,cfg,ks", [
    (512, 2048, 2048, False, 24, 2),   # prefill out_proj / o_proj: (2,1) tiles with k halves, 2 splits
    (512, 2048, 6144, False, 20, 4),   # prefill down: (4,1) tiles, 4 splits
    (120, 2048, 6144, False, 18, 8),   # question down: (2,1) tiles, 8 splits
    (120, 2048, 2048, False, 3, 4),    # question out_proj: 16x16 (2,1), 4 splits
    (120, 2048, 2048, False, 30, 4),   # the same, loads three steps ahead
    (120, 2048, 6144, False, 32, 4),   # 16x16 (4,1) three steps ahead, 4 splits
    # the measured plans' splits (M between 256 and 2560)
    (256, 2048, 2048, False, 18, 4),   # o_proj: (2,1), 4 splits
    (300, 2048, 6144, False, 26, 4),   # down: (3,1) with k halves, 4 splits
    (640, 2048, 6144, False, 26, 2),   # down: (3,1) with k halves, 2 splits
    (330, 2048, 6144, False, 25, 2),   # down: (4,1) with k halves, 2 splits
    (300, 2048, 6144, False, 21, 4),   # down: (3,1), 4 splits
    (300, 2048, 6144, False, 20, 2),   # down: (4,1), 2 splits
    (300, 2048, 6144, False, 19, 2),   # down: (2,2), 2 splits
    (300, 2048, 6144, False, 24, 4),   # down: (2,1) with k halves, 4 splits
    (300, 2048, 2048, False, 26, 1),   # o_proj: (3,1) with k halves, one slot
    (72, 2048, 2048, False, 31, 4),    # question batches: 16x16 (3,1) three steps ahead, 4 splits
    (150, 2048, 6144, False, 31, 4),
    (150, 2048, 2048, False, 31, 2),
    (240, 2048, 6144, False, 24, 4),   # (2,1) with k halves, 4 splits
    (8, 2048, 2048, True, -1, 2),      # GEMV partials
    (8, 2048, 6144, True, -1, 4),
    (20, 2048, 2048, True, -1, 1),
])
def test_split_partials(sdamd, synth, oracle, M, N, K, exact, cfg, ks):
    """The split-K partial slots the residual add consumes: summed in slot order and rounded to f16
    they are within one f16 ulp of the oracle's product."""
    rng = np.random.default_rng(M + N + K + ks)
    A, W, S = gemm_case(synth, rng, M, N, K)
    dA, dW, dS = dev(A), dev(W), dev(S)
    dP = torch.empty(ks * M * N * 4, dtype=torch.uint8, device="cuda")
    sdamd.op_matmul_split(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dP.data_ptr(), M, N, K, exact, cfg, ks)
    torch.cuda.synchronize()
    Y = split_sum(host(dP, np.float32, (ks * M * N,)), ks, M, N)
    check_gemm(oracle, A, W, S, Y, N, K, exact)


@pytest.mark.parametrize("M,exact,cfg", [(8, True, -1), (17, True, -1), (120, False, 24), (120, False, 30),
                                         (120, False, 33), (200, False, 30), (512, False, 18),
                                         # the measured plans' tiles: (4,1) with k halves, (4,2),
                                         # (3,1), (4,1)
                                         (256, False, 25), (300, False, 23), (384, False, 21), (330, False, 20),
                                         # question batches: 16x16 (3,2) three steps ahead, (3,1)
                                         # with k halves
                                         (80, False, 34), (150, False, 26)])
def test_gate_up_silu(sdamd, synth, oracle, M, exact, cfg):
    """gate_up with silu * mul in the epilogue (the engine's fused form).  (1) Against silu_mul of the
    same kernel family's unfused gate_up output: within one f16 ulp (the epilogue itself).  (2)
    Against the oracle's gate_up then silu_mul: one f16 ulp of gate or up (the product's own
    tolerance) moves silu(g) u by |d/dg| ulp(g) + |d/du| ulp(u), and the two roundings of the output
    can fall in neighbouring binades (2 ulp)."""
    import ctypes
    N, K = 12288, 2048
    rng = np.random.default_rng(M + exact)
    A, W, S = gemm_case(synth, rng, M, N, K)
    dA, dW, dS = dev(A), dev(W), dev(S)
    dmid = torch.empty(M * N, dtype=torch.uint8, device="cuda")
    sdamd.op_gate_up_silu(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dmid.data_ptr(), M, N, K, exact, cfg)
    torch.cuda.synchronize()
    got = host(dmid, np.float16, (M, N // 2)).astype(np.float32)

    def silu_mul(big16):
        mid = np.empty((M, N // 2), np.uint16)
        oracle.lib().or_silu_mul(oracle.P(np.ascontiguousarray(big16)), ctypes.c_int(M), ctypes.c_int(N // 2),
                                 oracle.P(mid))
        return oracle.h2f(mid)

    # the same kernel configuration without the epilogue: one f32 partial slot (ks = 1) rounded to
    # f16 holds exactly the gate and up values the fused epilogue sees (GEMV rows, the 32x32 tiles
    # (24: (2,1) with k halves, 18: (2,1)), the 16x16 three-steps-ahead tiles (30: (2,1), pairs
    # meeting in LDS; 33: (2,2), pairs in one wave))
    dP = torch.empty(M * N * 4, dtype=torch.uint8, device="cuda")
    sdamd.op_matmul_split(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dP.data_ptr(), M, N, K, exact, cfg, 1)
    torch.cuda.synchronize()
    gpu_big = host(dP, np.float32, (M, N)).astype(np.float16).view(np.uint16)
    own = silu_mul(gpu_big)
    err = np.abs(got - own)
    assert (err <= 1.01 * f16_ulp(own) + 1e-6).all(), f"epilogue: max err {err.max()} vs silu of its own gate_up"

    big = oracle.matmul(A.view(np.uint16), W, S.view(np.uint16), N, K, f16_deq=not exact)
    want = silu_mul(big)
    g = oracle.h2f(big[:, :N // 2]).astype(np.float64)
    u = oracle.h2f(big[:, N // 2:]).astype(np.float64)
    sig = 1 / (1 + np.exp(-g))
    dsilu = sig * (1 + g * (1 - sig))
    # gate and up each within the product's own tolerance (check_gemm): one f16 ulp plus 2e-5, the
    # f32 accumulation error of 2048 terms that cancel to a value near zero
    dg, du = 1.01 * f16_ulp(g) + 2e-5, 1.01 * f16_ulp(u) + 2e-5
    tol = 2.01 * f16_ulp(want) + np.abs(dsilu * u) * dg + np.abs(g * sig) * du + 1e-6
    err = np.abs(got - want)
    assert (err <= tol).all(), f"{(err > tol).sum()} beyond tolerance; max err {err.max()}"

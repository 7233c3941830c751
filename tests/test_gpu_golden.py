"""The HIP kernels against the committed golden fixtures (written from float64 brute force and
transformers' gated delta rule by tests/golden/make_golden.py), through the C ABI."""
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


def dev(a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def golden(name):
    return np.load(os.path.join(HERE, "golden", name + ".npz"))


@pytest.mark.parametrize("name", ["m_int4_small", "m_int4_tiled"])
@pytest.mark.parametrize("exact", [True, False])
def test_matmul_matches_golden(sdamd, name, exact):
    """exact: the GEMV's f32 dequant (src/kernels.rs:572, 620); else the tiled kernel's f16
    dequant (src/kernels.rs:668-672); both accumulate in f32 and round the output to f16 once."""
    c = cases.matmul_inputs(name)
    g = golden("matmul")
    assert str(g[f"{name}.digest"]) == cases.digest(c["A"], c["W"], c["S"], c["B"])
    M, N, K = c["M"], c["N"], c["K"]
    want = g[f"{name}.{'y32' if exact else 'y16'}"].astype(np.float32)
    dA, dW, dS = dev(c["A"]), dev(c["W"]), dev(c["S"])
    configs = [-1] + list(range(sdamd_configs(sdamd)))
    for cfg in configs:
        dY = torch.empty(M * N * 2, dtype=torch.uint8, device="cuda")
        try:
            sdamd.op_matmul(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dY.data_ptr(), M, N, K, exact, cfg)
        except sdamd.EngineError as e:
            # a configuration of the other dequant mode, a 64-wide-step one given K / ks not a
            # multiple of 256, or a three-steps-ahead one given K / ks not a multiple of 512
            assert "does not match" in str(e) or "multiple of 256" in str(e) or "multiple of 512" in str(e)
            continue
        torch.cuda.synchronize()
        got = dY.cpu().numpy().view(np.float16).reshape(M, N).astype(np.float32)
        err = np.abs(got - want)
        assert (err <= 1.001 * f16_ulp(want) + 1e-6).all(), f"cfg {cfg}: max err {err.max()}"


def sdamd_configs(sdamd):
    """Number of GEMM configurations: the first index the library rejects."""
    n = 0
    M, N, K = 1, 64, 128
    A = torch.zeros(M * K * 2, dtype=torch.uint8, device="cuda")  # f16
    W = torch.zeros(N * K // 2, dtype=torch.uint8, device="cuda")  # int4
    S = torch.zeros(N * K // 32 * 2, dtype=torch.uint8, device="cuda")  # f16 per 32
    Y = torch.zeros(M * N * 2, dtype=torch.uint8, device="cuda")
    while n < 64:
        try:
            sdamd.op_matmul(A.data_ptr(), W.data_ptr(), S.data_ptr(), Y.data_ptr(), M, N, K, False, n)
        except sdamd.EngineError as e:
            if "no configuration" in str(e):
                break
        n += 1
    torch.cuda.synchronize()
    return n


@pytest.mark.parametrize("name", [n for n, v in cases.GDN_CASES.items() if v[2] == 128 and v[3] == 128])
def test_gdn_matches_golden(sdamd, name):
    c = cases.gdn_inputs(name)
    g = golden("gdn")
    assert str(g[f"{name}.digest"]) == cases.digest(c["qkv"], c["big"], c["negA"], c["dtb"], c["state0"])
    L, H = c["L"], c["H"]
    dq, db, dn, dd, dst = dev(c["qkv"]), dev(c["big"]), dev(c["negA"]), dev(c["dtb"]), dev(c["state0"])
    do = torch.empty(L * H * 128 * 4, dtype=torch.uint8, device="cuda")
    sdamd.op_gdn(dq.data_ptr(), db.data_ptr(), c["stride"], c["a_off"], c["b_off"], dn.data_ptr(), dd.data_ptr(), L, H,
                 128, 128, dst.data_ptr(), c["load"], do.data_ptr())
    torch.cuda.synchronize()
    o = do.cpu().numpy().view(np.float32).reshape(L, H * 128)
    st = dst.cpu().numpy().view(np.float32).reshape(H, 128, 128)
    np.testing.assert_allclose(o, g[f"{name}.o"], rtol=2e-4, atol=2e-4)
    np.testing.assert_allclose(st[:, ::cases.STATE_ROW_STEP], g[f"{name}.state"], rtol=2e-4, atol=2e-4)

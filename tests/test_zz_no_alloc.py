"""sd_op_matmul_noalloc (no counterpart in the reference; for callers that cannot allocate device
memory) against sd_op_matmul, the entry point it mirrors, on two calls in a row (the second one
smaller, over the same scratch array), through the C ABI.  Both use the same plan and kernels, so
the outputs are bit-identical."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def case(synth, rng, M, N, K):
    A = rng.standard_normal((M, K)).astype(np.float16)
    W = synth.pack_nibbles(rng.integers(0, 16, size=(N, K), dtype=np.uint32))
    S = rng.uniform(0.005, 0.02, size=(N, K // 32)).astype(np.float16)
    return dev(A), dev(W), dev(S)


def both(sdamd, dA, dW, dS, M, N, K, exact):
    """(sd_op_matmul, sd_op_matmul_noalloc) outputs for the same packed weights."""
    y0 = torch.zeros(M * N * 2, dtype=torch.uint8, device="cuda")
    y1 = torch.full((M * N * 2,), 0xAB, dtype=torch.uint8, device="cuda")
    sdamd.op_matmul(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), y0.data_ptr(), M, N, K, exact, -1, True)
    sdamd.op_matmul_noalloc(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), y1.data_ptr(), M, N, K, exact)
    torch.cuda.synchronize()
    return y0.cpu().numpy(), y1.cpu().numpy()


@pytest.mark.parametrize("first,second", [
    ((512, 2048, 6144, False), (120, 2048, 2048, False)),   # 4 split-K slots filling the array, then 4 smaller
    ((128, 6144, 2048, False), (64, 512, 2048, False)),     # BASELINE configs[0], then a split 16x16 tile
    ((8, 8256, 2048, True), (3, 2048, 2048, True)),        # the GEMV rows (no scratch)
])
def test_noalloc_matches_matmul_twice(sdamd, synth, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for (M, N, K, exact) in (first, second):
        dA, dW, dS = case(synth, rng, M, N, K)
        sdamd.op_repack_w4(dW.data_ptr(), dS.data_ptr(), N, K)
        y0, y1 = both(sdamd, dA, dW, dS, M, N, K, exact)
        assert np.array_equal(y0, y1), f"M={M} N={N} K={K}: outputs differ"


def test_noalloc_fits_a_large_split_into_the_array(sdamd, synth):
    """A prefill shape whose split-K slots under sd_op_matmul's plan exceed the 16 MiB array runs with
    a smaller split.  Its slots add in another order, so each output is within one f16 rounding of
    sd_op_matmul's, plus the f32 summation-order difference that shows where the K = 6144 terms
    (partial sums of magnitude ~4) cancel to a tiny output (measured on MI355X: at most a few 1e-6,
    at outputs of 1e-4 .. 2e-3); both stay within one f16 ulp of the float64 product.  The next,
    smaller call is again bit-identical to sd_op_matmul."""
    from conftest import f16_ulp
    rng = np.random.default_rng(9)
    M, N, K = 1024, 2048, 6144  # sd_op_matmul: 4 slots of 1024 x 2048 f32 = 32 MiB
    dA, dW, dS = case(synth, rng, M, N, K)
    sdamd.op_repack_w4(dW.data_ptr(), dS.data_ptr(), N, K)
    y0, y1 = both(sdamd, dA, dW, dS, M, N, K, False)
    a, b = y0.view(np.float16).astype(np.float32), y1.view(np.float16).astype(np.float32)
    assert np.isfinite(b).all()
    SUM_ORDER = 1e-4  # f32 summation-order bound over K = 6144 at these magnitudes, absolute
    ulp = f16_ulp(np.maximum(np.abs(a), np.abs(b)))
    assert (np.abs(a - b) <= ulp + SUM_ORDER).all(), f"max excess {(np.abs(a - b) - ulp).max()}"
    assert (np.abs(a - b) > ulp).mean() < 1e-3  # only the near-cancelled outputs differ by more
    M2 = 256
    dA2 = dev(rng.standard_normal((M2, K)).astype(np.float16))
    y0, y1 = both(sdamd, dA2, dW, dS, M2, N, K, False)
    assert np.array_equal(y0, y1)


@pytest.mark.parametrize("M,N,K", [(512, 2048, 6144), (120, 8256, 2048)])
def test_noalloc_under_graph_capture(sdamd, synth, M, N, K):
    """Captured into a graph (after one call outside the capture, which looks up the array's address)
    and replayed several times with eager work and synchronizations between the replays: every
    replay is bit-identical to the eager sd_op_matmul result."""
    rng = np.random.default_rng(M + N)
    dA, dW, dS = case(synth, rng, M, N, K)
    sdamd.op_repack_w4(dW.data_ptr(), dS.data_ptr(), N, K)
    want, _ = both(sdamd, dA, dW, dS, M, N, K, False)  # also the warm-up call of the noalloc entry point
    y = torch.zeros(M * N * 2, dtype=torch.uint8, device="cuda")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            sdamd.op_matmul_noalloc(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), y.data_ptr(), M, N, K, False,
                                    stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    for r in range(4):
        y.fill_(0xCD)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want), f"replay {r} differs from the eager result"

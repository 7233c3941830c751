"""Seeded inputs of the golden cases.  The fixtures in this folder hold only the expected outputs
(plus a digest of the inputs); the inputs are regenerated here from numpy's PCG64 streams, which
are stable across platforms and numpy versions.

Layouts follow the oracle / C ABI:
  matmul  A [M][K] f16, W [N][K/32] blocks of `bits` u32 words, scales (and asym biases) f16
          per group (src/kernels.rs:550-576, 668-672)
  gdn     qkv [L][2*H*dk + H*dv] f32 (q | k | v), big [L][2H] f16 with a at column h and b at H + h,
          negA [H], dt_bias [H], state [H][dk][dv] f32 (src/kernels.rs:257-302)
  attn    Q [HQ][L][HD] f16, K and V [HK][LT][HD] f16, big [L][HQ*2*HD] f16 whose gate for head h is
          columns h*2*HD + HD .. (src/kernels.rs:453-541)
"""
from __future__ import annotations

import hashlib

import numpy as np


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


# ---- quantized matmul -------------------------------------------------------------------------

MATMUL_CASES = {
    # name: (M, N, K, bits, group, asym)
    "m_int4_small": (3, 64, 256, 4, 32, False),
    "m_int4_tiled": (33, 96, 384, 4, 32, False),
    "m_int3_asym_g64": (2, 32, 128, 3, 64, True),
    "m_int2_g128": (2, 32, 128, 2, 128, False),
}


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Codes [N][K] -> u32 words [N][K/32][bits]: int4 puts element e of a 32-block in word e/8 at
    bit 4(e%8); int2 in word e/16 at bit 2(e%16); int3 is int2 low bits plus a third word whose
    bit e is the code's bit 2 (src/kernels.rs:63-70, 562-573)."""
    N, K = codes.shape
    c = codes.astype(np.uint64).reshape(N, K // 32, 32)
    words = np.zeros((N, K // 32, bits), np.uint64)
    if bits == 4:
        for e in range(32):
            words[:, :, e // 8] |= c[:, :, e] << np.uint64(4 * (e % 8))
    else:
        lo = c & np.uint64(3)
        for e in range(32):
            words[:, :, e // 16] |= lo[:, :, e] << np.uint64(2 * (e % 16))
        if bits == 3:
            for e in range(32):
                words[:, :, 2] |= ((c[:, :, e] >> np.uint64(2)) & np.uint64(1)) << np.uint64(e)
    return words.astype(np.uint32)


def matmul_inputs(name: str):
    M, N, K, bits, group, asym = MATMUL_CASES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    A = rng.standard_normal((M, K)).astype(np.float16)
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint32)
    W = pack_codes(codes, bits)
    ng = N * K // group
    # scales with full 10-bit mantissas, so (q - 8) * s usually needs more than f16's 11 bits
    S = rng.uniform(0.005, 0.02, size=ng).astype(np.float16)
    B = rng.uniform(-0.05, 0.05, size=ng).astype(np.float16) if asym else None
    return dict(M=M, N=N, K=K, bits=bits, group=group, asym=asym, A=A, codes=codes, W=W, S=S, B=B)


# ---- gated delta rule ----------------------------------------------------------------------

GDN_CASES = {
    # name: (L, H, dk, dv, load_state, negA, dt_bias, a_scale)
    "g_l70_h1": (70, 1, 128, 128, False, (-1.0,), (0.0,), 1.0),
    "g_l5_h1_state": (5, 1, 128, 128, True, (-16.0,), (0.0,), 3.0),
    "g_l33_h2_rect": (33, 2, 32, 48, True, (-0.5, -8.0), (1.0, 0.5), 1.0),
    "g_l130_h1": (130, 1, 128, 128, True, (-2.0,), (1.0,), 1.5),
}
STATE_ROW_STEP = 8  # the fixtures keep key rows 0, 8, 16, ... of the final state


def gdn_inputs(name: str):
    L, H, dk, dv, load, negA, dtb, a_scale = GDN_CASES[name]
    rng = np.random.default_rng(1000 + sum(map(ord, name)))
    C = 2 * H * dk + H * dv
    qkv = rng.standard_normal((L, C)).astype(np.float32)
    big = np.zeros((L, 2 * H), np.float16)
    big[:, :H] = (a_scale * rng.standard_normal((L, H))).astype(np.float16)
    big[:, H:] = rng.standard_normal((L, H)).astype(np.float16)
    state0 = (0.1 * rng.standard_normal((H, dk, dv))).astype(np.float32) if load else np.zeros((H, dk, dv), np.float32)
    return dict(L=L, H=H, dk=dk, dv=dv, load=load, qkv=qkv, big=big, stride=2 * H, a_off=0, b_off=H,
                negA=np.asarray(negA, np.float32), dtb=np.asarray(dtb, np.float32), state0=state0)


# ---- attention -----------------------------------------------------------------------------

ATTN_CASES = {
    # name: (HQ, HK, HD, L, P, LT)
    "a_gqa_prefix": (4, 2, 64, 6, 9, 16),
    "a_first_token": (2, 1, 64, 1, 0, 4),
    "a_long": (4, 1, 64, 40, 100, 160),
}


def attn_inputs(name: str):
    HQ, HK, HD, L, P, LT = ATTN_CASES[name]
    rng = np.random.default_rng(2000 + sum(map(ord, name)))
    Q = rng.standard_normal((HQ, L, HD)).astype(np.float16)
    K = np.zeros((HK, LT, HD), np.float16)
    V = np.zeros((HK, LT, HD), np.float16)
    K[:, :P + L] = rng.standard_normal((HK, P + L, HD)).astype(np.float16)
    V[:, :P + L] = rng.standard_normal((HK, P + L, HD)).astype(np.float16)
    big = rng.standard_normal((L, HQ * 2 * HD)).astype(np.float16)
    return dict(HQ=HQ, HK=HK, HD=HD, L=L, P=P, LT=LT, Q=Q, K=K, V=V, big=big, stride=HQ * 2 * HD)

"""Writes the golden fixtures of this folder from libraries that share no code with the oracle or
the engine:

  matmul.npz  brute force in float64 numpy over a weight decode written from the format
              description (src/kernels.rs:550-576): Y = f16(sum_k A[m,k] * w[n,k]); w in f32
              (the GEMV's dequant, src/kernels.rs:572, 620) and w rounded to f16 (the tiled
              kernel's dequant, src/kernels.rs:668-672)
  gdn.npz     transformers' `torch_recurrent_gated_delta_rule` (Qwen3.5's torch path, with its
              own l2norm at eps 1e-6 inside the sqrt, as src/kernels.rs:280-283), checked here
              against transformers' chunked `torch_chunk_gated_delta_rule`
  attn.npz    float64 torch softmax attention with a causal offset and GQA head sharing, times
              sigmoid(gate) (src/kernels.rs:453-541)

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import cases  # noqa: E402


def decode(codes, S, B, N, K, bits, group, asym):
    """deq(W)[N,K] in float64 from the codes: asym q*s + b, else (q - 2^(bits-1)) * s."""
    g = np.arange(K) // group
    s = S.astype(np.float64).reshape(N, K // group)[:, g]
    q = codes.astype(np.float64)
    if asym:
        return q * s + B.astype(np.float64).reshape(N, K // group)[:, g]
    return (q - 2 ** (bits - 1)) * s


def make_matmul():
    out = {}
    for name in cases.MATMUL_CASES:
        c = cases.matmul_inputs(name)
        w64 = decode(c["codes"], c["S"], c["B"], c["N"], c["K"], c["bits"], c["group"], c["asym"])
        w32 = w64.astype(np.float32)  # one rounding: the f32 product (or fma) of the reference's GEMV
        w16 = w32.astype(np.float16)  # the tiled kernel stores the f32 value as f16
        A = c["A"].astype(np.float64)
        # the dequantized weights must match bit for bit: a digest keeps the fixture small
        out[f"{name}.deq32"] = np.array(cases.digest(w32))
        out[f"{name}.deq16"] = np.array(cases.digest(w16.astype(np.float32)))
        out[f"{name}.y32"] = (A @ w32.astype(np.float64).T).astype(np.float16)
        out[f"{name}.y16"] = (A @ w16.astype(np.float64).T).astype(np.float16)
        out[f"{name}.digest"] = np.array(cases.digest(c["A"], c["W"], c["S"], c["B"]))
    np.savez_compressed(os.path.join(HERE, "matmul.npz"), **out)


def make_gdn():
    import torch
    from transformers.models.qwen3_5.modeling_qwen3_5 import (torch_chunk_gated_delta_rule,
                                                               torch_recurrent_gated_delta_rule)
    out = {}
    for name in cases.GDN_CASES:
        c = cases.gdn_inputs(name)
        L, H, dk, dv = c["L"], c["H"], c["dk"], c["dv"]
        qkv = torch.from_numpy(c["qkv"])
        q = qkv[:, :H * dk].reshape(1, L, H, dk)
        k = qkv[:, H * dk:2 * H * dk].reshape(1, L, H, dk)
        v = qkv[:, 2 * H * dk:].reshape(1, L, H, dv)
        big = torch.from_numpy(c["big"].astype(np.float32))
        a, b = big[:, :H], big[:, H:]
        g = (torch.from_numpy(c["negA"]) * torch.nn.functional.softplus(a + torch.from_numpy(c["dtb"]))).reshape(1, L, H)
        beta = torch.sigmoid(b).reshape(1, L, H)
        s0 = torch.from_numpy(c["state0"]).reshape(1, H, dk, dv) if c["load"] else None
        o, st = torch_recurrent_gated_delta_rule(q, k, v, g, beta, s0, True, use_qk_l2norm_in_kernel=True)
        oc, stc = torch_chunk_gated_delta_rule(q, k, v, g, beta, 64, s0, True, use_qk_l2norm_in_kernel=True)
        assert torch.allclose(o, oc, rtol=1e-4, atol=1e-4), name
        assert torch.allclose(st, stc, rtol=1e-4, atol=1e-4), name
        out[f"{name}.o"] = o.reshape(L, H * dv).numpy()
        # every 8th key row of the final state keeps the fixture small
        out[f"{name}.state"] = st.reshape(H, dk, dv).numpy()[:, ::cases.STATE_ROW_STEP]
        out[f"{name}.digest"] = np.array(cases.digest(c["qkv"], c["big"], c["negA"], c["dtb"], c["state0"]))
    np.savez_compressed(os.path.join(HERE, "gdn.npz"), **out)


def make_attn():
    import torch
    out = {}
    for name in cases.ATTN_CASES:
        c = cases.attn_inputs(name)
        HQ, HK, HD, L, P = c["HQ"], c["HK"], c["HD"], c["L"], c["P"]
        # the reference scales q by 1/sqrt(hd) and stores it as f16; 1/8 for hd = 64 is exact
        q = torch.from_numpy(c["Q"].astype(np.float64)) / np.sqrt(HD)
        k = torch.from_numpy(c["K"][:, :P + L].astype(np.float64)).repeat_interleave(HQ // HK, dim=0)
        v = torch.from_numpy(c["V"][:, :P + L].astype(np.float64)).repeat_interleave(HQ // HK, dim=0)
        s = q @ k.transpose(1, 2)
        t = torch.arange(L)[:, None]
        j = torch.arange(P + L)[None, :]
        s = s.masked_fill(j > P + t, float("-inf"))
        o = torch.softmax(s, dim=-1) @ v  # [HQ, L, HD]
        gate = torch.from_numpy(c["big"].astype(np.float64)).reshape(L, HQ, 2, HD)[:, :, 1]
        y = o.transpose(0, 1) * torch.sigmoid(gate)
        out[f"{name}.out"] = y.reshape(L, HQ * HD).numpy().astype(np.float16)
        out[f"{name}.digest"] = np.array(cases.digest(c["Q"], c["K"], c["V"], c["big"]))
    np.savez_compressed(os.path.join(HERE, "attn.npz"), **out)


if __name__ == "__main__":
    make_matmul()
    make_gdn()
    make_attn()
    for f in ("matmul.npz", "gdn.npz", "attn.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")

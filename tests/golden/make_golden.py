"""Writes tests/golden/attn_small.npz: small paged decode-attention cases with
expected outputs from torch's scaled_dot_product_attention in float64 — an
independent library routine, not the oracle — used to pin the oracle's
attention (oracle/pkv_oracle.c orc_attn_decode / orc_attn_prefill).

Each case: bf16 (uint16) q [T][Hq][256], K/V pools [slots][Hkv][256] filled
through a shuffled block table, and per (t, h) the fp64 attention output over
keys 0..pos[t] (causal prefill rows use their own pos). Run from the repo root:
    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
D, BS = 256, 16


def bf16_bits(x):
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bits_to_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def case(seed, lens, Hq, Hkv, scale_val):
    rng = np.random.default_rng(seed)
    B = len(lens)
    max_blocks = max((L + BS - 1) // BS for L in lens)
    pages = B * max_blocks + 3
    perm = rng.permutation(pages).astype(np.int32)
    bt = perm[:B * max_blocks].reshape(B, max_blocks)
    kc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * scale_val)
    vc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * scale_val)
    q = bf16_bits(rng.standard_normal((B, Hq, D)) * scale_val)
    pos = np.array([L - 1 for L in lens], np.int32)
    scale = 1.0 / np.sqrt(D)
    G = Hq // Hkv
    expect = np.zeros((B, Hq, D), np.float64)
    for s, L in enumerate(lens):
        slots = bt[s, np.arange(L) // BS] * BS + np.arange(L) % BS
        K = torch.from_numpy(bits_to_f64(kc[slots]))  # [L][Hkv][D]
        V = torch.from_numpy(bits_to_f64(vc[slots]))
        Q = torch.from_numpy(bits_to_f64(q[s]))       # [Hq][D]
        Kh = K.permute(1, 0, 2).repeat_interleave(G, 0)  # [Hq][L][D]
        Vh = V.permute(1, 0, 2).repeat_interleave(G, 0)
        o = F.scaled_dot_product_attention(Q[:, None, :], Kh, Vh, scale=float(scale))
        expect[s] = o[:, 0, :].numpy()
    return dict(q=q, kc=kc, vc=vc, bt=bt, pos=pos, expect=expect, Hq=np.int32(Hq), Hkv=np.int32(Hkv))


def main():
    cases = {
        "a": case(1, [1, 17, 40], 8, 2, 0.5),
        "b": case(2, [33, 5], 16, 4, 1.0),
        "c": case(3, [64], 4, 1, 2.0),
    }
    flat = {}
    for name, c in cases.items():
        for k, v in c.items():
            flat[f"{name}_{k}"] = v
    np.savez_compressed(os.path.join(HERE, "attn_small.npz"), **flat)
    print("wrote", os.path.join(HERE, "attn_small.npz"))


if __name__ == "__main__":
    main()

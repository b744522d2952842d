"""GPU parity: attention input preparation (pkv_attn_prep, and the
reference-named attn_prep kernel of pkv_kernels.hsaco) against the oracle
(oracle/pkv_oracle.c orc_attn_prep, restating qwen35.cu:1067-1128).

Bar: v rows bit-exact at their slots, untouched slots unchanged; normalised
and rotated q / k within 1 bf16 ulp everywhere (the rounding points are the
reference's; the f32 order of the squared sum and the last bits of device
cosf / sinf are not pinned) and bit-exact on at least 99 % of elements."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import bf16_bits
from pkv.refabi import F, I, P, RefKernels

pytestmark = pytest.mark.gpu
D = 256


def mono(bits):
    b = bits.astype(np.int64)
    return np.where(b < 0x8000, b, -(b & 0x7FFF))


def ulp_ok(got, want):
    if got.size == 0:
        return 0, 1.0
    diff = np.abs(mono(got) - mono(want))
    return int(diff.max()), float((diff == 0).mean())


def case(T, Hq, Hkv, seed, pool):
    rng = np.random.default_rng(seed)
    qstride = (2 * Hq + 2 * Hkv) * D
    slots = rng.permutation(pool)[:T].astype(np.int32)
    slots[::7] = -1  # padding rows: no k / v write
    rope = np.tile(rng.integers(0, 131072, size=T), (3, 1)).astype(np.int32)
    rope[1, ::3] += 17   # some tokens with distinct height / width positions
    rope[2, ::3] += 101
    return dict(qkv=bf16_bits(rng.standard_normal((T, qstride)) * 2), qstride=qstride, Hq=Hq, Hkv=Hkv,
                q_norm=(1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
                k_norm=(1 + 0.1 * rng.standard_normal(D)).astype(np.float32), rope=rope, slots=slots,
                inv_freq=(1.0 / 1e7 ** (2 * np.arange(32) / 64.0)).astype(np.float32), T=T, pool=pool)


def check(c, qout, kc, vc, kc0, vc0):
    T, Hq, Hkv, pool = c["T"], c["Hq"], c["Hkv"], c["pool"]
    wq = np.zeros((T, Hq, D), np.uint16)
    wk, wv = kc0.copy(), vc0.copy()
    oracle.attn_prep(c["qkv"], c["qstride"], Hq, Hkv, c["q_norm"], c["k_norm"], c["rope"], T, 11, 11, c["slots"],
                     c["inv_freq"], 1e-6, wq, wk, wv)
    assert np.array_equal(vc, wv)  # v bit for bit, other slots untouched
    written = np.zeros(pool, bool)
    written[c["slots"][c["slots"] >= 0]] = True
    assert np.array_equal(kc[~written], kc0[~written])
    for name, g, w in (("q", qout, wq), ("k", kc[written], wk[written])):
        worst, exact = ulp_ok(g, w)
        assert worst <= 1 and exact >= 0.99, f"{name}: max ulp {worst}, exact {exact:.4f}"


@pytest.mark.parametrize("T,Hq,Hkv,seed", [(37, 16, 4, 0), (64, 8, 2, 1), (1, 4, 1, 2), (20, 24, 4, 3), (9, 32, 4, 4), (5, 2, 2, 5)])
def test_prep_matches_oracle(dev, T, Hq, Hkv, seed):
    print(f"case prep T={T} Hq={Hq} Hkv={Hkv}", flush=True)
    c = case(T, Hq, Hkv, seed, pool=128)
    rng = np.random.default_rng(seed + 100)
    kc0 = bf16_bits(rng.standard_normal((c["pool"], Hkv, D)))
    vc0 = bf16_bits(rng.standard_normal((c["pool"], Hkv, D)))
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    qout = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    kc, vc = t16(kc0), t16(vc0)
    pkv.attn_prep(t16(c["qkv"]), c["qstride"], Hq, Hkv, torch.from_numpy(c["q_norm"]).to(dev),
                  torch.from_numpy(c["k_norm"]).to(dev), torch.from_numpy(c["rope"]).to(dev), T, 11, 11,
                  torch.from_numpy(c["slots"]).to(dev), torch.from_numpy(c["inv_freq"]).to(dev), qout, kc, vc,
                  1e-6, T, c["pool"])
    torch.cuda.synchronize()
    n = lambda x: x.cpu().numpy().view(np.uint16)
    check(c, n(qout), n(kc), n(vc), kc0, vc0)


def test_reference_named_attn_prep(dev):
    """attn_prep of the code object, launched as model.rs:2340-2365 does:
    grid (T, Hq + 2 Hkv), 128 threads, 18 argument slots."""
    print("case refabi attn_prep", flush=True)
    T, Hq, Hkv = 37, 16, 4
    c = case(T, Hq, Hkv, 3, pool=64)
    rng = np.random.default_rng(7)
    kc0 = bf16_bits(rng.standard_normal((c["pool"], Hkv, D)))
    vc0 = bf16_bits(rng.standard_normal((c["pool"], Hkv, D)))
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    qout = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    kc, vc = t16(kc0), t16(vc0)
    rk = RefKernels()
    rk.launch("attn_prep", (T, Hq + 2 * Hkv, 1), 128, 0,
              [P(t16(c["qkv"])), I(c["qstride"]), I(Hq), I(Hkv), P(torch.from_numpy(c["q_norm"]).to(dev)),
               P(torch.from_numpy(c["k_norm"]).to(dev)), P(torch.from_numpy(c["rope"]).to(dev)), I(T), I(11), I(11),
               P(torch.from_numpy(c["slots"]).to(dev)), P(torch.from_numpy(c["inv_freq"]).to(dev)), P(qout), P(kc),
               P(vc), P(None), P(None), F(1e-6)])
    torch.cuda.synchronize()
    n = lambda x: x.cpu().numpy().view(np.uint16)
    check(c, n(qout), n(kc), n(vc), kc0, vc0)

"""Pins the CPU oracle (oracle/pkv_oracle.c) before it is trusted as the
checker: against the torch-fp64 golden fixtures (tests/golden/), closed forms
and brute force. A plausible mistake in the oracle (a dropped scale, a wrong
kv-head index, a transposed operand, a wrong causal bound) fails one of these.
CPU only."""
import os

import numpy as np
import pytest
import torch

import oracle
from _util import BS, D, bf16_bits, decode_case, hash_bf16

GOLD = os.path.join(os.path.dirname(__file__), "golden", "attn_small.npz")


def test_f2b_matches_torch_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf],
                                 np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f2b(x), want)
    # the C helper agrees with the numpy one
    for v in x[:200]:
        assert oracle._lib.orc_f2b(float(v)) == oracle.f2b(np.array([v]))[0]


def test_hash_inputs_match_reference_formula_small_cases():
    # bench-attn inputs (main.rs:739-748) computed by hand for i = 0, 1, seed 1:
    # h = (i ^ 0x9e3779b9) * 2654435761 mod 2^64; x = (h % 2001) / 1000 - 1
    for i in (0, 1, 7):
        h = ((i ^ 0x9E3779B9) * 2654435761) % (1 << 64)
        x = np.float32((h % 2001)) / np.float32(1000.0) - np.float32(1.0)
        assert hash_bf16(8, 1)[i] == bf16_bits(np.array([x]))[0]


@pytest.mark.parametrize("row", [(2, 64, np.float32), (4, 256, np.uint16)])
def test_append_gather_roundtrip_and_closed_form(row):
    Hkv, Dh, dt = row
    rng = np.random.default_rng(1)
    pages = 64
    lens = rng.integers(1, 201, size=4)
    perm = rng.permutation(pages)
    bt = np.zeros((4, 13), np.int32)
    at = 0
    for s, L in enumerate(lens):
        n = (L + BS - 1) // BS
        bt[s, :n] = perm[at:at + n]
        at += n
    kc = np.zeros((pages * BS, Hkv, Dh), dt)
    vc = np.zeros((pages * BS, Hkv, Dh), dt)
    dense = []
    for s, L in enumerate(lens):
        k = rng.standard_normal((L, Hkv, Dh)).astype(np.float32)
        v = rng.standard_normal((L, Hkv, Dh)).astype(np.float32)
        if dt == np.uint16:
            k, v = bf16_bits(k), bf16_bits(v)
        slot = (bt[s, np.arange(L) // BS] * BS + np.arange(L) % BS).astype(np.int32)
        oracle.append(k, v, slot, kc, vc)
        # closed form: the rows sit exactly at their slots
        assert np.array_equal(kc[slot], k) and np.array_equal(vc[slot], v)
        dense.append((k, v))
    for s, L in enumerate(lens):
        ko, vo = oracle.gather(kc, vc, bt[s], int(L), BS)
        assert np.array_equal(ko, dense[s][0]) and np.array_equal(vo, dense[s][1])


def test_append_skips_padding_slots():
    kc = np.zeros((32, 1, 4), np.float32)
    vc = np.zeros_like(kc)
    k = np.ones((3, 1, 4), np.float32)
    oracle.append(k, k * 2, np.array([5, -1, 7], np.int32), kc, vc)
    assert kc[5].sum() == 4 and kc[7].sum() == 4 and kc.sum() == 8 and vc.sum() == 16


def test_page_copy_closed_form():
    rng = np.random.default_rng(2)
    kc = rng.standard_normal((8 * BS, 2, 8)).astype(np.float32)
    vc = rng.standard_normal((8 * BS, 2, 8)).astype(np.float32)
    k0, v0 = kc.copy(), vc.copy()
    page_bytes = BS * 2 * 8 * 4
    oracle.page_copy(kc, vc, [1, 3], [6, 0], page_bytes)
    ref_k, ref_v = k0.copy(), v0.copy()
    ref_k[6 * BS:7 * BS] = k0[BS:2 * BS]
    ref_k[0:BS] = k0[3 * BS:4 * BS]
    ref_v[6 * BS:7 * BS] = v0[BS:2 * BS]
    ref_v[0:BS] = v0[3 * BS:4 * BS]
    assert np.array_equal(kc, ref_k) and np.array_equal(vc, ref_v)


@pytest.mark.parametrize("name", ["a", "b", "c"])
def test_decode_oracle_matches_torch_sdpa_golden(name):
    g = np.load(GOLD)
    c = {k[2:]: g[k] for k in g.files if k.startswith(name + "_")}
    Hq, Hkv = int(c["Hq"]), int(c["Hkv"])
    B = len(c["pos"])
    qstride = (2 * Hq + 2 * Hkv) * D
    gate = np.zeros((B, qstride), np.uint16)  # gate 0 -> sigmoid 1/2
    out, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], gate, qstride, Hq, Hkv, c["pos"],
                                  np.arange(B, dtype=np.int32), c["bt"], c["bt"].shape[1], BS, 1.0 / 16.0)
    np.testing.assert_allclose(raw, c["expect"], rtol=1e-5, atol=1e-6)
    # gated epilogue: bf16(bf16(o) * 0.5) == bf16(o) * 0.5 exactly (a power of two)
    want = bf16_bits(oracle.b2f(bf16_bits(raw)) * 0.5)
    assert np.array_equal(out, want)


def test_decode_gate_and_closed_forms():
    Hq, Hkv = 4, 1
    c = decode_case([1, 20, 20], Hq, Hkv, seed=3)
    # sequence 1: every key equal -> output = mean of v
    bt1 = c["bt"][1]
    slots = bt1[np.arange(20) // BS] * BS + np.arange(20) % BS
    c["kc"][slots] = c["kc"][slots[0]]
    # sequence 2: one key hugely aligned with q -> output = its v
    bt2 = c["bt"][2]
    slots2 = bt2[np.arange(20) // BS] * BS + np.arange(20) % BS
    qf = oracle.b2f(c["q"][2, 0])
    c["kc"][slots2[7], 0] = bf16_bits(qf * 64)
    c["kc"][slots2[np.arange(20) != 7], 0] = 0
    out, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"],
                                  c["bt"], c["max_blocks"], BS, 1.0 / 16.0)
    v = oracle.b2f(c["vc"])
    # one key: o = v of that key for every head
    np.testing.assert_allclose(raw[0], np.broadcast_to(v[c["bt"][0][0] * BS, 0], (Hq, D)), rtol=1e-6)
    np.testing.assert_allclose(raw[1], np.broadcast_to(v[slots, 0].astype(np.float64).mean(0), (Hq, D)),
                               rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(raw[2, 0], v[slots2[7], 0], rtol=1e-5, atol=1e-6)
    # gate: y = bf16(bf16(o) / (1 + exp(-gate)))
    gate = oracle.b2f(c["qkv"][:, :Hq * 2 * D].reshape(3, Hq, 2, D)[:, :, 1, :])
    want = bf16_bits(oracle.b2f(bf16_bits(raw)) / (np.float32(1) + np.exp(-gate, dtype=np.float32)))
    assert np.array_equal(out, want)


@pytest.mark.parametrize("lens,Hq,Hkv,seed", [([1, 17, 300], 16, 4, 11), ([900, 40], 24, 4, 12), ([64], 8, 8, 13)])
def test_decode_f32_scalar_port_within_tolerance_of_the_oracle(lens, Hq, Hkv, seed):
    """The one-pass f32 scalar decode (the CPU baseline's f32 leg) against the
    f64 oracle: within the attention tolerance; the golden fixtures' cases
    within it too (gates 0); a skipped prompt row is left untouched."""
    from _util import close
    c = decode_case(lens, Hq, Hkv, seed=seed)
    want, _ = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"],
                                 c["bt"], c["max_blocks"], BS, 1.0 / 16.0)
    got = oracle.attn_decode_f32(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"],
                                 c["bt"], c["max_blocks"], BS, 1.0 / 16.0)
    ok, err = close(got, want, what="f32 scalar port vs f64 oracle")
    assert ok, err
    g = np.load(GOLD)
    cg = {k[2:]: g[k] for k in g.files if k.startswith("a_")}
    Hq2, Hkv2 = int(cg["Hq"]), int(cg["Hkv"])
    B = len(cg["pos"])
    qstride = (2 * Hq2 + 2 * Hkv2) * D
    gate = np.zeros((B, qstride), np.uint16)
    got = oracle.attn_decode_f32(cg["q"], cg["kc"], cg["vc"], gate, qstride, Hq2, Hkv2, cg["pos"],
                                 np.arange(B, dtype=np.int32), cg["bt"], cg["bt"].shape[1], BS, 1.0 / 16.0)
    ok, err = close(got, bf16_bits(oracle.b2f(bf16_bits(cg["expect"])) * 0.5), what="f32 port vs SDPA golden")
    assert ok, err


def test_decode_wrong_head_mapping_would_fail():
    """GQA: q head h reads kv head h // G. Pools whose kv heads differ give
    different outputs per group, and equal outputs within a group only when q
    is equal."""
    Hq, Hkv = 8, 2
    c = decode_case([30], Hq, Hkv, seed=4)
    c["q"][0, :] = c["q"][0, 0]
    _, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"],
                                c["bt"], c["max_blocks"], BS, 0.0625)
    assert np.array_equal(raw[0, 0], raw[0, 3]) and not np.allclose(raw[0, 0], raw[0, 4])


def test_skip_prompts_and_spec_rows():
    Hq, Hkv = 4, 1
    c = decode_case([10, 12, 9], Hq, Hkv, seed=5)
    # sequence 0: 1 decode token; sequence 1: a 2-token prompt chunk; sequence 2: verifying (outs >= 0)
    pos = np.array([9, 10, 11, 7, 8], np.int32)
    tok_seq = np.array([0, 1, 1, 2, 2], np.int32)
    cu = np.array([0, 1, 3, 5], np.int32)
    outs = np.array([-1, -1, 4], np.int32)
    q = np.concatenate([c["q"], c["q"][:2]])
    qkv = np.concatenate([c["qkv"], c["qkv"][:2]])
    sentinel = np.full((5, Hq, D), 0x7777, np.uint16)
    out, _ = oracle.attn_decode(q, c["kc"], c["vc"], qkv, c["qstride"], Hq, Hkv, pos, tok_seq, c["bt"],
                                c["max_blocks"], BS, 0.0625, cu=cu, skip_prompts=1, outs=outs, spec=1,
                                out=sentinel.copy())
    assert (out[1:3] == 0x7777).all(), "prompt rows are left to prefill"
    assert not (out[0] == 0x7777).any() and not (out[3:] == 0x7777).any()


def test_split_merge_equals_unsplit():
    Hq, Hkv = 4, 1
    c = decode_case([300], Hq, Hkv, seed=6)
    L = 300
    M, S, A = oracle.attn_partial(c["q"], c["kc"], c["vc"], Hq, Hkv, 0, 2, c["bt"][0], BS, 0, L, 0.0625)
    for cuts in ([0, 100, 300], [0, 1, 64, 65, 299, 300], [0, 150, 300]):
        parts = [oracle.attn_partial(c["q"], c["kc"], c["vc"], Hq, Hkv, 0, 2, c["bt"][0], BS, a, b, 0.0625)
                 for a, b in zip(cuts[:-1], cuts[1:])]
        o = oracle.merge([p[0] for p in parts], [p[1] for p in parts], [p[2] for p in parts])
        np.testing.assert_allclose(o, A / S, rtol=1e-12, atol=1e-14)


def test_split_parts_examples():
    # model.rs:44-46 / qwen35.cu:1139-1141 at 256 CUs, ROCm min_chunk 64
    assert oracle.split_parts(4097, 64, 64) == 64
    assert oracle.split_parts(100, 4, 64) == 2
    assert oracle.split_parts(1, 4, 64) == 1
    assert oracle.split_parts(8193, 4, 64) == 4


def test_prefill_oracle_matches_causal_sdpa():
    """Prefill rows: causal over keys 0..pos[t]; q rounded to bf16 after
    scaling by scale*log2(e), exp2 softmax == SDPA(q', K, V, scale=ln 2)."""
    Hq, Hkv, n, ctx = 8, 2, 21, 13
    rng = np.random.default_rng(7)
    L = ctx + n
    c = decode_case([L], Hq, Hkv, seed=7)
    q = bf16_bits(rng.standard_normal((n, Hq, D)) * 0.5)
    qkv = np.zeros((n, c["qstride"]), np.uint16)
    pos = np.arange(ctx, ctx + n, dtype=np.int32)
    cu = np.array([0, n], np.int32)
    out = oracle.attn_prefill(q, c["kc"], c["vc"], qkv, c["qstride"], Hq, Hkv, pos, cu, 1, c["bt"], c["max_blocks"],
                              BS, 0.0625, p_tile=0)
    slots = c["bt"][0][np.arange(L) // BS] * BS + np.arange(L) % BS
    K = torch.from_numpy(oracle.b2f(c["kc"][slots]).astype(np.float64)).permute(1, 0, 2).repeat_interleave(4, 0)
    V = torch.from_numpy(oracle.b2f(c["vc"][slots]).astype(np.float64)).permute(1, 0, 2).repeat_interleave(4, 0)
    qs = oracle.b2f(bf16_bits(oracle.b2f(q) * np.float32(0.0625 * 1.4426950408889634)))
    Q = torch.from_numpy(qs.astype(np.float64)).permute(1, 0, 2)  # [Hq][n][D]
    mask = torch.from_numpy(np.arange(L)[None, :] <= pos[:, None])
    o = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=float(np.log(2.0)))
    want = bf16_bits(oracle.b2f(bf16_bits(o.permute(1, 0, 2).numpy().astype(np.float32))) * 0.5)
    got = oracle.b2f(out)
    assert np.abs(got - oracle.b2f(want)).max() <= 2 ** -9  # one bf16 rounding apart at most
    # the causal bound matters: the first row differs from attending all keys
    assert not np.allclose(o[:, 0], o[:, -1])


def _prefill_scores_case(scores, n_keys, seed=0):
    """One sequence of n_keys keys whose scores (exp2 domain) for its last
    two query rows are `scores` (dict key -> bf16-exact score, others 0):
    q = e_0 scaled by ln 2 (so q' = bf16(q * scale * log2 e) = e_0), K rows
    zero except dim 0 = score, V random; gates large (sigmoid = 1 in f32)."""
    Hq, Hkv = 4, 1
    rng = np.random.default_rng(seed)
    pages = (n_keys + BS - 1) // BS
    kc = np.zeros((pages * BS, Hkv, D), np.uint16)
    for j, sc in scores.items():
        kc[j, 0, 0] = bf16_bits(np.array([sc], np.float32))[0]
    vc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * 0.5)
    q = np.zeros((2, Hq, D), np.uint16)
    q[:, :, 0] = bf16_bits(np.float32(1.0))
    qstride = (2 * Hq + 2 * Hkv) * D
    qkv = np.zeros((2, qstride), np.uint16)
    for h in range(Hq):
        qkv[:, h * 2 * D + D:h * 2 * D + 2 * D] = bf16_bits(np.float32(30.0))
    pos = np.array([n_keys - 2, n_keys - 1], np.int32)
    bt = np.arange(pages, dtype=np.int32)[None, :]
    return dict(q=q, kc=kc, vc=vc, qkv=qkv, qstride=qstride, pos=pos, cu=np.array([0, 2], np.int32), bt=bt,
                pages=pages, Hq=Hq, Hkv=Hkv)


def test_prefill_oracle_reference_tiles_round_p_against_the_running_max():
    """The reference's prefill softmax (amd/attention.cuh:55-121, AM_BN = 32):
    per 32-key tile the anchor is the running max, P.V takes bf16(p) and the
    denominator the unrounded p. Three keys: scores 0 and r = bf16(-0.3) in
    the first tile, 0.5 at key 32 (a new max in the second tile). Closed
    form: A = (v0 + bf16(2^r) v1) 2^-0.5 + v32, S = (1 + 2^r) 2^-0.5 + 1.
    Anchoring every p on the final max instead, rounding the denominator
    too, or not rounding at all all give other bits; with p_tile = 0 the
    result is the textbook softmax."""
    r = float(oracle.b2f(bf16_bits(np.float32(-0.3))))
    n = 34  # keys 0..33 for the last row (key 33 score 0, like key 0)
    c = _prefill_scores_case({1: r, 32: 0.5}, n)
    args = (c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"], 1, c["bt"],
            c["pages"], BS, float(np.log(2.0)))
    got = oracle.attn_prefill(*args, p_tile=32)
    exact = oracle.attn_prefill(*args, p_tile=0)
    v = oracle.b2f(c["vc"][:, 0]).astype(np.float64)
    sc = np.zeros(n)
    sc[1], sc[32] = r, 0.5
    # row 1 (position 33): tile 1 = keys 0..31 (anchor 0), tile 2 = keys 32, 33 (anchor 0.5)
    p1 = 2.0 ** (sc[:32] - 0.0)
    p2 = 2.0 ** (sc[32:34] - 0.5)
    rb = lambda x: oracle.b2f(bf16_bits(np.asarray(x, np.float32))).astype(np.float64)
    A = (rb(p1) @ v[:32]) * 2 ** -0.5 + rb(p2) @ v[32:34]
    S = p1.sum() * 2 ** -0.5 + p2.sum()
    want = bf16_bits(oracle.b2f(bf16_bits((A / S).astype(np.float32))))
    for h in range(c["Hq"]):
        assert np.abs(oracle.b2f(got[1, h]) - oracle.b2f(want)).max() == 0
    # a final-max anchor rounds other values: the tiled result is not that
    p_fin = 2.0 ** (sc - 0.5)
    alt = bf16_bits(((rb(p_fin) @ v[:n]) / p_fin.sum()).astype(np.float32))
    assert not np.array_equal(got[1, 0], alt)
    # and differs from the textbook softmax by P rounding only
    assert not np.array_equal(got[1], exact[1])
    assert np.abs(oracle.b2f(got) - oracle.b2f(exact)).max() <= 2e-2


def test_prefill_oracle_tiles_equal_textbook_when_p_is_exact():
    """Scores whose differences are integers make every p a power of two
    (exact in bf16, exact under any anchor): the tiled softmax with rounding
    must then equal the textbook one bit for bit, across 5 tiles with the
    max moving up in tiles 2 and 4 (the rescale of earlier sums)."""
    scores = {3: -2.0, 40: 1.0, 77: -1.0, 100: 3.0, 140: -4.0}
    c = _prefill_scores_case(scores, 150, seed=3)
    args = (c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"], 1, c["bt"],
            c["pages"], BS, float(np.log(2.0)))
    assert np.array_equal(oracle.attn_prefill(*args, p_tile=32), oracle.attn_prefill(*args, p_tile=0))


def test_mtp_slots_closed_form():
    bt = np.array([[5, 9, 2], [7, 1, 0]], np.int32)
    dpos, dslot = oracle.mtp_slots([0, 1], [15, 3], bt, 3, BS, [47, 4], 2)
    assert list(dpos) == [17, 5]
    assert list(dslot) == [9 * 16 + 1, -1]


def test_mtp_next_closed_form():
    """Draft pass k = 2 over two sequences (rows 3 and 0 of the step): slot
    of position pos + 2 through the block table while within the limit (-1
    past it), rotary rows shifted by k per axis (rope_stride 5)."""
    bt = np.array([[5, 9, 2], [7, 1, 0]], np.int32)
    pos = np.array([3, 0, 0, 15], np.int32)      # rows 0..3
    rope = np.arange(15, dtype=np.int32) * 10    # 3 axes x stride 5
    dpos, dslot, drope = oracle.mtp_next([3, 0], pos, rope, 5, bt, 3, BS, [47, 4], 2)
    assert list(dpos) == [17, 5]
    assert list(dslot) == [9 * 16 + 1, -1]      # 17 <= 47: page 1 of row 0; 5 > 4
    assert drope.tolist() == [[32, 2], [82, 52], [132, 102]]


# ---- attn_prep (reference qwen35.cu:1067-1128) ----

def _prep_case(T, Hq, Hkv, rng, slots=None, sec=(11, 11, 10), theta=1e7):
    qstride = (2 * Hq + 2 * Hkv) * 256
    qkv = bf16_bits(rng.standard_normal((T, qstride)))
    inv_freq = (1.0 / theta ** (2 * np.arange(32) / 64.0)).astype(np.float32)
    return dict(qkv=qkv, qstride=qstride, Hq=Hq, Hkv=Hkv, q_norm=np.ones(256, np.float32),
                k_norm=np.ones(256, np.float32), rope=np.zeros((3, T), np.int32), sec=sec, inv_freq=inv_freq,
                slots=np.arange(T, dtype=np.int32) if slots is None else np.asarray(slots, np.int32))


def _run_prep(c, eps=1e-6, pool=None):
    T, Hq, Hkv = len(c["slots"]), c["Hq"], c["Hkv"]
    pool = pool or max(T, 1)
    qout = np.zeros((T, Hq, 256), np.uint16)
    kc = np.full((pool, Hkv, 256), 0x7777, np.uint16)
    vc = np.full((pool, Hkv, 256), 0x7777, np.uint16)
    oracle.attn_prep(c["qkv"], c["qstride"], Hq, Hkv, c["q_norm"], c["k_norm"], c["rope"], T, c["sec"][1],
                     c["sec"][2], c["slots"], c["inv_freq"], eps, qout, kc, vc)
    return qout, kc, vc


def test_prep_constant_rows_normalise_to_weights():
    """A constant head row with eps = 0 normalises to exactly w (position 0:
    no rotation): x * (1 / |x|) * w = w for w exact in bf16."""
    rng = np.random.default_rng(0)
    c = _prep_case(2, 4, 2, rng)
    c["qkv"][:] = bf16_bits(np.full(c["qkv"].shape, 0.75))
    c["q_norm"] = np.linspace(-2, 2, 256).astype(np.float32)
    c["q_norm"] = oracle.b2f(bf16_bits(c["q_norm"]))
    qout, kc, _ = _run_prep(c, eps=0.0)
    assert np.array_equal(oracle.b2f(qout[0, 0]), c["q_norm"])
    assert np.array_equal(oracle.b2f(kc[1, 1]), np.ones(256, np.float32))


def test_prep_position_zero_is_plain_rmsnorm_and_v_is_copied():
    rng = np.random.default_rng(1)
    c = _prep_case(3, 4, 2, rng, slots=[5, -1, 2])
    qout, kc, vc = _run_prep(c, pool=8)
    x = oracle.b2f(c["qkv"][0, :256]).astype(np.float64)
    y = x / np.sqrt((x * x).mean() + 1e-6)
    got = oracle.b2f(qout[0, 0]).astype(np.float64)
    assert np.abs(got - y).max() <= 2 ** -7 * np.abs(y).max()
    # v rows bit for bit at their slots; slot -1 writes nothing (q still written)
    voff = (2 * 4 + 2) * 256
    assert np.array_equal(vc[5].reshape(-1), c["qkv"][0, voff:voff + 512])
    assert np.array_equal(vc[2].reshape(-1), c["qkv"][2, voff:voff + 512])
    untouched = [i for i in range(8) if i not in (5, 2)]
    assert (vc[untouched] == 0x7777).all() and (kc[untouched] == 0x7777).all()
    assert not (qout[1] == 0).all()


def test_prep_rotation_keeps_pair_norms_and_angles():
    """Each pair (d, d + 32) turns by pos * inv_freq[d]: against a complex
    rotation of the position-0 result (within bf16 rounding)."""
    rng = np.random.default_rng(2)
    c = _prep_case(1, 1, 0, rng)
    base, _, _ = _run_prep(c)
    c["rope"][:] = 1234
    rot, _, _ = _run_prep(c)
    y0 = oracle.b2f(base[0, 0]).astype(np.float64)
    y1 = oracle.b2f(rot[0, 0]).astype(np.float64)
    ang = 1234.0 * c["inv_freq"].astype(np.float64)
    z0 = y0[:32] + 1j * y0[32:64]
    z1 = y1[:32] + 1j * y1[32:64]
    want = z0 * np.exp(1j * ang)
    assert np.abs(z1 - want).max() < 3 * 2 ** -8 * np.abs(z0).max()
    assert np.array_equal(y1[64:], y0[64:])  # dims past 64 are not rotated


def test_prep_axis_rule():
    """Frequencies d % 3 == 1 below 3 sec_h take the height position, d % 3
    == 2 below 3 sec_w the width position, the rest time (interleaved
    multimodal rotary). Each frequency's angle identifies its axis."""
    rng = np.random.default_rng(3)
    c = _prep_case(1, 1, 0, rng, sec=(11, 5, 3))
    base, _, _ = _run_prep(c)
    c["rope"][:, 0] = [1000, 2000, 3000]
    rot, _, _ = _run_prep(c)
    y0 = oracle.b2f(base[0, 0]).astype(np.float64)
    y1 = oracle.b2f(rot[0, 0]).astype(np.float64)
    z0 = y0[:32] + 1j * y0[32:64]
    z1 = y1[:32] + 1j * y1[32:64]
    for d in range(32):
        errs = [abs(z1[d] - z0[d] * np.exp(1j * p * float(c["inv_freq"][d]))) for p in (1000, 2000, 3000)]
        axis = int(np.argmin(errs))
        want = 1 if (d % 3 == 1 and d < 15) else 2 if (d % 3 == 2 and d < 9) else 0
        if abs(z0[d]) > 0.05 and float(c["inv_freq"][d]) * 1000 > 1e-2:
            assert axis == want, (d, errs)


# ---- E4M3 cache (reference store_e4m3 / attn_paged8, qwen35.cu:1055-1065, 1146-1309) ----

def test_e4m3_decode_all_codes_match_torch():
    import torch
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.e4m3_to_f(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert set(np.flatnonzero(nan)) == {0x7F, 0xFF}


def test_e4m3_encode_matches_torch_in_range_and_saturates():
    import torch
    rng = np.random.default_rng(0)
    grid = oracle.e4m3_to_f(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (grid[:-1] + grid[1:]) / 2  # exact ties
    x = np.concatenate([rng.standard_normal(4000) * 50, rng.standard_normal(2000) * 0.01, mids, -mids,
                        [0.0, -0.0, 448.0, -448.0, 2 ** -9, 2 ** -10, 3 * 2 ** -10]]).astype(np.float32)
    x = x[np.abs(x) < 464]  # torch overflows to NaN past the largest tie; the reference saturates
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.f_to_e4m3(x), want)
    assert list(oracle.f_to_e4m3(np.array([500.0, -1e9, 464.0], np.float32))) == [0x7E, 0xFE, 0x7E]
    assert oracle.f_to_e4m3(np.array([np.nan], np.float32))[0] == 0x7F


def test_e4m3_store_scale_and_zero_row():
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(256) * 3).astype(np.float32)
    b, sc = oracle.store_e4m3(v)
    assert sc == np.float32(np.abs(v).max()) / np.float32(448.0)
    assert np.abs(oracle.e4m3_to_f(b)).max() == 448.0  # the largest maps to E4M3's largest
    assert np.allclose(oracle.e4m3_to_f(b) * sc, v, rtol=2 ** -3, atol=sc * 2 ** -9)
    b0, sc0 = oracle.store_e4m3(np.zeros(256, np.float32))
    assert sc0 == 1.0 and not b0.any()


def test_decode8_equals_bf16_decode_on_the_e4m3_grid():
    """K and V whose values sit on the E4M3 grid (scale 1): E4M3 decode ==
    bf16 decode; a single key gives its scaled value."""
    from _util import decode_case
    c = decode_case([1, 37, 150], 16, 4, 5)
    rng = np.random.default_rng(5)
    grid = oracle.e4m3_to_f(np.arange(0x60, dtype=np.uint8))  # |v| < 16
    n = c["kc"].size
    k8 = rng.integers(0, 0x60, size=n).astype(np.uint8) | (rng.integers(0, 2, size=n).astype(np.uint8) << 7)
    v8 = rng.integers(0, 0x60, size=n).astype(np.uint8) | (rng.integers(0, 2, size=n).astype(np.uint8) << 7)
    kbf = bf16_bits(oracle.e4m3_to_f(k8)).reshape(c["kc"].shape)
    vbf = bf16_bits(oracle.e4m3_to_f(v8)).reshape(c["vc"].shape)
    slots = c["kc"].shape[0] * c["kc"].shape[1]
    ones = np.ones(slots, np.float32)
    got = oracle.attn_decode8(c["q"], k8, v8, ones, ones, c["qkv"], c["qstride"], 16, 4, c["pos"], c["tok_seq"],
                              c["bt"], c["max_blocks"], 16, 1 / 16)
    want, _ = oracle.attn_decode(c["q"], kbf, vbf, c["qkv"], c["qstride"], 16, 4, c["pos"], c["tok_seq"], c["bt"],
                                 c["max_blocks"], 16, 1 / 16)
    assert np.array_equal(got, want)
    # one key: output is its value times its scale, gated
    vs = np.full(slots, 0.5, np.float32)
    got1 = oracle.attn_decode8(c["q"], k8, v8, ones, vs, c["qkv"], c["qstride"], 16, 4, c["pos"], c["tok_seq"],
                               c["bt"], c["max_blocks"], 16, 1 / 16)
    want1, _ = oracle.attn_decode(c["q"], kbf, bf16_bits(oracle.b2f(vbf) * 0.5), c["qkv"], c["qstride"], 16, 4,
                                  c["pos"], c["tok_seq"], c["bt"], c["max_blocks"], 16, 1 / 16)
    assert np.array_equal(got1, want1)


def test_prefill8_is_prefill_of_the_dequantised_cache():
    """E4M3 prefill == bf16 prefill of bf16(e4m3 * scale) rows, and with
    unit scales on grid values == bf16 prefill of the same values."""
    from _util import decode_case
    rng = np.random.default_rng(8)
    c = decode_case([40, 70], 8, 2, 8)
    T = 12
    pos = np.concatenate([np.arange(28, 34), np.arange(64, 70)]).astype(np.int32)
    cu = np.array([0, 6, 12], np.int32)
    q = bf16_bits(rng.standard_normal((T, 8, 256)) * 0.5)
    qkv = bf16_bits(rng.standard_normal((T, c["qstride"])))
    k8 = rng.integers(0, 0x60, size=c["kc"].shape).astype(np.uint8)
    v8 = rng.integers(0, 0x60, size=c["vc"].shape).astype(np.uint8) | 0x80
    ks = rng.random(c["kc"].shape[:2]).astype(np.float32) * 0.1
    vs = rng.random(c["kc"].shape[:2]).astype(np.float32) * 0.1
    got = oracle.attn_prefill8(q, k8, v8, ks, vs, qkv, c["qstride"], 8, 2, pos, cu, 2, c["bt"], c["max_blocks"], 16,
                               1 / 16)
    kb = bf16_bits(oracle.e4m3_to_f(k8) * ks[:, :, None])
    vb = bf16_bits(oracle.e4m3_to_f(v8) * vs[:, :, None])
    want = oracle.attn_prefill(q, kb, vb, qkv, c["qstride"], 8, 2, pos, cu, 2, c["bt"], c["max_blocks"], 16, 1 / 16)
    assert np.array_equal(got, want)
    assert not (got == 0).all()


def test_mx_exp_is_the_smallest_exponent_fitting_448():
    """orc_mx_exp(a) is the smallest e with a / 2^e <= 448 (brute force over
    random amax, powers of two and 448 2^k exactly, where the frexp mantissa
    is 0.5), -127 for zero."""
    rng = np.random.default_rng(3)
    vals = list(np.float32(rng.random(2000) * 10.0 ** rng.integers(-6, 6, 2000)))
    vals += [np.float32(448 * 2.0 ** k) for k in range(-20, 20)] + [np.float32(2.0 ** k) for k in range(-20, 20)]
    vals += [np.nextafter(np.float32(448 * 2.0 ** k), np.float32(np.inf)) for k in range(-5, 5)]
    for a in vals:
        e = oracle.mx_exp(a)
        want = next(x for x in range(-127, 128) if np.float64(a) / 2.0 ** x <= 448)
        assert e == want, (a, e, want)
    assert oracle.mx_exp(0.0) == -127


def test_mx_index_is_the_128x4_tile_layout():
    """The Mx32 scale index is a bijection of (row, block) onto the tiles'
    bytes; inside a 128-row x 4-block tile of 512 bytes the 4 blocks of a row
    are adjacent and rows r, r + 32, r + 64, r + 96 share one 16-byte line
    (cuBLASLt's block-scale tile), tiles row-major over the column tiles."""
    T, KB = 300, 10
    kt = (KB + 3) // 4
    seen = set()
    for r in range(T):
        for kb in range(KB):
            i = oracle.mx_index(r, kb, KB)
            tile, within = divmod(i, 512)
            assert tile == (r // 128) * kt + kb // 4
            line, byte = divmod(within, 16)
            assert line == r % 32 and byte // 4 == (r % 128) // 32 and byte % 4 == kb % 4
            seen.add(i)
    assert len(seen) == T * KB


@pytest.mark.parametrize("mode", [1, 2])
def test_fp8_rows_round_trip(mode):
    """Bytes dequantise to within half an E4M3 step of v (relative 2^-4 for
    normals, absolute 2^-10 scale for subnormals); a row of E4M3 grid values
    with amax 448 comes back exactly (scale 1 / exponent 127 + 0), and a zero
    group gets scale 1 / exponent byte 0."""
    rng = np.random.default_rng(mode)
    T, K = 130, 512
    y = (rng.standard_normal((T, K)) * 10.0 ** rng.integers(-3, 3, (T, 1))).astype(np.float32)
    y[5, 128:256] = 0.0
    grid = oracle.e4m3_to_f(np.arange(0, 0x7F, dtype=np.uint8))
    y[7] = np.resize(grid, K) * np.where(np.arange(K) % 2, 1, -1)
    y[7, ::32] = 448.0
    q, s = oracle.fp8_rows(y, mode)
    gw = 128 if mode == 1 else 32
    for t in range(T):
        for e in range(0, K, gw):
            if mode == 1:
                sc = s[e // 128, t]
            else:
                sc = 2.0 ** (int(s[oracle.mx_index(t, e // 32, K // 32)]) - 127)
            v = y[t, e:e + gw].astype(np.float64)
            back = oracle.e4m3_to_f(q[t, e:e + gw]).astype(np.float64) * sc
            step = np.maximum(np.abs(v) * 2.0 ** -4, sc * 2.0 ** -10)
            assert (np.abs(back - v) <= step * 1.0001).all(), (t, e)
            if t == 5 and e == 128:
                assert (q[t, e:e + gw] == 0).all() and (sc == 1.0 if mode == 1 else
                                                        s[oracle.mx_index(t, 4, 16)] == 0)
            if t == 7:
                assert sc == 1.0 and (back == v).all(), (t, e)

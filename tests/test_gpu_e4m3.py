"""GPU parity of the E4M3 KV cache: pkv_attn_prep with scales (the
reference's store_e4m3 in attn_prep, qwen35.cu:1055-1128) and
pkv_attn_decode_e4m3 / pkv_attn_verify_e4m3 (attn_paged8_g4,
qwen35.cu:1146-1334 with F8) against the oracle (oracle/pkv_oracle.c orc_attn_prep8 / orc_attn_decode8).

Bars: v bytes and scales bit-exact (quantised from the exact bf16 inputs);
k bytes within one E4M3 code (the normed / rotated bf16 inputs may differ by
one bf16 ulp, see test_gpu_prep.py) with scales within 1 %; attention
outputs within max-abs 2e-3 and relative 1e-2 of the oracle. The hardware
conversions are OCP E4M3FN on gfx950; the oracle's are pinned against
torch.float8_e4m3fn in tests/test_oracle.py."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits, close, decode_case
from test_gpu_prep import case as prep_case
from test_gpu_verify import verify_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0


def t_(a, dev):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def test_prep_stores_e4m3(dev):
    print("case prep e4m3", flush=True)
    T, Hq, Hkv = 37, 16, 4
    c = prep_case(T, Hq, Hkv, 11, pool=64)
    pool = c["pool"]
    kc8 = np.full((pool, Hkv, D), 0x33, np.uint8)
    vc8 = np.full((pool, Hkv, D), 0x33, np.uint8)
    ks = np.full((pool, Hkv), -1.0, np.float32)
    vs = np.full((pool, Hkv), -1.0, np.float32)
    qout = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    kd, vd, ksd, vsd = t_(kc8, dev), t_(vc8, dev), t_(ks, dev), t_(vs, dev)
    pkv.attn_prep(t_(c["qkv"], dev), c["qstride"], Hq, Hkv, t_(c["q_norm"], dev), t_(c["k_norm"], dev),
                  t_(c["rope"], dev), T, 11, 11, t_(c["slots"], dev), t_(c["inv_freq"], dev), qout, kd, vd, 1e-6, T, pool,
                  kscale=ksd, vscale=vsd)
    torch.cuda.synchronize()
    wq = np.zeros((T, Hq, D), np.uint16)
    wk8, wv8, wks, wvs = kc8.copy(), vc8.copy(), ks.copy(), vs.copy()
    oracle.attn_prep8(c["qkv"], c["qstride"], Hq, Hkv, c["q_norm"], c["k_norm"], c["rope"], T, 11, 11, c["slots"],
                      c["inv_freq"], 1e-6, wq, wk8, wv8, wks, wvs)
    gk8, gv8, gks, gvs = kd.cpu().numpy(), vd.cpu().numpy(), ksd.cpu().numpy(), vsd.cpu().numpy()
    assert np.array_equal(gv8, wv8) and np.array_equal(gvs, wvs)  # untouched slots included
    written = np.zeros(pool, bool)
    written[c["slots"][c["slots"] >= 0]] = True
    assert np.array_equal(gk8[~written], wk8[~written]) and np.array_equal(gks[~written], wks[~written])
    assert np.allclose(gks[written], wks[written], rtol=1e-2)
    a, b = gk8[written].astype(np.int32), wk8[written].astype(np.int32)
    same_sign = (a >> 7) == (b >> 7)
    assert (np.abs(a - b)[same_sign] <= 1).all() and same_sign.mean() > 0.999
    assert (a == b).mean() > 0.97


def e4m3_cache(shape, rng):
    """Random E4M3 bytes (no NaN codes) and positive scales per slot row head."""
    b = rng.integers(0, 0x7F, size=shape).astype(np.uint8)  # 0x00 .. 0x7E
    return b | (rng.integers(0, 2, size=shape).astype(np.uint8) << 7)


def run_decode8(c, k8, v8, ks, vs, dev, skip=0, outs=None, spec=1, out_init=None, entry="decode"):
    """pkv_attn_decode_e4m3 (per-token ranges) or pkv_attn_verify_e4m3 (rows
    of a sequence grouped), each with its own workspace size."""
    T, Hq = len(c["pos"]), c["Hq"]
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev) if out_init is None else t_(out_init, dev)
    fn, wsf = ((pkv.attn_decode_e4m3, pkv.attn_decode_workspace) if entry == "decode" else
               (pkv.attn_verify_e4m3, pkv.attn_verify_workspace))
    ws = torch.empty(wsf(T, Hq), dtype=torch.uint8, device=dev)
    fn(t_(c["q"], dev), t_(k8, dev), t_(v8, dev), t_(ks, dev), t_(vs, dev), t_(c["qkv"], dev),
                         c["qstride"], Hq, c["Hkv"], t_(c["pos"].astype(np.int32), dev),
                         t_(c["tok_seq"].astype(np.int32), dev), t_(c["bt"], dev), c["max_blocks"], BS, out, SCALE,
                         t_(c["cu"].astype(np.int32), dev), skip, None if outs is None else t_(outs, dev), spec, T,
                         c["pages"], ws)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("entry", ["decode", "verify"])
@pytest.mark.parametrize("lens,Hkv,seed,min_range", [
    ([1, 2, 15, 16, 17], 4, 0, 32),
    ([513, 8193, 1000, 4000, 777, 64], 4, 1, 32),
    ([300, 5000], 2, 2, 32),
    ([900, 2000], 8, 3, 1 << 20),
    ([31, 32, 33, 47, 48, 49, 95], 4, 5, 16),
    ([5, 40, 17, 33] * 75, 4, 6, 32),     # 300 rows: more than a block's token tables
    ([100, 3, 47] * 30, 1, 7, 32),        # Hkv 1 (64-thread blocks), 90 rows
    ([600] * 56, 4, 8, 32),               # two ranges per CU: ~10 records per row, one-wave merge blocks
])
def test_decode_e4m3_matches_oracle(dev, entry, lens, Hkv, seed, min_range):
    print(f"case {entry} e4m3 lens={lens} Hkv={Hkv} min_range={min_range}", flush=True)
    pkv.attn_decode_config(1, min_range)
    try:
        c = decode_case(lens, 4 * Hkv, Hkv, seed)
        rng = np.random.default_rng(seed + 50)
        k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
        ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)  # |k| up to ~9
        vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
        got = run_decode8(c, k8, v8, ks, vs, dev, entry=entry)
        want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"],
                                   c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
        ok, err = close(got, want)
        assert ok, f"max |diff| {err}"
    finally:
        pkv.attn_decode_config(1, 32)


@pytest.mark.parametrize("entry", ["decode", "verify"])
def test_verify_e4m3_rows_and_prompt_skip(dev, entry):
    """Verify rows over the E4M3 cache (per token, or 4 rows per pass), a
    skipped prompt."""
    print(f"case verify rows e4m3 {entry}", flush=True)
    c = verify_case([(300, 4), (0, 9), (40, 4), (90, 1), (2000, 3)], 4, 12)
    rng = np.random.default_rng(12)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    outs = np.zeros(5, np.int32)
    outs[1] = -1
    init = np.full((c["T"], 16, D), 0x5555, np.uint16)
    got = run_decode8(c, k8, v8, ks, vs, dev, skip=1, outs=outs, out_init=init, entry=entry)
    assert (got[4:13] == 0x5555).all()
    want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], 16, 4, c["pos"], c["tok_seq"], c["bt"],
                               c["max_blocks"], BS, SCALE, cu=c["cu"], skip_prompts=1, outs=outs, out=init.copy())
    ok, err = close(got, want)
    assert ok, err


def test_decode_e4m3_equals_bf16_decode_on_grid_values(dev):
    """Config-3-like batch (64 sequences, 512..8192 keys): with unit scales
    the E4M3 cache holds exactly the bf16 cache's values, so E4M3 decode
    and bf16 decode agree (within the tolerance: different kernels)."""
    print("case decode e4m3 vs bf16 c3", flush=True)
    from pkv import synth
    lens = synth.c3_lengths(4, batch=64)
    meta = synth.decode_meta(lens - 1, 64 * 520, steps=1, seed=4)
    st = meta.step(0)
    Hq, Hkv = 16, 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    n = meta.num_pages * BS * Hkv * D
    k8 = torch.randint(0, 0x60, (n,), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
    v8 = torch.randint(0, 0x60, (n,), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
    k8 |= (torch.randint(0, 2, (n,), device=dev, generator=gen, dtype=torch.int32) << 7).to(torch.uint8)
    v8 |= (torch.randint(0, 2, (n,), device=dev, generator=gen, dtype=torch.int32) << 7).to(torch.uint8)
    kbf = k8.view(torch.float8_e4m3fn).to(torch.bfloat16).view(-1, Hkv, D)
    vbf = v8.view(torch.float8_e4m3fn).to(torch.bfloat16).view(-1, Hkv, D)
    ones = torch.ones(meta.num_pages * BS * Hkv, device=dev)
    B = len(lens)
    q = (torch.randn(B, Hq, D, device=dev, generator=gen) * 0.05).to(torch.bfloat16)
    qstride = synth.qkv_stride(Hq, Hkv)
    qkv = torch.randn(B, qstride, device=dev, generator=gen).to(torch.bfloat16)
    pos, ts, cu = (torch.from_numpy(st[k]).to(dev) for k in ("pos", "tok_seq", "cu"))
    bt = torch.from_numpy(meta.block_table).to(dev)
    o8 = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
    ob = torch.zeros_like(o8)
    ws = torch.empty(max(pkv.attn_verify_workspace(B, Hq), pkv.attn_decode_workspace(B, Hq)), dtype=torch.uint8,
                     device=dev)
    pkv.attn_decode(q, kbf, vbf, qkv, qstride, Hq, Hkv, pos, ts, bt, meta.max_blocks, BS, ob, SCALE, cu, 0, None, 1, B,
                    meta.num_pages, ws)
    bits = lambda x: x.cpu().view(torch.int16).numpy().view(np.uint16)
    for fn in (pkv.attn_decode_e4m3, pkv.attn_verify_e4m3):
        o8.zero_()
        fn(q, k8, v8, ones, ones, qkv, qstride, Hq, Hkv, pos, ts, bt, meta.max_blocks, BS, o8, SCALE, cu, 0, None, 1, B,
           meta.num_pages, ws)
        torch.cuda.synchronize()
        ok, err = close(bits(o8), bits(ob))
        assert ok, (fn.__name__, err)


@pytest.mark.parametrize("refabi_kernel", [False, True])
@pytest.mark.parametrize("ctxs,chunks,Hkv,seed", [
    ([0], [37], 4, 0),
    ([100, 16], [64, 130], 4, 1),
    ([1000, 33, 0], [70, 200, 65], 2, 3),
])
def test_prefill_e4m3_matches_oracle(dev, refabi_kernel, ctxs, chunks, Hkv, seed):
    """Chunked prefill over an E4M3 cache, through pkv_attn_prefill_e4m3 or
    the code object's attn_group8_g4_t2_k16 launched as the engine does."""
    print(f"case prefill e4m3 refabi={refabi_kernel} ctx={ctxs} chunk={chunks}", flush=True)
    from test_gpu_prefill import prefill_case
    from pkv.refabi import F, I, P, RefKernels, flash_launch
    c = prefill_case(ctxs, chunks, Hkv, seed, decode_rows=1)
    rng = np.random.default_rng(seed + 70)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    T, Hq = c["T"], c["Hq"]
    init = np.full((T, Hq, D), 0x3333, np.uint16)
    out = t_(init, dev)
    args = [t_(c["q"], dev), t_(k8, dev), t_(v8, dev), t_(ks, dev), t_(vs, dev), t_(c["qkv"], dev)]
    pos, cu, bt = t_(c["pos"], dev), t_(c["cu"], dev), t_(c["bt"], dev)
    if refabi_kernel:
        name, grid, threads, smem = flash_launch(T, c["seqs"], Hkv, fp8=True)
        RefKernels().launch(name, grid, threads, smem,
                            [P(args[0]), P(args[1]), P(args[2]), P(args[3]), P(args[4]), P(args[5]), I(c["qstride"]),
                             I(Hq), I(Hkv), P(pos), P(cu), I(c["seqs"]), P(bt), I(c["max_blocks"]), I(BS), P(out),
                             F(SCALE), P(None), I(1)])
    else:
        pkv.attn_prefill_e4m3(*args, c["qstride"], Hq, Hkv, pos, cu, c["seqs"], bt, c["max_blocks"], BS, out, SCALE,
                              None, 1, T, c["pages"])
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    assert (got[0] == 0x3333).all()  # the decode row is left to decode attention
    want = oracle.attn_prefill8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["cu"], c["seqs"],
                                c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("lens,Z", [([1, 2, 15, 16, 17], None), ([4097], None), ([513, 8193, 1000, 64], None),
                                    ([900, 70], 1), ([40, 3, 100] * 100, None)])
def test_reference_named_paged8(dev, lens, Z):
    """attn_paged8_g4 (+ attn_merge when split) of the code object, launched
    as model.rs:2366-2437 does for an E4M3 cache, against the oracle."""
    print(f"case refabi paged8 lens={lens} Z={Z}", flush=True)
    from pkv.refabi import F, I, P, RefKernels, SPLIT_MIN_KEYS, split_ranges
    rk = RefKernels()
    c = decode_case(lens, 16, 4, 21)
    rng = np.random.default_rng(21)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    T, Hq, Hkv = len(c["pos"]), 16, 4
    sms = torch.cuda.get_device_properties(0).multi_processor_count
    ranges = split_ranges(T, Hkv, sms) if Z is None else Z
    part = torch.full((T * ranges * Hq * (D + 2),), float("nan"), device=dev) if ranges > 1 else None
    q, qkv = t_(c["q"], dev), t_(c["qkv"], dev)
    pos, ts, bt, cu = (t_(c[k].astype(np.int32), dev) for k in ("pos", "tok_seq", "bt", "cu"))
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    rk.launch("attn_paged8_g4", (T, Hkv, ranges), 256, 0,
              [P(q), P(t_(k8, dev)), P(t_(v8, dev)), P(t_(ks, dev)), P(t_(vs, dev)), P(qkv), I(c["qstride"]), I(Hq),
               I(Hkv), P(pos), P(ts), P(bt), I(c["max_blocks"]), I(BS), P(out), F(SCALE), P(None), P(None), I(0), I(0),
               P(cu), I(0), I(SPLIT_MIN_KEYS), P(part), P(None), I(1)])
    if part is not None:
        rk.launch("attn_merge", (T, Hq, 1), 256, 0,
                  [P(part), I(ranges), I(SPLIT_MIN_KEYS), P(qkv), I(c["qstride"]), I(Hq), P(pos), P(ts), P(cu), I(0),
                   P(out), P(None), P(None), I(0), I(0), P(None), I(1)])
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"],
                               c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def nan_stale8(c, lens, k8, v8, ks, vs):
    """E4M3 bytes 0x7F (NaN) and NaN scales in every slot holding no key."""
    from _util import used_slots
    used = used_slots(c, lens)
    k8, v8, ks, vs = k8.copy(), v8.copy(), ks.copy(), vs.copy()
    k8[~used] = 0x7F
    v8[~used] = 0x7F
    ks[~used] = np.nan
    vs[~used] = np.nan
    return k8, v8, ks, vs


@pytest.mark.parametrize("kind", ["decode", "decode_split", "verify", "verify_rows_per_token"])
def test_e4m3_stale_slots_are_nan(dev, kind):
    """Decode / verify over an E4M3 cache whose slots holding no key are NaN
    bytes with NaN scales: no NaN reaches the outputs."""
    print(f"case e4m3 NaN stale slots {kind}", flush=True)
    pkv.attn_decode_config(1, 16 if kind == "decode_split" else 32)
    try:
        if kind.startswith("verify"):
            groups = [(12, 4), (301, 3), (0, 2)]
            c = verify_case(groups, 4, 14)
            lens = [L0 + n for L0, n in groups]
        else:
            lens = [1, 2, 15, 17, 33, 4097]
            c = decode_case(lens, 16, 4, 14)
        rng = np.random.default_rng(14)
        k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
        ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
        vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
        k8, v8, ks, vs = nan_stale8(c, lens, k8, v8, ks, vs)
        got = run_decode8(c, k8, v8, ks, vs, dev, entry="verify" if kind == "verify" else "decode")
        want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], 4, c["pos"],
                                   c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
        ok, err = close(got, want)
        assert ok, f"max |diff| {err}"
    finally:
        pkv.attn_decode_config(1, 32)


@pytest.mark.parametrize("refabi_kernel", [False, True])
def test_prefill_e4m3_stale_slots_are_nan(dev, refabi_kernel):
    """Chunked prefill over an E4M3 cache with NaN bytes and scales in every
    slot holding no key."""
    print(f"case prefill e4m3 NaN stale slots refabi={refabi_kernel}", flush=True)
    from test_gpu_prefill import prefill_case
    from pkv.refabi import F, I, P, RefKernels, flash_launch
    c = prefill_case([100, 5], [45, 130], 4, 15)
    rng = np.random.default_rng(15)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    lens = [int(c["pos"][c["cu"][s + 1] - 1]) + 1 for s in range(c["seqs"])]
    k8, v8, ks, vs = nan_stale8(c, lens, k8, v8, ks, vs)
    T, Hq, Hkv = c["T"], c["Hq"], 4
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    args = [t_(c["q"], dev), t_(k8, dev), t_(v8, dev), t_(ks, dev), t_(vs, dev), t_(c["qkv"], dev)]
    pos, cu, bt = t_(c["pos"], dev), t_(c["cu"], dev), t_(c["bt"], dev)
    if refabi_kernel:
        name, grid, threads, smem = flash_launch(T, c["seqs"], Hkv, fp8=True)
        RefKernels().launch(name, grid, threads, smem,
                            [P(args[0]), P(args[1]), P(args[2]), P(args[3]), P(args[4]), P(args[5]), I(c["qstride"]),
                             I(Hq), I(Hkv), P(pos), P(cu), I(c["seqs"]), P(bt), I(c["max_blocks"]), I(BS), P(out),
                             F(SCALE), P(None), I(1)])
    else:
        pkv.attn_prefill_e4m3(*args, c["qstride"], Hq, Hkv, pos, cu, c["seqs"], bt, c["max_blocks"], BS, out, SCALE,
                              None, 1, T, c["pages"])
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = oracle.attn_prefill8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["cu"], c["seqs"],
                                c["bt"], c["max_blocks"], BS, SCALE)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("Hkv,min_range", [(1, 16), (2, 16), (8, 32), (4, 1 << 20)])
def test_verify_e4m3_four_row_segments(dev, Hkv, min_range):
    """pkv_attn_verify_e4m3 with full 4-row segments (the NR = 4 columns of
    the E4M3 wave body) at Hkv 1 and 2 (fewer waves per block) and 8 (two
    kv-head groups), contexts long enough to cross several key ranges (small
    min_range), plus ragged 1..3-row tails; every row against the oracle."""
    print(f"case verify e4m3 4-row segments Hkv={Hkv} min_range={min_range}", flush=True)
    pkv.attn_decode_config(1, min_range)
    try:
        c = verify_case([(700, 4), (1500, 4), (33, 3), (2100, 8), (5, 1), (400, 6)], Hkv, 30 + Hkv)
        rng = np.random.default_rng(31 + Hkv)
        k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
        ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
        vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
        outs = np.zeros(6, np.int32)
        got = run_decode8(c, k8, v8, ks, vs, dev, skip=1, outs=outs, entry="verify")
        want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], 4 * Hkv, Hkv, c["pos"],
                                   c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"], skip_prompts=1,
                                   outs=outs)
        ok, err = close(got, want, what=f"verify e4m3 Hkv {Hkv}")
        assert ok, err
    finally:
        pkv.attn_decode_config(1, 32)


def test_ref_group8_short_dynamic_lds_writes_nothing(dev):
    """attn_group8_g4_t2_k16 keeps its three stages in the launch's dynamic
    shared memory: a launch with less than they take (96 KiB instead of the
    engine's 101,376 bytes; the stages need 100,608) returns before any work
    and leaves the output untouched."""
    print("case refabi group8 short dynamic LDS", flush=True)
    from test_gpu_prefill import prefill_case
    from pkv.refabi import F, I, P, RefKernels, flash_launch
    c = prefill_case([100], [64], 4, 5, decode_rows=1)
    rng = np.random.default_rng(5)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    T, Hq = c["T"], c["Hq"]
    name, grid, threads, smem = flash_launch(T, c["seqs"], 4, fp8=True)
    assert name == "attn_group8_g4_t2_k16" and smem >= 100608
    init = np.full((T, Hq, D), 0x3333, np.uint16)
    out = t_(init, dev)
    RefKernels().launch(name, grid, threads, 96 * 1024,
                        [P(t_(c["q"], dev)), P(t_(k8, dev)), P(t_(v8, dev)), P(t_(ks, dev)), P(t_(ks, dev)),
                         P(t_(c["qkv"], dev)), I(c["qstride"]), I(Hq), I(4), P(t_(c["pos"], dev)),
                         P(t_(c["cu"], dev)), I(c["seqs"]), P(t_(c["bt"], dev)), I(c["max_blocks"]), I(BS), P(out),
                         F(SCALE), P(None), I(1)])
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint16) == 0x3333).all()

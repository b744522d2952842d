"""GPU parity of the reference-ABI code object (pkv_kernels.hsaco): its
kernels, loaded by name with hipModuleLoadData and launched with the
reference engine's grids, blocks, shared memory and 8-byte argument slots
(src/model.rs:2366-2493, src/gpu.rs:903-930), against the oracle.

Tolerance (north star): bf16 outputs within max-abs 2e-3 and relative 1e-2,
|got - want| <= 2e-3 + 1e-2 * |want|. The split records are also merged on
the host with the reference's own attn_merge formula (natural-log maxima,
qwen35.cu:2255-2273), pinning the record format a mixed deployment would
exchange."""
import numpy as np
import pytest
import torch

import oracle
from _util import BS, D, bf16_bits, close, decode_case
from pkv.refabi import F, I, P, RefKernels, SPLIT_MIN_KEYS, flash_launch, split_ranges
from test_gpu_prefill import prefill_case
from test_gpu_verify import verify_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0


@pytest.fixture(scope="module")
def rk():
    return RefKernels()


def i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def ref_decode(rk, c, dev, Z=None, spec=1, skip=0, outs=None, out_init=None, keep_part=False, f8=None, fp8out=None):
    """attn_paged_g<G> (+ attn_merge when split) as model.rs:2366-2437 launches
    them: the kernel of the model's G = Hq / Hkv, 128 threads for G >= 6, else
    256. f8 = (k8, v8, kscale, vscale) launches attn_paged8_g<G> over an E4M3
    cache."""
    T, Hq, Hkv = len(c["pos"]), c["Hq"], c["Hkv"]
    G = Hq // Hkv
    sms = torch.cuda.get_device_properties(0).multi_processor_count
    ranges = split_ranges(T, Hkv, sms) if Z is None else Z
    seqs = len(c["cu"]) - 1
    part = (torch.full((seqs * spec * ranges * Hq * (D + 2),), float("nan"), device=dev) if ranges > 1 else None)
    q, qkv = i16(c["q"], dev), i16(c["qkv"], dev)
    if f8 is None:
        kc, vc, ks, vs = i16(c["kc"], dev), i16(c["vc"], dev), None, None
    else:
        kc, vc, ks, vs = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in f8)
    pos, ts, bt, cu = i32(c["pos"], dev), i32(c["tok_seq"], dev), i32(c["bt"], dev), i32(c["cu"], dev)
    outs_d = None if outs is None else i32(outs, dev)
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev) if out_init is None else i16(out_init, dev)
    # fp8out = (mode, frows): the FP8 activation copy buffers (fq [T][Hq 256]
    # bytes; fs: mode 1 f32 [Hq 256 / 128][frows], mode 2 the Mx32 tiles)
    fmode, frows = (0, 0) if fp8out is None else fp8out
    fq = fs = None
    if fmode:
        K = Hq * D
        fq = torch.full((T, K), 0x7F, dtype=torch.uint8, device=dev)
        fs = (torch.full((K // 128, frows), float("nan"), device=dev) if fmode == 1 else
              torch.full((((frows + 127) // 128) * ((K // 32 + 3) // 4) * 512,), 0xEE, dtype=torch.uint8, device=dev))
    rk.launch(f"attn_paged{'8' if f8 is not None else ''}_g{G}", (T, Hkv, ranges), 128 if G >= 6 else 256, 0,
              [P(q), P(kc), P(vc), P(ks), P(vs), P(qkv), I(c["qstride"]), I(Hq), I(Hkv), P(pos), P(ts), P(bt),
               I(c["max_blocks"]), I(BS), P(out), F(SCALE), P(fq), P(fs), I(fmode), I(frows), P(cu), I(skip),
               I(SPLIT_MIN_KEYS), P(part), P(outs_d), I(spec)])
    if part is not None:
        rk.launch("attn_merge", (T, Hq, 1), 256, 0,
                  [P(part), I(ranges), I(SPLIT_MIN_KEYS), P(qkv), I(c["qstride"]), I(Hq), P(pos), P(ts), P(cu),
                   I(skip), P(out), P(fq), P(fs), I(fmode), I(frows), P(outs_d), I(spec)])
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    if fmode:
        return got, fq.cpu().numpy(), fs.cpu().numpy()
    if keep_part:
        return got, (None if part is None else part.cpu().numpy()), ranges
    return got


def oracle_decode(c, **kw):
    out, _ = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"],
                                c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"], **kw)
    return out


@pytest.mark.parametrize("lens,Hkv,seed,Z", [
    ([1, 2, 15, 16, 17], 4, 0, None),          # page edges; 52 ranges offered, 1 used
    ([4097], 4, 1, None),                      # config 2: 64 ranges of 65 keys
    ([513, 8193, 1000, 4000, 777, 64], 4, 2, None),
    ([300, 5000], 2, 3, None),                 # Hkv 2
    ([900, 70, 4000], 4, 4, 1),                # no split: part = 0, gated output in place
    ([200] * 300, 4, 5, None),                 # 300 tokens: split_ranges gives 1
])
def test_ref_decode_matches_oracle(dev, rk, lens, Hkv, seed, Z):
    print(f"case refabi decode lens={lens[:6]} Hkv={Hkv} Z={Z}", flush=True)
    c = decode_case(lens, 4 * Hkv, Hkv, seed)
    ok, err = close(ref_decode(rk, c, dev, Z=Z), oracle_decode(c))
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G,Hkv", [(1, 4), (2, 2), (6, 4), (6, 1), (8, 2), (8, 8)])
@pytest.mark.parametrize("lens,seed,Z", [
    ([1, 2, 15, 16, 17, 33], 0, None),
    ([513, 4097, 1000, 64], 1, None),
    ([900, 70, 4000], 2, 1),
    ([40, 3, 100] * 100, 3, None),             # 300 tokens: more than a block's threads to order
])
def test_ref_decode_groups_match_oracle(dev, rk, G, Hkv, lens, seed, Z):
    """attn_paged_g1/g2/g6/g8: the reference loads attn_paged_g<Hq / Hkv>
    (model.rs:1053-1054)."""
    print(f"case refabi decode G={G} Hkv={Hkv} lens={lens[:6]} Z={Z}", flush=True)
    c = decode_case(lens, G * Hkv, Hkv, seed)
    want, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"],
                                   c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    ok, err = close(ref_decode(rk, c, dev, Z=Z), want,
                    explain=dict(raw=raw, qkv=c["qkv"], qstride=c["qstride"], Hq=c["Hq"]))
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G,Hkv", [(1, 4), (2, 2), (4, 4), (6, 4), (8, 2)])
def test_ref_paged8_groups_match_oracle(dev, rk, G, Hkv):
    print(f"case refabi paged8 G={G} Hkv={Hkv}", flush=True)
    from test_gpu_e4m3 import e4m3_cache
    c = decode_case([1, 17, 513, 4097, 64, 900], G * Hkv, Hkv, 30 + G)
    rng = np.random.default_rng(31 + G)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    got = ref_decode(rk, c, dev, f8=(k8, v8, ks, vs))
    want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"], c["tok_seq"],
                               c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_ref_paged_wrong_block_writes_nothing(dev, rk):
    """attn_paged_g6 launched with 64 threads (not the engine's 128) returns
    before any work. (A block above the kernel's 128-thread bound is refused
    by the runtime at launch.)"""
    print("case refabi paged g6 wrong block", flush=True)
    c = decode_case([100, 40], 24, 4, 9)
    init = np.full((2, 24, D), 0x3333, np.uint16)
    out = i16(init, dev)
    rk.launch("attn_paged_g6", (2, 4, 1), 64, 0,
              [P(i16(c["q"], dev)), P(i16(c["kc"], dev)), P(i16(c["vc"], dev)), P(None), P(None),
               P(i16(c["qkv"], dev)), I(c["qstride"]), I(24), I(4), P(i32(c["pos"], dev)), P(i32(c["tok_seq"], dev)),
               P(i32(c["bt"], dev)), I(c["max_blocks"]), I(BS), P(out), F(SCALE), P(None), P(None), I(0), I(0),
               P(i32(c["cu"], dev)), I(0), I(SPLIT_MIN_KEYS), P(None), P(None), I(1)])
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint16) == 0x3333).all()


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("G,Hkv,Z", [(4, 4, 1), (4, 4, None), (6, 4, 1), (6, 4, None), (8, 2, 1)])
def test_ref_fp8_output_copies(dev, rk, mode, G, Hkv, Z):
    """fq / fs / fmode / frows (the reference's Fp8Out, fp8.cuh:50-85): the
    gated f32 outputs as E4M3 bytes with Block128 f32 scales (mode 1) or
    Mx32 E8M0 exponents in the 128 x 4 tiles (mode 2), written by
    attn_paged_g<G> unsplit (Z = 1) or by attn_merge after a split. Against
    the oracle's quantisation of its own gated outputs: every element
    dequantises to within one E4M3 step of the oracle's f32 output (the two
    f32 outputs differ by the attention tolerance), bytes and scales agree
    almost everywhere, and nothing outside the rows' bytes and scales is
    written."""
    print(f"case refabi fp8 copies mode={mode} G={G} Hkv={Hkv} Z={Z}", flush=True)
    lens = [1, 17, 700, 4097, 130, 2000]
    c = decode_case(lens, G * Hkv, Hkv, 50 + mode + G)
    T, Hq, K = len(lens), G * Hkv, G * Hkv * D
    frows = 200  # the engine's row capacity, above T
    got, fq, fs = ref_decode(rk, c, dev, Z=Z, fp8out=(mode, frows))
    want_bits, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"],
                                        c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    ok, err = close(got, want_bits)
    assert ok, err
    y = oracle.gate_rows(raw, c["qkv"], c["qstride"], Hq).reshape(T, K)
    wq, ws = oracle.fp8_rows(y, mode, rows=frows)
    gw = 128 if mode == 1 else 32
    # per-element scales of the kernel's and the oracle's copies
    if mode == 1:
        sg, sw = fs[:, :T].T, ws[:, :T].T                            # [T][K / 128]
        assert np.isnan(fs[:, T:]).all()                             # rows past T untouched
    else:
        idx = np.array([[oracle.mx_index(t, kb, K // 32) for kb in range(K // 32)] for t in range(T)])
        sg, sw = 2.0 ** (fs[idx].astype(np.float64) - 127), 2.0 ** (ws[idx].astype(np.float64) - 127)
        mask = np.ones(fs.shape, bool)
        mask[idx.reshape(-1)] = False
        assert (fs[mask] == 0xEE).all()                              # other tile bytes untouched
    deq = oracle.e4m3_to_f(fq).astype(np.float64) * np.repeat(sg, gw, axis=1)
    step = np.repeat(sw, gw, axis=1) * 2.0 ** -9 + np.abs(y) * 2.0 ** -4
    bf_ulp = np.abs(y) * 2.0 ** -8
    assert (np.abs(deq - y) <= step + bf_ulp + 2e-3 + 1e-2 * np.abs(y)).all()
    assert (fq == wq).mean() > 0.99, (fq == wq).mean()
    # scales: f32 amax / 448 (mode 1) follows the f32 outputs' last bits (the
    # kernel's exp against the oracle's expf), so within 1e-5 for most
    # groups; E8M0 exponents (mode 2) agree almost everywhere
    rel = np.abs(sg / sw - 1)
    assert (rel <= 1e-2).all()
    assert ((rel <= 1e-5).mean() > 0.95) if mode == 1 else ((sg == sw).mean() > 0.99), (rel <= 1e-5).mean()


def test_ref_spec_rows_and_prompt_skip(dev, rk):
    """Speculative rows (spec = 4 rows per sequence, partial rows indexed
    s * spec + row) verified; a prompt sequence's rows skipped."""
    print("case refabi spec rows", flush=True)
    c = verify_case([(300, 4), (0, 9), (40, 4), (90, 1), (2000, 3)], 4, 6)
    outs = np.zeros(5 * 4, np.int32)  # outs[s * spec] >= 0: sequence s verifies drafts
    outs[1 * 4] = -1                   # sequence 1 (9 rows) is a prompt: skipped before any write
    init = np.full((c["T"], 16, D), 0x5555, np.uint16)
    got = ref_decode(rk, c, dev, spec=4, skip=1, outs=outs, out_init=init)
    assert (got[4:13] == 0x5555).all()
    want = oracle_decode(c, skip_prompts=1, outs=outs, spec=4, out=init.copy())
    ok, err = close(got, want)
    assert ok, err


def test_ref_records_merge_with_reference_formula(dev, rk):
    """The split records are the reference's: [M (natural log), S, A[256]] at
    ((s * spec + t - cu[s]) * Hq + h) * Z + z. Merged on the host with
    attn_merge's formula they give the kernel's output."""
    print("case refabi records", flush=True)
    c = decode_case([4097, 1500, 130], 16, 4, 7)
    got, part, Z = ref_decode(rk, c, dev, keep_part=True)
    assert Z > 1
    T, Hq = 3, 16
    rec = part.reshape(T, Hq, Z, D + 2).astype(np.float64)
    for t, L in enumerate(c["pos"] + 1):
        nz = max(1, min(Z, -(-int(L) // SPLIT_MIN_KEYS)))
        r = rec[t, :, :nz]
        assert np.isfinite(r).all()
        M = r[:, :, 0].max(axis=1, keepdims=True)
        f = np.exp(r[:, :, 0] - M)
        S = (r[:, :, 1] * f).sum(axis=1)
        A = (r[:, :, 2:] * f[:, :, None]).sum(axis=1) / S[:, None]
        o = oracle.b2f(oracle.f2b(A.astype(np.float32)))
        gate = oracle.b2f(c["qkv"][t][:Hq * 2 * D].reshape(Hq, 2, D)[:, 1]).astype(np.float64)
        want = oracle.f2b((o / (1 + np.exp(-gate))).astype(np.float32))
        ok, err = close(got[t], want)
        assert ok, f"token {t}: {err}"


@pytest.mark.parametrize("mfma", [False, True])
@pytest.mark.parametrize("ctxs,chunks,Hkv,seed", [
    ([0], [37], 4, 0),
    ([100], [64], 4, 1),
    ([16, 5], [130, 2], 1, 2),
    ([1000, 33, 0], [70, 200, 65], 2, 3),
])
def test_ref_prefill_matches_oracle(dev, rk, mfma, ctxs, chunks, Hkv, seed):
    print(f"case refabi prefill mfma={mfma} ctx={ctxs} chunk={chunks} Hkv={Hkv}", flush=True)
    c = prefill_case(ctxs, chunks, Hkv, seed, decode_rows=1)
    T, Hq = c["T"], c["Hq"]
    name, grid, threads, smem = flash_launch(T, c["seqs"], Hkv, mfma=mfma)
    init = np.full((T, Hq, D), 0x3333, np.uint16)
    out = i16(init, dev)
    rk.launch(name, grid, threads, smem,
              [P(i16(c["q"], dev)), P(i16(c["kc"], dev)), P(i16(c["vc"], dev)), P(None), P(None),
               P(i16(c["qkv"], dev)), I(c["qstride"]), I(Hq), I(Hkv), P(i32(c["pos"], dev)), P(i32(c["cu"], dev)),
               I(c["seqs"]), P(i32(c["bt"], dev)), I(c["max_blocks"]), I(BS), P(out), F(SCALE), P(None), I(1)])
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    assert (got[0] == 0x3333).all()  # the decode row is left to decode attention
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_ref_prefill_short_dynamic_lds_writes_nothing(dev, rk):
    """attn_groupr_g4_t2_k32 keeps its stages in the launch's dynamic shared
    memory: a launch that passes less than they take (here 32 KiB instead of
    the engine's 67,584 bytes) returns before any work, like a launch with
    another block size, and leaves the output untouched."""
    print("case refabi prefill short dynamic LDS", flush=True)
    c = prefill_case([100], [64], 4, 5, decode_rows=1)
    T, Hq = c["T"], c["Hq"]
    name, grid, threads, smem = flash_launch(T, c["seqs"], 4)
    assert name == "attn_groupr_g4_t2_k32" and smem >= 67328
    init = np.full((T, Hq, D), 0x3333, np.uint16)
    out = i16(init, dev)
    rk.launch(name, grid, threads, 32 * 1024,
              [P(i16(c["q"], dev)), P(i16(c["kc"], dev)), P(i16(c["vc"], dev)), P(None), P(None),
               P(i16(c["qkv"], dev)), I(c["qstride"]), I(Hq), I(4), P(i32(c["pos"], dev)), P(i32(c["cu"], dev)),
               I(c["seqs"]), P(i32(c["bt"], dev)), I(c["max_blocks"]), I(BS), P(out), F(SCALE), P(None), I(1)])
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint16) == 0x3333).all()

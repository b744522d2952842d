"""GPU parity for the query-head groups other than 4 (G = Hq / Hkv in 1, 2,
6, 8: the reference instantiates attn_paged_g<G> / attn_paged8_g<G> for
these, src/kernels/qwen35.cu:1326-1334, and loads the one of the model's
ratio, src/model.rs:1054). bf16 and E4M3 caches, per-token decode and
grouped verify rows, against the oracle, which takes any G.

Tolerance (north star): bf16 outputs within max-abs 2e-3 and relative 1e-2,
|got - want| <= 2e-3 + 1e-2 * |want|."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, close, decode_case, nan_stale
from test_gpu_decode import dev_i16, dev_i32, run_gpu, run_oracle
from test_gpu_e4m3 import e4m3_cache, run_decode8
from test_gpu_verify import run_oracle as run_oracle_v, run_verify, verify_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0

# (G, Hkv): the reference's 27B shape is 24 query heads over 4 kv heads.
GROUPS = [(1, 4), (2, 2), (6, 4), (6, 1), (8, 2), (8, 8)]


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)


@pytest.mark.parametrize("G,Hkv", GROUPS)
@pytest.mark.parametrize("lens,seed,min_range", [
    ([1, 2, 15, 16, 17, 33], 0, 32),        # page edges, one key
    ([513, 4097, 1000, 64], 1, 32),         # split over ranges
    ([700, 2000], 2, 1 << 20),              # whole tokens per range
])
def test_decode_groups_match_oracle(dev, G, Hkv, lens, seed, min_range):
    print(f"case decode G={G} Hkv={Hkv} lens={lens} min_range={min_range}", flush=True)
    pkv.attn_decode_config(1, min_range)
    c = decode_case(lens, G * Hkv, Hkv, seed)
    ok, err = close(run_gpu(c, dev), run_oracle(c, cu=c["cu"]))
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G,Hkv", GROUPS)
def test_verify_groups_match_oracle(dev, G, Hkv):
    """Rows of a sequence share a pass: 4 rows per segment for G <= 4, 2
    for G = 6 and 8; ragged row counts, one skipped prompt."""
    print(f"case verify G={G} Hkv={Hkv}", flush=True)
    c = verify_case([(300, 4), (0, 9), (40, 3), (90, 1), (2000, 5), (12, 2)], Hkv, 20 + G, G=G)
    outs = np.array([0, -1, 0, 0, 0, 0], np.int32)
    init = np.full((c["T"], c["Hq"], D), 0x5555, np.uint16)
    got = run_verify(c, dev, skip=1, outs=outs, out_init=init)
    assert (got[4:13] == 0x5555).all()
    want = run_oracle_v(c, skip_prompts=1, outs=outs, spec=1, out=init.copy())
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G,Hkv", [(6, 4), (8, 2)])
def test_groups_stale_slots_are_nan(dev, G, Hkv):
    print(f"case decode G={G} NaN stale slots", flush=True)
    lens = [1, 17, 130, 2049]
    c = nan_stale(decode_case(lens, G * Hkv, Hkv, 40 + G), lens)
    ok, err = close(run_gpu(c, dev), run_oracle(c, cu=c["cu"]))
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("entry", ["decode", "verify"])
@pytest.mark.parametrize("G,Hkv", GROUPS)
def test_e4m3_groups_match_oracle(dev, entry, G, Hkv):
    print(f"case {entry} e4m3 G={G} Hkv={Hkv}", flush=True)
    if entry == "verify":
        c = verify_case([(300, 4), (40, 3), (90, 1), (2000, 5), (12, 2)], Hkv, 60 + G, G=G)
    else:
        c = decode_case([1, 16, 17, 513, 4097, 64], G * Hkv, Hkv, 60 + G)
    rng = np.random.default_rng(70 + G)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    got = run_decode8(c, k8, v8, ks, vs, dev, entry=entry)
    want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"], c["tok_seq"],
                               c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_fused_step_rejects_unsupported_groups(dev):
    """The fused append + decode step serves G in {1, 2, 4, 6, 8}; another
    group (G = 5) gets PKV_ERR_UNSUPPORTED before any launch."""
    c = decode_case([40, 50], 20, 4, 3)
    T = 2
    q = torch.zeros(T, 20, D, dtype=torch.int16, device=dev)
    kc = torch.zeros(c["pages"] * BS, 4, D, dtype=torch.int16, device=dev)
    rows = torch.zeros(T, 4 * D, dtype=torch.int16, device=dev)
    qkv = torch.zeros(T, c["qstride"], dtype=torch.int16, device=dev)
    i = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, 20), dtype=torch.uint8, device=dev)
    with pytest.raises(pkv.PkvError, match="unsupported"):
        pkv.attn_decode_step(rows, rows, 4 * D * 2, i([0, 16]), q, kc, kc, qkv, c["qstride"], 20, 4, i(c["pos"]),
                             i(c["tok_seq"]), i(c["bt"]), c["max_blocks"], BS, q, SCALE, i(c["cu"]), 0, None, 1, T,
                             c["pages"], ws)


PREFILL_CASES = [
    ([0], [37], 0),                     # no prefix, partial query tile
    ([100, 16], [64, 130], 1),          # tiles crossing a tile edge after a prefix
    ([1000, 33, 0], [70, 200, 65], 2),  # three prompts, a decode row first
]


def _prefill(c, dev, entry, f8=None):
    """entry: "lib" (pkv_attn_prefill[_e4m3]) or "ref" (the code object's
    kernel for this group, launched as the engine's fa_shape picks it)."""
    from pkv.refabi import F, I, P, RefKernels, flash_launch
    T, Hq, Hkv = c["T"], c["Hq"], c["Hkv"]
    init = np.full((T, Hq, D), 0x3333, np.uint16)
    out = torch.from_numpy(init.view(np.int16).copy()).to(dev)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16
                                   else np.ascontiguousarray(a)).to(dev)
    kc, vc = (t(c["kc"]), t(c["vc"])) if f8 is None else (t(f8[0]), t(f8[1]))
    ks, vs = (None, None) if f8 is None else (t(f8[2]), t(f8[3]))
    q, qkv, pos, cu, bt = t(c["q"]), t(c["qkv"]), t(c["pos"]), t(c["cu"]), t(c["bt"])
    if entry == "ref":
        name, grid, threads, smem = flash_launch(T, c["seqs"], Hkv, g=Hq // Hkv, fp8=f8 is not None)
        print(f"  kernel {name} grid {grid} threads {threads} smem {smem}", flush=True)
        RefKernels().launch(name, grid, threads, smem,
                            [P(q), P(kc), P(vc), P(ks), P(vs), P(qkv), I(c["qstride"]), I(Hq), I(Hkv), P(pos), P(cu),
                             I(c["seqs"]), P(bt), I(c["max_blocks"]), I(BS), P(out), F(SCALE), P(None), I(1)])
    elif f8 is None:
        pkv.attn_prefill(q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, cu, c["seqs"], bt, c["max_blocks"], BS, out,
                         SCALE, None, 1, T, c["pages"])
    else:
        pkv.attn_prefill_e4m3(q, kc, vc, ks, vs, qkv, c["qstride"], Hq, Hkv, pos, cu, c["seqs"], bt, c["max_blocks"],
                              BS, out, SCALE, None, 1, T, c["pages"])
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16), init


@pytest.mark.parametrize("entry", ["lib", "ref"])
@pytest.mark.parametrize("G,Hkv", [(1, 4), (2, 2), (6, 4), (6, 1), (8, 2)])
@pytest.mark.parametrize("ctxs,chunks,seed", PREFILL_CASES)
def test_prefill_groups_match_oracle(dev, entry, G, Hkv, ctxs, chunks, seed):
    """Prompt attention for G = 1, 2, 6, 8: the library's kernels and the
    code object's attn_groupr_g6_t1_k32 / attn_group_g{1,2,8}_t*_k16."""
    print(f"case prefill {entry} G={G} Hkv={Hkv} ctx={ctxs} chunk={chunks}", flush=True)
    from test_gpu_prefill import prefill_case
    c = prefill_case(ctxs, chunks, Hkv, seed, decode_rows=1, G=G)
    got, init = _prefill(c, dev, entry)
    assert (got[0] == 0x3333).all()  # the decode row is left to decode attention
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("entry", ["lib", "ref"])
@pytest.mark.parametrize("G,Hkv", [(1, 4), (2, 2), (6, 4), (8, 2)])
@pytest.mark.parametrize("ctxs,chunks,seed", PREFILL_CASES[1:])
def test_prefill_e4m3_groups_match_oracle(dev, entry, G, Hkv, ctxs, chunks, seed):
    print(f"case prefill e4m3 {entry} G={G} Hkv={Hkv} ctx={ctxs} chunk={chunks}", flush=True)
    from test_gpu_prefill import prefill_case
    c = prefill_case(ctxs, chunks, Hkv, seed, decode_rows=1, G=G)
    rng = np.random.default_rng(seed + 90 + G)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    got, init = _prefill(c, dev, entry, f8=(k8, v8, ks, vs))
    assert (got[0] == 0x3333).all()
    want = oracle.attn_prefill8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"], c["cu"],
                                c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def paged_prompt_case(ctxs, chunks, Hkv, G, bs, seed):
    """Prompt sequences (ctx cached tokens + a chunk, all in the cache) over
    pages of `bs` keys from a seeded permutation."""
    rng = np.random.default_rng(seed)
    Hq = G * Hkv
    lens = [c + n for c, n in zip(ctxs, chunks)]
    mb = max((L + bs - 1) // bs for L in lens)
    pages = len(lens) * mb + 3
    perm = rng.permutation(pages).astype(np.int32)
    bt = np.zeros((len(lens), mb), np.int32)
    at = 0
    for s, L in enumerate(lens):
        n = (L + bs - 1) // bs
        bt[s, :n] = perm[at:at + n]
        at += n
    pos, cu = [], [0]
    for ctx, n in zip(ctxs, chunks):
        pos.extend(range(ctx, ctx + n))
        cu.append(cu[-1] + n)
    T = len(pos)
    qstride = (2 * Hq + 2 * Hkv) * D
    from _util import bf16_bits
    return dict(q=bf16_bits(rng.standard_normal((T, Hq, D)) * 0.5),
                kc=bf16_bits(rng.standard_normal((pages * bs, Hkv, D)) * 0.5),
                vc=bf16_bits(rng.standard_normal((pages * bs, Hkv, D)) * 0.5),
                qkv=bf16_bits(rng.standard_normal((T, qstride))), qstride=qstride, bt=bt, max_blocks=mb, pages=pages,
                pos=np.array(pos, np.int32), cu=np.array(cu, np.int32), seqs=len(lens), T=T, Hq=Hq, Hkv=Hkv)


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("e4m3", [False, True])
@pytest.mark.parametrize("G,Hkv", [(4, 4), (6, 4), (1, 4), (8, 2)])
@pytest.mark.parametrize("bs", [1, 2, 4, 8, 32, 64])
def test_prefill_block_sizes_match_oracle(dev, e4m3, G, Hkv, bs, split):
    """Pages of 1 / 2 / 4 / 8 / 32 / 64 keys (any power of two; the reference
    engine uses 16): below 16 keys the tiles load through registers with a
    page id per key (pages smaller than the loading threads' key groups; at
    G = 6, whose 6 waves load in key pairs, pages of 1 key) or per key group
    (G = 6: per wave key pair from 2 keys up), at 32 and 64 by LDS DMA (bf16)
    — for every group shape; and the same through the split-key entry points
    (these small grids split)."""
    print(f"case prefill bs={bs} G={G} Hkv={Hkv} e4m3={e4m3} split={split}", flush=True)
    c = paged_prompt_case([100, 0, 37], [70, 33, 130], Hkv, G, bs, 200 + bs + G)
    T, Hq = c["T"], c["Hq"]
    ws = None
    if split:
        nbytes = pkv.attn_prefill_workspace(T, Hq, Hkv, c["seqs"])
        assert nbytes > 0
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    init = np.full((T, Hq, D), 0x3333, np.uint16)
    out = torch.from_numpy(init.view(np.int16).copy()).to(dev)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16
                                   else np.ascontiguousarray(a)).to(dev)
    pos, cu, bt = t(c["pos"]), t(c["cu"]), t(c["bt"])
    if e4m3:
        rng = np.random.default_rng(bs + G)
        k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
        ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
        vs = (rng.random(c["vc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
        pkv.attn_prefill_e4m3(t(c["q"]), t(k8), t(v8), t(ks), t(vs), t(c["qkv"]), c["qstride"], Hq, Hkv, pos, cu,
                              c["seqs"], bt, c["max_blocks"], bs, out, SCALE, None, 1, T, c["pages"], workspace=ws)
        want = oracle.attn_prefill8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["cu"],
                                    c["seqs"], c["bt"], c["max_blocks"], bs, SCALE, out=init.copy())
    else:
        pkv.attn_prefill(t(c["q"]), t(c["kc"]), t(c["vc"]), t(c["qkv"]), c["qstride"], Hq, Hkv, pos, cu, c["seqs"],
                         bt, c["max_blocks"], bs, out, SCALE, None, 1, T, c["pages"], workspace=ws)
        want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["cu"],
                                   c["seqs"], c["bt"], c["max_blocks"], bs, SCALE, out=init.copy())
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("fmode", [0, 1, 2])
def test_groups_graph_replay_matches_eager(dev, fmode):
    """The G = 6 decode route (range kernels + merge, optionally with FP8
    output copies) captured into a HIP graph and replayed 4 times, with eager
    launches and synchronizations in between, reproduces the eager outputs
    and copies bit for bit each time."""
    print(f"case decode G=6 graph replay fmode={fmode}", flush=True)
    from _util import fp8_buffers
    c = decode_case([513, 4097, 1000, 64, 17], 24, 4, 70 + fmode)
    T, Hq = len(c["pos"]), c["Hq"]
    q, kc, vc, qkv = (dev_i16(c[k], dev) for k in ("q", "kc", "vc", "qkv"))
    pos, ts, bt, cu = (dev_i32(c[k], dev) for k in ("pos", "tok_seq", "bt", "cu"))
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)
    fq, fs = fp8_buffers(T, Hq * D, fmode or 1, T, dev)
    fq0, fs0 = fq.clone(), fs.clone()  # sentinels; Mx32 scales pad to 128 rows

    def launch():
        if fmode:
            pkv.attn_fp8_next(fq, fs, fmode, T)
        pkv.attn_decode(q, kc, vc, qkv, c["qstride"], Hq, c["Hkv"], pos, ts, bt, c["max_blocks"], BS, out, SCALE,
                        cu, 0, None, 1, T, c["pages"], ws)

    def snap():
        torch.cuda.synchronize()
        return out.cpu().numpy().copy(), fq.cpu().numpy().copy(), fs.cpu().numpy().copy()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch()  # eager reference, outside capture
    torch.cuda.current_stream().wait_stream(s)
    e_out, e_fq, e_fs = snap()
    ok, err = close(e_out.view(np.uint16), run_oracle(c, cu=c["cu"]))
    assert ok, f"eager max |diff| {err}"
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for r in range(4):
        if r % 2:
            launch()  # eager work between replays
            torch.cuda.synchronize()
        out.fill_(0)
        fq.copy_(fq0)
        fs.copy_(fs0)
        g.replay()
        g_out, g_fq, g_fs = snap()
        assert np.array_equal(g_out, e_out), f"replay {r} out"
        if fmode:
            assert np.array_equal(g_fq, e_fq), f"replay {r} fq"
            assert np.array_equal(g_fs.view(np.uint8), e_fs.view(np.uint8)), f"replay {r} fs"


@pytest.mark.parametrize("G,Hkv", [(4, 4), (6, 4), (8, 2)])
def test_groups_more_rows_than_a_block(dev, G, Hkv):
    """More rows than a workgroup has threads (the range search's two-pass
    scan and per-row metadata read from memory): 90 sequences of 1..7 draft
    rows (over 256 rows, segments of every fill) through pkv_attn_verify, and
    300 single rows through pkv_attn_decode (G != 4 runs the verify kernels),
    and the verify rows over an E4M3 cache, all against the oracle."""
    rng = np.random.default_rng(80 + G)
    groups = [(int(rng.integers(0, 400)), int(rng.integers(1, 8))) for _ in range(90)]
    print(f"case verify G={G} Hkv={Hkv} rows={sum(n for _, n in groups)}", flush=True)
    c = verify_case(groups, Hkv, 81 + G, G=G)
    assert c["T"] > 256

    def want_raw(c):
        out, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"],
                                      c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
        return out, dict(raw=raw, qkv=c["qkv"], qstride=c["qstride"], Hq=c["Hq"])

    want, ex = want_raw(c)
    ok, err = close(run_verify(c, dev), want, explain=ex)
    assert ok, f"verify max |diff| {err}"
    lens = [int(x) for x in rng.integers(1, 300, 300)]
    print(f"case decode G={G} Hkv={Hkv} tokens=300", flush=True)
    d = decode_case(lens, G * Hkv, Hkv, 82 + G)
    want, ex = want_raw(d)
    ok, err = close(run_gpu(d, dev), want, explain=ex)
    assert ok, f"decode max |diff| {err}"
    # the same verify rows over an E4M3 cache
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    want, raw = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"],
                                    c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"], return_raw=True)
    ok, err = close(run_decode8(c, k8, v8, ks, vs, dev, entry="verify"), want,
                    explain=dict(raw=raw, qkv=c["qkv"], qstride=c["qstride"], Hq=c["Hq"]))
    assert ok, f"verify e4m3 max |diff| {err}"


def test_prefill_g6_library_kernel_all_rows(dev):
    """The G = 6 library prompt kernel (four LDS stages, a barrier every
    second key tile) on a grid that covers the CUs, every row against the
    oracle: a 1,070-token chunk after 1,000 cached keys and a 1,025-token
    prompt (odd and even tile counts, partial last tiles)."""
    print("case prefill G=6 library kernel all rows", flush=True)
    from test_gpu_prefill import prefill_case
    c = prefill_case([1000, 0], [1070, 1025], 4, 181, G=6)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert ((c["T"] + 31) // 32 + c["seqs"]) * 4 >= cus
    got, init = _prefill(c, dev, "lib")
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], 4, c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G,nseq", [(1, 16), (2, 16), (4, 9), (6, 9), (8, 9)])
def test_prefill_many_tiles_sampled_rows(dev, G, nseq):
    """Prompts with enough query tiles for the library's full-size kernel
    (nseq prompts of 1,000 tokens: at least CUs workgroups for G <= 6, 4 x
    CUs for G = 8; smaller grids take the fine-tile kernel, which the cases
    above cover), all rows computed, 2-row groups at 24 places checked
    against the oracle."""
    print(f"case prefill many tiles G={G} seqs={nseq}", flush=True)
    from test_gpu_prefill import prefill_case
    c = prefill_case([0] * nseq, [1000] * nseq, 4, 170 + G, G=G)
    bq = 32 if G >= 6 else 256 // G
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert ((c["T"] + bq - 1) // bq + c["seqs"]) * 4 >= (4 if G == 8 else 1) * cus
    got, _ = _prefill(c, dev, "lib")
    rng = np.random.default_rng(171 + G)
    for _ in range(24):
        s = int(rng.integers(0, nseq))
        j = int(rng.integers(0, 999))
        rows = np.array([c["cu"][s] + j, c["cu"][s] + j + 1])
        want = oracle.attn_prefill(np.ascontiguousarray(c["q"][rows]), c["kc"], c["vc"],
                                   np.ascontiguousarray(c["qkv"][rows]), c["qstride"], c["Hq"], 4, c["pos"][rows],
                                   np.array([0, 2], np.int32), 1, np.ascontiguousarray(c["bt"][s:s + 1]),
                                   c["max_blocks"], BS, SCALE)
        ok, err = close(got[rows], want)
        assert ok, f"seq {s} rows {rows}: max |diff| {err}"

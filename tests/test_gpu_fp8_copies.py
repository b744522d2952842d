"""FP8 output copies through the C-ABI (pkv_attn_fp8_next): the reference's
fq / fs / fmode / frows of attn_paged_g<G> / attn_merge (Fp8Out / quant8,
src/kernels/fp8.cuh:29-85). The bf16 outputs must be bit for bit those of the
same call without copies (a row finished by the merge from one record is the
in-place arithmetic), and the copies must match the oracle's quantisation of
its gated f32 outputs (tests/_util.py check_fp8_copies)."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, check_fp8_copies, close, decode_case, fp8_buffers
from test_gpu_e4m3 import e4m3_cache
from test_gpu_verify import verify_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0
FROWS = 300


def t_(a, dev):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)
    pkv.attn_fp8_next(None, None, 0, 0)


def run(c, dev, entry, fp8=None, f8cache=None, outs=None, skip=0):
    T, Hq, Hkv = len(c["pos"]), c["Hq"], c["Hkv"]
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    ws = torch.empty(max(pkv.attn_decode_workspace(T, Hq), pkv.attn_verify_workspace(T, Hq)), dtype=torch.uint8,
                     device=dev)
    if fp8 is not None:
        pkv.attn_fp8_next(fp8[0], fp8[1], fp8[2], FROWS)
    q, qkv = t_(c["q"], dev), t_(c["qkv"], dev)
    pos, ts, bt, cu = (t_(np.asarray(c[k], np.int32), dev) for k in ("pos", "tok_seq", "bt", "cu"))
    outs_d = None if outs is None else t_(np.asarray(outs, np.int32), dev)
    if f8cache is not None:
        k8, v8, ks, vs = (t_(a, dev) for a in f8cache)
        fn = pkv.attn_decode_e4m3 if entry == "decode" else pkv.attn_verify_e4m3
        fn(q, k8, v8, ks, vs, qkv, c["qstride"], Hq, Hkv, pos, ts, bt, c["max_blocks"], BS, out, SCALE, cu, skip,
           outs_d, 1, T, c["pages"], ws)
    elif entry == "step":
        kc, vc = t_(c["kc"], dev), t_(c["vc"], dev)
        # the step's rows are the keys already in the cache at pos (written back unchanged)
        slot = (c["bt"][c["tok_seq"], c["pos"] // BS] * BS + c["pos"] % BS).astype(np.int32)
        rows = np.concatenate([c["kc"][slot].reshape(T, -1), c["vc"][slot].reshape(T, -1)], axis=1)
        rows_d = t_(rows, dev)
        k_rows = rows_d.data_ptr()
        v_rows = k_rows + Hkv * D * 2
        pkv.attn_decode_step(k_rows, v_rows, 2 * Hkv * D * 2, t_(slot, dev), q, kc, vc, qkv, c["qstride"], Hq, Hkv,
                             pos, ts, bt, c["max_blocks"], BS, out, SCALE, cu, skip, outs_d, 1, T, c["pages"], ws)
    elif entry == "split":
        # pkv_attn_decode_split, then pkv_attn_decode_merge (a copy request
        # set before the split is kept for the merge)
        kc, vc = t_(c["kc"], dev), t_(c["vc"], dev)
        for phase in ("split", "merge"):
            pkv.attn_decode(q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, ts, bt, c["max_blocks"], BS, out, SCALE, cu,
                            skip, outs_d, 1, T, c["pages"], ws, phase=phase)
    else:
        fn = pkv.attn_decode if entry == "decode" else pkv.attn_verify
        fn(q, t_(c["kc"], dev), t_(c["vc"], dev), qkv, c["qstride"], Hq, Hkv, pos, ts, bt, c["max_blocks"], BS, out,
           SCALE, cu, skip, outs_d, 1, T, c["pages"], ws)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("G", [4, 6])
def test_split_then_merge_matches_decode(dev, mode, G):
    """pkv_attn_decode_split followed by pkv_attn_decode_merge gives the bytes
    of one pkv_attn_decode call (G = 4: decode ranges; G = 6: the verify
    route), FP8 copies included."""
    print(f"case split + merge G={G} fp8 mode={mode}", flush=True)
    c = decode_case([1, 17, 700, 4097, 130, 2000], G * 4, 4, 90 + G)
    T, K = len(c["pos"]), G * 4 * D
    bufs = [fp8_buffers(T, K, mode, FROWS, dev) if mode else (None, None) for _ in range(2)]
    one = run(c, dev, "decode", fp8=(bufs[0][0], bufs[0][1], mode) if mode else None)
    two = run(c, dev, "split", fp8=(bufs[1][0], bufs[1][1], mode) if mode else None)
    assert np.array_equal(one, two)
    if mode:
        assert torch.equal(bufs[0][0], bufs[1][0]) and torch.equal(bufs[0][1].view(torch.uint8),
                                                                    bufs[1][1].view(torch.uint8))
    ok, err = close(one, oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], 4, c["pos"],
                                            c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])[0])
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("entry,G,min_range", [("decode", 4, 32), ("decode", 4, 1 << 20), ("step", 4, 32),
                                               ("verify", 4, 32), ("decode", 6, 32), ("verify", 8, 1 << 20)])
def test_fp8_copies_bf16_cache(dev, mode, entry, G, min_range):
    print(f"case fp8 copies mode={mode} {entry} G={G} min_range={min_range}", flush=True)
    pkv.attn_decode_config(1, min_range)
    Hkv = 2 if G == 8 else 4
    if entry == "verify":
        c = verify_case([(300, 4), (0, 9), (40, 3), (2000, 5), (12, 2)], Hkv, 80 + G, G=G)
    else:
        c = decode_case([1, 17, 700, 4097, 130, 2000], G * Hkv, Hkv, 81 + G)
    T, Hq = len(c["pos"]), c["Hq"]
    plain = run(c, dev, entry)
    fq, fs = fp8_buffers(T, Hq * D, mode, FROWS, dev)
    got = run(c, dev, entry, fp8=(fq, fs, mode))
    assert np.array_equal(got, plain)
    want, raw = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"],
                                   c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    ok, err = close(got, want)
    assert ok, err
    y = oracle.gate_rows(raw, c["qkv"], c["qstride"], Hq).reshape(T, Hq * D)
    check_fp8_copies(fq.cpu().numpy(), fs.cpu().numpy(), y, mode, FROWS)


@pytest.mark.parametrize("entry", ["decode", "verify"])
def test_fp8_copies_e4m3_cache_and_skipped_rows(dev, entry):
    """E4M3 cache, Mx32 copies; a skipped prompt's rows get no copy."""
    print(f"case fp8 copies e4m3 {entry}", flush=True)
    c = verify_case([(300, 4), (0, 9), (40, 4), (90, 1), (2000, 3)], 4, 12)
    rng = np.random.default_rng(13)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    outs = np.array([0, -1, 0, 0, 0], np.int32)
    T, Hq = c["T"], 16
    plain = run(c, dev, entry, f8cache=(k8, v8, ks, vs), outs=outs, skip=1)
    fq, fs = fp8_buffers(T, Hq * D, 2, FROWS, dev)
    got = run(c, dev, entry, fp8=(fq, fs, 2), f8cache=(k8, v8, ks, vs), outs=outs, skip=1)
    assert np.array_equal(got, plain)
    _, raw = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], Hq, 4, c["pos"], c["tok_seq"],
                                 c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"], skip_prompts=1, outs=outs,
                                 return_raw=True)
    y = oracle.gate_rows(raw, c["qkv"], c["qstride"], Hq).reshape(T, Hq * D)
    rows = [t for t in range(T) if not 4 <= t < 13]
    fqh = fq.cpu().numpy()
    assert (fqh[4:13] == 0x7F).all()
    check_fp8_copies(fqh, fs.cpu().numpy(), y, 2, FROWS, rows=rows)


def test_fp8_next_is_cleared_by_the_merging_call(dev):
    """The request covers one call: the following call writes no copies."""
    print("case fp8 request cleared", flush=True)
    c = decode_case([300, 40], 16, 4, 5)
    fq, fs = fp8_buffers(2, 16 * D, 1, FROWS, dev)
    run(c, dev, "decode", fp8=(fq, fs, 1))
    fq2, fs2 = fp8_buffers(2, 16 * D, 1, FROWS, dev)
    pkv.attn_fp8_next(fq2, fs2, 1, FROWS)
    pkv.attn_fp8_next(None, None, 0, 0)  # cleared again before the call
    run(c, dev, "decode")
    torch.cuda.synchronize()
    assert (fq2.cpu().numpy() == 0x7F).all() and torch.isnan(fs2).all()
    assert (fq.cpu().numpy() != 0x7F).any()
    with pytest.raises(pkv.PkvError):
        pkv.attn_fp8_next(fq, None, 1, FROWS)


@pytest.mark.parametrize("entry", ["decode", "step", "step_noalloc_bad_group"])
def test_fp8_request_consumed_by_a_failing_call(dev, entry):
    """A merging call that fails its argument checks still consumes the
    pending request: the next valid call writes no copies through the stale
    fq / fs (they may have been freed after the error)."""
    print(f"case fp8 request consumed by failing {entry}", flush=True)
    c = decode_case([300, 40, 17], 16, 4, 6)
    T = len(c["pos"])
    fq, fs = fp8_buffers(T, 16 * D, 1, FROWS, dev)
    pkv.attn_fp8_next(fq, fs, 1, 2)  # frows 2 < T: the merging call must refuse it
    with pytest.raises(pkv.PkvError):
        run(c, dev, "step" if entry.startswith("step") else "decode")
    if entry == "step_noalloc_bad_group":
        # a second request, refused by the no-allocation step's group check (G = 5)
        pkv.attn_fp8_next(fq, fs, 1, FROWS)
        cc = decode_case([50], 20, 4, 7)
        q, qkv = t_(cc["q"], dev), t_(cc["qkv"], dev)
        pos, ts, bt, cu = (t_(np.asarray(cc[k], np.int32), dev) for k in ("pos", "tok_seq", "bt", "cu"))
        kc, vc = t_(cc["kc"], dev), t_(cc["vc"], dev)
        out = torch.zeros(1, 20, D, dtype=torch.int16, device=dev)
        slot = t_(np.zeros(1, np.int32), dev)
        with pytest.raises(pkv.PkvError):
            pkv.attn_decode_step_noalloc(qkv.data_ptr(), qkv.data_ptr(), 2 * 4 * D * 2, slot, q, kc, vc, qkv,
                                         cc["qstride"], 20, 4, pos, ts, bt, cc["max_blocks"], BS, out, SCALE, cu, 0,
                                         None, 1, 1, cc["pages"])
    got = run(c, dev, "decode")
    torch.cuda.synchronize()
    assert (fq.cpu().numpy() == 0x7F).all() and torch.isnan(fs).all()
    ok, err = close(got, oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], 16, 4, c["pos"],
                                            c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])[0])
    assert ok, err

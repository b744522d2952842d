"""GPU parity: draft-verify attention (pkv_attn_verify) against the oracle's
paged decode attention (oracle/pkv_oracle.c orc_attn_decode): each row of a
sequence that feeds several tokens attends causally to keys 0..pos[t].

Tolerance (north star): bf16 outputs within max-abs 2e-3 and relative 1e-2,
|got - want| <= 2e-3 + 1e-2 * |want|. The verify kernel rounds the softmax
weights to bf16 before P.V (the oracle keeps them in double), which the
tolerance covers. Config 5 at full size (16 sequences of 32k..128k keys, 4
rows each) is checked against the decode kernel on the same cache and, on
every row, against the oracle."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits, close, host_pages, nan_stale, oracle_decode_rows

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0


def i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)


def verify_case(groups, Hkv, seed, G=4):
    """groups: (L0, n) per sequence: n rows at positions L0 .. L0 + n - 1,
    every key already cached; pages from a seeded permutation; G query
    heads per kv head."""
    rng = np.random.default_rng(seed)
    Hq = G * Hkv
    need = [(L0 + n + BS - 1) // BS for L0, n in groups]
    mb = max(need)
    pages = sum(need) + 3
    perm = rng.permutation(pages).astype(np.int32)
    bt = np.zeros((len(groups), mb), np.int32)
    at = 0
    for s, k in enumerate(need):
        bt[s, :k] = perm[at:at + k]
        at += k
    pos, ts, cu = [], [], [0]
    for s, (L0, n) in enumerate(groups):
        pos.extend(range(L0, L0 + n))
        ts.extend([s] * n)
        cu.append(cu[-1] + n)
    T = len(pos)
    qstride = (2 * Hq + 2 * Hkv) * D
    return dict(q=bf16_bits(rng.standard_normal((T, Hq, D)) * 0.5),
                kc=bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * 0.5),
                vc=bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * 0.5),
                qkv=bf16_bits(rng.standard_normal((T, qstride))), qstride=qstride, bt=bt, max_blocks=mb, pages=pages,
                pos=np.array(pos, np.int32), tok_seq=np.array(ts, np.int32), cu=np.array(cu, np.int32), T=T, Hq=Hq,
                Hkv=Hkv)


def run_verify(c, dev, skip=0, outs=None, spec=1, out_init=None):
    T, Hq = c["T"], c["Hq"]
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev) if out_init is None else i16(out_init, dev)
    ws = torch.empty(pkv.attn_verify_workspace(T, Hq), dtype=torch.uint8, device=dev)
    pkv.attn_verify(i16(c["q"], dev), i16(c["kc"], dev), i16(c["vc"], dev), i16(c["qkv"], dev), c["qstride"], Hq,
                    c["Hkv"], i32(c["pos"], dev), i32(c["tok_seq"], dev), i32(c["bt"], dev), c["max_blocks"], BS, out,
                    SCALE, i32(c["cu"], dev), skip, None if outs is None else i32(outs, dev), spec, T, c["pages"], ws)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


def run_oracle(c, **kw):
    out, _ = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"],
                                c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"], **kw)
    return out


@pytest.mark.parametrize("groups,Hkv,seed,min_range", [
    ([(0, 4)], 4, 0, 32),                                   # first rows: 1..4 keys
    ([(12, 4), (16, 4), (29, 4)], 4, 1, 32),                # drafts crossing a page edge
    ([(100, 1), (50, 2), (70, 3), (200, 4), (33, 5), (64, 7)], 4, 2, 32),  # ragged rows, 2 segments
    ([(5000, 4), (300, 4), (9000, 4)], 4, 3, 32),           # long, split over many ranges
    ([(5000, 4), (300, 4), (9000, 4)], 4, 3, 1 << 20),      # the same unsplit (one range)
    ([(700, 4), (1500, 3)], 2, 4, 32),                      # Hkv 2
    ([(900, 4), (2000, 2)], 8, 5, 32),                      # two kv-head groups
])
def test_verify_matches_oracle(dev, groups, Hkv, seed, min_range):
    print(f"case verify groups={groups} Hkv={Hkv} min_range={min_range}", flush=True)
    pkv.attn_decode_config(1, min_range)
    c = verify_case(groups, Hkv, seed)
    got = run_verify(c, dev)
    want = run_oracle(c)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("groups,min_range", [([(12, 4), (29, 3), (0, 2)], 32), ([(5000, 4), (301, 4)], 32)])
def test_verify_stale_slots_are_nan(dev, groups, min_range):
    """Slots holding no key of a sequence are NaN in K and V (the drafts'
    own later keys are real keys, masked causally): no NaN reaches the
    outputs."""
    print(f"case verify NaN stale slots groups={groups}", flush=True)
    pkv.attn_decode_config(1, min_range)
    c = verify_case(groups, 4, 13)
    c = nan_stale(c, [L0 + n for L0, n in groups])
    got = run_verify(c, dev)
    want = run_oracle(c)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_verify_skips_prompt_rows(dev):
    """With skip_prompts, rows of prompt sequences (several rows, not
    speculative: outs[s * spec] < 0) are left to prefill and untouched;
    speculative sequences' rows are verified."""
    print("case verify skip prompts", flush=True)
    c = verify_case([(300, 4), (0, 9), (40, 4), (90, 1)], 4, 6)
    outs = np.array([0, -1, 0, 0], np.int32)  # spec = 1
    init = np.full((c["T"], c["Hq"], D), 0x5555, np.uint16)
    got = run_verify(c, dev, skip=1, outs=outs, out_init=init)
    assert (got[4:13] == 0x5555).all()
    want = run_oracle(c, skip_prompts=1, outs=outs, spec=1, out=init.copy())
    ok, err = close(got, want)
    assert ok, err


def test_verify_c5_full_size(dev):
    """Config 5: 16 sequences with 32,768..131,072 cached tokens verify 4
    drafts each (positions L .. L + 3). Against the decode kernel on the same
    cache (every row), and against the oracle for the shortest sequence."""
    print("case verify c5 full", flush=True)
    Hq, Hkv, B, n = 16, 4, 16, 4
    rng = np.random.default_rng(21)
    L0 = rng.integers(32768, 131072 + 1, size=B)
    need = (L0 + n + BS - 1) // BS
    pages = int(need.sum()) + 16
    mb = int(need.max())
    perm = rng.permutation(pages).astype(np.int32)
    bt = np.zeros((B, mb), np.int32)
    at = 0
    for s in range(B):
        bt[s, :need[s]] = perm[at:at + need[s]]
        at += need[s]
    gen = torch.Generator(device=dev)
    gen.manual_seed(21)
    kc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    T = B * n
    pos = np.concatenate([np.arange(L, L + n) for L in L0]).astype(np.int32)
    ts = np.repeat(np.arange(B), n).astype(np.int32)
    cu = (np.arange(B + 1) * n).astype(np.int32)
    q = (torch.randn(T, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = (2 * Hq + 2 * Hkv) * D
    qkv = torch.randn(T, qstride, device=dev, generator=gen).to(torch.bfloat16)
    pos_d, ts_d, bt_d, cu_d = i32(pos, dev), i32(ts, dev), i32(bt, dev), i32(cu, dev)
    outs_d = i32(np.zeros(B, np.int32), dev)
    vout = torch.zeros(T, Hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(pkv.attn_verify_workspace(T, Hq), dtype=torch.uint8, device=dev)
    pkv.attn_verify(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d, ts_d, bt_d, mb, BS, vout, SCALE, cu_d, 1, outs_d, 1, T,
                    pages, ws)
    dout = torch.zeros_like(vout)
    wsd = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)
    pkv.attn_decode(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d, ts_d, bt_d, mb, BS, dout, SCALE, cu_d, 1, outs_d, 1, T,
                    pages, wsd)
    torch.cuda.synchronize()
    bits = lambda x: x.cpu().view(torch.int16).numpy().view(np.uint16)
    ok, err = close(bits(vout), bits(dout))
    assert ok, f"verify vs decode: {err}"
    # every row (16 sequences x 4 drafts x 16 heads) against the oracle
    kc_h, vc_h, bt_h, _ = host_pages(kc, vc, bt, need)
    want = oracle_decode_rows(bits(q), kc_h, vc_h, bits(qkv), qstride, Hq, Hkv, pos, ts, bt_h, mb, SCALE)
    del kc_h, vc_h
    ok, err = close(bits(vout), want, what="c5 full, all 64 x 16 rows")
    assert ok, f"verify vs oracle: {err}"

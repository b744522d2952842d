"""GPU parity: chunked-prefill attention over paged context (MFMA bf16,
pkv_attn_prefill) against the oracle (oracle/pkv_oracle.c orc_attn_prefill).

Tolerance (north star): bf16 outputs within max-abs 2e-3 and relative 1e-2,
i.e. |got - want| <= 2e-3 + 1e-2 * |want|. The oracle keeps P in double; the
reference (and this kernel) round P to bf16 before P.V — that rounding is
the part of parity left to the tolerance. Full config-4 size is checked on
sampled rows (prefill == decode with q pre-rounded to bf16(q * scale *
log2 e) and scale ln 2, an identity of the two oracles) and by the
reference's own bench-attn --check idea: a prompt chunk's last row equals
paged decode attention for that token."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits, close, decode_case, nan_stale

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0
LN2 = float(np.log(2.0))
LOG2E = 1.4426950408889634


def i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def prefill_case(ctxs, chunks, Hkv, seed, decode_rows=0):
    """Sequences with ctx cached tokens feeding a chunk of n tokens (all
    already in the cache, as after pkv_append); optional extra one-token
    decode sequences first."""
    Hq = 4 * Hkv
    lens = [c + n for c, n in zip(ctxs, chunks)]
    dec = [40 + 13 * i for i in range(decode_rows)]
    c = decode_case(dec + lens, Hq, Hkv, seed)
    rng = np.random.default_rng(seed + 7)
    pos, tok_seq, cu = [], [], [0]
    for s, L in enumerate(dec):
        pos.append(L - 1)
        tok_seq.append(s)
        cu.append(cu[-1] + 1)
    for i, (ctx, n) in enumerate(zip(ctxs, chunks)):
        s = decode_rows + i
        pos.extend(range(ctx, ctx + n))
        tok_seq.extend([s] * n)
        cu.append(cu[-1] + n)
    T = len(pos)
    q = bf16_bits(rng.standard_normal((T, Hq, D)) * 0.5)
    qkv = bf16_bits(rng.standard_normal((T, c["qstride"])))
    return dict(c, q=q, qkv=qkv, pos=np.array(pos, np.int32), tok_seq=np.array(tok_seq, np.int32),
                cu=np.array(cu, np.int32), T=T, seqs=len(cu) - 1, Hq=Hq, Hkv=Hkv)


def run_prefill(c, dev, out_init=None):
    T, Hq = c["T"], c["Hq"]
    out = (torch.zeros(T, Hq, D, dtype=torch.int16, device=dev) if out_init is None else i16(out_init, dev))
    pkv.attn_prefill(i16(c["q"], dev), i16(c["kc"], dev), i16(c["vc"], dev), i16(c["qkv"], dev), c["qstride"], Hq,
                     c["Hkv"], i32(c["pos"], dev), i32(c["cu"], dev), c["seqs"], i32(c["bt"], dev), c["max_blocks"],
                     BS, out, SCALE, None, 1, T, c["pages"])
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("ctxs,chunks,Hkv,seed", [
    ([0], [37], 4, 0),             # no prefix, partial query tile
    ([100], [64], 4, 1),           # one full 64-query tile after a prefix
    ([16, 5], [130, 2], 1, 2),     # tiles crossing 64, a 2-token prompt
    ([1000, 33, 0], [70, 200, 65], 2, 3),
])
def test_prefill_matches_oracle(dev, ctxs, chunks, Hkv, seed):
    print(f"case prefill ctx={ctxs} chunk={chunks} Hkv={Hkv}", flush=True)
    c = prefill_case(ctxs, chunks, Hkv, seed)
    got = run_prefill(c, dev)
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_prefill_late_dominant_key(dev):
    """A key in a late tile whose score exceeds every earlier score by 92
    (log2 units): the running maximum jumps and the accumulators are
    rescaled; the output is that key's value (against the oracle)."""
    print("case prefill dominant late key", flush=True)
    c = prefill_case([300], [70], 4, 9)
    s0 = 0
    hot = 200  # a key well past the first 32-key tile
    bt = c["bt"][s0]
    slot = bt[hot // BS] * BS + hot % BS
    rng = np.random.default_rng(9)
    u = np.where(rng.random(D) < 0.5, -0.5, 0.5)
    q = c["q"].copy()
    q[:, 0] = bf16_bits(np.broadcast_to(u, (c["T"], D)))  # query head 0 of every row: u
    kc = c["kc"].copy()
    kc[slot, 0] = bf16_bits(16 * u)  # its score: 16 |u|^2 / 16 * log2 e = 92 (log2 units) above ~0
    c = dict(c, kc=kc, q=q)
    got = run_prefill(c, dev)
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("ctxs,chunks", [([0], [37]), ([100], [45]), ([16, 5], [130, 2])])
def test_prefill_stale_slots_are_nan(dev, ctxs, chunks):
    """Every cache slot that holds no key of a sequence (past its length in
    its last page, unused pages) is NaN in K and V: keys at or past the
    length must not reach the output, not even as 0 x NaN."""
    print(f"case prefill NaN stale slots ctx={ctxs} chunk={chunks}", flush=True)
    c = prefill_case(ctxs, chunks, 4, 11)
    c = nan_stale(c, [int(c["pos"][c["cu"][s + 1] - 1]) + 1 for s in range(c["seqs"])])
    got = run_prefill(c, dev)
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_prefill_leaves_decode_rows_untouched(dev):
    """Decode rows (one token) and verifying rows are left to decode attention."""
    print("case prefill skips decode rows", flush=True)
    c = prefill_case([50, 20], [40, 3], 4, 4, decode_rows=2)
    init = np.full((c["T"], c["Hq"], D), 0x7777, np.uint16)
    got = run_prefill(c, dev, out_init=init)
    assert (got[:2] == 0x7777).all()
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    ok, err = close(got, want)
    assert ok, err


def test_prefill_c4_shared_prefix_sampled_rows(dev):
    """Config 4: 8 sequences share a 16,384-token cached prefix (the same
    1,024 pages in every block table) and each feeds a 2,048-token chunk.
    Sampled rows against the oracle; each chunk's last row against the paged
    decode kernel on the same cache."""
    print("case prefill c4", flush=True)
    Hq, Hkv, B, P, N = 16, 4, 8, 16384, 2048
    pp, cp = P // BS, N // BS
    pages = pp + B * cp + 8
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    kc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    rng = np.random.default_rng(11)
    perm = rng.permutation(pages).astype(np.int32)
    shared = perm[:pp]
    bt = np.zeros((B, pp + cp), np.int32)
    for s in range(B):
        bt[s, :pp] = shared
        bt[s, pp:] = perm[pp + s * cp:pp + (s + 1) * cp]
    T = B * N
    pos = np.tile(np.arange(P, P + N, dtype=np.int32), B)
    cu = (np.arange(B + 1) * N).astype(np.int32)
    q = (torch.randn(T, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = (2 * Hq + 2 * Hkv) * D
    qkv = torch.randn(T, qstride, device=dev, generator=gen).to(torch.bfloat16)
    out = torch.zeros(T, Hq, D, dtype=torch.bfloat16, device=dev)
    bt_d, pos_d, cu_d = i32(bt, dev), i32(pos, dev), i32(cu, dev)
    pkv.attn_prefill(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d, cu_d, B, bt_d, pp + cp, BS, out, SCALE, None, 1, T,
                     pages)
    torch.cuda.synchronize()
    # (1) the last row of every chunk against paged decode attention (the
    # decode kernel does not round q; within tolerance of each other)
    last = cu[1:] - 1
    dout = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(B, Hq), dtype=torch.uint8, device=dev)
    pkv.attn_decode(q[last], kc, vc, qkv[last], qstride, Hq, Hkv, pos_d[last], torch.arange(B, dtype=torch.int32,
                    device=dev), bt_d, pp + cp, BS, dout, SCALE, i32(np.arange(B + 1), dev), 0, None, 1, B, pages, ws)
    torch.cuda.synchronize()
    ok, err = close(out[last].cpu().view(torch.int16).numpy().view(np.uint16),
                    dout.cpu().view(torch.int16).numpy().view(np.uint16))
    assert ok, f"prefill last rows vs decode: {err}"
    # (2) sampled rows against the oracle, as decode rows with q pre-rounded
    rows = np.concatenate([[0, 1, 63, 64, 2047], rng.integers(0, T, size=7)])
    seqs = rows // N
    need = [(pos[r] + BS) // BS for r in rows]
    sub = np.unique(np.concatenate([bt[s, :n] for s, n in zip(seqs, need)]))
    idx = torch.from_numpy(sub).to(dev).long()
    kc_h = kc.view(pages, BS, Hkv, D)[idx].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1, Hkv, D)
    vc_h = vc.view(pages, BS, Hkv, D)[idx].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1, Hkv, D)
    remap = {int(p_): i for i, p_ in enumerate(sub)}
    bt_r = np.zeros((len(rows), pp + cp), np.int32)
    for i, (s, n) in enumerate(zip(seqs, need)):
        bt_r[i, :n] = [remap[int(p_)] for p_ in bt[s, :n]]
    qh = q[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    q_r = bf16_bits(qh * np.float32(SCALE * LOG2E))
    qkv_h = qkv[torch.from_numpy(rows).to(dev)].cpu().view(torch.int16).numpy().view(np.uint16)
    want, _ = oracle.attn_decode(q_r, kc_h, vc_h, qkv_h, qstride, Hq, Hkv, pos[rows],
                                 np.arange(len(rows), dtype=np.int32), bt_r, pp + cp, BS, LN2)
    got = out[torch.from_numpy(rows).to(dev)].cpu().view(torch.int16).numpy().view(np.uint16)
    ok, err = close(got, want)
    assert ok, f"sampled rows vs oracle: {err}"

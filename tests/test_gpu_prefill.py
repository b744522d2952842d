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
from _util import BS, D, bf16_bits, bits, close, decode_case, host_pages, nan_stale, run_threads

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0
LN2 = float(np.log(2.0))
LOG2E = 1.4426950408889634


def i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def prefill_case(ctxs, chunks, Hkv, seed, decode_rows=0, G=4):
    """Sequences with ctx cached tokens feeding a chunk of n tokens (all
    already in the cache, as after pkv_append); optional extra one-token
    decode sequences first; G query heads per kv head."""
    Hq = G * Hkv
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


def test_prefill_c4_through_kv_manager(dev):
    """Config 4 through the KV manager at full size, with a prefix that ends
    inside a page (16,392 tokens): a seed sequence holds the prefix (written
    by pkv_append) and caches its whole 64-token units; 8 sequences share
    its pages (pkv_kv_share), copy the shared partial page on write
    (pkv_kv_prepare_write + pkv_page_copy) and feed a 2,048-token chunk
    each (pkv_kv_fill's slots, pkv_append, pkv_attn_prefill). Checks: the
    copies' bytes (the prefix's 8 slots as the seed wrote them, then the
    chunk's first rows) and the seed's page left as it was; refcounts (the
    prefix's whole pages at 9 = the cache entry + 8 sequences once the seed
    is released, each copy at 1, the seed's partial page freed); 1,024 rows
    (4 in every 64-row query tile of every sequence) against the oracle's
    prefill; each chunk's last row against the paged decode kernel."""
    from pkv import synth
    print("case prefill c4 through the KV manager, prefix 16392", flush=True)
    Hq, Hkv, B, P, N = 16, 4, 8, 16392, 2048
    qstride = (2 * Hq + 2 * Hkv) * D
    per_seq = (P + N + BS - 1) // BS
    pages = (P + BS - 1) // BS + B * (per_seq - P // BS) + 16
    kv = pkv.Kv(pages, BS)
    plan = synth.c4_kv_plan(kv, P, N, B, seed=11, release_seed=False)
    st, mb = plan["step"], plan["max_blocks"]
    assert not plan["via_cache"] and len(plan["cow"]) == B
    partial = plan["seed_blocks"][-1]
    assert all(src_ == partial for src_, _ in plan["cow"])
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    kc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    pk = (torch.randn(P, Hkv * D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    pv = (torch.randn(P, Hkv * D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    T = B * N
    q = (torch.randn(T, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qkv = torch.randn(T, qstride, device=dev, generator=gen).to(torch.bfloat16)
    out = torch.zeros(T, Hq, D, dtype=torch.bfloat16, device=dev)
    pos, slot, cu, bt = st["pos"], st["slot_map"], st["cu"], st["block_table"]
    pos_d, cu_d, bt_d = i32(pos, dev), i32(cu, dev), i32(bt, dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D
    # device work in stream order: prefix rows, copies on write, the chunk, prefill
    pkv.append(pk, pv, Hkv * D * 2, i32(plan["prefix_slots"], dev), P, Hkv, D * 2, kc, vc, pages * BS)
    page_before = (bits(kc.view(pages, BS, Hkv, D)[partial]), bits(vc.view(pages, BS, Hkv, D)[partial]))
    src = [c_[0] for c_ in plan["cow"]]
    dst = [c_[1] for c_ in plan["cow"]]
    pkv.page_copy(kc, vc, i32(src, dev), i32(dst, dev), B, BS * Hkv * D * 2, pages)
    pkv.append(k_rows, v_rows, qstride * 2, i32(slot, dev), T, Hkv, D * 2, kc, vc, pages * BS)
    pkv.attn_prefill(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d, cu_d, B, bt_d, mb, BS, out, SCALE, None, 1, T, pages)
    torch.cuda.synchronize()
    # copies on write: bytes and the tables
    off = P % BS
    kq = bits(qkv[:, 2 * Hq * D:2 * Hq * D + Hkv * D]).reshape(T, Hkv, D)
    vq = bits(qkv[:, 2 * Hq * D + Hkv * D:2 * Hq * D + 2 * Hkv * D]).reshape(T, Hkv, D)
    assert np.array_equal(bits(kc.view(pages, BS, Hkv, D)[partial]), page_before[0]), "seed's page changed"
    assert np.array_equal(bits(vc.view(pages, BS, Hkv, D)[partial]), page_before[1])
    for s, d_ in enumerate(dst):
        assert bt[s, P // BS] == d_ and d_ not in plan["seed_blocks"]
        for cache, pre, new in ((kc, page_before[0], kq), (vc, page_before[1], vq)):
            got_page = bits(cache.view(pages, BS, Hkv, D)[d_])
            assert np.array_equal(got_page[:off], pre[:off]), f"sequence {s}: copied prefix slots differ"
            assert np.array_equal(got_page[off:], new[cu[s]:cu[s] + BS - off]), f"sequence {s}: chunk slots differ"
    kv.release(plan["seed_id"])
    whole = plan["seed_blocks"][:P // BS]
    assert all(kv.refs(b_) == B + 1 for b_ in whole), "prefix pages: cache entry + 8 sequences"
    assert kv.refs(partial) == 0 and all(kv.refs(d_) == 1 for d_ in dst)
    assert all((bt[s, :P // BS] == whole).all() for s in range(B))
    # (1) the last row of every chunk against paged decode attention
    last = cu[1:] - 1
    dout = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(B, Hq), dtype=torch.uint8, device=dev)
    pkv.attn_decode(q[last], kc, vc, qkv[last], qstride, Hq, Hkv, pos_d[last], torch.arange(B, dtype=torch.int32,
                    device=dev), bt_d, mb, BS, dout, SCALE, i32(np.arange(B + 1), dev), 0, None, 1, B, pages, ws)
    torch.cuda.synchronize()
    ok, err = close(bits(out[last]), bits(dout), what="c4 last rows, prefill vs decode kernel")
    assert ok, f"prefill last rows vs decode: {err}"
    # (2) 4 rows in every 64-row query tile of every sequence against the
    # oracle's prefill (groups of 8 rows run in parallel on host pages)
    rng = np.random.default_rng(12)
    tiles = N // 64
    picks = np.sort(np.stack([rng.choice(64, 4, replace=False) + 64 * j for j in range(tiles)]).reshape(-1))
    kc_h, vc_h, bt_h, _ = host_pages(kc, vc, bt, np.full(B, per_seq))
    q_h, qkv_h = bits(q), bits(qkv)
    groups = [(s, cu[s] + picks[i:i + 8]) for s in range(B) for i in range(0, len(picks), 8)]

    def one(g):
        s, rows = g
        return rows, oracle.attn_prefill(np.ascontiguousarray(q_h[rows]), kc_h, vc_h,
                                         np.ascontiguousarray(qkv_h[rows]), qstride, Hq, Hkv, pos[rows],
                                         np.array([0, len(rows)], np.int32), 1, np.ascontiguousarray(bt_h[s:s + 1]),
                                         mb, BS, SCALE, threads=1)

    rows_all = np.concatenate([g[1] for g in groups])
    want = np.zeros((len(rows_all), Hq, D), np.uint16)
    at = 0
    for rows, o in run_threads(one, groups):
        want[at:at + len(rows)] = o
        at += len(rows)
    got = bits(out)[rows_all]
    assert len(rows_all) == 1024
    ok, err = close(got, want, what="c4 through the KV manager, 1024 rows (4 per tile, all 8 x 32 tiles)")
    assert ok, f"sampled rows vs oracle: {err}"

"""GPU parity: paged decode attention through the C-ABI against the oracle.

Tolerance (north star): bf16 outputs within max-abs 2e-3 and relative 1e-2 of
the oracle, i.e. |got - want| <= 2e-3 + 1e-2 * |want| elementwise. Oracle-sized
cases compare every output; the full batch-64 configuration is checked
through properties that do not need the oracle (page placement invariance,
split-configuration invariance, constant-V closed form)."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits, bits, close, decode_case, hash_bf16, host_pages, nan_stale, oracle_decode_rows
from pkv import synth

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0


def dev_i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def dev_i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def run_gpu(c, dev, cu=None, skip=0, outs=None, spec=1, out_init=None, T=None):
    T = len(c["pos"]) if T is None else T
    q, kc, vc, qkv = (dev_i16(c[k], dev) for k in ("q", "kc", "vc", "qkv"))
    pos, ts, bt = dev_i32(c["pos"], dev), dev_i32(c["tok_seq"], dev), dev_i32(c["bt"], dev)
    cu_d = dev_i32(c["cu"] if cu is None else cu, dev)
    outs_d = None if outs is None else dev_i32(outs, dev)
    out = (torch.zeros(T, c["Hq"], D, dtype=torch.int16, device=dev) if out_init is None
           else dev_i16(out_init, dev))
    ws = torch.empty(pkv.attn_decode_workspace(T, c["Hq"]), dtype=torch.uint8, device=dev)
    pkv.attn_decode(q, kc, vc, qkv, c["qstride"], c["Hq"], c["Hkv"], pos, ts, bt, c["max_blocks"], BS, out, SCALE,
                    cu_d, skip, outs_d, spec, T, c["pages"], ws)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


def run_oracle(c, **kw):
    out, _ = oracle.attn_decode(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"],
                                c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, **kw)
    return out


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)


@pytest.mark.parametrize("lens,Hkv,seed", [
    ([1, 2, 15, 16, 17], 4, 0),          # page edges, single key
    ([200, 37, 150, 3], 2, 1),           # config 1 restated in bf16 (Hkv 2, G 4)
    ([4097], 4, 2),                      # config 2 shape (one sequence, 4096 + 1 keys)
    ([513, 8193, 1000, 4000, 777, 64], 4, 3),
    ([33] * 40, 4, 4),                   # many short sequences per range
    ([300, 5000], 8, 5),                 # two kv-head groups (Hkv 8)
    ([700] * 24, 4, 9),                  # one-wave merge blocks at its bound (24 x 16 heads, ~12 records each)
    ([700] * 16, 4, 10),                 # merge blocks of 4 waves (16 x 16 heads, ~17 records each)
])
def test_decode_matches_oracle(dev, lens, Hkv, seed):
    print(f"case decode lens={lens[:6]} Hkv={Hkv} seed={seed}", flush=True)
    c = decode_case(lens, 4 * Hkv, Hkv, seed)
    got = run_gpu(c, dev)
    want = run_oracle(c)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("lens,wg,mr", [([1, 2, 15, 17, 33], 1, 32), ([4097, 40], 4, 16), ([513, 8193, 1000], 1, 32)])
def test_decode_stale_slots_are_nan(dev, lens, wg, mr):
    """Slots holding no key (past each length in its last page, unused
    pages) are NaN in K and V; masked keys must not reach the output, not
    even as 0 x NaN, whole-token or split over ranges."""
    print(f"case decode NaN stale slots lens={lens} wg={wg} mr={mr}", flush=True)
    pkv.attn_decode_config(wg, mr)
    c = nan_stale(decode_case(lens, 16, 4, 12), lens)
    got = run_gpu(c, dev)
    want = run_oracle(c)
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_decode_bench_attn_inputs_reversed_table(dev):
    """The reference's bench-attn --check inputs (main.rs:739-763): hash-based
    bf16 in [-1, 1] and each sequence's blocks in reverse order."""
    print("case decode bench-attn inputs", flush=True)
    Hq, Hkv, seqs, ctx = 16, 4, 3, 700
    L = ctx + 1
    mb = (L + BS - 1) // BS
    slots = seqs * mb * BS
    qstride = (2 * Hq + 2 * Hkv) * D
    bt = np.array([[s * mb + mb - 1 - b for b in range(mb)] for s in range(seqs)], np.int32)
    c = dict(q=hash_bf16(seqs * Hq * D, 1).reshape(seqs, Hq, D), qkv=hash_bf16(seqs * qstride, 2).reshape(seqs, -1),
             kc=hash_bf16(slots * Hkv * D, 3).reshape(slots, Hkv, D),
             vc=hash_bf16(slots * Hkv * D, 4).reshape(slots, Hkv, D), qstride=qstride, bt=bt, max_blocks=mb,
             pages=seqs * mb, pos=np.full(seqs, ctx, np.int32), tok_seq=np.arange(seqs, dtype=np.int32),
             cu=np.arange(seqs + 1, dtype=np.int32), Hq=Hq, Hkv=Hkv)
    ok, err = close(run_gpu(c, dev), run_oracle(c))
    assert ok, err


def test_decode_skip_prompts_and_spec_rows(dev):
    """Prompt rows are left untouched with skip_prompts; verifying rows
    (outs >= 0) are decoded, each with its own causal length."""
    print("case decode skip/spec", flush=True)
    c = decode_case([100, 120, 90], 16, 4, seed=7)
    pos = np.array([99, 100, 101, 60, 61, 62], np.int32)
    tok_seq = np.array([0, 1, 1, 2, 2, 2], np.int32)
    cu = np.array([0, 1, 3, 6], np.int32)
    outs = np.array([-1, -1, 5], np.int32)
    q = np.concatenate([c["q"], c["q"], c["q"]])[:6]
    qkv = np.concatenate([c["qkv"], c["qkv"]])[:6]
    c2 = dict(c, q=q, qkv=qkv, pos=pos, tok_seq=tok_seq)
    init = np.full((6, 16, D), 0x7777, np.uint16)
    got = run_gpu(c2, dev, cu=cu, skip=1, outs=outs, spec=1, out_init=init)
    want = run_oracle(c2, cu=cu, skip_prompts=1, outs=outs, spec=1, out=init.copy())
    assert (got[1:3] == 0x7777).all()
    ok, err = close(got, want)
    assert ok, err


@pytest.mark.parametrize("wg,mr", [(1, 16), (4, 64), (8, 16), (2, 100000)])
def test_decode_split_configuration_invariance(dev, wg, mr):
    """Outputs do not depend on how the keys are cut into ranges (one range
    per token with min_range 100000 is the unsplit computation)."""
    print(f"case decode config wg={wg} mr={mr}", flush=True)
    c = decode_case([1000, 3000, 17, 2048], 16, 4, seed=8)
    want = run_oracle(c)
    pkv.attn_decode_config(wg, mr)
    got = run_gpu(c, dev)
    ok, err = close(got, want)
    assert ok, err


def test_decode_c3_batch64_properties(dev):
    """Config 3 at full size (B = 64, contexts U[512, 8192], pages scattered
    over a 65,536-page pool): (1) moving every page to another place in the
    pool and rewriting the tables leaves the outputs bit-identical; (2) with
    V constant per (kv head, dim), the output is bf16(rbf(v) * sigmoid(gate))
    exactly up to f32 rounding of sum(p v) / sum(p); (3) all 64
    sequences match the oracle (every row)."""
    print("case decode c3 full", flush=True)
    Hq, Hkv, pages = 16, 4, 65536
    lens = synth.c3_lengths(seed=9)
    meta = synth.decode_meta(lens, pages, steps=1, seed=9)
    st = meta.step(0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    kc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    B = meta.B
    q = (torch.randn(B, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = synth.qkv_stride(Hq, Hkv)
    qkv = torch.randn(B, qstride, device=dev, generator=gen).to(torch.bfloat16)
    pos, ts, cu = dev_i32(st["pos"], dev), dev_i32(st["tok_seq"], dev), dev_i32(st["cu"], dev)
    bt = dev_i32(meta.block_table, dev)
    ws = torch.empty(pkv.attn_decode_workspace(B, Hq), dtype=torch.uint8, device=dev)

    def run(kc_, vc_, bt_):
        out = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
        pkv.attn_decode(q, kc_, vc_, qkv, qstride, Hq, Hkv, pos, ts, bt_, meta.max_blocks, BS, out, SCALE, cu, 0,
                        None, 1, B, pages, ws)
        torch.cuda.synchronize()
        return out

    out0 = run(kc, vc, bt)
    # (1) page placement invariance: page p moves to perm[p]
    perm = torch.randperm(pages, device=dev, generator=gen)
    kc2 = torch.empty_like(kc)
    vc2 = torch.empty_like(vc)
    kc2.view(pages, BS, Hkv, D)[perm] = kc.view(pages, BS, Hkv, D)
    vc2.view(pages, BS, Hkv, D)[perm] = vc.view(pages, BS, Hkv, D)
    bt2 = perm.to(torch.int32)[bt.long()]
    out1 = run(kc2, vc2, bt2)
    assert torch.equal(out0.view(torch.int16), out1.view(torch.int16))
    del kc2, vc2
    # (3) every row (64 tokens x 16 heads) against the oracle, on host
    # copies of the pages the sequences use, rows run in parallel
    need = (st["pos"] + BS) // BS
    kc_h, vc_h, bt_h, _ = host_pages(kc, vc, meta.block_table, need)
    want = oracle_decode_rows(bits(q), kc_h, vc_h, bits(qkv), qstride, Hq, Hkv, st["pos"], st["tok_seq"], bt_h,
                              meta.max_blocks, SCALE)
    del kc_h, vc_h
    ok, err = close(bits(out0), want, what="c3 full batch, all 64 x 16 rows")
    assert ok, err
    # (2) constant V per (kv head, dim)
    row = (torch.randn(Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    vc.copy_(row.expand_as(vc))
    out2 = run(kc, vc, bt).float()
    gate = qkv[:, :Hq * 2 * D].view(B, Hq, 2, D)[:, :, 1, :].float()
    vrow = row.float().repeat_interleave(4, 0)  # q head h reads kv head h // 4
    want2 = (vrow[None] / (1 + torch.exp(-gate))).to(torch.bfloat16).float()
    err = (out2 - want2).abs().max().item()
    assert err <= 2e-3 + 1e-2 * want2.abs().max().item(), err

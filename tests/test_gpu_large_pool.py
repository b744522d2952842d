"""Pools past 4 GiB. The kernels address a cache page by a 64-bit page base
(buffer descriptors, LDS-DMA bases) plus 32-bit offsets inside the page, so
sequences whose pages sit at the top of a pool of 262,144 + 1,024 pages
(8.6 GB per bf16 pool, 4.3 GB per E4M3 pool) must read exactly what they
read from a compact pool: the outputs are compared bit for bit. Each case
moves a small step's pages (decode, G = 6 decode on the verify kernel, E4M3
decode, bf16 and E4M3 prompts) to the pool's last page ids, in reverse
order."""
import numpy as np
import pytest
import torch

import pkv
from _util import BS, D, decode_case
from test_gpu_e4m3 import e4m3_cache
from test_gpu_groups import paged_prompt_case

pytestmark = pytest.mark.gpu

BIG = 262144 + 1024
SCALE = 1.0 / 16.0


def t_(a, dev):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


def to_top(pool, pages, dev, dtype=np.uint16):
    """The compact pool `pool` ([pages * BS, Hkv, ...]) placed at the last
    page ids of a BIG-page device pool (page i at BIG - 1 - i); returns the
    device pool and the page-id map."""
    row = pool.shape[1:]
    tdt = torch.int16 if dtype == np.uint16 else (torch.uint8 if dtype == np.uint8 else torch.float32)
    big = torch.empty((BIG * BS,) + row, dtype=tdt, device=dev)
    ids = torch.arange(BIG - 1, BIG - 1 - pages, -1, device=dev)
    big.view((BIG, BS) + row)[ids] = t_(pool, dev).view((pages, BS) + row)
    return big, (BIG - 1 - np.arange(pages)).astype(np.int32)


def remap(bt, ids, lens):
    """Block table rows through the page-id map (entries past a row's pages
    stay as they were: never read)."""
    out = bt.copy()
    for s, L in enumerate(lens):
        n = (L + BS - 1) // BS
        out[s, :n] = ids[bt[s, :n]]
    return out


@pytest.mark.parametrize("G", [4, 6])
def test_decode_top_of_a_large_pool(dev, G):
    print(f"case large pool decode G={G}", flush=True)
    Hkv = 4
    lens = [300, 4097, 17, 1500, 2049]
    c = decode_case(lens, G * Hkv, Hkv, 80 + G)
    T, Hq = len(lens), c["Hq"]
    pos, ts, cu = t_(c["pos"], dev), t_(c["tok_seq"], dev), t_(c["cu"], dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)

    def run(kc, vc, bt, pages):
        out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
        pkv.attn_decode(t_(c["q"], dev), kc, vc, t_(c["qkv"], dev), c["qstride"], Hq, Hkv, pos, ts, t_(bt, dev),
                        c["max_blocks"], BS, out, SCALE, cu, 0, None, 1, T, pages, ws)
        torch.cuda.synchronize()
        return out.cpu()

    want = run(t_(c["kc"], dev), t_(c["vc"], dev), c["bt"], c["pages"])
    kb, ids = to_top(c["kc"], c["pages"], dev)
    vb, _ = to_top(c["vc"], c["pages"], dev)
    got = run(kb, vb, remap(c["bt"], ids, lens), BIG)
    del kb, vb
    assert torch.equal(got, want)


def test_decode_e4m3_top_of_a_large_pool(dev):
    print("case large pool decode e4m3", flush=True)
    Hkv = 4
    lens = [300, 4097, 17, 1500, 2049]
    c = decode_case(lens, 16, Hkv, 90)
    T, Hq = len(lens), c["Hq"]
    rng = np.random.default_rng(91)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    pos, ts, cu = t_(c["pos"], dev), t_(c["tok_seq"], dev), t_(c["cu"], dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)

    def run(kc, vc, ksc, vsc, bt, pages):
        out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
        pkv.attn_decode_e4m3(t_(c["q"], dev), kc, vc, ksc, vsc, t_(c["qkv"], dev), c["qstride"], Hq, Hkv, pos, ts,
                             t_(bt, dev), c["max_blocks"], BS, out, SCALE, cu, 0, None, 1, T, pages, ws)
        torch.cuda.synchronize()
        return out.cpu()

    want = run(t_(k8, dev), t_(v8, dev), t_(ks, dev), t_(vs, dev), c["bt"], c["pages"])
    kb, ids = to_top(k8, c["pages"], dev, np.uint8)
    vb, _ = to_top(v8, c["pages"], dev, np.uint8)
    ksb, _ = to_top(ks, c["pages"], dev, np.float32)
    vsb, _ = to_top(vs, c["pages"], dev, np.float32)
    got = run(kb, vb, ksb, vsb, remap(c["bt"], ids, lens), BIG)
    del kb, vb
    assert torch.equal(got, want)


@pytest.mark.parametrize("e4m3", [False, True])
def test_prefill_top_of_a_large_pool(dev, e4m3):
    print(f"case large pool prefill e4m3={e4m3}", flush=True)
    G, Hkv = 4, 4
    ctxs, chunks = [100, 0, 37], [70, 33, 130]
    c = paged_prompt_case(ctxs, chunks, Hkv, G, BS, 95)
    lens = [a + b for a, b in zip(ctxs, chunks)]
    T, Hq = c["T"], c["Hq"]
    pos, cu = t_(c["pos"], dev), t_(c["cu"], dev)

    def run(pools, bt, pages):
        out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
        if e4m3:
            kc, vc, ksc, vsc = pools
            pkv.attn_prefill_e4m3(t_(c["q"], dev), kc, vc, ksc, vsc, t_(c["qkv"], dev), c["qstride"], Hq, Hkv, pos,
                                  cu, c["seqs"], t_(bt, dev), c["max_blocks"], BS, out, SCALE, None, 1, T, pages)
        else:
            kc, vc = pools
            pkv.attn_prefill(t_(c["q"], dev), kc, vc, t_(c["qkv"], dev), c["qstride"], Hq, Hkv, pos, cu, c["seqs"],
                             t_(bt, dev), c["max_blocks"], BS, out, SCALE, None, 1, T, pages)
        torch.cuda.synchronize()
        return out.cpu()

    if e4m3:
        rng = np.random.default_rng(96)
        k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
        ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
        vs = (rng.random(c["vc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
        want = run((t_(k8, dev), t_(v8, dev), t_(ks, dev), t_(vs, dev)), c["bt"], c["pages"])
        kb, ids = to_top(k8, c["pages"], dev, np.uint8)
        vb, _ = to_top(v8, c["pages"], dev, np.uint8)
        ksb, _ = to_top(ks, c["pages"], dev, np.float32)
        vsb, _ = to_top(vs, c["pages"], dev, np.float32)
        got = run((kb, vb, ksb, vsb), remap(c["bt"], ids, lens), BIG)
    else:
        want = run((t_(c["kc"], dev), t_(c["vc"], dev)), c["bt"], c["pages"])
        kb, ids = to_top(c["kc"], c["pages"], dev)
        vb, _ = to_top(c["vc"], c["pages"], dev)
        got = run((kb, vb), remap(c["bt"], ids, lens), BIG)
    del kb, vb
    assert torch.equal(got, want)

"""GPU: the host KV manager driving the device path — copy-on-write of a
shared partial page (pkv_kv_prepare_write + pkv_page_copy + pkv_append) and
speculative rollback (pkv_kv_truncate) — bit-exact against the same
operations on the oracle's host copy of the pool, and decode attention over
the resulting tables within the north-star tolerance (max-abs 2e-3,
rel 1e-2)."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits, close

pytestmark = pytest.mark.gpu
HKV, HQ = 4, 16
ROW = HKV * D  # elements per slot row
PAGE_BYTES = BS * ROW * 2


def i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


class Pools:
    """Device pools and their host mirror, updated by the same operations."""

    def __init__(self, pages, dev, seed):
        rng = np.random.default_rng(seed)
        self.kh = bf16_bits(rng.standard_normal((pages * BS, HKV, D)) * 0.5)
        self.vh = bf16_bits(rng.standard_normal((pages * BS, HKV, D)) * 0.5)
        self.kd, self.vd = i16(self.kh, dev), i16(self.vh, dev)
        self.pages, self.dev = pages, dev

    def copy_pages(self, src, dst):
        if not src:
            return
        pkv.page_copy(self.kd, self.vd, i32(src, self.dev), i32(dst, self.dev), len(src), PAGE_BYTES, self.pages)
        oracle.page_copy(self.kh, self.vh, src, dst, PAGE_BYTES)

    def append(self, rows_k, rows_v, slots):
        T = len(slots)
        kd, vd = i16(rows_k, self.dev), i16(rows_v, self.dev)
        pkv.append(kd, vd, ROW * 2, i32(slots, self.dev), T, HKV, D * 2, self.kd, self.vd, self.pages * BS)
        oracle.append(rows_k.reshape(T, -1), rows_v.reshape(T, -1), slots, self.kh.reshape(-1, ROW),
                      self.vh.reshape(-1, ROW))

    def gather(self, blocks, L):
        bt = i32(blocks, self.dev)
        ko = torch.empty(L, HKV, D, dtype=torch.int16, device=self.dev)
        vo = torch.empty_like(ko)
        pkv.gather(self.kd, self.vd, bt, L, BS, HKV, D * 2, self.pages, ko, vo)
        torch.cuda.synchronize()
        return ko.cpu().numpy().view(np.uint16), vo.cpu().numpy().view(np.uint16)

    def synced(self):
        torch.cuda.synchronize()
        return (np.array_equal(self.kd.cpu().numpy().view(np.uint16), self.kh) and
                np.array_equal(self.vd.cpu().numpy().view(np.uint16), self.vh))


def test_copy_on_write_of_shared_partial_page(dev):
    print("case kv cow", flush=True)
    rng = np.random.default_rng(1)
    pools = Pools(32, dev, 1)
    kv = pkv.Kv(32, BS)
    a = kv.new_seq()
    kv.reserve(a, 40)
    # a writes 40 tokens
    slots = np.array([kv.blocks(a)[p // BS] * BS + p % BS for p in range(40)], np.int32)
    pools.append(bf16_bits(rng.standard_normal((40, HKV, D))), bf16_bits(rng.standard_normal((40, HKV, D))), slots)
    kv.set_len(a, 40)
    before_a = pools.gather(kv.blocks(a), 40)
    # b shares the 40-token prefix (2 full pages + a partial one), then writes position 40
    b = kv.new_seq()
    kv.share(b, a, 40)
    src, dst = kv.prepare_write(b, 40, 1)
    assert len(src) == 1 and src[0] == kv.blocks(a)[2]
    pools.copy_pages(src, dst)
    kb = bf16_bits(rng.standard_normal((1, HKV, D)))
    vb = bf16_bits(rng.standard_normal((1, HKV, D)))
    slot_b = kv.blocks(b)[2] * BS + 40 % BS
    pools.append(kb, vb, np.array([slot_b], np.int32))
    kv.set_len(b, 41)
    # a is untouched; b holds a's 40 tokens then its own
    assert all(np.array_equal(x, y) for x, y in zip(pools.gather(kv.blocks(a), 40), before_a))
    gk, gv = pools.gather(kv.blocks(b), 41)
    assert np.array_equal(gk[:40], before_a[0]) and np.array_equal(gv[:40], before_a[1])
    assert np.array_equal(gk[40], kb[0]) and np.array_equal(gv[40], vb[0])
    assert pools.synced()
    # decode attention over both tables (b's through the copied page)
    m = kv.fill([(a, 0), (b, 0)], max_tokens=2, max_blocks=4)
    pos = np.array([39, 40], np.int32)
    q = bf16_bits(rng.standard_normal((2, HQ, D)) * 0.5)
    qstride = (2 * HQ + 2 * HKV) * D
    qkv = bf16_bits(rng.standard_normal((2, qstride)))
    out = torch.zeros(2, HQ, D, dtype=torch.int16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(2, HQ), dtype=torch.uint8, device=dev)
    pkv.attn_decode(i16(q, dev), pools.kd, pools.vd, i16(qkv, dev), qstride, HQ, HKV, i32(pos, dev),
                    i32([0, 1], dev), i32(m["block_table"], dev), 4, BS, out, 1 / 16, i32([0, 1, 2], dev), 0, None,
                    1, 2, pools.pages, ws)
    torch.cuda.synchronize()
    want, _ = oracle.attn_decode(q, pools.kh, pools.vh, qkv, qstride, HQ, HKV, pos, np.array([0, 1]),
                                 m["block_table"], 4, BS, 1 / 16)
    ok, err = close(out.cpu().numpy().view(np.uint16), want)
    assert ok, err


@pytest.mark.parametrize("accepted,free_pages", [(0, False), (2, True), (3, False)])
def test_verify_then_truncate(dev, accepted, free_pages):
    """A sequence at 62 tokens appends 1 + 3 draft tokens (positions 62..65,
    crossing a page), runs the fused verify step (each position attends
    causally), accepts `accepted` drafts and truncates to 63 + accepted. The
    kept positions' K/V are byte-identical after truncation; with page
    freeing, pages wholly past the new length return to the pool."""
    print(f"case kv verify+truncate accepted={accepted} free={free_pages}", flush=True)
    rng = np.random.default_rng(2 + accepted)
    pools = Pools(16, dev, 2)
    kv = pkv.Kv(16, BS)
    s, _ = kv.admit(list(range(1, 63)), 10)  # reserves ceil(72 / 16) = 5 pages
    slots = np.array([kv.blocks(s)[p // BS] * BS + p % BS for p in range(62)], np.int32)
    pools.append(bf16_bits(rng.standard_normal((62, HKV, D))), bf16_bits(rng.standard_normal((62, HKV, D))), slots)
    kv.set_len(s, 62)
    T = 4
    m = kv.fill([(s, T)], max_tokens=T, max_blocks=8)
    qstride = (2 * HQ + 2 * HKV) * D
    qkv = bf16_bits(rng.standard_normal((T, qstride)) * 0.5)
    q = bf16_bits(rng.standard_normal((T, HQ, D)) * 0.5)
    out = torch.zeros(T, HQ, D, dtype=torch.int16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, HQ), dtype=torch.uint8, device=dev)
    qkv_d = i16(qkv, dev)
    k_rows = qkv_d.data_ptr() + 2 * (2 * HQ * D)
    v_rows = k_rows + 2 * HKV * D
    pkv.attn_decode_step(k_rows, v_rows, qstride * 2, i32(m["slot_map"], dev), i16(q, dev), pools.kd, pools.vd,
                         qkv_d, qstride, HQ, HKV, i32(m["pos"], dev), i32(m["tok_seq"], dev),
                         i32(m["block_table"], dev), 8, BS, out, 1 / 16, i32(m["cu"], dev), 0, i32([0], dev), 1, T,
                         pools.pages, ws)
    oracle.append(np.ascontiguousarray(qkv[:, 2 * HQ * D:2 * HQ * D + ROW]),
                  np.ascontiguousarray(qkv[:, 2 * HQ * D + ROW:2 * HQ * D + 2 * ROW]), m["slot_map"],
                  pools.kh.reshape(-1, ROW), pools.vh.reshape(-1, ROW))
    assert pools.synced()
    want, _ = oracle.attn_decode(q, pools.kh, pools.vh, qkv, qstride, HQ, HKV, m["pos"], m["tok_seq"],
                                 m["block_table"], 8, BS, 1 / 16, cu=m["cu"], skip_prompts=0,
                                 outs=np.array([0], np.int32), spec=1)
    ok, err = close(out.cpu().numpy().view(np.uint16), want)
    assert ok, err
    kv.set_len(s, 62 + T)
    keep = 63 + accepted
    before = pools.gather(kv.blocks(s), keep)
    free0 = kv.free_count()
    kv.truncate(s, keep, free_pages=free_pages)
    after = pools.gather(kv.blocks(s), keep)
    assert all(np.array_equal(x, y) for x, y in zip(before, after))
    n_pages = -(-keep // BS)
    assert len(kv.blocks(s)) == (n_pages if free_pages else 5)
    assert kv.free_count() == free0 + (5 - n_pages if free_pages else 0)

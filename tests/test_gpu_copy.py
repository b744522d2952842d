"""GPU parity: append, gather and page copy through the C-ABI, bit-exact
against the oracle (oracle/pkv_oracle.c)."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def as_i16(a):
    return np.ascontiguousarray(a).view(np.int16)


def test_c1_plumbing_append_gather_f32(dev):
    """Config 1: Hkv 2, head_dim 64, f32, page 16; 4 sequences of U[1, 200]
    tokens; tables from a seeded permutation of a 64-page pool; append all,
    gather back bit-exact, then single-query attention of each sequence's
    last token over its gathered rows on the GPU (pkv_attn_dense_f32)
    against the oracle's fp64 attention over the paged cache: within 1e-5
    absolute + 1e-5 relative (f32 scores, exp and sums against fp64)."""
    print("case c1 f32 append/gather", flush=True)
    rng = np.random.default_rng(11)
    Hkv, Dh, pages = 2, 64, 64
    lens = rng.integers(1, 201, size=4)
    perm = rng.permutation(pages).astype(np.int32)
    mb = 13
    bt = np.zeros((4, mb), np.int32)
    at = 0
    for s, L in enumerate(lens):
        n = (L + BS - 1) // BS
        bt[s, :n] = perm[at:at + n]
        at += n
    kc_d = torch.zeros(pages * BS, Hkv, Dh, dtype=torch.float32, device=dev)
    vc_d = torch.zeros_like(kc_d)
    kc_h = np.zeros((pages * BS, Hkv, Dh), np.float32)
    vc_h = np.zeros_like(kc_h)
    data = []
    for s, L in enumerate(lens):
        k = rng.standard_normal((L, Hkv, Dh)).astype(np.float32)
        v = rng.standard_normal((L, Hkv, Dh)).astype(np.float32)
        slot = (bt[s, np.arange(L) // BS] * BS + np.arange(L) % BS).astype(np.int32)
        kd, vd, sd = to_dev(k, dev), to_dev(v, dev), to_dev(slot, dev)
        pkv.append(kd, vd, Hkv * Dh * 4, sd, int(L), Hkv, Dh * 4, kc_d, vc_d, pages * BS)
        oracle.append(k, v, slot, kc_h, vc_h)
        data.append((k, v))
    torch.cuda.synchronize()
    assert np.array_equal(kc_d.cpu().numpy(), kc_h) and np.array_equal(vc_d.cpu().numpy(), vc_h)
    dense = []
    for s, L in enumerate(lens):
        ko = torch.empty(L, Hkv, Dh, dtype=torch.float32, device=dev)
        vo = torch.empty_like(ko)
        btd = to_dev(bt[s], dev)
        pkv.gather(kc_d, vc_d, btd, int(L), BS, Hkv, Dh * 4, pages, ko, vo)
        torch.cuda.synchronize()
        assert np.array_equal(ko.cpu().numpy(), data[s][0]) and np.array_equal(vo.cpu().numpy(), data[s][1])
        dense.append((ko, vo))
    k_all = torch.cat([d[0] for d in dense]).contiguous()
    v_all = torch.cat([d[1] for d in dense]).contiguous()
    off = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    for Hq in (2, 8):
        q = rng.standard_normal((4, Hq, Dh)).astype(np.float32)
        out = torch.full((4, Hq, Dh), float("nan"), device=dev)
        pkv.attn_dense_f32(to_dev(q, dev), k_all, v_all, to_dev(off, dev), to_dev(lens.astype(np.int32), dev), 4, Hq,
                           Hkv, Dh, 0.125, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for s, L in enumerate(lens):
            want = oracle.attn_single(q[s], kc_h, vc_h, Dh, Hq, Hkv, bt[s], int(L), BS, 0.125)
            err = np.abs(got[s] - want)
            assert (err <= 1e-5 + 1e-5 * np.abs(want)).all(), (Hq, s, float(err.max()))


@pytest.mark.parametrize("T,Hkv", [(1, 4), (64, 4), (513, 4), (7, 8), (130, 16), (3, 2)])
def test_append_bf16_from_qkv_rows_with_padding(dev, T, Hkv):
    """Append K/V straight out of qkv projection rows (stride (2Hq + 2Hkv)
    * 256 elements), with padding rows (slot -1), slots past the pool and
    ragged T (token counts that do not fill the whole-row kernel's blocks of
    4); rows of 2, 4 and 8 KiB take the whole-row kernel, 1 KiB the generic
    one."""
    print(f"case append bf16 T={T} Hkv={Hkv}", flush=True)
    rng = np.random.default_rng(T)
    Hq, pages = 4 * Hkv, 128
    qstride = (2 * Hq + 2 * Hkv) * D
    qkv = bf16_bits(rng.standard_normal((T, qstride)))
    slots = rng.permutation(pages * BS)[:T].astype(np.int32)
    slots[rng.random(T) < 0.1] = -1
    if T > 2:
        slots[1] = pages * BS + 5  # past the pool: skipped like padding
    kc_h = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)))
    vc_h = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)))
    kc_d, vc_d = to_dev(as_i16(kc_h), dev), to_dev(as_i16(vc_h), dev)
    qkv_d, sl_d = to_dev(as_i16(qkv), dev), to_dev(slots, dev)
    k_off, v_off = 2 * Hq * D, 2 * Hq * D + Hkv * D
    pkv.append(qkv_d.data_ptr() + 2 * k_off, qkv_d.data_ptr() + 2 * v_off, qstride * 2, sl_d, T, Hkv, D * 2,
               kc_d, vc_d, pages * BS)
    k_rows = np.ascontiguousarray(qkv[:, k_off:k_off + Hkv * D])
    v_rows = np.ascontiguousarray(qkv[:, v_off:v_off + Hkv * D])
    # the C-ABI skips slots outside the pool; the oracle takes them as padding
    oracle.append(k_rows, v_rows, np.where(slots < pages * BS, slots, -1), kc_h, vc_h)
    torch.cuda.synchronize()
    assert np.array_equal(kc_d.cpu().numpy().view(np.uint16), kc_h)
    assert np.array_equal(vc_d.cpu().numpy().view(np.uint16), vc_h)


def test_append_out_of_pool_slot_is_skipped(dev):
    print("case append out-of-pool", flush=True)
    kc = torch.zeros(32, 4, dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    k = torch.ones(3, 4, dtype=torch.float32, device=dev)
    slots = torch.tensor([1, 32, 1 << 30], dtype=torch.int32, device=dev)
    pkv.append(k, k, 16, slots, 3, 1, 16, kc, vc, 32)
    torch.cuda.synchronize()
    assert kc.sum().item() == 4 and vc.sum().item() == 4


def test_gather_odd_row_bytes(dev):
    """Rows that are not a multiple of 16 bytes use the narrow copy paths."""
    print("case gather odd rows", flush=True)
    rng = np.random.default_rng(3)
    pages, Hkv, hb = 6, 3, 6  # 18-byte rows -> 2-byte aligned, byte copies
    kc = rng.integers(0, 255, size=(pages * BS, Hkv * hb), dtype=np.uint8)
    vc = rng.integers(0, 255, size=(pages * BS, Hkv * hb), dtype=np.uint8)
    bt = np.array([4, 0, 5], np.int32)
    L = 40
    ko = torch.empty(L, Hkv * hb, dtype=torch.uint8, device=dev)
    vo = torch.empty_like(ko)
    pkv.gather(to_dev(kc, dev), to_dev(vc, dev), to_dev(bt, dev), L, BS, Hkv, hb, pages, ko, vo)
    torch.cuda.synchronize()
    wk, wv = oracle.gather(kc, vc, bt, L, BS)
    assert np.array_equal(ko.cpu().numpy(), wk) and np.array_equal(vo.cpu().numpy(), wv)


def test_page_copy_bit_exact(dev):
    print("case page copy", flush=True)
    rng = np.random.default_rng(4)
    pages, Hkv = 40, 4
    kc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)))
    vc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)))
    src = np.array([3, 17, 0, 39], np.int32)
    dst = np.array([21, 2, 38, 5], np.int32)
    kd, vd = to_dev(as_i16(kc), dev), to_dev(as_i16(vc), dev)
    page_bytes = BS * Hkv * D * 2
    pkv.page_copy(kd, vd, to_dev(src, dev), to_dev(dst, dev), 4, page_bytes, pages)
    oracle.page_copy(kc, vc, src, dst, page_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy().view(np.uint16), kc)
    assert np.array_equal(vd.cpu().numpy().view(np.uint16), vc)

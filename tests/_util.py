"""Shared builders for the tests (numpy-side synthetic inputs)."""
import numpy as np

D = 256
BS = 16


def bf16_bits(x):
    """float array -> bf16 bits (uint16), round to nearest even."""
    import oracle
    return oracle.f2b(np.asarray(x, np.float32))


def hash_bf16(n, seed, scale=1.0):
    """The reference bench-attn's deterministic inputs (src/main.rs:739-748):
    h = (i ^ seed * 0x9e3779b9) * 2654435761 (64-bit wrapping),
    x = ((h % 2001) / 1000 - 1) * scale, as bf16."""
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = (i ^ np.uint64((seed * 0x9E3779B9) % (1 << 64))) * np.uint64(2654435761)
    x = ((h % np.uint64(2001)).astype(np.float32) / np.float32(1000.0) - np.float32(1.0)) * np.float32(scale)
    return bf16_bits(x)


def decode_case(lens, Hq, Hkv, seed, pages=None, scale_val=0.5, skip=None, spec_rows=None):
    """A decode step: one token per sequence at position len - 1 (its key is
    already in the cache), pages from a seeded permutation; all bf16 bits."""
    rng = np.random.default_rng(seed)
    B = len(lens)
    max_blocks = max((L + BS - 1) // BS for L in lens)
    if pages is None:
        pages = B * max_blocks + 5
    perm = rng.permutation(pages).astype(np.int32)
    bt = np.zeros((B, max_blocks), np.int32)
    at = 0
    for s, L in enumerate(lens):
        n = (L + BS - 1) // BS
        bt[s, :n] = perm[at:at + n]
        at += n
    kc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * scale_val)
    vc = bf16_bits(rng.standard_normal((pages * BS, Hkv, D)) * scale_val)
    q = bf16_bits(rng.standard_normal((B, Hq, D)) * scale_val)
    qstride = (2 * Hq + 2 * Hkv) * D
    qkv = bf16_bits(rng.standard_normal((B, qstride)))
    return dict(q=q, kc=kc, vc=vc, qkv=qkv, qstride=qstride, bt=bt, max_blocks=max_blocks, pages=pages,
                pos=np.array([L - 1 for L in lens], np.int32), tok_seq=np.arange(B, dtype=np.int32),
                cu=np.arange(B + 1, dtype=np.int32), Hq=Hq, Hkv=Hkv)


def close(got_bits, want_bits, atol=2e-3, rtol=1e-2):
    """The north-star attention tolerance on bf16 outputs:
    |got - want| <= atol + rtol * |want| elementwise (max-abs 2e-3, relative 1e-2)."""
    import oracle
    g = oracle.b2f(got_bits).astype(np.float64)
    w = oracle.b2f(want_bits).astype(np.float64)
    err = np.abs(g - w)
    ok = err <= atol + rtol * np.abs(w)
    return bool(ok.all()), float(err.max()) if err.size else 0.0


def used_slots(c, lens):
    """Slots holding a key of a sequence (sequence s has keys
    0 .. lens[s] - 1 through block table row s)."""
    used = np.zeros(c["kc"].shape[0], bool)
    for s, L in enumerate(lens):
        for k in range(int(L)):
            used[c["bt"][s][k // BS] * BS + k % BS] = True
    return used


def nan_stale(c, lens):
    """K / V caches of case c with every slot that holds no key of a
    sequence set to bf16 NaN: stale or never-written slots must not reach
    any output."""
    used = used_slots(c, lens)
    kc, vc = c["kc"].copy(), c["vc"].copy()
    kc[~used] = 0x7FC0
    vc[~used] = 0x7FC0
    return dict(c, kc=kc, vc=vc)

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


ATOL, RTOL = 2e-3, 1e-2

# Every close() call of this process: (test id, what, elements, max-abs,
# max-rel over |want| > ATOL, elements above ATOL); conftest prints them at
# the end of the run.
PARITY_LOG = []
EXPLAIN_LOG = []  # (test, line) of explain_beyond


class Closeness(tuple):
    """(ok, max_abs) plus max_rel (largest |got - want| / |want| over
    elements with |want| > ATOL), max_ulp (largest |got - want| in units of
    the bf16 spacing at want, over the same elements), n (elements compared) and n_either (elements
    beyond both max-abs ATOL and relative RTOL on their own, which the
    additive bound admits)."""

    def __new__(cls, ok, max_abs, max_rel, max_ulp, n, n_either):
        self = super().__new__(cls, (ok, max_abs))
        self.ok, self.max_abs, self.max_rel, self.max_ulp = ok, max_abs, max_rel, max_ulp
        self.n, self.n_either = n, n_either
        return self


def bf16_ulp(w):
    """Spacing of bf16 values at |w| (2^(e - 7) for |w| in [2^e, 2^(e+1)),
    the subnormal spacing below the smallest normal)."""
    a = np.maximum(np.abs(np.asarray(w, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(a)) - 7)


def explain_beyond(got_bits, want_bits, raw, qkv, qstride, Hq, atol=ATOL, rtol=RTOL):
    """For every element beyond both bounds alone (|d| > max(atol, rtol
    |want|)): its (row, head, dim), want, got, the oracle's unrounded output
    o (raw, f32 of the f64 value), its bf16 rounding rbf(o), how far o lies
    from that rounding's nearest tie point (in bf16 ulps of o), and which of
    rbf(o) - 1 ulp, rbf(o), rbf(o) + 1 ulp gives `got` once gated as the
    epilogue does: bf16(rbf * sigmoid(gate)). Returns the lines."""
    import oracle
    g = oracle.b2f(got_bits).astype(np.float64)
    w = oracle.b2f(want_bits).astype(np.float64)
    err = np.abs(g - w)
    idx = np.argwhere(err > np.maximum(atol, rtol * np.abs(w)))
    lines = []
    for t, h, d in idx:
        o = np.float32(raw[t, h, d])
        gate = float(oracle.b2f(np.array([qkv[t, h * 512 + 256 + d]], np.uint16))[0])
        r = float(oracle.b2f(oracle.f2b(np.array([o], np.float32)))[0])
        ulp = float(bf16_ulp(r))
        tie = r + ulp / 2 if o >= r else r - ulp / 2
        which = []
        for k, cand in ((-1, r - ulp), (0, r), (1, r + ulp)):
            y = np.float32(cand) / (np.float32(1) + np.exp(np.float32(-gate), dtype=np.float32))
            if float(oracle.b2f(oracle.f2b(np.array([y], np.float32)))[0]) == g[t, h, d]:
                which.append(k)
        lines.append(f"beyond both: (row {t}, head {h}, dim {d}) want {w[t, h, d]:.6g} got {g[t, h, d]:.6g} "
                     f"|diff| {err[t, h, d]:.3e} rel {err[t, h, d] / abs(w[t, h, d]):.3e}; oracle o {float(o):.8g}, "
                     f"rbf(o) {r:.6g}, |o - tie| {abs(float(o) - tie) / ulp:.4f} ulp, gate {gate:.4g}; got = gated "
                     f"rbf(o) {'/'.join(f'{k:+d}' for k in which) if which else '(none of +-1)'} ulp")
    return lines


def close(got_bits, want_bits, atol=ATOL, rtol=RTOL, what="", explain=None):
    """The north-star attention tolerance on bf16 outputs (max-abs 2e-3,
    relative 1e-2) in the numpy / torch allclose form: every element with
    |got - want| <= atol + rtol * |want|. The additive form is needed by the
    gated epilogue's double rounding: bf16(rbf(o) * sigmoid(gate)) turns a
    one-ulp flip of rbf(o) (an f32 vs f64 accumulation difference at a
    rounding boundary) into two output ulps when the gate moves the value to
    a lower binade. Returns a Closeness (unpacks as ok, max_abs) and logs
    max-abs, max-rel, max ulps and the elements beyond either bound alone."""
    import os

    import oracle
    g = oracle.b2f(got_bits).astype(np.float64)
    w = oracle.b2f(want_bits).astype(np.float64)
    err = np.abs(g - w)
    big = np.abs(w) > atol
    rel = err[big] / np.abs(w[big])
    ok = bool((err <= atol + rtol * np.abs(w)).all()) and not np.isnan(g).any()
    ulps = err[big] / bf16_ulp(w[big])
    r = Closeness(ok, float(err.max()) if err.size else 0.0, float(rel.max()) if rel.size else 0.0,
                  float(ulps.max()) if ulps.size else 0.0, int(err.size),
                  int((err > np.maximum(atol, rtol * np.abs(w))).sum()))
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    PARITY_LOG.append((test, what, r.n, r.max_abs, r.max_rel, r.max_ulp, r.n_either))
    print(f"parity {what}: {r.n} elements, max-abs {r.max_abs:.3e}, max-rel {r.max_rel:.3e} (|want| > {atol}), "
          f"max {r.max_ulp:.0f} ulp, {r.n_either} beyond both bounds alone", flush=True)
    if explain is not None and r.n_either:
        for line in explain_beyond(got_bits, want_bits, atol=atol, rtol=rtol, **explain):
            print(line, flush=True)
            EXPLAIN_LOG.append((test, line))
    return r


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


def oracle_threads():
    """Worker threads for oracle runs: the host's cores, at most 16 (one
    GPU box's CPU share)."""
    import os
    return max(1, min(16, os.cpu_count() or 1))


def balanced_sets(weights, n):
    """Indices 0..len(weights)-1 split into at most n sets of similar total
    weight (heaviest first into the lightest set); each set sorted."""
    sets = [[] for _ in range(max(1, min(n, len(weights))))]
    load = [0] * len(sets)
    for i in sorted(range(len(weights)), key=lambda i: -int(weights[i])):
        j = load.index(min(load))
        sets[j].append(i)
        load[j] += int(weights[i])
    return [np.array(sorted(s), np.int64) for s in sets if s]


def run_threads(fn, items):
    """fn over items on oracle_threads() threads (the oracle's C calls
    release the GIL); results in item order."""
    import concurrent.futures
    with concurrent.futures.ThreadPoolExecutor(oracle_threads()) as ex:
        return list(ex.map(fn, items))


def oracle_decode_rows(q, kc, vc, qkv, qstride, Hq, Hkv, pos, tok_seq, bt, max_blocks, scale, decode8=None):
    """oracle.attn_decode over every row (bf16 bits), rows split into
    key-balanced sets run in parallel; returns out [T][Hq][256] uint16.
    decode8 = (kscale, vscale) runs oracle.attn_decode8 over E4M3 caches."""
    import oracle
    T = len(pos)
    out = np.zeros((T, Hq, D), np.uint16)

    def one(ids):
        args = (np.ascontiguousarray(q[ids]), kc, vc) + ((decode8[0], decode8[1]) if decode8 else ()) + (
            np.ascontiguousarray(qkv[ids]), qstride, Hq, Hkv, np.ascontiguousarray(pos[ids], np.int32),
            np.ascontiguousarray(tok_seq[ids], np.int32), bt, max_blocks, BS, scale)
        if decode8:
            return ids, oracle.attn_decode8(*args, threads=1)
        return ids, oracle.attn_decode(*args, threads=1)[0]  # the sets already run on threads

    for ids, o in run_threads(one, balanced_sets(np.asarray(pos) + 1, 4 * oracle_threads())):
        out[ids] = o
    return out


def host_pages(kc, vc, bt, need):
    """Host copies of the pages sequences use: pages bt[s, :need[s]] of the
    device pools kc / vc ([pages * 16][Hkv][256], any 2-byte or 1-byte
    dtype) gathered once each, with bt remapped to them. Returns (kc_h,
    vc_h, bt_h) as numpy (uint16 for 2-byte pools, uint8 otherwise)."""
    import torch
    rows = [bt[s, :int(n)] for s, n in enumerate(need)]
    sub = np.unique(np.concatenate(rows))
    Hkv, Dd = kc.shape[1], kc.shape[2]
    idx = torch.from_numpy(sub.astype(np.int64)).to(kc.device)

    def grab(c):
        x = c.view(-1, BS, Hkv, Dd)[idx].cpu()
        if x.element_size() == 2:
            return x.view(torch.int16).numpy().view(np.uint16).reshape(-1, Hkv, Dd)
        return x.view(torch.uint8).numpy().reshape(-1, Hkv, Dd)

    where = np.full(int(bt.max()) + 1, -1, np.int64)
    where[sub] = np.arange(len(sub))
    bt_h = np.zeros_like(bt, dtype=np.int32)
    for s, r in enumerate(rows):
        bt_h[s, :len(r)] = where[r]
    return grab(kc), grab(vc), bt_h, sub


def bits(x):
    """A bf16 / int16 device tensor as host uint16 bits."""
    import torch
    return x.cpu().view(torch.int16).numpy().view(np.uint16)


def fp8_buffers(T, K, mode, frows, dev):
    """fq / fs for FP8 output copies, filled with sentinels (0x7F bytes, NaN
    scales, 0xEE exponent bytes) so untouched entries are visible."""
    import torch
    fq = torch.full((T, K), 0x7F, dtype=torch.uint8, device=dev)
    fs = (torch.full((K // 128, frows), float("nan"), device=dev) if mode == 1 else
          torch.full((((frows + 127) // 128) * ((K // 32 + 3) // 4) * 512,), 0xEE, dtype=torch.uint8, device=dev))
    return fq, fs


def check_fp8_copies(fq, fs, y, mode, frows, rows=None):
    """FP8 copies (fq [T][K] E4M3 bytes, fs scales) of f32 outputs y [T][K]
    against the oracle's quantisation of y (oracle.fp8_rows): every element
    dequantises to within one E4M3 step of y (plus the attention tolerance,
    since y is the oracle's own output), > 99 % of bytes identical, scales
    within 1e-2 (f32 Block128 scales within 1e-5 for > 95 % of groups, Mx32
    exponents identical for > 99 %), and rows outside `rows` untouched."""
    import oracle
    T, K = y.shape
    rows = np.arange(T) if rows is None else np.asarray(rows)
    wq, ws = oracle.fp8_rows(y, mode, rows=frows)
    gw = 128 if mode == 1 else 32
    if mode == 1:
        sg, sw = fs[:, :T].T.astype(np.float64), ws[:, :T].T.astype(np.float64)
        untouched = np.isnan(fs[:, [t for t in range(frows) if t not in set(rows.tolist())]])
        assert untouched.all()
    else:
        idx = np.array([[oracle.mx_index(t, kb, K // 32) for kb in range(K // 32)] for t in range(T)])
        sg, sw = 2.0 ** (fs[idx].astype(np.float64) - 127), 2.0 ** (ws[idx].astype(np.float64) - 127)
        mask = np.ones(fs.shape, bool)
        mask[idx[rows].reshape(-1)] = False
        assert (fs[mask] == 0xEE).all()
    sg, sw, fq, wq, y = sg[rows], sw[rows], fq[rows], wq[rows], y[rows]
    deq = oracle.e4m3_to_f(fq).astype(np.float64) * np.repeat(sg, gw, axis=1)
    step = np.repeat(sw, gw, axis=1) * 2.0 ** -9 + np.abs(y) * 2.0 ** -4
    assert (np.abs(deq - y) <= step + np.abs(y) * 2.0 ** -8 + 2e-3 + 1e-2 * np.abs(y)).all()
    assert (fq == wq).mean() > 0.99, (fq == wq).mean()
    rel = np.abs(sg / sw - 1)
    assert (rel <= 1e-2).all()
    assert ((rel <= 1e-5).mean() > 0.95) if mode == 1 else ((sg == sw).mean() > 0.99)

"""CPU oracle for the paged KV cache hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, as the checker (or the timed CPU baseline). The product
(libpkv.so, pocket-engine_amd/pkv) never imports it.

numpy wrappers over liboracle.so (pkv_oracle.c, a scalar C restatement of
the reference's semantics; see the header of that file for the reference
lines each function follows and how each is pinned) plus the allocator
restatement in alloc.py.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build():
    r = subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout + r.stderr)
    return LIB_PATH


if not os.path.exists(LIB_PATH):
    build()
_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_lib.orc_f2b.restype = ctypes.c_uint16
_lib.orc_f2b.argtypes = [_F]
_lib.orc_b2f.restype = _F
_lib.orc_b2f.argtypes = [ctypes.c_uint16]
_lib.orc_append.argtypes = [_P, _P, _L, _P, _I, _I, _I, _P, _P]
_lib.orc_gather.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P, _P]
_lib.orc_page_copy.argtypes = [_P, _P, _P, _P, _I, _L]
_lib.orc_attn_decode.restype = _I
_lib.orc_attn_decode.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _P, _F, _P, _I, _P, _I, _I, _P]
_lib.orc_attn_single.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P, _I, _I, _F, _P]
_lib.orc_split_parts.restype = _I
_lib.orc_split_parts.argtypes = [_I, _I, _I]
_lib.orc_attn_partial.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P, _I, _I, _I, _F, _P, _P, _P]
_lib.orc_merge.argtypes = [_P, _P, _P, _I, _P]
_lib.orc_attn_prefill.restype = _I
_lib.orc_attn_prefill.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P, _I, _P, _I, _I, _P, _F, _P, _I]
_lib.orc_attn_prefill_t.restype = _I
_lib.orc_attn_prefill_t.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P, _I, _P, _I, _I, _P, _F, _P, _I, _I]
_lib.orc_attn_decode_f32.restype = _I
_lib.orc_attn_decode_f32.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _P, _F, _P, _I, _P, _I, _I]
_lib.orc_attn_prefill_part.restype = _I
_lib.orc_attn_prefill_part.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P, _I, _P, _I, _I, _P, _F, _P, _I, _I, _I, _I,
                                       _I, _I]
_lib.orc_dequant_e4m3.restype = None
_lib.orc_dequant_e4m3.argtypes = [_P, _P, _L, _P]
_lib.orc_mtp_slots.argtypes = [_P, _P, _P, _I, _I, _P, _I, _P, _P, _I]
_lib.orc_mtp_next.argtypes = [_P, _P, _P, _I, _P, _I, _I, _P, _I, _P, _P, _P, _I]
_lib.orc_attn_prep.argtypes = [_P, _I, _I, _I, _P, _P, _P, _I, _I, _I, _P, _P, _F, _I, _L, _P, _P, _P]
_lib.orc_e4m3_to_f.restype = _F
_lib.orc_e4m3_to_f.argtypes = [ctypes.c_uint8]
_lib.orc_f_to_e4m3.restype = ctypes.c_uint8
_lib.orc_f_to_e4m3.argtypes = [_F]
_lib.orc_store_e4m3.argtypes = [_P, _P, _P]
_lib.orc_mx_index.restype = ctypes.c_size_t
_lib.orc_mx_index.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
_lib.orc_mx_exp.restype = ctypes.c_int
_lib.orc_mx_exp.argtypes = [_F]
_lib.orc_fp8_rows.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, _P]
_lib.orc_gate_rows.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
_lib.orc_attn_prep8.argtypes = [_P, _I, _I, _I, _P, _P, _P, _I, _I, _I, _P, _P, _F, _I, _L, _P, _P, _P, _P, _P]
_lib.orc_attn_prefill8.restype = _I
_lib.orc_attn_prefill8.argtypes = [_P, _P, _P, _P, _P, _L, _P, _I, _I, _I, _P, _P, _I, _P, _I, _I, _P, _F, _I]
_lib.orc_attn_decode8.restype = _I
_lib.orc_attn_decode8.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _P, _F, _P, _I, _P, _I, _I, _P]


def _p(a):
    """Pointer to a C-contiguous numpy array. The caller keeps the array
    referenced until the C call returns (never pass a temporary)."""
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags.c_contiguous, "oracle takes C-contiguous numpy arrays"
    return a.ctypes.data


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def f2b(x):
    """f32 -> bf16 bits, round to nearest even (numpy, vectorised)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def b2f(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def append(k_src, v_src, slot_map, kcache, vcache):
    """k_src/v_src: [T][row] arrays (any dtype); kcache/vcache: [slots][row]; in place."""
    T = k_src.shape[0]
    row_bytes = k_src[0].nbytes
    slot_map = _i32(slot_map)
    _lib.orc_append(_p(k_src), _p(v_src), row_bytes, _p(slot_map), T, 1, row_bytes, _p(kcache), _p(vcache))


def gather(kcache, vcache, bt_row, L, block_size):
    """Returns dense (k, v) of shape [L] + kcache.shape[1:]."""
    ko = np.empty((L,) + kcache.shape[1:], kcache.dtype)
    vo = np.empty((L,) + vcache.shape[1:], vcache.dtype)
    row_bytes = kcache[0].nbytes
    bt_row = _i32(bt_row)
    _lib.orc_gather(_p(kcache), _p(vcache), _p(bt_row), L, block_size, 1, row_bytes, _p(ko), _p(vo))
    return ko, vo


def page_copy(kcache, vcache, src, dst, page_bytes):
    src, dst = _i32(src), _i32(dst)
    _lib.orc_page_copy(_p(kcache), _p(vcache), _p(src), _p(dst), len(src), page_bytes)


def attn_decode(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks, block_size, scale,
                cu=None, skip_prompts=0, outs=None, spec=1, out=None, threads=None):
    """bf16 (uint16) arrays in; returns (out uint16 [T][Hq][256], o_raw f32).
    threads: host threads over row ranges (None: up to 16)."""
    T = len(pos)
    if out is None:
        out = np.zeros((T, Hq, 256), np.uint16)
    raw = np.zeros((T, Hq, 256), np.float32)
    cu, outs, pos, tok_seq, block_table = _i32(cu), _i32(outs), _i32(pos), _i32(tok_seq), _i32(block_table)
    q, kcache, vcache, qkv = (np.ascontiguousarray(a) for a in (q, kcache, vcache, qkv))
    q, qkv = q.reshape(T, -1), qkv.reshape(T, -1)

    def run(t0, t1):
        qs, qk, ps, ts, os_, rs = q[t0:t1], qkv[t0:t1], pos[t0:t1], tok_seq[t0:t1], out[t0:t1], raw[t0:t1]
        _lib.orc_attn_decode(_p(qs), _p(kcache), _p(vcache), _p(qk), qstride, Hq, Hkv, _p(ps), _p(ts),
                             _p(block_table), max_blocks, block_size, _p(os_), scale, _p(cu), skip_prompts, _p(outs),
                             spec, t1 - t0, _p(rs))

    _row_parts(pos, threads, run)
    return out, raw


def attn_decode_f32(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks, block_size,
                    scale, cu=None, skip_prompts=0, outs=None, spec=1, out=None):
    """orc_attn_decode_f32: the one-pass f32 scalar decode (the CPU
    baseline's f32 leg; the f64 attn_decode is the checker). One thread."""
    T = len(pos)
    if out is None:
        out = np.zeros((T, Hq, 256), np.uint16)
    cu, outs, pos, tok_seq, block_table = _i32(cu), _i32(outs), _i32(pos), _i32(tok_seq), _i32(block_table)
    q, kcache, vcache, qkv = (np.ascontiguousarray(a) for a in (q, kcache, vcache, qkv))
    _lib.orc_attn_decode_f32(_p(q), _p(kcache), _p(vcache), _p(qkv), qstride, Hq, Hkv, _p(pos), _p(tok_seq),
                             _p(block_table), max_blocks, block_size, _p(out), scale, _p(cu), skip_prompts, _p(outs),
                             spec, T)
    return out


def _row_parts(pos, threads, run):
    """Runs run(t0, t1) over contiguous row ranges balanced by attended keys
    (pos + 1), on up to `threads` host threads (None: up to 16; ctypes
    releases the GIL). The decode oracles' rows are independent: a row reads
    only its own q, qkv, pos, tok_seq and writes only its own outputs."""
    T = len(pos)
    if T == 0:
        return
    nthr = max(1, min(threads or 16, os.cpu_count() or 1, T))
    cum = np.concatenate([[0], np.cumsum(np.asarray(pos, np.int64) + 1)])
    tb = sorted(set([0] + [int(np.searchsorted(cum, cum[-1] * i / nthr)) for i in range(1, nthr)] + [T]))
    parts = [(tb[i], tb[i + 1]) for i in range(len(tb) - 1) if tb[i] < tb[i + 1]]
    if len(parts) == 1:
        run(*parts[0])
        return
    import concurrent.futures
    with concurrent.futures.ThreadPoolExecutor(len(parts)) as ex:
        list(ex.map(lambda tt: run(*tt), parts))


def attn_single(q, kcache, vcache, D, Hq, Hkv, bt_row, L, block_size, scale):
    """One query (q: [Hq][D], f32 or bf16-as-uint16) -> f32 [Hq][D], ungated."""
    dtype = 1 if q.dtype == np.float32 else 0
    o = np.zeros((Hq, D), np.float32)
    bt_row = _i32(bt_row)
    _lib.orc_attn_single(_p(q), _p(kcache), _p(vcache), dtype, D, Hq, Hkv, _p(bt_row), L, block_size, scale, _p(o))
    return o


def split_parts(L, Z, min_chunk):
    return _lib.orc_split_parts(L, Z, min_chunk)


def attn_partial(q, kcache, vcache, Hq, Hkv, t, h, bt_row, block_size, j0, j1, scale):
    M = np.zeros(1, np.float64)
    S = np.zeros(1, np.float64)
    A = np.zeros(256, np.float64)
    bt_row = _i32(bt_row)
    _lib.orc_attn_partial(_p(q), _p(kcache), _p(vcache), Hq, Hkv, t, h, _p(bt_row), block_size, j0, j1, scale,
                          _p(M), _p(S), _p(A))
    return M[0], S[0], A


def merge(Ms, Ss, As):
    Ms = np.ascontiguousarray(Ms, np.float64)
    Ss = np.ascontiguousarray(Ss, np.float64)
    As = np.ascontiguousarray(As, np.float64)
    o = np.zeros(256, np.float64)
    _lib.orc_merge(_p(Ms), _p(Ss), _p(As), len(Ms), _p(o))
    return o


P_TILE = 32  # the reference's prefill key tile (AM_BN, amd/attention.cuh:10)


def attn_prefill(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks, block_size, scale,
                 outs=None, spec=1, out=None, p_tile=P_TILE, threads=None):
    """Chunked prefill. p_tile = 32 (default): the reference's tiled softmax
    with P rounded to bf16 for P.V; p_tile = 0: P in double (textbook)."""
    T = len(pos)
    if out is None:
        out = np.zeros((T, Hq, 256), np.uint16)
    pos, cu, block_table, outs = _i32(pos), _i32(cu), _i32(block_table), _i32(outs)
    q, kcache, vcache, qkv = (np.ascontiguousarray(a) for a in (q, kcache, vcache, qkv))
    # (row range, head range) parts, balanced by attended keys, run on
    # threads (ctypes releases the GIL; every part writes its own outputs)
    nthr = max(1, min(threads or 16, os.cpu_count() or 1))
    hparts = min(Hq, nthr)
    hb = [Hq * i // hparts for i in range(hparts + 1)]
    tparts = max(1, min(T, (2 * nthr + hparts - 1) // hparts))
    cum = np.concatenate([[0], np.cumsum(pos.astype(np.int64) + 1)])
    tb = [0] + [int(np.searchsorted(cum, cum[-1] * i / tparts)) for i in range(1, tparts)] + [T]
    jobs = [(tb[i], tb[i + 1], hb[j], hb[j + 1]) for i in range(tparts) for j in range(hparts) if tb[i] < tb[i + 1]]

    def run(job):
        t0, t1, h0, h1 = job
        _lib.orc_attn_prefill_part(_p(q), _p(kcache), _p(vcache), _p(qkv), qstride, Hq, Hkv, _p(pos), _p(cu), seqs,
                                   _p(block_table), max_blocks, block_size, _p(out), scale, _p(outs), spec, p_tile, t0,
                                   t1, h0, h1)

    if len(jobs) == 1:
        run(jobs[0])
    else:
        import concurrent.futures
        with concurrent.futures.ThreadPoolExecutor(min(nthr, len(jobs))) as ex:
            list(ex.map(run, jobs))
    return out


def mtp_slots(rows, pos, block_table, max_blocks, block_size, limits, k):
    S = len(rows)
    dpos = np.zeros(S, np.int32)
    dslot = np.zeros(S, np.int32)
    rows, pos, block_table, limits = _i32(rows), _i32(pos), _i32(block_table), _i32(limits)
    _lib.orc_mtp_slots(_p(rows), _p(pos), _p(block_table), max_blocks, block_size, _p(limits), k, _p(dpos),
                       _p(dslot), S)
    return dpos, dslot


def mtp_next(rows, pos, rope, rope_stride, block_table, max_blocks, block_size, limits, k):
    """(dpos, dslot, drope [3, S]) of draft pass k (qwen35.cu:2633-2650)."""
    S = len(rows)
    dpos = np.zeros(S, np.int32)
    dslot = np.zeros(S, np.int32)
    drope = np.zeros((3, S), np.int32)
    rows, pos, rope, block_table, limits = _i32(rows), _i32(pos), _i32(rope), _i32(block_table), _i32(limits)
    _lib.orc_mtp_next(_p(rows), _p(pos), _p(rope), rope_stride, _p(block_table), max_blocks, block_size, _p(limits), k,
                      _p(dpos), _p(dslot), _p(drope), S)
    return dpos, dslot, drope


def attn_prep(qkv, qstride, Hq, Hkv, q_norm, k_norm, rope, rope_stride, sec_h, sec_w, slot_map, inv_freq, eps,
              qout, kcache, vcache):
    """Reference attn_prep restated (qwen35.cu:1067-1128); writes qout (uint16
    [T][Hq][256]) and the k/v slots of kcache/vcache (uint16) in place."""
    T = len(slot_map)
    qkv = np.ascontiguousarray(qkv, np.uint16)
    q_norm = np.ascontiguousarray(q_norm, np.float32)
    k_norm = np.ascontiguousarray(k_norm, np.float32)
    rope = _i32(rope)
    slot_map = _i32(slot_map)
    inv_freq = np.ascontiguousarray(inv_freq, np.float32)
    num_slots = kcache.size // (max(Hkv, 1) * 256)
    _lib.orc_attn_prep(_p(qkv), qstride, Hq, Hkv, _p(q_norm), _p(k_norm), _p(rope), rope_stride, sec_h, sec_w,
                       _p(slot_map), _p(inv_freq), eps, T, num_slots, _p(qout),
                       _p(kcache), _p(vcache))


def e4m3_to_f(codes):
    """E4M3FN bytes -> float32 (OCP: bias 7, max 448, 0x7F / 0xFF NaN)."""
    codes = np.asarray(codes, np.uint8)
    return np.array([_lib.orc_e4m3_to_f(int(c)) for c in codes.reshape(-1)], np.float32).reshape(codes.shape)


def f_to_e4m3(x):
    """float32 -> E4M3FN bytes, nearest-even, saturating to +-448."""
    x = np.asarray(x, np.float32)
    return np.array([_lib.orc_f_to_e4m3(float(v)) for v in x.reshape(-1)], np.uint8).reshape(x.shape)


def store_e4m3(v):
    """One head's 256 floats -> (bytes, scale) as the reference's store_e4m3."""
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(256, np.uint8)
    sc = np.zeros(1, np.float32)
    _lib.orc_store_e4m3(_p(v), _p(out), _p(sc))
    return out, float(sc[0])


def attn_prep8(qkv, qstride, Hq, Hkv, q_norm, k_norm, rope, rope_stride, sec_h, sec_w, slot_map, inv_freq, eps,
               qout, kcache8, vcache8, kscale, vscale):
    """attn_prep with an E4M3 cache (bytes + f32 scale per slot and kv head)."""
    T = len(slot_map)
    qkv = np.ascontiguousarray(qkv, np.uint16)
    q_norm = np.ascontiguousarray(q_norm, np.float32)
    k_norm = np.ascontiguousarray(k_norm, np.float32)
    rope = _i32(rope)
    slot_map = _i32(slot_map)
    inv_freq = np.ascontiguousarray(inv_freq, np.float32)
    num_slots = kcache8.size // (max(Hkv, 1) * 256)
    _lib.orc_attn_prep8(_p(qkv), qstride, Hq, Hkv, _p(q_norm), _p(k_norm), _p(rope), rope_stride, sec_h, sec_w,
                        _p(slot_map), _p(inv_freq), eps, T, num_slots, _p(qout), _p(kcache8), _p(vcache8),
                        _p(kscale), _p(vscale))


def attn_decode8(q, kcache8, vcache8, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks,
                 block_size, scale, cu=None, skip_prompts=0, outs=None, spec=1, out=None, return_raw=False,
                 threads=None):
    """Decode attention over an E4M3 cache (reference attn_paged8 semantics).
    Returns out, or (out, o_raw f32 ungated) with return_raw. threads: host
    threads over row ranges (None: up to 16)."""
    T = len(pos)
    if out is None:
        out = np.zeros((T, Hq, 256), np.uint16)
    raw = np.zeros((T, Hq, 256), np.float32)
    cu, outs, pos, tok_seq, block_table = _i32(cu), _i32(outs), _i32(pos), _i32(tok_seq), _i32(block_table)
    kscale = np.ascontiguousarray(kscale, np.float32)
    vscale = np.ascontiguousarray(vscale, np.float32)
    q, kcache8, vcache8, qkv = (np.ascontiguousarray(a) for a in (q, kcache8, vcache8, qkv))
    q, qkv = q.reshape(T, -1), qkv.reshape(T, -1)

    def run(t0, t1):
        qs, qk, ps, ts, os_, rs = q[t0:t1], qkv[t0:t1], pos[t0:t1], tok_seq[t0:t1], out[t0:t1], raw[t0:t1]
        _lib.orc_attn_decode8(_p(qs), _p(kcache8), _p(vcache8), _p(kscale), _p(vscale), _p(qk), qstride, Hq, Hkv,
                              _p(ps), _p(ts), _p(block_table), max_blocks, block_size, _p(os_), scale, _p(cu),
                              skip_prompts, _p(outs), spec, t1 - t0, _p(rs))

    _row_parts(pos, threads, run)
    return (out, raw) if return_raw else out


def attn_prefill8(q, kcache8, vcache8, kscale, vscale, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks,
                  block_size, scale, out=None, p_tile=P_TILE, threads=None):
    """Chunked prefill over an E4M3 cache (reference attn_group8)."""
    T = len(pos)
    if out is None:
        out = np.zeros((T, Hq, 256), np.uint16)
    kscale = np.ascontiguousarray(kscale, np.float32)
    vscale = np.ascontiguousarray(vscale, np.float32)
    kcache8, vcache8 = np.ascontiguousarray(kcache8), np.ascontiguousarray(vcache8)
    n = kcache8.size // 256
    kb, vb = np.empty((n, 256), np.uint16), np.empty((n, 256), np.uint16)
    # orc_attn_prefill8's dequantisation, then the bf16 prefill (in parts)
    _lib.orc_dequant_e4m3(_p(kcache8), _p(kscale), n, _p(kb))
    _lib.orc_dequant_e4m3(_p(vcache8), _p(vscale), n, _p(vb))
    return attn_prefill(q, kb, vb, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks, block_size, scale,
                        out=out, p_tile=p_tile, threads=threads)


def mx_index(r, kb, KB):
    """Byte offset of the Mx32 scale of (row r, 32-column block kb)."""
    return _lib.orc_mx_index(r, kb, KB)


def mx_exp(amax):
    return _lib.orc_mx_exp(float(amax))


def fp8_rows(y, mode, rows=None):
    """f32 rows y [T][K] -> (E4M3 bytes [T][K], scales): mode 1 f32
    [K / 128][rows], mode 2 uint8 Mx32 bytes (tiled, ceil(T / 128) row tiles)."""
    y = np.ascontiguousarray(y, np.float32)
    T, K = y.shape
    rows = T if rows is None else rows
    q = np.zeros((T, K), np.uint8)
    if mode == 1:
        s = np.zeros((K // 128, rows), np.float32)
    else:
        s = np.zeros(((T + 127) // 128) * ((K // 32 + 3) // 4) * 512, np.uint8)
    _lib.orc_fp8_rows(_p(y), T, K, mode, rows, _p(q), _p(s))
    return q, s


def gate_rows(raw, qkv, qstride, Hq):
    """Gated f32 outputs y = rbf(o) / (1 + expf(-gate)) of raw attention
    outputs [T][Hq][256] (the values an FP8 copy quantises)."""
    raw = np.ascontiguousarray(raw, np.float32)
    T = raw.shape[0]
    y = np.zeros_like(raw)
    _lib.orc_gate_rows(_p(raw), _p(np.ascontiguousarray(qkv)), qstride, T, Hq, _p(y))
    return y

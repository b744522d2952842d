"""pkv: MI355X paged KV cache — Python host mirror over libpkv.so (ctypes).

Device arguments are torch tensors on the GPU (their data_ptr is passed) or
raw integer device addresses; `stream` defaults to torch's current stream.
Every call raises PkvError on a non-zero status. There is no fallback: if
libpkv.so is missing or fails to load, importing this module raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# PKV_LIBRARY selects another build of the same library (A/B measurements).
LIB_PATH = os.environ.get("PKV_LIBRARY") or os.path.join(_HERE, "libpkv.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"libpkv.so not built at {LIB_PATH}: run __graft_entry__.build()")
# One HIP runtime per process. torch ships its own libamdhip64 (same SONAME,
# libamdhip64.so.7); loading torch first makes libpkv's dependency resolve to
# that already-loaded runtime, so device pointers and streams from torch are
# valid in libpkv. Without torch the system ROCm runtime is used.
try:
    import torch  # noqa: F401
except ImportError:
    pass
_lib = ctypes.CDLL(LIB_PATH)

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 801
ERR_NO_BLOCKS = 802

_c_int, _c_i64, _c_p, _c_f, _c_sz = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t

_SIGS = {
    "pkv_strerror": (ctypes.c_char_p, [_c_int]),
    "pkv_version": (_c_int, []),
    "pkv_append": (_c_int, [_c_p, _c_p, _c_i64, _c_p, _c_int, _c_int, _c_int, _c_p, _c_p, _c_i64, _c_p]),
    "pkv_gather": (_c_int, [_c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_p, _c_p, _c_p]),
    "pkv_page_copy": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_i64, _c_i64, _c_p]),
    "pkv_attn_fp8_next": (_c_int, [_c_p, _c_p, _c_int, _c_int]),
    "pkv_attn_dense_f32": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_int, _c_f, _c_p,
                                    _c_p]),
    "pkv_mtp_next": (_c_int, [_c_p, _c_p, _c_p, _c_int, _c_p, _c_int, _c_int, _c_p, _c_int, _c_p, _c_p, _c_p, _c_int,
                              _c_p]),
    "pkv_attn_decode_workspace": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "pkv_attn_decode": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_p, _c_p, _c_p, _c_int, _c_int,
                                 _c_p, _c_f, _c_p, _c_int, _c_p, _c_int, _c_int, _c_i64, _c_p, _c_sz, _c_p]),
    "pkv_attn_decode_config": (_c_int, [_c_int, _c_int]),
    "pkv_time_next_range_kernel": (_c_int, [_c_p, _c_p]),
    "pkv_time_next_prefill_kernel": (_c_int, [_c_p, _c_p]),
    "pkv_attn_prefill": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_p, _c_p, _c_int, _c_p, _c_int,
                                  _c_int, _c_p, _c_f, _c_p, _c_int, _c_int, _c_i64, _c_p]),
    "pkv_attn_prefill_workspace": (_c_int, [_c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "pkv_attn_prefill_e4m3_split": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_p, _c_p,
                                             _c_int, _c_p, _c_int, _c_int, _c_p, _c_f, _c_p, _c_int, _c_int, _c_i64,
                                             _c_p, _c_sz, _c_p]),
    "pkv_attn_prefill_split": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_p, _c_p, _c_int, _c_p,
                                        _c_int, _c_int, _c_p, _c_f, _c_p, _c_int, _c_int, _c_i64, _c_p, _c_sz, _c_p]),
    "pkv_attn_decode_step": (_c_int, [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_p,
                                      _c_p, _c_p, _c_int, _c_int, _c_p, _c_f, _c_p, _c_int, _c_p, _c_int, _c_int,
                                      _c_i64, _c_p, _c_sz, _c_p]),
    "pkv_pool_create": (_c_p, [_c_i64]),
    "pkv_pool_destroy": (None, [_c_p]),
    "pkv_pool_take": (_c_int, [_c_p, _c_int, ctypes.POINTER(ctypes.c_uint32)]),
    "pkv_pool_unref": (_c_int, [_c_p, ctypes.POINTER(ctypes.c_uint32), _c_int]),
    "pkv_pool_ref": (_c_int, [_c_p, ctypes.POINTER(ctypes.c_uint32), _c_int]),
    "pkv_pool_free_count": (_c_i64, [_c_p]),
    "pkv_pool_total": (_c_i64, [_c_p]),
    "pkv_pool_refs": (_c_int, [_c_p, ctypes.c_uint32]),
    "pkv_pool_free_list": (_c_i64, [_c_p, ctypes.POINTER(ctypes.c_uint32), _c_i64]),
    "pkv_kv_create": (_c_p, [_c_i64, _c_int, _c_i64]),
    "pkv_kv_destroy": (None, [_c_p]),
    "pkv_kv_pool": (_c_p, [_c_p]),
    "pkv_kv_admit": (_c_int, [_c_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32), _c_i64, _c_i64, _c_int,
                              ctypes.POINTER(_c_int), ctypes.POINTER(_c_i64)]),
    "pkv_kv_lookup": (_c_int, [_c_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32), _c_i64,
                               ctypes.POINTER(_c_i64)]),
    "pkv_kv_cache_add": (_c_int, [_c_p, _c_int, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32), _c_i64]),
    "pkv_kv_evict_one": (_c_int, [_c_p]),
    "pkv_kv_cache_entries": (_c_i64, [_c_p]),
    "pkv_kv_release": (_c_int, [_c_p, _c_int]),
    "pkv_kv_new_seq": (_c_int, [_c_p, ctypes.POINTER(_c_int)]),
    "pkv_kv_reserve": (_c_int, [_c_p, _c_int, _c_i64]),
    "pkv_kv_share": (_c_int, [_c_p, _c_int, _c_int, _c_i64]),
    "pkv_kv_prepare_write": (_c_int, [_c_p, _c_int, _c_i64, _c_int, ctypes.POINTER(ctypes.c_int32),
                                      ctypes.POINTER(ctypes.c_int32), _c_int, ctypes.POINTER(_c_int)]),
    "pkv_kv_set_len": (_c_int, [_c_p, _c_int, _c_i64]),
    "pkv_kv_truncate": (_c_int, [_c_p, _c_int, _c_i64, _c_int]),
    "pkv_kv_len": (_c_i64, [_c_p, _c_int]),
    "pkv_kv_blocks": (_c_i64, [_c_p, _c_int, ctypes.POINTER(ctypes.c_uint32), _c_i64]),
    "pkv_kv_fill": (_c_int, [_c_p, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int), _c_int, _c_int, _c_int] +
                    [ctypes.POINTER(ctypes.c_int32)] * 6),
    "pkv_kv_pad": (_c_int, [_c_int] * 6 + [ctypes.POINTER(ctypes.c_int32)] * 6),
    "pkv_meta_layout": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
}
_SIGS["pkv_attn_decode_step_noalloc"] = (_c_int, _SIGS["pkv_attn_decode_step"][1][:-3] + [_c_p])
_SIGS["pkv_attn_decode_split"] = _SIGS["pkv_attn_decode"]
_SIGS["pkv_attn_verify"] = _SIGS["pkv_attn_decode"]
_SIGS["pkv_attn_prefill_e4m3"] = (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p] + _SIGS["pkv_attn_prefill"][1][3:])
_SIGS["pkv_attn_decode_e4m3"] = (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p] + _SIGS["pkv_attn_decode"][1][3:])
_SIGS["pkv_attn_verify_e4m3"] = _SIGS["pkv_attn_decode_e4m3"]
_SIGS["pkv_attn_prep"] = (_c_int, [_c_p, _c_int, _c_int, _c_int, _c_p, _c_p, _c_p, _c_int, _c_int, _c_int, _c_p, _c_p,
                                   _c_p, _c_p, _c_p, _c_p, _c_p, ctypes.c_float, _c_int, ctypes.c_int64, _c_p])
_SIGS["pkv_attn_verify_workspace"] = _SIGS["pkv_attn_decode_workspace"]
_SIGS["pkv_attn_decode_merge"] = _SIGS["pkv_attn_decode"]
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(_lib, _name)
    _f.restype = _res
    _f.argtypes = _args


class PkvError(RuntimeError):
    def __init__(self, status, what):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} ({status})")


def strerror(status):
    return _lib.pkv_strerror(status).decode()


def version():
    return _lib.pkv_version()


def _check(status, what):
    if status != OK:
        raise PkvError(status, what)


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(stream):
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    import torch
    return torch.cuda.current_stream().cuda_stream


def append(k_rows, v_rows, row_stride, slot_map, T, Hkv, head_bytes, kcache, vcache, num_slots, stream=None):
    """KV append; row_stride in bytes (see include/pkv.h)."""
    _check(_lib.pkv_append(_ptr(k_rows), _ptr(v_rows), row_stride, _ptr(slot_map), T, Hkv, head_bytes,
                           _ptr(kcache), _ptr(vcache), num_slots, _stream(stream)), "pkv_append")


def gather(kcache, vcache, bt_row, L, block_size, Hkv, head_bytes, num_blocks, k_out, v_out, stream=None):
    _check(_lib.pkv_gather(_ptr(kcache), _ptr(vcache), _ptr(bt_row), L, block_size, Hkv, head_bytes, num_blocks,
                           _ptr(k_out), _ptr(v_out), _stream(stream)), "pkv_gather")


def attn_fp8_next(fq, fs, fmode, frows):
    """FP8 output copies for this thread's next decode / verify call (see include/pkv.h)."""
    _check(_lib.pkv_attn_fp8_next(_ptr(fq), _ptr(fs), fmode, frows), "pkv_attn_fp8_next")


def attn_dense_f32(q, k, v, off, lens, S, Hq, Hkv, D, scale, out, stream=None):
    """Single-query attention over dense f32 rows (see include/pkv.h)."""
    _check(_lib.pkv_attn_dense_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(off), _ptr(lens), S, Hq, Hkv, D, scale, _ptr(out),
                                   _stream(stream)), "pkv_attn_dense_f32")


def page_copy(kcache, vcache, src, dst, n, page_bytes, num_blocks, stream=None):
    _check(_lib.pkv_page_copy(_ptr(kcache), _ptr(vcache), _ptr(src), _ptr(dst), n, page_bytes, num_blocks,
                              _stream(stream)), "pkv_page_copy")


def mtp_next(rows, pos, rope, rope_stride, block_table, max_blocks, block_size, limits, k, dpos, dslot, drope, S,
             stream=None):
    """Draft pass k's positions, KV slots (-1 past limits) and rotary rows
    (reference mtp_next, qwen35.cu:2633-2650); device int32 arrays."""
    _check(_lib.pkv_mtp_next(_ptr(rows), _ptr(pos), _ptr(rope), rope_stride, _ptr(block_table), max_blocks, block_size,
                             _ptr(limits), k, _ptr(dpos), _ptr(dslot), _ptr(drope), S, _stream(stream)),
           "pkv_mtp_next")


def attn_decode_workspace(T, Hq):
    n = _c_sz(0)
    _check(_lib.pkv_attn_decode_workspace(T, Hq, ctypes.byref(n)), "pkv_attn_decode_workspace")
    return n.value


def attn_verify_workspace(T, Hq):
    n = _c_sz(0)
    _check(_lib.pkv_attn_verify_workspace(T, Hq, ctypes.byref(n)), "pkv_attn_verify_workspace")
    return n.value


def time_next_range_kernel(start_event, stop_event):
    """Have the next key-range kernel record these torch.cuda.Event objects
    (or raw hipEvent_t ints) at its start and end."""
    h = lambda e: e if (e is None or isinstance(e, int)) else e.cuda_event
    _check(_lib.pkv_time_next_range_kernel(h(start_event), h(stop_event)), "pkv_time_next_range_kernel")


def time_next_prefill_kernel(start_event, stop_event):
    h = lambda e: e if (e is None or isinstance(e, int)) else e.cuda_event
    _check(_lib.pkv_time_next_prefill_kernel(h(start_event), h(stop_event)), "pkv_time_next_prefill_kernel")


def attn_decode_config(wg_per_cu=1, min_range=32):
    _check(_lib.pkv_attn_decode_config(wg_per_cu, min_range), "pkv_attn_decode_config")


def attn_decode_step(k_rows, v_rows, row_stride, slot_map, q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, tok_seq,
                     block_table, max_blocks, block_size, out, scale, cu, skip_prompts, outs, spec, T, num_blocks,
                     workspace, workspace_bytes=None, stream=None):
    """Fused KV append + paged decode attention (see include/pkv.h)."""
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size()
    _check(_lib.pkv_attn_decode_step(_ptr(k_rows), _ptr(v_rows), row_stride, _ptr(slot_map), _ptr(q), _ptr(kcache),
                                     _ptr(vcache), _ptr(qkv), qstride, Hq, Hkv, _ptr(pos), _ptr(tok_seq),
                                     _ptr(block_table), max_blocks, block_size, _ptr(out), scale, _ptr(cu),
                                     int(skip_prompts), _ptr(outs), spec, T, num_blocks, _ptr(workspace),
                                     workspace_bytes, _stream(stream)), "pkv_attn_decode_step")


def attn_decode_step_noalloc(k_rows, v_rows, row_stride, slot_map, q, kcache, vcache, qkv, qstride, Hq, Hkv, pos,
                             tok_seq, block_table, max_blocks, block_size, out, scale, cu, skip_prompts, outs, spec, T,
                             num_blocks, stream=None):
    """pkv_attn_decode_step with the library's per-GPU device array as its
    workspace: allocates nothing; calls overlapping on one GPU race."""
    _check(_lib.pkv_attn_decode_step_noalloc(_ptr(k_rows), _ptr(v_rows), row_stride, _ptr(slot_map), _ptr(q),
                                             _ptr(kcache), _ptr(vcache), _ptr(qkv), qstride, Hq, Hkv, _ptr(pos),
                                             _ptr(tok_seq), _ptr(block_table), max_blocks, block_size, _ptr(out),
                                             scale, _ptr(cu), int(skip_prompts), _ptr(outs), spec, T, num_blocks,
                                             _stream(stream)), "pkv_attn_decode_step_noalloc")


def attn_decode(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks, block_size, out,
                scale, cu, skip_prompts, outs, spec, T, num_blocks, workspace, workspace_bytes=None, stream=None,
                phase="both"):
    """Paged decode attention (reference attn_paged_g4 + attn_merge semantics).
    phase: "both", "split" (key-range kernel only) or "merge"."""
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size()
    fn = {"both": _lib.pkv_attn_decode, "split": _lib.pkv_attn_decode_split, "merge": _lib.pkv_attn_decode_merge}[phase]
    _check(fn(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(qkv), qstride, Hq, Hkv, _ptr(pos),
                                _ptr(tok_seq), _ptr(block_table), max_blocks, block_size, _ptr(out), scale,
                                _ptr(cu), int(skip_prompts), _ptr(outs), spec, T, num_blocks, _ptr(workspace),
                                workspace_bytes, _stream(stream)), "pkv_attn_decode")


def attn_verify(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks, block_size, out,
                scale, cu, skip_prompts, outs, spec, T, num_blocks, workspace, workspace_bytes=None, stream=None):
    """Draft-verify attention: decode semantics per row, up to 4 rows of a
    sequence per pass over its pages (workspace: attn_verify_workspace)."""
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size()
    _check(_lib.pkv_attn_verify(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(qkv), qstride, Hq, Hkv, _ptr(pos),
                                _ptr(tok_seq), _ptr(block_table), max_blocks, block_size, _ptr(out), scale, _ptr(cu),
                                int(skip_prompts), _ptr(outs), spec, T, num_blocks, _ptr(workspace), workspace_bytes,
                                _stream(stream)), "pkv_attn_verify")


def attn_prep(qkv, qstride, Hq, Hkv, q_norm, k_norm, rope, rope_stride, sec_h, sec_w, slot_map, inv_freq, qout,
              kcache, vcache, eps, T, num_slots, kscale=None, vscale=None, stream=None):
    """Attention input preparation (reference attn_prep): q/k RMSNorm +
    interleaved multimodal rotary, q to qout, k/v into their cache slots."""
    _check(_lib.pkv_attn_prep(_ptr(qkv), qstride, Hq, Hkv, _ptr(q_norm), _ptr(k_norm), _ptr(rope), rope_stride, sec_h,
                              sec_w, _ptr(slot_map), _ptr(inv_freq), _ptr(qout), _ptr(kcache), _ptr(vcache),
                              _ptr(kscale), _ptr(vscale), eps, T, num_slots, _stream(stream)), "pkv_attn_prep")


def _e4m3_call(name, q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks,
               block_size, out, scale, cu, skip_prompts, outs, spec, T, num_blocks, workspace, workspace_bytes, stream):
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size()
    _check(getattr(_lib, name)(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(kscale), _ptr(vscale), _ptr(qkv), qstride,
                               Hq, Hkv, _ptr(pos), _ptr(tok_seq), _ptr(block_table), max_blocks, block_size,
                               _ptr(out), scale, _ptr(cu), int(skip_prompts), _ptr(outs), spec, T, num_blocks,
                               _ptr(workspace), workspace_bytes, _stream(stream)), name)


def attn_decode_e4m3(q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks,
                     block_size, out, scale, cu, skip_prompts, outs, spec, T, num_blocks, workspace,
                     workspace_bytes=None, stream=None):
    """Per-token decode attention over an E4M3 cache (reference attn_paged8 +
    attn_merge); workspace: attn_decode_workspace(T, Hq) bytes."""
    _e4m3_call("pkv_attn_decode_e4m3", q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq,
               block_table, max_blocks, block_size, out, scale, cu, skip_prompts, outs, spec, T, num_blocks,
               workspace, workspace_bytes, stream)


def attn_verify_e4m3(q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks,
                     block_size, out, scale, cu, skip_prompts, outs, spec, T, num_blocks, workspace,
                     workspace_bytes=None, stream=None):
    """The same with each sequence's rows sharing one pass over its pages
    (as attn_verify; `cu` required); workspace: attn_verify_workspace(T, Hq)."""
    _e4m3_call("pkv_attn_verify_e4m3", q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq,
               block_table, max_blocks, block_size, out, scale, cu, skip_prompts, outs, spec, T, num_blocks,
               workspace, workspace_bytes, stream)


def attn_prefill_e4m3(q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks,
                      block_size, out, scale, outs, spec, T, num_blocks, stream=None, workspace=None):
    """Causal chunked-prefill attention over an E4M3 cache (reference attn_group8);
    with a workspace (attn_prefill_workspace bytes), pkv_attn_prefill_e4m3_split."""
    if workspace is not None:
        _check(_lib.pkv_attn_prefill_e4m3_split(
            _ptr(q), _ptr(kcache), _ptr(vcache), _ptr(kscale), _ptr(vscale), _ptr(qkv), qstride, Hq, Hkv, _ptr(pos),
            _ptr(cu), seqs, _ptr(block_table), max_blocks, block_size, _ptr(out), scale, _ptr(outs), spec, T,
            num_blocks, _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(stream)),
            "pkv_attn_prefill_e4m3_split")
        return
    _check(_lib.pkv_attn_prefill_e4m3(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(kscale), _ptr(vscale), _ptr(qkv),
                                      qstride, Hq, Hkv, _ptr(pos), _ptr(cu), seqs, _ptr(block_table), max_blocks,
                                      block_size, _ptr(out), scale, _ptr(outs), spec, T, num_blocks, _stream(stream)),
           "pkv_attn_prefill_e4m3")


def attn_prefill(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks, block_size, out,
                 scale, outs, spec, T, num_blocks, stream=None, workspace=None):
    """Causal chunked-prefill attention over paged context (MFMA bf16);
    with a workspace (attn_prefill_workspace bytes), pkv_attn_prefill_split."""
    if workspace is not None:
        _check(_lib.pkv_attn_prefill_split(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(qkv), qstride, Hq, Hkv,
                                           _ptr(pos), _ptr(cu), seqs, _ptr(block_table), max_blocks, block_size,
                                           _ptr(out), scale, _ptr(outs), spec, T, num_blocks, _ptr(workspace),
                                           workspace.numel() * workspace.element_size(), _stream(stream)),
               "pkv_attn_prefill_split")
        return
    _check(_lib.pkv_attn_prefill(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(qkv), qstride, Hq, Hkv, _ptr(pos),
                                 _ptr(cu), seqs, _ptr(block_table), max_blocks, block_size, _ptr(out), scale,
                                 _ptr(outs), spec, T, num_blocks, _stream(stream)), "pkv_attn_prefill")


def attn_prefill_workspace(T, Hq, Hkv, seqs):
    """Workspace bytes of pkv_attn_prefill_split / _e4m3_split for these shapes."""
    n = _c_sz(0)
    _check(_lib.pkv_attn_prefill_workspace(T, Hq, Hkv, seqs, ctypes.byref(n)), "pkv_attn_prefill_workspace")
    return n.value


class Pool:
    """Block allocator (reference Scheduler.free_blocks/block_refs,
    src/sched.rs:461-465, 515, 801-817)."""

    def __init__(self, n_blocks):
        self._lib = _lib  # keeps the library alive until this handle is destroyed
        self._h = _lib.pkv_pool_create(n_blocks)
        if not self._h:
            raise PkvError(ERR_INVALID, "pkv_pool_create")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.pkv_pool_destroy(h)
            self._h = None

    @staticmethod
    def _ids(ids):
        ids = list(ids)
        return (ctypes.c_uint32 * max(1, len(ids)))(*ids), len(ids)

    def take(self, n):
        buf = (ctypes.c_uint32 * max(1, n))()
        _check(_lib.pkv_pool_take(self._h, n, buf), "pkv_pool_take")
        return list(buf[:n])

    def unref(self, ids):
        buf, n = self._ids(ids)
        _check(_lib.pkv_pool_unref(self._h, buf, n), "pkv_pool_unref")

    def ref(self, ids):
        buf, n = self._ids(ids)
        _check(_lib.pkv_pool_ref(self._h, buf, n), "pkv_pool_ref")

    def free_count(self):
        return _lib.pkv_pool_free_count(self._h)

    def total(self):
        return _lib.pkv_pool_total(self._h)

    def refs(self, i):
        r = _lib.pkv_pool_refs(self._h, i)
        if r < 0:
            raise PkvError(-r, "pkv_pool_refs")
        return r

    def free_list(self):
        n = self.free_count()
        buf = (ctypes.c_uint32 * max(1, n))()
        _lib.pkv_pool_free_list(self._h, buf, n)
        return list(buf[:n])


def _u32(tokens):
    tokens = list(tokens)
    return (ctypes.c_uint32 * max(1, len(tokens)))(*tokens), len(tokens)


class Kv:
    """KV manager: block tables, prefix cache, step metadata, copy-on-write
    and truncation (include/pkv.h pkv_kv_*; the reference Scheduler's KV
    bookkeeping, src/sched.rs)."""

    def __init__(self, n_blocks, block_size=16, max_entries=0):
        self._lib = _lib
        self._h = _lib.pkv_kv_create(n_blocks, block_size, max_entries)
        if not self._h:
            raise PkvError(ERR_INVALID, "pkv_kv_create")
        self.block_size = block_size

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.pkv_kv_destroy(h)
            self._h = None

    def free_count(self):
        return _lib.pkv_pool_free_count(_lib.pkv_kv_pool(self._h))

    def refs(self, page):
        return _lib.pkv_pool_refs(_lib.pkv_kv_pool(self._h), page)

    def admit(self, prompt, max_new, use_cache=True, adapter=0):
        """Returns (seq_id, cached_tokens); raises PkvError(ERR_NO_BLOCKS) when the request must wait."""
        buf, n = _u32(prompt)
        sid, cached = _c_int(0), _c_i64(0)
        _check(_lib.pkv_kv_admit(self._h, adapter, buf, n, max_new, int(use_cache), ctypes.byref(sid),
                                 ctypes.byref(cached)), "pkv_kv_admit")
        return sid.value, cached.value

    def lookup(self, prompt, adapter=0):
        buf, n = _u32(prompt)
        hit = _c_i64(0)
        _check(_lib.pkv_kv_lookup(self._h, adapter, buf, n, ctypes.byref(hit)), "pkv_kv_lookup")
        return hit.value

    def cache_add(self, seq, tokens, adapter=0):
        buf, n = _u32(tokens)
        _check(_lib.pkv_kv_cache_add(self._h, seq, adapter, buf, n), "pkv_kv_cache_add")

    def evict_one(self):
        return bool(_lib.pkv_kv_evict_one(self._h))

    def entries(self):
        return _lib.pkv_kv_cache_entries(self._h)

    def release(self, seq):
        _check(_lib.pkv_kv_release(self._h, seq), "pkv_kv_release")

    def new_seq(self):
        sid = _c_int(0)
        _check(_lib.pkv_kv_new_seq(self._h, ctypes.byref(sid)), "pkv_kv_new_seq")
        return sid.value

    def reserve(self, seq, n_tokens):
        _check(_lib.pkv_kv_reserve(self._h, seq, n_tokens), "pkv_kv_reserve")

    def share(self, dst, src, n_tokens):
        _check(_lib.pkv_kv_share(self._h, dst, src, n_tokens), "pkv_kv_share")

    def prepare_write(self, seq, pos, n, cap=64):
        """Returns the (src, dst) page copies copy-on-write needs before writing [pos, pos + n)."""
        src, dst, k = (ctypes.c_int32 * cap)(), (ctypes.c_int32 * cap)(), _c_int(0)
        _check(_lib.pkv_kv_prepare_write(self._h, seq, pos, n, src, dst, cap, ctypes.byref(k)), "pkv_kv_prepare_write")
        return list(src[:k.value]), list(dst[:k.value])

    def set_len(self, seq, n):
        _check(_lib.pkv_kv_set_len(self._h, seq, n), "pkv_kv_set_len")

    def truncate(self, seq, new_len, free_pages=False):
        _check(_lib.pkv_kv_truncate(self._h, seq, new_len, int(free_pages)), "pkv_kv_truncate")

    def len(self, seq):
        n = _lib.pkv_kv_len(self._h, seq)
        if n < 0:
            raise PkvError(-n, "pkv_kv_len")
        return n

    def blocks(self, seq):
        n = _lib.pkv_kv_blocks(self._h, seq, None, 0)
        if n < 0:
            raise PkvError(-n, "pkv_kv_blocks")
        buf = (ctypes.c_uint32 * max(1, n))()
        _lib.pkv_kv_blocks(self._h, seq, buf, n)
        return list(buf[:n])

    def fill(self, rows, max_tokens, max_blocks, max_rows=None):
        """rows: [(seq, ntok)]. Returns a dict of numpy int32 arrays (pos, slot_map, tok_seq, cu, limits,
        block_table) sized for max_rows rows (default len(rows)), the reference's Meta arrays for the step."""
        import numpy as np
        nrows = len(rows)
        max_rows = max(nrows, max_rows or 0)
        ids = (_c_int * max(1, nrows))(*[r[0] for r in rows])
        nt = (_c_int * max(1, nrows))(*[r[1] for r in rows])
        out = {k: np.zeros(n, np.int32) for k, n in (("pos", max_tokens), ("slot_map", max_tokens),
                                                       ("tok_seq", max_tokens), ("cu", max_rows + 1),
                                                       ("limits", max(1, max_rows)),
                                                       ("block_table", max(1, max_rows) * max_blocks))}
        P = ctypes.POINTER(ctypes.c_int32)
        args = [out[k].ctypes.data_as(P) for k in ("pos", "slot_map", "tok_seq", "cu", "limits", "block_table")]
        _check(_lib.pkv_kv_fill(self._h, ids, nt, nrows, max_tokens, max_blocks, *args), "pkv_kv_fill")
        out["block_table"] = out["block_table"].reshape(-1, max_blocks)
        return out


_META_FIELDS = ("ids", "pos", "slot_map", "tok_seq", "emb_src", "rope", "mtp_ids", "mtp_src", "cu", "slots", "fresh",
                "outs", "ocu", "last", "temps", "seeds", "top_ks", "top_ps", "min_ps", "pen_cu", "limits", "snaps",
                "block_table", "lora", "masks", "words")


def meta_layout(max_tokens, max_seqs, max_blocks, spec=1):
    """Offsets (int32 words) of the reference's per-step metadata buffer
    (Meta, model.rs:1245-1354), and its length as "words"."""
    arr = (ctypes.c_int64 * len(_META_FIELDS))()
    _check(_lib.pkv_meta_layout(max_tokens, max_seqs, max_blocks, spec, ctypes.byref(arr)), "pkv_meta_layout")
    return dict(zip(_META_FIELDS, arr))


def pad_rows(meta, frm, to, n):
    """Writes padding rows [frm, to) of n tokens into a fill() dict in place."""
    import ctypes as C
    P = C.POINTER(C.c_int32)
    max_rows, max_tokens = len(meta["cu"]) - 1, len(meta["pos"])
    max_blocks = meta["block_table"].shape[1]
    bt = meta["block_table"]
    args = [meta[k].ctypes.data_as(P) for k in ("pos", "slot_map", "tok_seq", "cu", "limits")] + [bt.ctypes.data_as(P)]
    _check(_lib.pkv_kv_pad(frm, to, n, max_rows, max_tokens, max_blocks, *args), "pkv_kv_pad")


def exported_symbols():
    """Names of every entry point declared in include/pkv.h that this library exports."""
    return [n for n in _SIGS if hasattr(_lib, n)]

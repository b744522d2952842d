// C-ABI entry points of libpkv.so (declared in include/pkv.h). Every entry
// point validates its shapes on the host before launching: a kernel only
// ever sees arguments its indexing was written for.
#include "pkv_copy.hip"
#include "pkv_decode.hip"
#include "pkv_decode8.hip"
#include "pkv_prefill.hip"
#include "pkv_verify.hip"
#include "pkv_prep.hip"
#include "../../include/pkv.h"

#include <hip/hip_ext.h>

#include <mutex>
#include <set>

namespace {

// Query heads per kv head the attention kernels serve (the
// reference instantiates attn_paged_g<G> for the same groups,
// qwen35.cu:1326-1334).
bool supported_group(int G) { return G == 1 || G == 2 || G == 4 || G == 6 || G == 8; }
template <class K>
K by_group(int G, K g1, K g2, K g4, K g6, K g8) {
    return G == 1 ? g1 : G == 2 ? g2 : G == 4 ? g4 : G == 6 ? g6 : g8;
}


int status_of(hipError_t e) { return e == hipSuccess ? PKV_OK : (int)e; }

int launch_status() { return status_of(hipGetLastError()); }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int vec_mode(const void* a, const void* b, const void* c, const void* d, int64_t stride, int row_bytes) {
    if (row_bytes % 16 == 0 && stride % 16 == 0 && aligned(a, 16) && aligned(b, 16) && aligned(c, 16) &&
        aligned(d, 16))
        return 2;
    if (row_bytes % 4 == 0 && stride % 4 == 0 && aligned(a, 4) && aligned(b, 4) && aligned(c, 4) && aligned(d, 4))
        return 1;
    return 0;
}

// Compute units of the current device, cached per device.
int device_cus() {
    static std::mutex mu;
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> g(mu);
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

int g_wg_per_cu = 1;
int g_min_range = 32;
// Events the next key-range launch of this thread records at its start and
// end (hipExtLaunchKernelGGL), then forgets.
thread_local hipEvent_t t_ev_start = nullptr, t_ev_stop = nullptr;
thread_local hipEvent_t t_pf_start = nullptr, t_pf_stop = nullptr;  // same for the prefill kernel
// FP8 output copies requested for this thread's next decode / verify call
// (pkv_attn_fp8_next); cleared by the call that runs the merge.
thread_local pkv::Fp8Out t_fp8 = {nullptr, nullptr, 0, 0};

int decode_n_wg() { return device_cus() * g_wg_per_cu; }
// The E4M3 decode kernel runs two workgroups per CU (252 VGPRs and 72.8 KB
// of LDS each: two waves per SIMD), so one wave's conversions and MFMAs
// overlap the other's loads (measured at C3: 111-112 us against 117-121
// with one).
constexpr int F8_WG_PER_CU = 2;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Workspace: [offs: T + 2 ints][part_ms][part_acc].
struct DecodeLayout {
    size_t offs, ms, acc, total;
};

// Partial rows: (T + n_wg) indices x Hq heads, times 4 query rows per index
// for the verify kernel.
// verify: the verify kernels' records, one per segment row (vf_rows(G); the
// workspace queries, which do not know G, size for the most, VF_ROWS).
DecodeLayout decode_layout(int T, int Hq, int n_wg, bool verify = false, int G = 0) {
    DecodeLayout d;
    const size_t rows = (size_t)(T + n_wg) * Hq * (verify ? (G > 0 ? pkv::vf_rows(G) : pkv::VF_ROWS) : 1);
    d.offs = 0;
    d.ms = round_up((size_t)(T + 2) * 4, 256);
    d.acc = d.ms + round_up(rows * 2 * 4, 256);
    d.total = d.acc + rows * pkv::HEAD_DIM * 4;
    return d;
}

}  // namespace

extern "C" {

const char* pkv_strerror(int status) {
    switch (status) {
        case PKV_OK: return "ok";
        case PKV_ERR_INVALID: return "invalid argument";
        case PKV_ERR_UNSUPPORTED: return "unsupported shape";
        case PKV_ERR_NO_BLOCKS: return "not enough free KV blocks";
        default: return hipGetErrorString((hipError_t)status);
    }
}

int pkv_version(void) { return 1; }

int pkv_append(const void* k_rows, const void* v_rows, int64_t row_stride, const int32_t* slot_map, int T, int Hkv,
               int head_bytes, void* kcache, void* vcache, int64_t num_slots, void* stream) {
    if (T < 0 || Hkv <= 0 || head_bytes <= 0 || num_slots <= 0) return PKV_ERR_INVALID;
    if (T == 0) return PKV_OK;
    if (!k_rows || !v_rows || !slot_map || !kcache || !vcache) return PKV_ERR_INVALID;
    const int64_t row_bytes = (int64_t)Hkv * head_bytes;
    if (row_bytes > (1 << 24) || row_stride < row_bytes || T > (1 << 30)) return PKV_ERR_INVALID;
    const int vec = vec_mode(k_rows, v_rows, kcache, vcache, row_stride, (int)row_bytes);
    if (vec == 2 && (row_bytes == 2048 || row_bytes == 4096 || row_bytes == 8192)) {
        // whole-row moves, APP_TOK tokens per block
        const dim3 grid((T + pkv::APP_TOK - 1) / pkv::APP_TOK);
        auto k = row_bytes == 2048 ? pkv::append_rows_kernel<1>
                 : row_bytes == 4096 ? pkv::append_rows_kernel<2> : pkv::append_rows_kernel<4>;
        hipLaunchKernelGGL(k, grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)k_rows, (const uint8_t*)v_rows,
                           (long)row_stride, slot_map, T, (uint8_t*)kcache, (uint8_t*)vcache, (long)num_slots);
        return launch_status();
    }
    hipLaunchKernelGGL(pkv::append_kernel, dim3(T, 2), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)k_rows,
                       (const uint8_t*)v_rows, (long)row_stride, slot_map, (int)row_bytes, (uint8_t*)kcache,
                       (uint8_t*)vcache, (long)num_slots, vec);
    return launch_status();
}

int pkv_gather(const void* kcache, const void* vcache, const int32_t* bt_row, int L, int block_size, int Hkv,
               int head_bytes, int64_t num_blocks, void* k_out, void* v_out, void* stream) {
    if (L < 0 || block_size <= 0 || Hkv <= 0 || head_bytes <= 0 || num_blocks <= 0) return PKV_ERR_INVALID;
    if (L == 0) return PKV_OK;
    if (!kcache || !vcache || !bt_row || !k_out || !v_out) return PKV_ERR_INVALID;
    const int64_t row_bytes = (int64_t)Hkv * head_bytes;
    if (row_bytes > (1 << 24)) return PKV_ERR_INVALID;
    const int vec = vec_mode(kcache, vcache, k_out, v_out, row_bytes, (int)row_bytes);
    hipLaunchKernelGGL(pkv::gather_kernel, dim3((L + 3) / 4, 2), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)kcache, (const uint8_t*)vcache, bt_row, L, block_size, (int)row_bytes,
                       (long)num_blocks, (uint8_t*)k_out, (uint8_t*)v_out, vec);
    return launch_status();
}

int pkv_attn_dense_f32(const float* q, const float* k, const float* v, const int32_t* off, const int32_t* len,
                       int S, int Hq, int Hkv, int D, float scale, float* out, void* stream) {
    if (S < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || D > 256) return PKV_ERR_INVALID;
    if (S == 0) return PKV_OK;
    if (!q || !k || !v || !off || !len || !out) return PKV_ERR_INVALID;
    hipLaunchKernelGGL(pkv::attn_dense_f32_kernel, dim3(S, Hq), dim3(256), 0, (hipStream_t)stream, q, k, v, off, len,
                       Hq, Hkv, D, scale, out);
    return launch_status();
}

int pkv_page_copy(void* kcache, void* vcache, const int32_t* src, const int32_t* dst, int n, int64_t page_bytes,
                  int64_t num_blocks, void* stream) {
    if (n < 0 || page_bytes <= 0 || page_bytes % 16 != 0 || num_blocks <= 0) return PKV_ERR_INVALID;
    if (n == 0) return PKV_OK;
    if (!kcache || !vcache || !src || !dst || !aligned(kcache, 16) || !aligned(vcache, 16)) return PKV_ERR_INVALID;
    const int slices = (int)std::min<int64_t>(16, std::max<int64_t>(1, page_bytes / 4096));
    hipLaunchKernelGGL(pkv::page_copy_kernel, dim3(n, 2, slices), dim3(256), 0, (hipStream_t)stream,
                       (uint8_t*)kcache, (uint8_t*)vcache, src, dst, (long)page_bytes, (long)num_blocks, slices);
    return launch_status();
}

int pkv_mtp_next(const int32_t* rows, const int32_t* pos, const int32_t* rope, int rope_stride,
                 const int32_t* block_table, int max_blocks, int block_size, const int32_t* limits, int k,
                 int32_t* dpos, int32_t* dslot, int32_t* drope, int S, void* stream) {
    if (S < 0 || max_blocks <= 0 || block_size <= 0 || rope_stride < 0) return PKV_ERR_INVALID;
    if (S == 0) return PKV_OK;
    if (!rows || !pos || !rope || !block_table || !limits || !dpos || !dslot || !drope) return PKV_ERR_INVALID;
    hipLaunchKernelGGL(pkv::mtp_next_kernel, dim3((S + 255) / 256), dim3(256), 0, (hipStream_t)stream, rows, pos, rope,
                       rope_stride, block_table, max_blocks, block_size, limits, k, dpos, dslot, drope, S);
    return launch_status();
}

int pkv_attn_prep(const void* qkv, int qstride, int Hq, int Hkv, const float* q_norm, const float* k_norm,
                  const int32_t* rope, int rope_stride, int sec_h, int sec_w, const int32_t* slot_map,
                  const float* inv_freq, void* qout, void* kcache, void* vcache, const float* kscale,
                  const float* vscale, float eps, int T, int64_t num_slots, void* stream) {
    if (T < 0 || Hq <= 0 || Hkv < 0 || num_slots < 0 || rope_stride < 0) return PKV_ERR_INVALID;
    if ((kscale == nullptr) != (vscale == nullptr)) return PKV_ERR_INVALID;  // both (E4M3 cache) or neither
    if (T == 0) return PKV_OK;
    if (!qkv || !q_norm || !rope || !slot_map || !inv_freq || !qout) return PKV_ERR_INVALID;
    if (Hkv > 0 && (!k_norm || !kcache || !vcache)) return PKV_ERR_INVALID;
    if (rope_stride < T || qstride < (2 * Hq + 2 * Hkv) * pkv::HEAD_DIM || qstride % 4 != 0) return PKV_ERR_INVALID;
    if (!aligned(qkv, 8) || !aligned(qout, 8) || !aligned(q_norm, 16) || (k_norm && !aligned(k_norm, 16)) ||
        (kcache && !aligned(kcache, 8)) || (vcache && !aligned(vcache, 8)) || (kscale && !aligned(kscale, 4)) ||
        (vscale && !aligned(vscale, 4)))
        return PKV_ERR_INVALID;
    pkv::PrepArgs a;
    a.qkv = (const uint16_t*)qkv;
    a.qstride = qstride;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.rope = rope;
    a.rope_stride = rope_stride;
    a.sec_h = sec_h;
    a.sec_w = sec_w;
    a.slot_map = slot_map;
    a.inv_freq = inv_freq;
    a.qout = (uint16_t*)qout;
    a.kcache = (uint16_t*)kcache;
    a.vcache = (uint16_t*)vcache;
    a.kscale = (float*)kscale;
    a.vscale = (float*)vscale;
    a.eps = eps;
    a.num_slots = (long)num_slots;
    hipLaunchKernelGGL(pkv::prep_kernel, dim3(T, (Hq + 2 * Hkv + 3) / 4), dim3(256), 0, (hipStream_t)stream, a);
    return launch_status();
}

}  // extern "C"

namespace {

// Workspace of pkv_attn_prefill_split: BQ x G records, of (max, sum) then
// 256 weighted values (f32), per split workgroup. The kernel takes the
// query tile count R from cu; the host bounds it by U = ceil(T / BQ) + seqs
// (each prompt rounds up once), so a split grid (parts x R x Hkv < 2 cus
// workgroups, and no more than max(2 R Hkv, cus)) holds at most
// max(2 min(U Hkv, cus - 1), cus) workgroups: the workspace's bound, cap.
struct PrefillSplitLayout {
    int64_t cap;
    size_t plan, ms, acc, total;
};
PrefillSplitLayout prefill_split_layout(int T, int Hq, int Hkv, int seqs) {
    const int G = Hq / Hkv, bq = pkv::pf_lib_bq(G);
    const int64_t cus = device_cus(), w = ((int64_t)(T + bq - 1) / bq + seqs) * Hkv;
    PrefillSplitLayout l;
    l.cap = std::max<int64_t>(2 * std::min<int64_t>(w, cus - 1), cus);
    const size_t recs = (size_t)l.cap * bq * G;
    l.plan = 0;  // the split plan (2 ints) in the first 256 bytes
    l.ms = 256;
    l.acc = round_up(l.ms + recs * 2 * 4, 256);
    l.total = l.acc + recs * pkv::HEAD_DIM * 4;
    return l;
}

int attn_prefill(const void* q, const void* kcache, const void* vcache, const float* kscale, const float* vscale,
                 const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos, const int32_t* cu, int seqs,
                 const int32_t* block_table, int max_blocks, int block_size, void* out, float scale,
                 const int32_t* outs, int spec, int T, int64_t num_blocks, void* stream, void* workspace = nullptr,
                 size_t workspace_bytes = 0) {
    if (T < 0 || seqs < 0 || Hq <= 0 || Hkv <= 0 || max_blocks <= 0 || block_size <= 0 || num_blocks <= 0 ||
        spec < 1)
        return PKV_ERR_INVALID;
    const int G = Hq % Hkv == 0 ? Hq / Hkv : 0;
    if (!supported_group(G) || (block_size & (block_size - 1)) != 0) return PKV_ERR_UNSUPPORTED;
    if (T == 0 || seqs == 0) return PKV_OK;
    if (!q || !kcache || !vcache || !qkv || !pos || !cu || !block_table || !out) return PKV_ERR_INVALID;
    if (qstride < 2 * Hq * pkv::HEAD_DIM || qstride % 8 != 0) return PKV_ERR_INVALID;
    if (!aligned(q, 16) || !aligned(kcache, 16) || !aligned(vcache, 16) || !aligned(qkv, 16) || !aligned(out, 16))
        return PKV_ERR_INVALID;
    const bool f8 = kscale != nullptr;
    if (f8 && (!vscale || !aligned(kscale, 4) || !aligned(vscale, 4))) return PKV_ERR_INVALID;
    if (workspace && !aligned(workspace, 256)) return PKV_ERR_INVALID;
    using PrefillKernel = void (*)(pkv::PrefillParams);
    const PrefillKernel kern =
        f8 ? by_group<PrefillKernel>(G, pkv::prefill_e4m3_kernel<1>, pkv::prefill_e4m3_kernel<2>,
                                     pkv::prefill_e4m3_kernel<4>, pkv::prefill_e4m3_kernel<6>,
                                     pkv::prefill_e4m3_kernel<8>)
           : by_group<PrefillKernel>(G, pkv::prefill_kernel<1>, pkv::prefill_kernel<2>, pkv::prefill_kernel<4>,
                                     pkv::prefill_kernel<6>, pkv::prefill_kernel<8>);
    int bq = pkv::pf_lib_bq(G);
    int threads = pkv::pf_lib_threads(G);
    size_t smem = pkv::prefill_smem_bytes(f8 ? pkv::pf_lib_nst_f8(G) : pkv::pf_lib_nst(G), threads);
    // Upper bound on query tiles: each prompt sequence rounds up once.
    int tiles = (T + bq - 1) / bq + seqs;
    // Few query tiles (one prompt, or one sequence's chunk, of a few
    // thousand tokens): the fine-tile kernel, half the queries per
    // workgroup and two workgroups per CU, fills and balances the CUs.
    // (G != 8: when the library's workgroups would not cover the CUs once;
    // G = 8, whose 8 waves hold fewer queries: below four rounds. At G = 6
    // the library kernel's two-tile steps beat the fine kernel once its
    // workgroups cover the CUs: 2,048 / 3,072 / 6,000-token prompts 121 /
    // 226 / 546 us against 136 / 236 / 571.)
    PrefillKernel kern_run = kern;
    // With a workspace: the split kernel, which splits every query tile's
    // keys over several workgroups when the prompt's tiles leave CUs idle
    // (it counts them from cu), then the merge. G = 6 / 8 without a sure
    // split (the bound U Hkv already covers the CUs) where the fine kernel
    // would run keeps the fine kernel.
    // Without drafts to verify (outs null) every sequence of two or more
    // rows is a prompt, so at least T - seqs rows are: when their tiles
    // alone fill the CUs no split can happen, and the call runs as without
    // a workspace (no merge launch).
    const int64_t cus = device_cus();
    const bool fine = !f8 && block_size >= 16 && (int64_t)tiles * Hkv < (G == 8 ? 4 : 1) * cus;
    const bool no_split = !outs && (int64_t)(T - seqs + bq - 1) / bq * Hkv >= cus;
    const bool split = workspace && !no_split && !(fine && G >= 6 && (int64_t)tiles * Hkv >= cus);
    PrefillSplitLayout lay{};
    if (split) {
        lay = prefill_split_layout(T, Hq, Hkv, seqs);
        if (workspace_bytes < lay.total) return PKV_ERR_INVALID;
        kern_run = f8 ? by_group<PrefillKernel>(G, pkv::prefill_split_kernel<1, true>,
                                                pkv::prefill_split_kernel<2, true>, pkv::prefill_split_kernel<4, true>,
                                                pkv::prefill_split_kernel<6, true>, pkv::prefill_split_kernel<8, true>)
                      : by_group<PrefillKernel>(G, pkv::prefill_split_kernel<1>, pkv::prefill_split_kernel<2>,
                                                pkv::prefill_split_kernel<4>, pkv::prefill_split_kernel<6>,
                                                pkv::prefill_split_kernel<8>);
    } else if (fine) {
        kern_run = by_group<PrefillKernel>(G, pkv::prefill_fine_kernel<1>, pkv::prefill_fine_kernel<2>,
                                           pkv::prefill_fine_kernel<4>, pkv::prefill_fine_kernel<6>,
                                           pkv::prefill_fine_kernel<8>);
        bq = pkv::pf_fine_bq(G);
        threads = pkv::pf_fine_threads(G);
        smem = pkv::pf_fine_smem_bytes(G);
        tiles = (T + bq - 1) / bq + seqs;
    }
    // per process: the kernels' LDS above the 64 KiB default, once per kernel
    static std::mutex attr_mu;
    static std::set<const void*> attr_set;
    {
        std::lock_guard<std::mutex> lk(attr_mu);
        if (!attr_set.count((const void*)kern_run)) {
            const int st = status_of(
                hipFuncSetAttribute((const void*)kern_run, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            if (st != PKV_OK) return st;
            attr_set.insert((const void*)kern_run);
        }
    }
    pkv::PrefillParams p;
    p.q = (const uint16_t*)q;
    p.kc = (const uint16_t*)kcache;
    p.vc = (const uint16_t*)vcache;
    p.qkv = (const uint16_t*)qkv;
    p.qstride = qstride;
    p.Hq = Hq;
    p.Hkv = Hkv;
    p.pos = pos;
    p.cu = cu;
    p.seqs = seqs;
    p.block_table = block_table;
    p.max_blocks = max_blocks;
    p.block_size = block_size;
    p.bs_log2 = __builtin_ctz((unsigned)block_size);
    p.out = (uint16_t*)out;
    p.scale = scale;
    p.outs = outs;
    p.spec = spec;
    p.num_blocks = (long)num_blocks;
    p.kscale = kscale;
    p.vscale = vscale;
    p.cus = (int)cus;
    p.split_cap = split ? (int)lay.cap : 0;
    p.part_ms = split ? (float*)((char*)workspace + lay.ms) : nullptr;
    p.part_acc = split ? (float*)((char*)workspace + lay.acc) : nullptr;
    p.split_plan = split ? (int*)((char*)workspace + lay.plan) : nullptr;
    hipEvent_t e0 = t_pf_start, e1 = t_pf_stop;
    t_pf_start = t_pf_stop = nullptr;
    // the split kernel: a 1-D grid over both of its launches' shapes
    const dim3 grid = split ? dim3((unsigned)std::max<int64_t>((int64_t)tiles * Hkv, 2 * cus)) : dim3(tiles, Hkv);
    hipExtLaunchKernelGGL(kern_run, grid, dim3(threads), smem, (hipStream_t)stream, e0, e1, 0, p);
    if (split) {
        int st = launch_status();
        if (st != PKV_OK) return st;
        using MergeKernel = void (*)(pkv::PrefillParams);
        const MergeKernel mk = by_group<MergeKernel>(G, pkv::prefill_merge_kernel<1>, pkv::prefill_merge_kernel<2>,
                                                     pkv::prefill_merge_kernel<4>, pkv::prefill_merge_kernel<6>,
                                                     pkv::prefill_merge_kernel<8>);
        hipLaunchKernelGGL(mk, dim3(T, Hkv), dim3(64 * G), 0, (hipStream_t)stream, p);
    }
    return launch_status();
}

}  // namespace

extern "C" {

int pkv_attn_prefill(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                     int Hkv, const int32_t* pos, const int32_t* cu, int seqs, const int32_t* block_table,
                     int max_blocks, int block_size, void* out, float scale, const int32_t* outs, int spec, int T,
                     int64_t num_blocks, void* stream) {
    return attn_prefill(q, kcache, vcache, nullptr, nullptr, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table,
                        max_blocks, block_size, out, scale, outs, spec, T, num_blocks, stream);
}

int pkv_attn_prefill_workspace(int T, int Hq, int Hkv, int seqs, size_t* bytes) {
    if (T < 0 || Hq <= 0 || Hkv <= 0 || seqs < 0 || Hq % Hkv != 0 || !bytes) return PKV_ERR_INVALID;
    *bytes = prefill_split_layout(T, Hq, Hkv, seqs).total;
    return PKV_OK;
}

int pkv_attn_prefill_split(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                           int Hkv, const int32_t* pos, const int32_t* cu, int seqs, const int32_t* block_table,
                           int max_blocks, int block_size, void* out, float scale, const int32_t* outs, int spec,
                           int T, int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream) {
    return attn_prefill(q, kcache, vcache, nullptr, nullptr, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table,
                        max_blocks, block_size, out, scale, outs, spec, T, num_blocks, stream, workspace,
                        workspace_bytes);
}

int pkv_attn_prefill_e4m3_split(const void* q, const void* kcache, const void* vcache, const float* kscale,
                                const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                                const int32_t* cu, int seqs, const int32_t* block_table, int max_blocks,
                                int block_size, void* out, float scale, const int32_t* outs, int spec, int T,
                                int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream) {
    if (!kscale || !vscale) return PKV_ERR_INVALID;
    return attn_prefill(q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table,
                        max_blocks, block_size, out, scale, outs, spec, T, num_blocks, stream, workspace,
                        workspace_bytes);
}

int pkv_attn_prefill_e4m3(const void* q, const void* kcache, const void* vcache, const float* kscale,
                          const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                          const int32_t* cu, int seqs, const int32_t* block_table, int max_blocks, int block_size,
                          void* out, float scale, const int32_t* outs, int spec, int T, int64_t num_blocks,
                          void* stream) {
    if (!kscale || !vscale) return PKV_ERR_INVALID;
    return attn_prefill(q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table,
                        max_blocks, block_size, out, scale, outs, spec, T, num_blocks, stream);
}



int pkv_time_next_range_kernel(void* start_event, void* stop_event) {
    t_ev_start = (hipEvent_t)start_event;
    t_ev_stop = (hipEvent_t)stop_event;
    return PKV_OK;
}

int pkv_attn_fp8_next(void* fq, void* fs, int fmode, int frows) {
    if (fmode < 0 || fmode > 2) return PKV_ERR_INVALID;
    if (fmode && (!fq || !fs || frows <= 0)) return PKV_ERR_INVALID;
    t_fp8 = {(uint8_t*)fq, fs, fmode, fmode ? frows : 0};
    return PKV_OK;
}

int pkv_time_next_prefill_kernel(void* start_event, void* stop_event) {
    t_pf_start = (hipEvent_t)start_event;
    t_pf_stop = (hipEvent_t)stop_event;
    return PKV_OK;
}

int pkv_attn_decode_config(int wg_per_cu, int min_range) {
    if (wg_per_cu < 1 || wg_per_cu > 64 || min_range < 1 || min_range > (1 << 20)) return PKV_ERR_INVALID;
    g_wg_per_cu = wg_per_cu;
    g_min_range = min_range;
    return PKV_OK;
}


int pkv_attn_decode_workspace(int T, int Hq, size_t* bytes) {
    if (T < 0 || Hq <= 0 || !bytes) return PKV_ERR_INVALID;
    // Groups other than 4 query heads per kv head run the verify kernels'
    // records, so the size covers both layouts.
    *bytes = std::max(decode_layout(T, Hq, decode_n_wg() * F8_WG_PER_CU).total,
                      decode_layout(T, Hq, decode_n_wg() * F8_WG_PER_CU, true).total);
    return PKV_OK;
}

int pkv_attn_verify_workspace(int T, int Hq, size_t* bytes) {
    if (T < 0 || Hq <= 0 || !bytes) return PKV_ERR_INVALID;
    *bytes = decode_layout(T, Hq, decode_n_wg() * F8_WG_PER_CU, true).total;
    return PKV_OK;
}

}  // extern "C"

namespace {

struct AppendArgs {
    const void* k_rows;
    const void* v_rows;
    int64_t row_stride;  // bytes
    const int32_t* slot_map;
};

// phase bit 1: key-range kernel; bit 2: merge kernel; bit 4: the key-range
// kernel with the step's append fused in (needs `app`); bit 8: the verify
// kernels (rows grouped by sequence, 4 per page pass) instead of per-token
// decode (with bits 1 and 2).
int attn_decode_phases(int phases, const AppendArgs* app, const float* kscale, const float* vscale, const void* q, const void* kcache, const void* vcache,
                       const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos, const int32_t* tok_seq,
                       const int32_t* block_table, int max_blocks, int block_size, void* out, float scale,
                       const int32_t* cu, int skip_prompts, const int32_t* outs, int spec, int T, int64_t num_blocks,
                       void* workspace, size_t workspace_bytes, void* stream) {
    // A call that merges consumes a pending FP8 output request before any
    // check, so a call that fails leaves no request behind for the next one.
    pkv::Fp8Out fo = {nullptr, nullptr, 0, 0};
    if (phases & 6) {
        fo = t_fp8;
        t_fp8 = {nullptr, nullptr, 0, 0};
    }
    if (T < 0 || Hq <= 0 || Hkv <= 0 || max_blocks <= 0 || num_blocks <= 0 || spec < 1) return PKV_ERR_INVALID;
    const int G = Hkv > 0 && Hq % Hkv == 0 ? Hq / Hkv : 0;
    if (!supported_group(G) || block_size != 16 || (Hkv > 4 && Hkv % 4 != 0)) return PKV_ERR_UNSUPPORTED;
    if (num_blocks > (int64_t)INT32_MAX / 16) return PKV_ERR_INVALID;
    if (T == 0) return PKV_OK;
    if (!q || !kcache || !vcache || !qkv || !pos || !tok_seq || !block_table || !out || !workspace)
        return PKV_ERR_INVALID;
    const bool f8 = kscale != nullptr;
    // bf16 decode for G != 4 runs the verify kernels (each row of a
    // sequence's consecutive rows attends its own keys, the same results as
    // one token at a time), which read cu.
    // The fused step (bit 4) for G != 4 is the verify kernel with the
    // append fused in, then the verify merge.
    if (G != 4 && !f8 && (phases & 7)) phases |= 8;
    if ((skip_prompts || (phases & 8)) && !cu) return PKV_ERR_INVALID;
    const bool verify = phases & 8;
    if (verify && (phases & 4) && G == 4) return PKV_ERR_INVALID;
    if (f8 && ((phases & 4) || !vscale || !aligned(kscale, 4) || !aligned(vscale, 4))) return PKV_ERR_INVALID;
    if (qstride < 2 * Hq * pkv::HEAD_DIM || qstride % 8 != 0) return PKV_ERR_INVALID;
    if (!aligned(q, 16) || !aligned(kcache, 16) || !aligned(vcache, 16) || !aligned(qkv, 16) || !aligned(out, 16) ||
        !aligned(workspace, 256))
        return PKV_ERR_INVALID;
    const int groups = (Hkv + 3) / 4, threads = 64 * std::min(Hkv, 4);
    if (phases & 4) {
        if (!app || !app->k_rows || !app->v_rows || !app->slot_map || !cu) return PKV_ERR_INVALID;
        if (!aligned(app->k_rows, 16) || !aligned(app->v_rows, 16) || app->row_stride % 16 != 0 ||
            app->row_stride < (int64_t)Hkv * pkv::HEAD_DIM * 2)
            return PKV_ERR_INVALID;
    }
    const int n_wg = decode_n_wg() * (f8 ? F8_WG_PER_CU : 1);
    const DecodeLayout lay = decode_layout(T, Hq, n_wg, verify, G);
    if (workspace_bytes < lay.total) return PKV_ERR_INVALID;
    if (fo.mode && T > fo.rows) return PKV_ERR_INVALID;
    pkv::DecodeParams p;
    p.fo = fo;
    p.q = (const uint16_t*)q;
    p.kc = (uint16_t*)kcache;
    p.vc = (uint16_t*)vcache;
    p.qkv = (const uint16_t*)qkv;
    p.qstride = qstride;
    p.Hq = Hq;
    p.Hkv = Hkv;
    p.max_blocks = max_blocks;
    p.out = (uint16_t*)out;
    p.scale = scale;
    p.skip_prompts = skip_prompts;
    p.spec = spec;
    p.T = T;
    p.num_blocks = (long)num_blocks;
    char* ws = (char*)workspace;
    p.offs = (int*)(ws + lay.offs);
    p.part_ms = (float*)(ws + lay.ms);
    p.part_acc = (float*)(ws + lay.acc);
    p.n_wg = n_wg;
    p.min_range = g_min_range;
    p.k_rows = app ? (const uint16_t*)app->k_rows : nullptr;
    p.v_rows = app ? (const uint16_t*)app->v_rows : nullptr;
    p.row_stride = app ? (long)(app->row_stride / 2) : 0;
    p.kscale = kscale;
    p.vscale = vscale;
    const int32_t* slot_map = app ? app->slot_map : nullptr;
    if (phases & 5) {
        hipEvent_t e0 = t_ev_start, e1 = t_ev_stop;
        t_ev_start = t_ev_stop = nullptr;
        using RangeKernel = void (*)(pkv::DecodeParams, const int*, const int*, const int*, const int*, const int*);
        using RangeKernelS =
            void (*)(pkv::DecodeParams, const int*, const int*, const int*, const int*, const int*, const int*);
        const RangeKernel rk = verify && f8 ? by_group<RangeKernel>(G, pkv::verify_range8_kernel<1>,
                                                                    pkv::verify_range8_kernel<2>,
                                                                    pkv::verify_range8_kernel<4>,
                                                                    pkv::verify_range8_kernel<6>,
                                                                    pkv::verify_range8_kernel<8>)
                               : f8 ? by_group<RangeKernel>(G, pkv::decode_range8_kernel<1>,
                                                            pkv::decode_range8_kernel<2>,
                                                            pkv::decode_range8_kernel<4>,
                                                            pkv::decode_range8_kernel<6>,
                                                            pkv::decode_range8_kernel<8>)
                                    : nullptr;
        const RangeKernelS vk = !verify || f8 ? nullptr
                                : (phases & 4) ? by_group<RangeKernelS>(G, pkv::verify_range_kernel<1, true>,
                                                                        pkv::verify_range_kernel<2, true>,
                                                                        pkv::verify_range_kernel<4, true>,
                                                                        pkv::verify_range_kernel<6, true>,
                                                                        pkv::verify_range_kernel<8, true>)
                                               : by_group<RangeKernelS>(G, pkv::verify_range_kernel<1>,
                                                                        pkv::verify_range_kernel<2>,
                                                                        pkv::verify_range_kernel<4>,
                                                                        pkv::verify_range_kernel<6>,
                                                                        pkv::verify_range_kernel<8>);
        if (rk)
            hipExtLaunchKernelGGL(rk, dim3(n_wg, groups), dim3(threads), 0, (hipStream_t)stream, e0, e1, 0, p, pos,
                                  tok_seq, block_table, cu, outs);
        else if (vk)
            hipExtLaunchKernelGGL(vk, dim3(n_wg, groups), dim3(threads), 0, (hipStream_t)stream, e0, e1, 0, p, pos,
                                  tok_seq, block_table, cu, outs, slot_map);
        else if (phases & 4)
            hipExtLaunchKernelGGL((pkv::decode_range_kernel<4, true>), dim3(n_wg, groups), dim3(threads), 0,
                                  (hipStream_t)stream, e0, e1, 0, p, pos, tok_seq, block_table, cu, outs, slot_map);
        else
            hipExtLaunchKernelGGL((pkv::decode_range_kernel<4, false>), dim3(n_wg, groups), dim3(threads), 0,
                                  (hipStream_t)stream, e0, e1, 0, p, pos, tok_seq, block_table, cu, outs, slot_map);
        const int st = launch_status();
        if (st != PKV_OK) return st;
    }
    if ((phases & 2) && verify) {
        // waves per (row, head) block chosen as for decode_merge_kernel below
        using MergeKernel = void (*)(pkv::DecodeParams, const int*, const int*, const int*, const int*);
        const int nw = (int64_t)T * Hq < device_cus() ? 16 : (int64_t)T + n_wg <= 12 * (int64_t)T ? 1 : 4;
        const bool r4 = pkv::vf_rows(G) == 4;
        const MergeKernel mk = nw == 16 ? (r4 ? pkv::verify_merge_kernel<4, 16> : pkv::verify_merge_kernel<2, 16>)
                               : nw == 1 ? (r4 ? pkv::verify_merge_kernel<4, 1> : pkv::verify_merge_kernel<2, 1>)
                                         : (r4 ? pkv::verify_merge_kernel<4, 4> : pkv::verify_merge_kernel<2, 4>);
        hipLaunchKernelGGL(mk, dim3(T, Hq), dim3(64 * nw), 0, (hipStream_t)stream, p, pos, tok_seq, cu, outs);
        return launch_status();
    }
    if (phases & 2) {
        // Waves per (token, head) block: 16 when there are fewer blocks than
        // CUs (a head's records, up to one per range, load in one round);
        // one when a token has at most 12 records on average ((T + n_wg) / T:
        // one wave folds 16 per round and skips the cross-wave combine;
        // measured faster at 9, the E4M3 C3 step's two ranges per CU, and
        // slower at 17); else 4. Any count is correct; this only picks the
        // faster launch.
        if ((int64_t)T * Hq < device_cus())
            hipLaunchKernelGGL(pkv::decode_merge_kernel<16>, dim3(T, Hq), dim3(1024), 0, (hipStream_t)stream, p);
        else if ((int64_t)T + n_wg <= 12 * (int64_t)T)
            hipLaunchKernelGGL(pkv::decode_merge_kernel<1>, dim3(T, Hq), dim3(64), 0, (hipStream_t)stream, p);
        else
            hipLaunchKernelGGL(pkv::decode_merge_kernel<4>, dim3(T, Hq), dim3(256), 0, (hipStream_t)stream, p);
        return launch_status();
    }
    return PKV_OK;
}

}  // namespace

extern "C" {

#define PKV_DECODE_ARGS                                                                                            \
    const void *q, const void *kcache, const void *vcache, const void *qkv, int qstride, int Hq, int Hkv,          \
        const int32_t *pos, const int32_t *tok_seq, const int32_t *block_table, int max_blocks, int block_size,    \
        void *out, float scale, const int32_t *cu, int skip_prompts, const int32_t *outs, int spec, int T,         \
        int64_t num_blocks, void *workspace, size_t workspace_bytes, void *stream
#define PKV_DECODE_PASS                                                                                           \
    q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks, block_size, out, scale, cu,  \
        skip_prompts, outs, spec, T, num_blocks, workspace, workspace_bytes, stream

int pkv_attn_decode(PKV_DECODE_ARGS) { return attn_decode_phases(3, nullptr, nullptr, nullptr, PKV_DECODE_PASS); }
int pkv_attn_decode_split(PKV_DECODE_ARGS) {
    return attn_decode_phases(1, nullptr, nullptr, nullptr, PKV_DECODE_PASS);
}
int pkv_attn_decode_merge(PKV_DECODE_ARGS) {
    return attn_decode_phases(2, nullptr, nullptr, nullptr, PKV_DECODE_PASS);
}

int pkv_attn_verify(PKV_DECODE_ARGS) { return attn_decode_phases(8 | 3, nullptr, nullptr, nullptr, PKV_DECODE_PASS); }

int pkv_attn_decode_e4m3(const void* q, const void* kcache, const void* vcache, const float* kscale,
                         const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                         const int32_t* tok_seq, const int32_t* block_table, int max_blocks, int block_size, void* out,
                         float scale, const int32_t* cu, int skip_prompts, const int32_t* outs, int spec, int T,
                         int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream) {
    if (!kscale || !vscale) {
        t_fp8 = {nullptr, nullptr, 0, 0};  // the failed call still consumes a pending FP8 request
        return PKV_ERR_INVALID;
    }
    return attn_decode_phases(3, nullptr, kscale, vscale, PKV_DECODE_PASS);
}

int pkv_attn_verify_e4m3(const void* q, const void* kcache, const void* vcache, const float* kscale,
                         const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                         const int32_t* tok_seq, const int32_t* block_table, int max_blocks, int block_size, void* out,
                         float scale, const int32_t* cu, int skip_prompts, const int32_t* outs, int spec, int T,
                         int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream) {
    if (!kscale || !vscale) {
        t_fp8 = {nullptr, nullptr, 0, 0};
        return PKV_ERR_INVALID;
    }
    return attn_decode_phases(8 | 3, nullptr, kscale, vscale, PKV_DECODE_PASS);
}

int pkv_attn_decode_step(const void* k_rows, const void* v_rows, int64_t row_stride, const int32_t* slot_map,
                         PKV_DECODE_ARGS) {
    const AppendArgs app{k_rows, v_rows, row_stride, slot_map};
    return attn_decode_phases(4 | 2, &app, nullptr, nullptr, PKV_DECODE_PASS);
}

}  // extern "C"

// Scratch of pkv_attn_decode_step_noalloc: the decode workspace (key offsets
// and split partials) in a file-scope device array, so the call allocates
// nothing. Each device holds its own copy for the life of the process. In
// host code `scratch` names a host-side stand-in, never the device array:
// kernels get the address hipGetSymbolAddress returns for the current
// device, looked up once per device and kept in g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[PKV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {nullptr};

// The current device's scratch address (looked up on the device's first
// call, with that device current).
int scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return status_of(e);
    if (dev < 0 || dev >= MAX_DEVICES) return PKV_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return status_of(e);
        if (!p) return PKV_ERR_INVALID;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return PKV_OK;
}

}  // namespace

extern "C" {

int pkv_attn_decode_step_noalloc(const void* k_rows, const void* v_rows, int64_t row_stride, const int32_t* slot_map,
                                 const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride,
                                 int Hq, int Hkv, const int32_t* pos, const int32_t* tok_seq,
                                 const int32_t* block_table, int max_blocks, int block_size, void* out, float scale,
                                 const int32_t* cu, int skip_prompts, const int32_t* outs, int spec, int T,
                                 int64_t num_blocks, void* stream) {
    // G = 4 runs the decode records, other groups the verify records
    const bool vrec = Hkv > 0 && Hq != 4 * Hkv;
    if (T < 0 || Hq <= 0 ||
        decode_layout(T, Hq, decode_n_wg(), vrec, Hkv > 0 && Hq % Hkv == 0 ? Hq / Hkv : 0).total >
            PKV_NOALLOC_SCRATCH_BYTES) {
        t_fp8 = {nullptr, nullptr, 0, 0};  // the failed call still consumes a pending FP8 request
        return T < 0 || Hq <= 0 ? PKV_ERR_INVALID : PKV_ERR_UNSUPPORTED;
    }
    // The fused step runs the bf16 key-range kernel (decode_n_wg() ranges);
    // its layout must fit the array. Nothing in it needs clearing: the range
    // kernel writes every offset and partial the merge reads.
    void* workspace = nullptr;
    const int st = scratch_ptr(&workspace);
    if (st != PKV_OK) {
        t_fp8 = {nullptr, nullptr, 0, 0};
        return st;
    }
    const size_t workspace_bytes = PKV_NOALLOC_SCRATCH_BYTES;
    const AppendArgs app{k_rows, v_rows, row_stride, slot_map};
    return attn_decode_phases(4 | 2, &app, nullptr, nullptr, PKV_DECODE_PASS);
}

}  // extern "C"

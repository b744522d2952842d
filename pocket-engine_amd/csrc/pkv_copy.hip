// Byte-exact data movement of the paged KV cache: append (scatter by slot),
// gather (through a block table) and page copy (copy-on-write).
//
// Cache layout (reference model.rs:1166-1197): K and V pools of
// [pages * block_size][Hkv][head_dim]; one slot row (all kv heads) is
// `row_bytes` = Hkv * head_bytes contiguous bytes, so a page is
// block_size * row_bytes contiguous bytes. Every kernel copies whole slot
// rows with 16-byte vector accesses when rows and pointers allow it.
#pragma once
#include "pkv_common.h"

namespace pkv {

template <typename V>
__device__ __forceinline__ void copy_row(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, int n,
                                         int tid, int nthr) {
    V* d = reinterpret_cast<V*>(dst);
    const V* s = reinterpret_cast<const V*>(src);
    for (int i = tid; i < n; i += nthr) d[i] = s[i];
}

// KV append (reference attn_prep's cache stores, qwen35.cu:1090-1100 and
// 1120-1127, without the norm and rotary which the caller has applied):
// for token t with slot = slot_map[t] >= 0, cache[slot] := row t. One block
// per (token, K|V); `vec` selects 16-byte (2), 4-byte (1) or byte (0) moves.
// Slots outside [0, num_slots) are skipped like padding rows (slot < 0).
__global__ void __launch_bounds__(256) append_kernel(const uint8_t* __restrict__ ksrc,
                                                     const uint8_t* __restrict__ vsrc, long stride,
                                                     const int* __restrict__ slot_map, int row_bytes,
                                                     uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
                                                     long num_slots, int vec) {
    const int t = blockIdx.x;
    const long slot = slot_map[t];
    if (slot < 0 || slot >= num_slots) return;
    const bool is_v = blockIdx.y != 0;
    const uint8_t* src = (is_v ? vsrc : ksrc) + (size_t)t * stride;
    uint8_t* dst = (is_v ? vc : kc) + (size_t)slot * row_bytes;
    if (vec == 2)
        copy_row<uint4>(dst, src, row_bytes >> 4, threadIdx.x, blockDim.x);
    else if (vec == 1)
        copy_row<uint32_t>(dst, src, row_bytes >> 2, threadIdx.x, blockDim.x);
    else
        copy_row<uint8_t>(dst, src, row_bytes, threadIdx.x, blockDim.x);
}

// The same for rows of 256 * CPT / 2 16-byte chunks (2, 4 or 8 KiB: Hkv 4,
// 8 or 16 at head_dim 256 in bf16), 16-byte aligned: a block of 256 threads
// takes APP_TOK tokens, thread i moving chunk i (then i + 256, ...) of the
// token's K row followed by its V row, and issues all of its loads (read-once
// source rows: nontemporal) before its stores, so each thread keeps
// APP_TOK * CPT 16-byte moves in flight.
constexpr int APP_TOK = 4;
template <int CPT>
__global__ void __launch_bounds__(256) append_rows_kernel(const uint8_t* __restrict__ ksrc,
                                                          const uint8_t* __restrict__ vsrc, long stride,
                                                          const int* __restrict__ slot_map, int T,
                                                          uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
                                                          long num_slots) {
    constexpr int N = 128 * CPT;  // 16-byte chunks per row
    const int t0 = blockIdx.x * APP_TOK, tid = threadIdx.x;
    uint4 buf[APP_TOK][CPT];
    long slot[APP_TOK];
#pragma unroll
    for (int u = 0; u < APP_TOK; u++) {
        const int t = t0 + u;
        slot[u] = t < T ? slot_map[t] : -1;
        if (slot[u] < 0 || slot[u] >= num_slots) continue;
#pragma unroll
        for (int c = 0; c < CPT; c++) {
            const int i = c * 256 + tid;  // < 2 N
            const uint8_t* src = (i < N ? ksrc : vsrc) + (size_t)t * stride + 16 * (i < N ? i : i - N);
            buf[u][c] = load_nt(src);
        }
    }
#pragma unroll
    for (int u = 0; u < APP_TOK; u++) {
        if (slot[u] < 0 || slot[u] >= num_slots) continue;
#pragma unroll
        for (int c = 0; c < CPT; c++) {
            const int i = c * 256 + tid;
            uint8_t* dst = (i < N ? kc : vc) + (size_t)slot[u] * (16 * N) + 16 * (i < N ? i : i - N);
            *reinterpret_cast<uint4*>(dst) = buf[u][c];
        }
    }
}

// Gather one sequence's first L slot rows into dense [L][row] buffers:
// dense[j] = cache[bt[j / bs] * bs + j % bs]. Four rows per block of 256.
// Page ids outside [0, num_blocks) are clamped into the pool (garbage in,
// garbage out, never an out-of-bounds access).
__global__ void __launch_bounds__(256) gather_kernel(const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc,
                                                     const int* __restrict__ bt, int L, int bs, int row_bytes,
                                                     long num_blocks, uint8_t* __restrict__ ko,
                                                     uint8_t* __restrict__ vo, int vec) {
    const int sub = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = blockIdx.x * 4 + sub;
    if (j >= L) return;
    long page = bt[j / bs];
    page = page < 0 ? 0 : page >= num_blocks ? num_blocks - 1 : page;
    const size_t slot = (size_t)page * bs + j % bs;
    const bool is_v = blockIdx.y != 0;
    const uint8_t* src = (is_v ? vc : kc) + slot * row_bytes;
    uint8_t* dst = (is_v ? vo : ko) + (size_t)j * row_bytes;
    if (vec == 2)
        copy_row<uint4>(dst, src, row_bytes >> 4, lane, 64);
    else if (vec == 1)
        copy_row<uint32_t>(dst, src, row_bytes >> 2, lane, 64);
    else
        copy_row<uint8_t>(dst, src, row_bytes, lane, 64);
}

// Page copy for copy-on-write: page dst[i] := page src[i] in the K and V
// pools. One block per (pair, K|V, slice of the page); 16-byte moves.
// Pairs whose ids fall outside the pool are skipped.
__global__ void __launch_bounds__(256) page_copy_kernel(uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
                                                        const int* __restrict__ src, const int* __restrict__ dst,
                                                        long page_bytes, long num_blocks, int slices) {
    const int i = blockIdx.x;
    const long s = src[i], d = dst[i];
    if (s < 0 || d < 0 || s >= num_blocks || d >= num_blocks) return;
    uint8_t* pool = blockIdx.y ? vc : kc;
    const long n = page_bytes >> 4, per = (n + slices - 1) / slices;
    const long b = blockIdx.z * per, e = min(n, b + per);
    const uint4* sp = reinterpret_cast<const uint4*>(pool + s * page_bytes);
    uint4* dp = reinterpret_cast<uint4*>(pool + d * page_bytes);
    for (long k = b + threadIdx.x; k < e; k += blockDim.x) dp[k] = sp[k];
}

// Draft-pass metadata (reference mtp_next, qwen35.cu:2633-2650): for
// sequence s (step row rows[s]) and draft pass k, the position p =
// pos[rows[s]] + k, its cache slot through the block table while p <=
// limits[s] (-1 past the limit: the draft layer writes no KV there), and the
// three rotary position rows shifted by k. One thread per sequence. A page
// index past max_blocks maps to -1 (the reference reads past the row there).
__device__ __forceinline__ void mtp_next_one(int s, const int* __restrict__ rows, const int* __restrict__ pos,
                                             const int* __restrict__ rope, int rope_stride,
                                             const int* __restrict__ block_table, int max_blocks, int block_size,
                                             const int* __restrict__ limits, int k, int* __restrict__ dpos,
                                             int* __restrict__ dslot, int* __restrict__ drope, int S) {
    const int r = rows[s], p = pos[r] + k;
    dpos[s] = p;
    const int pi = p / block_size;
    dslot[s] = p <= limits[s] && pi < max_blocks
                   ? block_table[(size_t)s * max_blocks + pi] * block_size + p % block_size
                   : -1;
#pragma unroll
    for (int axis = 0; axis < 3; axis++) drope[axis * S + s] = rope[(size_t)axis * rope_stride + r] + k;
}

__global__ void __launch_bounds__(256) mtp_next_kernel(const int* __restrict__ rows, const int* __restrict__ pos,
                                                       const int* __restrict__ rope, int rope_stride,
                                                       const int* __restrict__ block_table, int max_blocks,
                                                       int block_size, const int* __restrict__ limits, int k,
                                                       int* __restrict__ dpos, int* __restrict__ dslot,
                                                       int* __restrict__ drope, int S) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s < S)
        mtp_next_one(s, rows, pos, rope, rope_stride, block_table, max_blocks, block_size, limits, k, dpos, dslot,
                     drope, S);
}

}  // namespace pkv

namespace pkv {

// Single-query attention over dense f32 rows (the check path of the
// reference's CPU plumbing configuration: a sequence gathered to
// [L][Hkv][D], its last token's query): block (s, h) computes
// out[s][h][d] = sum_j e^(x_j - max) v_j[d] / sum_j e^(x_j - max),
// x_j = scale * q[s][h] . k_j over the sequence's rows off[s] .. off[s] +
// len[s] - 1, kv head h / (Hq / Hkv). Keys in chunks of 256 (a thread per
// key for the scores, a thread per dim for the weighted sum), with the
// running max and sum rescaled per chunk; f32 throughout.
__global__ void __launch_bounds__(256) attn_dense_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                             const float* __restrict__ v,
                                                             const int* __restrict__ off,
                                                             const int* __restrict__ len, int Hq, int Hkv, int D,
                                                             float scale, float* __restrict__ out) {
    __shared__ float sq[256];
    __shared__ float sp[256];
    __shared__ float red[4];
    const int s = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int kvh = h / (Hq / Hkv), L = len[s];
    const float* qrow = q + ((size_t)s * Hq + h) * D;
    if (tid < D) sq[tid] = qrow[tid];
    __syncthreads();
    float m = -INFINITY, l = 0.f, acc = 0.f;  // acc: dim tid
    auto block_max = [&](float x) {
        for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
        if (lane == 0) red[w] = x;
        __syncthreads();
        x = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        return x;
    };
    auto block_sum = [&](float x) {
        for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
        if (lane == 0) red[w] = x;
        __syncthreads();
        x = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
        return x;
    };
    for (int j0 = 0; j0 < L; j0 += 256) {
        const int j = j0 + tid;
        float x = -INFINITY;
        if (j < L) {
            const float* krow = k + ((size_t)(off[s] + j) * Hkv + kvh) * D;
            float d0 = 0.f;
            for (int d = 0; d < D; d++) d0 = fmaf(sq[d], krow[d], d0);
            x = scale * d0;
        }
        const float mn = fmaxf(m, block_max(x));
        const float p = j < L ? expf(x - mn) : 0.f;
        const float corr = m == -INFINITY ? 0.f : expf(m - mn);
        sp[tid] = p;
        l = l * corr + block_sum(p);  // block_sum's barriers also publish sp
        m = mn;
        if (tid < D) {
            float a = acc * corr;
            const int n = min(256, L - j0);
            const float* vcol = v + ((size_t)(off[s] + j0) * Hkv + kvh) * D + tid;
            for (int i = 0; i < n; i++) a = fmaf(sp[i], vcol[(size_t)i * Hkv * D], a);
            acc = a;
        }
        __syncthreads();  // sp is rewritten by the next chunk
    }
    if (tid < D) out[((size_t)s * Hq + h) * D + tid] = L > 0 ? acc / l : 0.f;
}

}  // namespace pkv

// Chunked-prefill attention over the paged cache on gfx950 matrix cores.
// Same results as the reference's attn_mfma_g4_t2 / attn_flash_group
// (amd/attention.cuh:12-136, qwen35.cu:1364-1585): for every prompt sequence
// (more than one token, not verifying drafts), every token t at position
// pos[t] and every query head, causal attention over keys 0 .. pos[t]; q is
// scaled by scale * log2(e) and rounded to bf16, scores are in exp2 units,
// P is rounded to bf16 for the P.V product, and the output is gated
// bf16(rbf(O / l) * sigmoid(gate)).
//
// Tiling (this build's own). A workgroup takes BQ consecutive query
// positions of one sequence and one kv head with its G query heads; its
// BQ x G (query, head) columns go 32 to a wave: a wave per (query head,
// block of 32 queries) when BQ >= 32 (G = 4: 64 queries, 8 waves), or per
// (2 heads, 16 queries) on grids of 16-query tiles. Keys stream in tiles of 32 (two pages) staged in LDS
// once for all waves (GQA sharing), K and V both row-major [key][d]. Per
// tile a wave computes
//   S^T[32 keys][32 queries] = K Q^T     16 x v_mfma_f32_32x32x16_bf16
//   O^T[256 d][32 queries] += V^T P^T    16 x v_mfma_f32_32x32x16_bf16
// Computing S transposed leaves each lane with one query's 16 scores (keys
// 8 (r / 4) + 4 (lane / 32) + r % 4), so the online softmax is in-lane plus
// one cross-half shuffle, and the probabilities are already the B operand of
// the second product once the matching V^T fragments are read (keys
// 16 kk + 4 (lane / 32) + {0..3, 8..11}; transposed on the LDS read by
// ds_read_b64_tr_b16). Page ids of full tiles are uniform loads, so the
// staging costs a handful of ALU instructions per tile. q stays in registers (64 VGPRs),
// O^T takes 128 accumulators. The next tile's K/V are loaded into registers
// while the current one is multiplied (double-buffered LDS).
#pragma once
#include "pkv_common.h"
#include "pkv_decode.hip"

namespace pkv {

struct PrefillParams {
    const uint16_t* q;        // [T][Hq][256]
    const uint16_t* kc;       // [pages * bs][Hkv][256]
    const uint16_t* vc;
    const uint16_t* qkv;      // gate: qkv[t * qstride + h * 512 + 256 + d]
    int qstride, Hq, Hkv;
    const int* pos;
    const int* cu;
    int seqs;
    const int* block_table;
    int max_blocks, block_size, bs_log2;
    uint16_t* out;
    float scale;
    const int* outs;
    int spec;
    long num_blocks;
    // E4M3 cache (prefill_tile<.., true>): kc / vc hold bytes, one f32 scale
    // per (slot, kv head)
    const float* kscale;
    const float* vscale;
    // Split keys (prefill_split_kernel): the device's CUs (the split fills
    // them), the workgroups whose records part_ms / part_acc hold, and the
    // records: (max in log2 units, sum) at part_ms[r * 2] and the
    // unnormalised weighted values at part_acc[r * 256], r = workgroup *
    // BQ * G + query * G + head in group (pf_split_rec)
    int cus, split_cap;
    float* part_ms;
    float* part_acc;
    // the split kernel's plan for prefill_merge_kernel: parts and the
    // prompt's query tiles R, written by the split grid's workgroup 0
    int* split_plan;
};

// 8 bytes / 4 bytes by raw buffer loads, as buf_load16 (the base in the
// descriptor, the offset one VGPR): the E4M3 register path's raw bytes and
// scales.
__device__ __forceinline__ uint2 buf_load8(const void* base, uint32_t off) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                                                       0x00020000);
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float buf_load4f(const void* base, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                                                       0x00020000);
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

constexpr int PF_BK = 32;  // keys per tile
// Tile layout in LDS (K and V alike, row-major [key][d]): keys r and r + 16
// are one 1,024-byte pair (one 64-lane global_load_lds_dwordx4 fills it) and
// pairs are padded: K pairs every 1,040 bytes, so the 16 rows a quarter-wave
// reads with ds_read_b128 start 16 bytes apart modulo 256 (distinct banks);
// V pairs every 1,088 bytes (64 modulo 256), so the 4 rows x 64 bytes of a
// half-wave's transposing ds_read_b64_tr_b16 land on distinct banks.
constexpr int PF_KPAIR = 520;  // elements
constexpr int PF_VPAIR = 544;
constexpr int PF_K_ELEMS = 16 * PF_KPAIR;
constexpr int PF_V_ELEMS = 16 * PF_VPAIR;
// Rows hold keys in the order key_of_row(r) = (r & 7) + 16 ((r >> 3) & 1) +
// 8 (r >> 4): the two rows of a pair (r, r + 16) are keys j and j + 8 of the
// same 16-key half, i.e. the same page whenever pages hold 16 keys or more,
// so one DMA of a pair reads from one page. (P and V^T share the row order,
// so only key positions, for masking, depend on it.)
__device__ __forceinline__ constexpr int pf_key_of_row(int r) { return (r & 7) + 16 * ((r >> 3) & 1) + 8 * (r >> 4); }
__device__ __forceinline__ constexpr int pf_row_of_key(int j) { return (j & 7) + 8 * ((j >> 4) & 1) + 16 * ((j >> 3) & 1); }
// Element offset of row r (0..31) of a K or V tile.
__device__ __forceinline__ constexpr int pf_krow(int r) { return (r & 15) * PF_KPAIR + (r >> 4) * HEAD_DIM; }
template <int VP = PF_VPAIR>
__device__ __forceinline__ constexpr int pf_vrow(int r) { return (r & 15) * VP + (r >> 4) * HEAD_DIM; }
// Elements of one K + V stage with V pairs VP elements apart.
__host__ __device__ constexpr int pf_stage(int vp) { return PF_K_ELEMS + 16 * vp; }

// Query positions per workgroup (BQ), query heads per kv head (G) and
// 32-query blocks per wave (NQB): waves = G x BQ / (32 NQB). NQB = 2 feeds
// every K / V^T fragment read from LDS into two MFMAs (half the LDS traffic
// per MFMA) at the cost of 128 q + 256 accumulator registers per wave (one
// wave per SIMD).
#ifndef PKV_PF_NQB
#define PKV_PF_NQB 1
#endif
constexpr int PF_BQ = 64;
constexpr int PF_NQB = PKV_PF_NQB;
constexpr int pf_threads(int bq, int nqb, int G = 4) { return 64 * G * bq / 32 / nqb; }
constexpr int PF_THREADS = pf_threads(PF_BQ, PF_NQB);
constexpr int pow2_floor(int x) { return x >= 1024 ? 1024 : x >= 512 ? 512 : x >= 256 ? 256 : x >= 128 ? 128 : 64; }
// Threads that load and store tiles through registers: a power of two
// (whole 16-byte chunks each); any others only compute.
constexpr int pf_load_threads(int threads) { return pow2_floor(threads); }
constexpr bool pf_pow2(int x) { return (x & (x - 1)) == 0; }
constexpr int pf_log2(int x) { return x <= 1 ? 0 : 1 + pf_log2(x / 2); }
// Register tile paths of a workgroup whose thread count is not a power of
// two (G = 6: 6 or 3 waves) load through every thread, each wave taking
// key pairs (2 w, 2 w + 1) + KPU u of the tile (KPU = threads / 32), so a
// wave's chunk u lies in one page whenever pages hold 2 keys or more.
// Otherwise the first pf_load_threads() threads load KPU-key groups, one
// page each, when pages hold KPU keys or more. Smallest page (log2) that
// takes the uniform-page path:
constexpr int pf_upage_log2(int threads) { return pf_pow2(threads) ? pf_log2(pf_load_threads(threads) / 32) : 1; }
// Waves that issue the DMA path's tile loads (pairs per wave 16 / that: 2,
// 4 or 8).
constexpr int pf_dma_waves(int threads) { return pow2_floor(threads) / 64 > 8 ? 8 : pow2_floor(threads) / 64; }
constexpr int PF_STAGE = PF_K_ELEMS + PF_V_ELEMS;
// LDS stages of K / V tiles: 3 (one barrier per tile) unless the launch's
// shared memory only holds 2 (two barriers per tile).
constexpr int PF_NST = 3;
// Stages of the library's bf16 prompt kernel (LDS-DMA tiles): 4 with two
// tiles per barrier for G = 6, whose 6 waves sit 2, 2, 1, 1 on the SIMDs
// (the waves drift within a step and the lone ones fill in: C4 at 24 query
// heads 7.16 -> 6.68 ms), else 3 with a barrier per tile (4 stages measured
// 0.6-1.5 % slower at G = 2, 4 and 8, whose 8 waves sit two per SIMD).
constexpr int pf_lib_nst(int G) { return G == 6 ? 4 : 3; }
// The E4M3 prompt kernels (tiles through registers) take four stages and two
// tiles per barrier for every group: C4 over E4M3 at G = 4 / 6 / 8 4.84 /
// 10.39 / 9.55 -> 4.70 / 9.64 / 9.21 ms.
constexpr int pf_lib_nst_f8(int G) { return 4; }
// The DMA path's page-id ring after the stages: per DMA wave 4 slots x 4 ids.
constexpr int pf_ids_bytes(int threads) { return pf_dma_waves(threads) * 4 * 4 * 4; }
constexpr int PF_IDS_BYTES = pf_ids_bytes(PF_THREADS);
// The library's query positions per workgroup for G heads per kv head: 6 or
// 8 waves of 32 columns (G = 6: 6 waves, 32 queries), one workgroup per CU
// with 3 stages. (Over an E4M3 cache, G = 6 in 3 waves of 16 queries x 2
// heads with two workgroups per CU spills 584 bytes per lane at 256 VGPRs.)
constexpr int pf_lib_bq(int G) { return G >= 6 ? 32 : 256 / G; }
constexpr int pf_lib_nqb(int G) { return G == 4 ? PF_NQB : 1; }
constexpr int pf_lib_threads(int G) { return pf_threads(pf_lib_bq(G), pf_lib_nqb(G), G); }

// Split keys (prefill_split_kernel). R query tiles x Hkv kv heads = w
// workgroups leave CUs idle when w < cus: each tile's keys then go to
// max(2, cus / w) ranges (one round of cus workgroups for a small w; two
// for w >= cus / 2, where halving the ranges beats leaving them whole),
// never under PF_SPLIT_MIN key tiles each (a range then still amortises its
// query load and records). A split grid holds parts * w < 2 cus workgroups.
constexpr int PF_SPLIT_MIN = 4;
__host__ __device__ constexpr int pf_split_parts(int w, int cus) {
    return w <= 0 || w >= cus ? 1 : (cus / w > 2 ? cus / w : 2);
}
// Key tiles per range of a query tile of nt key tiles.
__host__ __device__ constexpr int pf_split_per(int nt, int parts) {
    return (nt + parts - 1) / parts > PF_SPLIT_MIN ? (nt + parts - 1) / parts : PF_SPLIT_MIN;
}
// Record of query q (in its tile) and head hh (in its group) from split
// workgroup wg.
template <int BQ, int G>
__device__ __forceinline__ size_t pf_split_rec(int wg, int q, int hh) {
    return ((size_t)wg * BQ + q) * G + hh;
}
// Split workgroup index of (query tile x, kv head kvh, range z) among R
// tiles.
__device__ __forceinline__ int pf_split_index(int x, int kvh, int z, int R, int Hkv) { return x + R * (kvh + Hkv * z); }
constexpr size_t prefill_smem_bytes(int nst = PF_NST, int threads = PF_THREADS) {
    return (size_t)nst * PF_STAGE * 2 + pf_ids_bytes(threads);
}
// V pairs 1,056 bytes apart (528 elements): two stages then take 67,072
// bytes, so two workgroups share a CU (the code object's attn_groupr
// kernels, and the library's fine-tile kernel below).
constexpr int PF_VPAIR_TIGHT = 528;
// The fine-tile prompt kernel: 128 / G queries per workgroup for G <= 4
// (4 waves of one head x 32 queries), 16 for G = 6 or 8 (a wave per 2
// heads x 16 queries), two stages with tight V pairs: two workgroups per CU.
constexpr int pf_fine_bq(int G) { return G >= 6 ? 16 : 128 / G; }
constexpr int pf_fine_threads(int G) { return pf_threads(pf_fine_bq(G), 1, G); }
constexpr size_t pf_fine_smem_bytes(int G) {
    return (size_t)2 * pf_stage(PF_VPAIR_TIGHT) * 2 + pf_ids_bytes(pf_fine_threads(G));
}

// NP LDS DMA pairs from one uniform base: pair j reads 16 bytes per lane at
// base + off[j] into LDS at m0 + j * lds_step (+ 16 x lane). The m0 writes
// (and the one wait state each needs) stay in one asm block.
template <int NP>
__device__ __forceinline__ void dma_pairs(const void* base, const uint32_t (&off)[NP], uint32_t m0,
                                          uint32_t lds_step) {
    static_assert(NP == 2 || NP == 4 || NP == 8, "2, 4 or 8 pairs");
    if constexpr (NP == 8) {
        const uint32_t lo[4] = {off[0], off[1], off[2], off[3]}, hi[4] = {off[4], off[5], off[6], off[7]};
        dma_pairs<4>(base, lo, m0, lds_step);
        dma_pairs<4>(base, hi, m0 + 4 * lds_step, lds_step);
    } else if constexpr (NP == 2) {
        asm volatile(
            "s_mov_b32 m0, %3\n\ts_nop 0\n\t"
            "global_load_lds_dwordx4 %1, %0\n\t"
            "s_add_u32 m0, m0, %4\n\ts_nop 0\n\t"
            "global_load_lds_dwordx4 %2, %0"
            :
            : "s"(base), "v"(off[0]), "v"(off[1]), "s"(__builtin_amdgcn_readfirstlane(m0)), "s"(lds_step)
            : "memory", "scc");
    } else {
        asm volatile(
            "s_mov_b32 m0, %5\n\ts_nop 0\n\t"
            "global_load_lds_dwordx4 %1, %0\n\t"
            "s_add_u32 m0, m0, %6\n\ts_nop 0\n\t"
            "global_load_lds_dwordx4 %2, %0\n\t"
            "s_add_u32 m0, m0, %6\n\ts_nop 0\n\t"
            "global_load_lds_dwordx4 %3, %0\n\t"
            "s_add_u32 m0, m0, %6\n\ts_nop 0\n\t"
            "global_load_lds_dwordx4 %4, %0"
            :
            : "s"(base), "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]),
              "s"(__builtin_amdgcn_readfirstlane(m0)), "s"(lds_step)
            : "memory", "scc");
    }
}

// The query tiles of sequence i (0 past the last): a prompt sequence
// (more than one row, not verifying drafts) has ceil(rows / BQ).
template <int BQ>
__device__ __forceinline__ int seq_tiles(const PrefillParams& p, int i) {
    if (i >= p.seqs) return 0;
    const int n = p.cu[i + 1] - p.cu[i];
    return n > 1 && !is_spec(p.outs, p.spec, i) ? (n + BQ - 1) / BQ : 0;
}

// The prompt's query tiles, summed by each wave over its lanes (64
// sequences a round: a mixed step's one-row decode sequences cost a load
// round per 64, not one each).
template <int BQ>
__device__ __forceinline__ int prompt_tiles(const PrefillParams& p) {
    const int lane = threadIdx.x & 63;
    int total = 0;
    for (int c = 0; c < p.seqs; c += 64) total += seq_tiles<BQ>(p, c + lane);
#pragma unroll
    for (int o = 32; o; o >>= 1) total += __shfl_xor(total, o);
    return __builtin_amdgcn_readfirstlane(total);
}

// The query tile of this workgroup among the prompt sequences: tile
// total - 1 - `tile` of the concatenated BQ-query tiles of the prompt
// sequences, found by each wave with a prefix sum over its lanes. Returns
// false if the grid has more blocks than tiles. Called by whole waves.
template <int BQ>
__device__ __forceinline__ bool find_prefill_tile(const PrefillParams& p, int tile, int& s, int& tb, int& nb,
                                                  int total = -1) {
    // Tiles are taken last first: a sequence's later tiles attend more keys,
    // so the longest work is dispatched first and the short tiles fill the
    // tail.
    if (total < 0) total = prompt_tiles<BQ>(p);
    if (tile >= total) return false;
    tile = total - 1 - tile;
    const int lane = threadIdx.x & 63;
    int base = 0;  // tiles of the sequences before this round
    s = -1;
    for (int c = 0; c < p.seqs; c += 64) {
        const int k = seq_tiles<BQ>(p, c + lane);
        int incl = k;  // inclusive prefix sum over lanes
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (lane >= o) incl += v;
        }
        // the first lane whose tiles reach past `tile`
        const unsigned long long hit = __ballot(base + incl > tile);
        if (hit) {
            const int l = __ffsll((long long)hit) - 1;
            s = c + l;
            tile -= base + __shfl(incl - k, l);
            break;
        }
        base += __shfl(incl, 63);
    }
    s = __builtin_amdgcn_readfirstlane(s);
    if (s < 0) return false;
    tile = __builtin_amdgcn_readfirstlane(tile);
    tb = p.cu[s] + tile * BQ;
    nb = min(BQ, p.cu[s + 1] - tb);
    return true;
}

// One workgroup's query tile (sequence s, rows tb .. tb + nb - 1, nb <= BQ);
// pf_smem holds prefill_smem_bytes(NST). UPAGE: every page holds at least
// THREADS / 32 keys. F8: an E4M3 cache, dequantised while
// the tiles load as the reference's attn_group8 does (qwen35.cu:1424-1436):
// K' = bf16(k * kscale), V' = bf16(v * vscale); the rest is unchanged.
//
// Workgroup (query tile, kv head kvh, key range part). SPL with parts > 1:
// this workgroup, number wg of the split grid, takes key range part of
// parts (pf_split_per key tiles each; an empty range returns at once) and
// leaves a record per (row, query head) for prefill_merge_kernel instead of
// the gated rows.
template <int G, int BQ, int NQB, bool F8, bool UPAGE, int NST, bool DMA, int VP = PF_VPAIR, bool SPL = false>
__device__ __forceinline__ void prefill_tile(const PrefillParams& p, uint16_t* pf_smem, int s, int tb, int nb,
                                             int kvh, int part = 0, int parts = 1, int wg = 0) {
    constexpr int THREADS = pf_threads(BQ, NQB, G);
    // BQ = 16: a wave's 32 columns are 2 heads x 16 queries
    constexpr bool PAIRED = BQ < 32;
    static_assert(!PAIRED || (BQ == 16 && NQB == 1 && G % 2 == 0), "16-query tiles pair heads");
    static_assert(PAIRED || BQ % (32 * NQB) == 0, "whole 32-query blocks");
    // Register paths: tiles load through the first LDT threads (a power of
    // two), or (WP) through every thread, in wave-sized key pairs.
    constexpr bool WP = !DMA && !pf_pow2(THREADS);
    constexpr int LDT = WP ? THREADS : pf_load_threads(THREADS);
    static_assert(WP || PF_BK * HEAD_DIM / 8 % LDT == 0, "whole 16-byte chunks per thread");
    static_assert(!WP || THREADS % 64 == 0, "whole waves");
    // Buffer b: K tile at pf_smem + b * STAGE, V tile right after it.
    constexpr int STAGE = pf_stage(VP);
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31,
              lh = lane >> 5;
    const bool loader = LDT == THREADS || tid < LDT;  // wave-uniform
    // This lane's query head, and the wave's first query block (BQ >= 32).
    const int h = kvh * G + (PAIRED ? 2 * wave + (lq >> 4) : wave % G);
    const int qb0 = PAIRED ? 0 : (wave / G) * NQB;
    // Query (index in the tile) of this lane's column in block qb, and the
    // first query of the block.
    auto qcol = [&](int qb) { return PAIRED ? (lq & 15) : (qb0 + qb) * 32 + lq; };
    auto qfirst = [&](int qb) { return PAIRED ? 0 : (qb0 + qb) * 32; };
    const int qp0 = p.pos[tb];
    const int L = qp0 + nb;  // keys this tile needs: 0 .. L - 1
    const int* bt = p.block_table + (size_t)s * p.max_blocks;
    const size_t row = (size_t)p.Hkv * HEAD_DIM;

    // This wave's queries: blocks qb0 + qb (queries 32 (qb0 + qb) + lq of the
    // tile), q^T operands scaled into log2 units.
    bf16x8 qf[NQB][16];
    // (called once the tile path has requested its first page ids, so the
    // q loads overlap that request)
    auto load_q = [&]() __attribute__((always_inline)) {
        const float f = p.scale * LOG2E;
#pragma unroll
        for (int qb = 0; qb < NQB; qb++) {
            const int myq = qcol(qb);
            const bool ok = myq < nb;
            const uint16_t* qrow = p.q + ((size_t)(tb + (ok ? myq : 0)) * p.Hq + h) * HEAD_DIM;
#pragma unroll
            for (int kk = 0; kk < 16; kk++) {
                uint4 raw = ok ? *reinterpret_cast<const uint4*>(qrow + 16 * kk + 8 * lh) : make_uint4(0, 0, 0, 0);
                // round to nearest even (the hardware conversion)
                raw = make_uint4(pack2_hw(bf_lo(raw.x) * f, bf_hi(raw.x) * f),
                                 pack2_hw(bf_lo(raw.y) * f, bf_hi(raw.y) * f),
                                 pack2_hw(bf_lo(raw.z) * f, bf_hi(raw.z) * f),
                                 pack2_hw(bf_lo(raw.w) * f, bf_hi(raw.w) * f));
                qf[qb][kk] = as_bf16x8(raw);
            }
        }
    };
    f32x16 o[NQB][8];
#pragma unroll
    for (int qb = 0; qb < NQB; qb++)
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[qb][db][r] = 0.f;
    float m[NQB], l[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
        m[qb] = -INFINITY;
        l[qb] = 0.f;
    }
    // the wave's last query position
    const int last = qp0 + min(nb, PAIRED ? BQ : (qb0 + NQB) * 32) - 1;

    // Tile loads: 32 keys x 256 dims of K and of V, both row-major in LDS,
    // NCH 16-byte chunks of each per thread: chunk u is key KPU u + kl0 of
    // the tile (KPU = THREADS / 32 consecutive keys per u), dims c8 .. c8 + 7.
    // When a page holds at least KPU keys, each u reads one page: its id is a
    // uniform (scalar) load and the lane's part of the address is the same
    // for every tile. Every load is issued unconditionally from a valid
    // address (page index clamped to the sequence's last key); keys at or
    // past L are zeroed when the tile is stored to LDS, so no load result is
    // overwritten while in flight.
    constexpr int KPU = LDT / 32;
    constexpr int NCH = (PF_BK + KPU - 1) / KPU;
    // chunk u of this thread holds a key of the tile (wave-uniform: WP
    // leaves the last chunk to the waves whose pairs fit)
    auto chunk_ok = [&](int u) {
        if constexpr (WP)
            return u * KPU + (tid >> 5) < PF_BK;
        else
            return true;
    };
    const int kl0 = tid >> 5, c8 = (tid & 31) * 8;
    uint4 kr[NCH], vr[NCH];
    // E4M3: the raw bytes and scales stay in registers until the tile is
    // stored, so the loads keep their lead over the conversion
    uint2 kw[F8 ? NCH : 1], vw[F8 ? NCH : 1];
    float ksv[F8 ? NCH : 1], vsv[F8 ? NCH : 1];
    // Block size is a power of two (checked on the host): shifts, no division.
    const int bs_log2 = p.bs_log2, bs_mask = (1 << bs_log2) - 1;
    const int last_pi = (L - 1) >> bs_log2;
    auto page_id = [&](int pi) -> size_t {
        long pg = bt[min(pi, last_pi)];
        pg = pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg;
        return (size_t)pg;
    };
    // 8 values at element `at` of a pool: bf16 as stored, or E4M3 bytes times
    // the slot's scale (at `scale_at`), rounded to bf16.
    // `slot` is the key's cache slot, or (fast path) the uniform slot of the
    // KPU-key group with the lane's key offset folded into at / scale_at.
    auto raw8 = [&](const uint16_t* pool, const float* scales, size_t slot, uint32_t at, uint32_t scale_at, uint2& w,
                    float& sc) {
        const uint8_t* base = reinterpret_cast<const uint8_t*>(pool) + slot * row;  // uniform on the fast path
        w = *reinterpret_cast<const uint2*>(base + at);
        sc = (scales + slot * p.Hkv)[scale_at];
    };
    auto cvt8 = [&](uint2 w, float sc) -> uint4 {
        const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w.x, false), b = __builtin_amdgcn_cvt_pk_f32_fp8(w.x, true);
        const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(w.y, false), d = __builtin_amdgcn_cvt_pk_f32_fp8(w.y, true);
        return make_uint4(pack2_hw(a.x * sc, a.y * sc), pack2_hw(b.x * sc, b.y * sc), pack2_hw(c.x * sc, c.y * sc),
                          pack2_hw(d.x * sc, d.y * sc));
    };
    auto load8 = [&](const uint16_t* pool, const float* scales, size_t slot, uint32_t at, uint32_t scale_at) -> uint4 {
        if constexpr (F8) {
            uint2 w;
            float sc;
            raw8(pool, scales, slot, at, scale_at, w, sc);
            return cvt8(w, sc);
        } else {
            // uniform base + 32-bit lane byte offset (the saddr addressing form)
            const uint8_t* base = reinterpret_cast<const uint8_t*>(pool + slot * row);
            return *reinterpret_cast<const uint4*>(base + 2 * at);
        }
    };
    // the lane's key within its group (WP: within its wave's pair)
    uint32_t lane_at, lane_sc;  // lane parts of an element offset and of a scale index
    if constexpr (WP) {
        lane_at = (uint32_t)((lane >> 5) * row + kvh * HEAD_DIM + c8);
        lane_sc = (uint32_t)((lane >> 5) * p.Hkv + kvh);
    } else {
        lane_at = (uint32_t)(kl0 * row + kvh * HEAD_DIM + c8);
        lane_sc = (uint32_t)(kl0 * p.Hkv + kvh);
    }
    // first key of the uniform-page group of chunk u, relative to the tile
    auto group_key = [&](int u) {
        if constexpr (WP)
            return u * KPU + 2 * wave;
        else
            return u * KPU;
    };
    // UPAGE: the page ids of the tile loaded next (uniform), fetched one
    // tile ahead so their latency hides behind a whole tile of work (the
    // block-table reads are vector loads: the barriers keep the compiler
    // from using the scalar cache).
    int ids[NCH];
    auto fetch_ids = [&](int k0) {
#pragma unroll
        for (int u = 0; u < NCH; u++) ids[u] = bt[min((k0 + group_key(u)) >> bs_log2, last_pi)];
    };
    auto load_tile = [&](int k0) {
        if constexpr (UPAGE) {
#pragma unroll
            for (int u = 0; u < NCH; u++) {
                if constexpr (WP) if (!chunk_ok(u)) continue;
                const int kg = k0 + group_key(u);
                long pg = __builtin_amdgcn_readfirstlane(ids[u]);
                pg = pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg;
                const size_t slot = ((size_t)pg << bs_log2) + (kg & bs_mask);  // uniform
                if constexpr (F8) {
                    // buffer loads: the slot row in the descriptor, the
                    // lane's byte and scale offsets one VGPR each
                    kw[u] = buf_load8(reinterpret_cast<const uint8_t*>(p.kc) + slot * row, lane_at);
                    vw[u] = buf_load8(reinterpret_cast<const uint8_t*>(p.vc) + slot * row, lane_at);
                    ksv[u] = buf_load4f(p.kscale + slot * p.Hkv, 4 * lane_sc);
                    vsv[u] = buf_load4f(p.vscale + slot * p.Hkv, 4 * lane_sc);
                } else {
                    // buffer loads: uniform base in the descriptor, the lane's
                    // 32-bit byte offset in one VGPR shared by K and V
                    kr[u] = buf_load16(p.kc + slot * row, 2 * lane_at);
                    vr[u] = buf_load16(p.vc + slot * row, 2 * lane_at);
                }
            }
            fetch_ids(k0 + PF_BK);
        } else {
#pragma unroll
            for (int u = 0; u < NCH; u++) {
                if constexpr (WP) if (!chunk_ok(u)) continue;
                const int kp = k0 + u * KPU + kl0;
                const size_t slot = (page_id(kp >> bs_log2) << bs_log2) + (kp & bs_mask);
                if constexpr (F8) {
                    raw8(p.kc, p.kscale, slot, kvh * HEAD_DIM + c8, kvh, kw[u], ksv[u]);
                    raw8(p.vc, p.vscale, slot, kvh * HEAD_DIM + c8, kvh, vw[u], vsv[u]);
                } else {
                    kr[u] = load8(p.kc, p.kscale, slot, kvh * HEAD_DIM + c8, kvh);
                    vr[u] = load8(p.vc, p.vscale, slot, kvh * HEAD_DIM + c8, kvh);
                }
            }
        }
    };
    auto store_tile = [&](int buf, int k0) {
        uint16_t* sk = pf_smem + buf * STAGE;
        uint16_t* sv = sk + PF_K_ELEMS;
        const bool tail = k0 + PF_BK > L;
        // one chunk at a time (E4M3: converted just before its store, so
        // only one chunk's bf16 values are live)
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            if constexpr (WP) if (!chunk_ok(u)) continue;
            uint4 kx, vx;
            if constexpr (F8) {
                kx = cvt8(kw[u], ksv[u]);
                vx = cvt8(vw[u], vsv[u]);
            } else {
                kx = kr[u];
                vx = vr[u];
            }
            if (tail && k0 + u * KPU + kl0 >= L) kx = vx = make_uint4(0, 0, 0, 0);
            // WP: the lane's LDS rows are recomputed per tile (an opaque
            // copy of kl0) instead of held across the loop, which costs a
            // few VALU where keeping them spilled the raw chunks
            int kl = kl0;
            if constexpr (WP) asm volatile("" : "+v"(kl));
            const int r = pf_row_of_key(u * KPU + kl);
            *reinterpret_cast<uint4*>(sk + pf_krow(r) + c8) = kx;
            *reinterpret_cast<uint4*>(sv + pf_vrow<VP>(r) + c8) = vx;
        }
    };
    // V^T fragments (A operand of O^T += V^T P^T, dims 32 db + lq, keys
    // 16 kk + 8 h + 4 lh + e) come from the row-major V tile through
    // ds_read_b64_tr_b16: in each 16-lane group, result lane i element e is
    // element i % 4 of what lane i / 4 + 4 e read, so lane s of the group
    // reads row 16 kk + 8 h + 4 lh + s / 4, dims 32 db + 16 (group & 1) +
    // 4 (s % 4) (row 16 kk + x sits at pf_vrow(x) + 256 kk).
    const int tr_at = (4 * lh + ((lane & 15) >> 2)) * VP + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // The key tiles this workgroup streams: [kbase, kbase + ntiles * 32).
    int ntiles = (L + PF_BK - 1) / PF_BK, kbase = 0;
    bool records = false;  // SPL: this tile takes more than one range
    if constexpr (SPL) {
        const int per = pf_split_per(ntiles, parts), t0 = part * per;
        records = parts > 1 && ntiles > per;
        ntiles = min(ntiles, t0 + per) - t0;
        kbase = t0 * PF_BK;
        if (ntiles <= 0) return;  // whole workgroup: nothing to merge from this range
    }
    // Tile k0 from stage buf: S^T, online softmax, O^T update.
    auto compute = [&](int buf, int k0) __attribute__((always_inline)) {
        if (k0 <= last) {
            const uint16_t* K = pf_smem + buf * STAGE;
            const uint16_t* Vt = K + PF_K_ELEMS;
            // S^T = K Q^T; each K fragment feeds the wave's NQB blocks. Lane
            // (lh, lq) ends with query lq's scores of keys
            // k0 + 8 (r / 4) + 4 lh + r % 4.
            f32x16 st[NQB];
#pragma unroll
            for (int qb = 0; qb < NQB; qb++)
#pragma unroll
                for (int r = 0; r < 16; r++) st[qb][r] = 0.f;
            const uint16_t* krow = K + pf_krow(lq) + 8 * lh;
            // The bf16 LDS-DMA tile paths (library, split, fine and
            // code-object kernels, G != 6) read K fragments four MFMAs ahead:
            // the scheduler left two, and each pair of MFMAs waited on its
            // reads (C4 +2 %, one 4,096-token prompt -4 %, a 2,048-token chunk
            // on the fine kernel and the code object -4 / -5 %). The E4M3 and
            // G = 6 kernels keep the scheduler's order (more scratch).
            constexpr bool KDEEP = DMA && !F8 && G != 6;
            if constexpr (KDEEP) {
                constexpr int KD = 4;  // K fragments in flight
                uint4 kf[KD];
#pragma unroll
                for (int i = 0; i < KD; i++) kf[i] = *reinterpret_cast<const uint4*>(krow + 16 * i);
#pragma unroll
                for (int kk = 0; kk < 16; kk++) {
                    const bf16x8 a = as_bf16x8(kf[kk % KD]);
                    if (kk + KD < 16) kf[kk % KD] = *reinterpret_cast<const uint4*>(krow + 16 * (kk + KD));
#pragma unroll
                    for (int qb = 0; qb < NQB; qb++)
                        st[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb][kk], st[qb], 0, 0, 0);
                }
                // 4 DS reads, then (MFMA, DS read) x 12, then 4 MFMAs
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
                for (int i = 0; i < 12; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            } else {
#pragma unroll
                for (int kk = 0; kk < 16; kk++) {
                    const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 16 * kk));
#pragma unroll
                    for (int qb = 0; qb < NQB; qb++)
                        st[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb][kk], st[qb], 0, 0, 0);
                }
            }
            uint4 pb[NQB][2];
#pragma unroll
            for (int qb = 0; qb < NQB; qb++) {
                const int qb_first = qp0 + qfirst(qb), qp = qp0 + qcol(qb);
                if (k0 + PF_BK - 1 > qb_first || k0 + PF_BK > L) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int kp = k0 + pf_key_of_row(8 * (r >> 2) + 4 * lh + (r & 3));
                        if (kp > qp || kp >= L) st[qb][r] = -INFINITY;
                    }
                }
                float mx = m[qb];
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, st[qb][r]);
                mx = max_xor32(mx);
                // A query with no key yet keeps -inf; it subtracts 0 so exp2 gives 0.
                const float bse = mx == -INFINITY ? 0.f : mx;
                const float corr = __builtin_amdgcn_exp2f(m[qb] - bse);
                float sum = 0.f;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    st[qb][r] = __builtin_amdgcn_exp2f(st[qb][r] - bse);
                    sum += st[qb][r];
                }
                sum = add_xor32(sum);
                l[qb] = l[qb] * corr + sum;
                m[qb] = mx;
                // Rescale only when some query's max moved (rare after the first tiles).
                if (__any(corr != 1.f)) {
#pragma unroll
                    for (int db = 0; db < 8; db++)
#pragma unroll
                        for (int r = 0; r < 16; r++) o[qb][db][r] *= corr;
                }
                // P^T (bf16) as the B operand: step kk, element e <-> key
                // 16 kk + 8 (e / 4) + 4 lh + e % 4, i.e. register 8 kk + e.
#pragma unroll
                for (int kk = 0; kk < 2; kk++)
                    pb[qb][kk] = make_uint4(pack2_hw(st[qb][8 * kk + 0], st[qb][8 * kk + 1]),
                                            pack2_hw(st[qb][8 * kk + 2], st[qb][8 * kk + 3]),
                                            pack2_hw(st[qb][8 * kk + 4], st[qb][8 * kk + 5]),
                                            pack2_hw(st[qb][8 * kk + 6], st[qb][8 * kk + 7]));
            }
            // O^T += V^T P^T; each V^T fragment feeds the wave's NQB blocks.
            typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
            const uint16_t* vtr = Vt + tr_at;
#pragma unroll
            for (int kk = 0; kk < 2; kk++)
#pragma unroll
                for (int db = 0; db < 8; db++) {
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(vtr + 256 * kk + 32 * db));
                    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(vtr + 8 * VP + 256 * kk + 32 * db));
                    const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                    for (int qb = 0; qb < NQB; qb++)
                        o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_bf16x8(pb[qb][kk]), o[qb][db], 0, 0, 0);
                }
        }
    };
    static_assert(NST >= 2 && NST <= 4, "2, 3 or 4 stages");
    if constexpr (DMA) {
        // Iteration i requests tile i + 2 (stage (i + 2) % 3, freed by the
        // barrier that ended iteration i - 1) and the page ids of tile i + 4,
        // computes tile i, waits for its own DMA of tile i + 1 (everything
        // but this iteration's requests), then one barrier publishes tile
        // i + 1 to all waves. Wave w DMAs pairs NPW w .. NPW w + NPW - 1 of K
        // and of V (keys key_of_row(r) and + 8, one page: pages hold 16 keys
        // or more on this path) and reads their page ids from its own 4-slot
        // ring, filled 4 tiles ahead by its own DMA, so the loop issues no
        // other vector memory reads.
        static_assert(!F8 && UPAGE, "bf16, 16-key pages");
        // The first NDW waves issue the DMA (the others only compute; their
        // waits below find nothing outstanding).
        constexpr int NDW = pf_dma_waves(THREADS);
        constexpr int NPW = 16 / NDW;  // pairs per DMA wave (2 with 8 waves, 4 with 4, 8 with 2)
        const bool dmaw = NDW * 64 == THREADS || wave < NDW;  // wave-uniform
        int* ring = reinterpret_cast<int*>(pf_smem + NST * STAGE) + (dmaw ? wave : 0) * 16;
        const int hi = lane >> 5;
        // Wave w's pairs are rows NPW w .. NPW w + NPW - 1: keys kb + j and
        // kb + j + 8 (j < NPW) of one 16-key half, i.e. one page per tile
        // (pages hold 16 keys or more here): one page id per tile, one
        // uniform base, lane offsets fixed for the loop.
        const int kb = pf_key_of_row(NPW * wave);
        const uint32_t row2 = (uint32_t)row * 2;
        const uint32_t lane_off = (uint32_t)(hi * 8 * row + kvh * HEAD_DIM + 8 * (lane & 31)) * 2;
        uint32_t offs[NPW];
#pragma unroll
        for (int j = 0; j < NPW; j++) offs[j] = lane_off + j * row2;
        const uint32_t lds_k = lds_addr(pf_smem) + (uint32_t)(pf_krow(NPW * wave)) * 2;
        const uint32_t lds_v = lds_addr(pf_smem) + (uint32_t)(PF_K_ELEMS + pf_vrow<VP>(NPW * wave)) * 2;
        auto dma_ids = [&](int k0, int slot) __attribute__((always_inline)) {
            if (dmaw && lane == 0) dma4(bt + min((k0 + kb) >> bs_log2, last_pi), lds_addr(ring + 4 * slot));
        };
        auto dma_tile = [&](int k0, int buf, int slot) __attribute__((always_inline)) {
            if (!dmaw) return;
            long pg = __builtin_amdgcn_readfirstlane(ring[4 * slot]);
            pg = pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg;
            const size_t at = (((size_t)pg << bs_log2) + ((k0 + kb) & bs_mask)) * row2;  // uniform
            const uint32_t so = (uint32_t)(buf * STAGE) * 2;
            dma_pairs<NPW>(reinterpret_cast<const char*>(p.kc) + at, offs, lds_k + so, PF_KPAIR * 2);
            dma_pairs<NPW>(reinterpret_cast<const char*>(p.vc) + at, offs, lds_v + so, VP * 2);
        };
        // V rows of keys at or past L (partial last tile) read stale slots:
        // the wave zeroes its own rows once its DMA has landed (P is 0 there,
        // but 0 x a stale NaN would not be).
        auto zero_tail = [&](int k0, int buf) __attribute__((always_inline)) {
            if (!dmaw || k0 + PF_BK <= L) return;
#pragma unroll
            for (int j = 0; j < NPW; j++) {
                const int r = NPW * wave + j + 16 * hi;
                if (k0 + pf_key_of_row(r) >= L)
                    *reinterpret_cast<uint4*>(pf_smem + buf * STAGE + PF_K_ELEMS + pf_vrow<VP>(r) + 8 * (lane & 31)) =
                        make_uint4(0, 0, 0, 0);
            }
        };
#pragma unroll
        for (int t = 0; t < 4; t++)
            if (t < ntiles) dma_ids(kbase + t * PF_BK, t);
        load_q();
        wait_vm<0>();
        dma_tile(kbase, 0, 0);
        if constexpr (NST == 2) {
            // Two stages: iteration i requests tile i + 1 into the stage the
            // barrier that ended iteration i - 1 freed (and the page ids of
            // tile i + 4), computes tile i, waits for its own DMA of tile
            // i + 1, then one barrier publishes it: one tile of lead.
            wait_vm<0>();
            zero_tail(kbase, 0);
            __syncthreads();
            int buf = 0;
            for (int it = 0; it < ntiles; it++) {
                const int k0 = kbase + it * PF_BK;
                const bool more1 = it + 1 < ntiles, more4 = it + 4 < ntiles;
                if (more1) dma_tile(k0 + PF_BK, buf ^ 1, (it + 1) & 3);
                if (more4) dma_ids(k0 + 4 * PF_BK, it & 3);
                compute(buf, k0);
                if (more1) {
                    if (more4) wait_vm<1>();
                    else wait_vm<0>();
                    buf ^= 1;
                    zero_tail(k0 + PF_BK, buf);
                    __syncthreads();
                }
            }
        } else if constexpr (NST == 4) {
            // Four stages, two tiles per barrier: step s (tiles i = 2 s and
            // i + 1) requests tiles i + 2 and i + 3 into the stages of tiles
            // i - 2 and i - 1 (freed by the barrier that ended step s - 1)
            // and the page ids of tiles i + 6 and i + 7 into the ring slots
            // tiles i + 2 and i + 3 were read from, computes tiles i and
            // i + 1 with no barrier between them, waits for its own
            // requests, then one barrier publishes tiles i + 2 and i + 3.
            if (ntiles > 1) dma_tile(kbase + PF_BK, 1, 1);
            if (ntiles > 4) dma_ids(kbase + 4 * PF_BK, 0);
            if (ntiles > 5) dma_ids(kbase + 5 * PF_BK, 1);
            wait_vm<0>();
            zero_tail(kbase, 0);
            if (ntiles > 1) zero_tail(kbase + PF_BK, 1);
            __syncthreads();
            for (int it = 0; it < ntiles; it += 2) {
                const int k0 = kbase + it * PF_BK;
                if (it + 2 < ntiles) dma_tile(k0 + 2 * PF_BK, (it + 2) & 3, (it + 2) & 3);
                if (it + 3 < ntiles) dma_tile(k0 + 3 * PF_BK, (it + 3) & 3, (it + 3) & 3);
                if (it + 6 < ntiles) dma_ids(k0 + 6 * PF_BK, (it + 2) & 3);
                if (it + 7 < ntiles) dma_ids(k0 + 7 * PF_BK, (it + 3) & 3);
                compute(it & 3, k0);
                if (it + 1 < ntiles) compute((it + 1) & 3, k0 + PF_BK);
                if (it + 2 < ntiles) {
                    wait_vm<0>();
                    zero_tail(k0 + 2 * PF_BK, (it + 2) & 3);
                    if (it + 3 < ntiles) zero_tail(k0 + 3 * PF_BK, (it + 3) & 3);
                    __syncthreads();
                }
            }
        } else {
        if (ntiles > 1) {
            dma_tile(kbase + PF_BK, 1, 1);
            wait_vm<2 * NPW>();
        } else {
            wait_vm<0>();
        }
        zero_tail(kbase, 0);
        __syncthreads();
        int buf = 0;
        for (int it = 0; it < ntiles; it++) {
            const int k0 = kbase + it * PF_BK;
            const bool more2 = it + 2 < ntiles, more4 = it + 4 < ntiles;
            if (more2) dma_tile(k0 + 2 * PF_BK, buf == 0 ? 2 : buf - 1, (it + 2) & 3);
            if (more4) dma_ids(k0 + 4 * PF_BK, it & 3);
            compute(buf, k0);
            if (it + 1 < ntiles) {
                // tile i + 1 landed: all but this iteration's requests
                if (more4) wait_vm<2 * NPW + 1>();
                else if (more2) wait_vm<2 * NPW>();
                else wait_vm<0>();
                buf = buf == 2 ? 0 : buf + 1;
                zero_tail(k0 + PF_BK, buf);
                __syncthreads();
            }
        }
        }
    } else {
    // Only the first LDT threads load and store tiles.
    if (UPAGE && loader) fetch_ids(kbase);
    load_q();
    if constexpr (NST == 4) {
        // Four stages, two tiles per barrier, one tile of registers: step s
        // (tiles i = 2 s and i + 1) stores tile i + 2 (requested during the
        // previous step) into the stage of tile i - 2, requests tile i + 3,
        // computes tile i, stores tile i + 3 into the stage of tile i - 1,
        // requests tile i + 4, computes tile i + 1, then one barrier
        // publishes tiles i + 2 and i + 3.
        if (loader) {
            load_tile(kbase);
            store_tile(0, kbase);
            if (ntiles > 1) {
                load_tile(kbase + PF_BK);
                store_tile(1, kbase + PF_BK);
            }
            if (ntiles > 2) load_tile(kbase + 2 * PF_BK);
        }
        __syncthreads();
        for (int it = 0; it < ntiles; it += 2) {
            const int k0 = kbase + it * PF_BK;
            if (loader && it + 2 < ntiles) {
                store_tile((it + 2) & 3, k0 + 2 * PF_BK);
                if (it + 3 < ntiles) load_tile(k0 + 3 * PF_BK);
            }
            compute(it & 3, k0);
            if (loader && it + 3 < ntiles) {
                store_tile((it + 3) & 3, k0 + 3 * PF_BK);
                if (it + 4 < ntiles) load_tile(k0 + 4 * PF_BK);
            }
            if (it + 1 < ntiles) compute((it + 1) & 3, k0 + PF_BK);
            if (it + 2 < ntiles) __syncthreads();
        }
    } else {
    // NST 3: iteration i stores tile i + 1 (loaded during iteration i - 1)
    // into the stage tile i - 2 used, requests tile i + 2, computes tile i,
    // then one barrier. NST 2: iteration i requests tile i + 1, computes
    // tile i, and stores between two barriers.
    if (loader) {
        load_tile(kbase);
        store_tile(0, kbase);
        if (NST == 3 && ntiles > 1) load_tile(kbase + PF_BK);
    }
    __syncthreads();
    int buf = 0;
    for (int it = 0; it < ntiles; it++) {
        const int k0 = kbase + it * PF_BK;
        if (loader) {
            if constexpr (NST == 3) {
                if (it + 1 < ntiles) {
                    store_tile(buf == 2 ? 0 : buf + 1, k0 + PF_BK);
                    if (it + 2 < ntiles) load_tile(k0 + 2 * PF_BK);
                }
            } else {
                if (it + 1 < ntiles) load_tile(k0 + PF_BK);
            }
        }
        compute(buf, k0);
        if constexpr (NST == 3) {
            if (it + 1 < ntiles) __syncthreads();  // tile i + 1 stored; tile i's stage free after the next store
            buf = buf == 2 ? 0 : buf + 1;
        } else if (it + 1 < ntiles) {
            __syncthreads();  // everyone is done with the buffer two tiles back
            if (loader) store_tile(buf ^ 1, k0 + PF_BK);
            __syncthreads();
            buf ^= 1;
        }
    }
    }
    }
    // a tile with one range writes its gated rows, as the unsplit kernel
    if (SPL && records) {
        // Records (f32) go out as the gated rows do: each wave stages its
        // 32 rows, 64 dims a pass (rows of 64 + 4 floats), and writes 16-byte
        // pieces with 16 lanes per 256 contiguous bytes of a record.
        constexpr int RR = 68;  // staged row stride (floats)
        static_assert(32 * RR * 4 * (THREADS / 64) <= PF_NST * PF_STAGE * 2, "record staging fits the stages");
        __syncthreads();  // every wave is past the last tile's stage
        float* rw = reinterpret_cast<float*>(pf_smem) + wave * 32 * RR;
        const int rr = lane >> 4, rc = lane & 15;  // read: rows rr + 4 k, floats 4 rc of the pass
#pragma unroll
        for (int qb = 0; qb < NQB; qb++) {
            auto row_q = [&](int r) { return PAIRED ? (r & 15) : (qb0 + qb) * 32 + r; };
            auto row_hh = [&](int r) { return PAIRED ? 2 * wave + (r >> 4) : wave % G; };
            if (lh == 0 && qcol(qb) < nb) {
                const size_t r = pf_split_rec<BQ, G>(wg, qcol(qb), h - kvh * G);
                *reinterpret_cast<float2*>(p.part_ms + r * 2) = make_float2(m[qb], l[qb]);
            }
#pragma unroll
            for (int ps = 0; ps < 4; ps++) {
#pragma unroll
                for (int db = 2 * ps; db < 2 * ps + 2; db++)
#pragma unroll
                    for (int g4 = 0; g4 < 4; g4++) {
                        const f32x16& oo = o[qb][db];
                        *reinterpret_cast<float4*>(rw + lq * RR + 32 * (db - 2 * ps) + 8 * g4 + 4 * lh) =
                            make_float4(oo[4 * g4], oo[4 * g4 + 1], oo[4 * g4 + 2], oo[4 * g4 + 3]);
                    }
                wave_sync();
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int r = rr + 4 * k, q = row_q(r);
                    const float4 v = *reinterpret_cast<const float4*>(rw + r * RR + 4 * rc);
                    if (q < nb)
                        *reinterpret_cast<float4*>(p.part_acc + pf_split_rec<BQ, G>(wg, q, row_hh(r)) * HEAD_DIM +
                                                   64 * ps + 4 * rc) = v;
                }
                wave_sync();  // the region is rewritten by the next pass
            }
        }
        return;
    }
    // Gated rows: bf16(rbf(O / l) * sigmoid(gate)). The wave's 32 columns
    // are 32 rows (query, head); lane (lq, lh) holds 4-dim pieces of row lq,
    // so stores straight from the accumulators would hit 32 rows per
    // instruction. Instead each wave stages rbf(O / l) as bf16 (hardware
    // round to nearest even, the same bits as rbf) in its own
    // LDS region, 64 dims at a time (rows of 64 + 8 elements), and reads it
    // back as 16-byte pieces: lane i takes row 8 k + i / 8, dims 8 (i % 8)
    // of the pass, so 8 lanes cover 128 contiguous bytes of a row, for the
    // gate loads and the output stores alike.
    constexpr int ER = 72;  // staged row stride (elements)
    static_assert(32 * ER * 2 * (THREADS / 64) <= 2 * pf_stage(PF_VPAIR_TIGHT) * 2, "epilogue staging fits 2 stages");
    __syncthreads();  // every wave is past the last tile's stage
    uint16_t* ew = pf_smem + wave * 32 * ER;
    const int er = lane >> 3, ec = lane & 7;  // read: rows er + 8 k, dims 8 ec of the pass
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
        const float inv = l[qb] > 0.f ? 1.f / l[qb] : 0.f;
        // row r of the staged tile is the column of lane lq = r
        auto row_q = [&](int r) { return PAIRED ? (r & 15) : (qb0 + qb) * 32 + r; };
        auto row_h = [&](int r) { return kvh * G + (PAIRED ? 2 * wave + (r >> 4) : wave % G); };
        // gate pieces of every pass, requested up front
        uint4 graw[4][4];
#pragma unroll
        for (int ps = 0; ps < 4; ps++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int r = er + 8 * k, q = row_q(r);
                const size_t t = (size_t)tb + (q < nb ? q : 0);
                graw[ps][k] = *reinterpret_cast<const uint4*>(p.qkv + t * p.qstride + (size_t)row_h(r) * 2 * HEAD_DIM +
                                                              HEAD_DIM + 64 * ps + 8 * ec);
            }
#pragma unroll
        for (int ps = 0; ps < 4; ps++) {
            // dims 64 ps + 32 (db - 2 ps) + 8 g4 + 4 lh of row lq
#pragma unroll
            for (int db = 2 * ps; db < 2 * ps + 2; db++)
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const f32x16& oo = o[qb][db];
                    *reinterpret_cast<uint2*>(ew + lq * ER + 32 * (db - 2 * ps) + 8 * g4 + 4 * lh) =
                        make_uint2(pack2_hw(oo[4 * g4] * inv, oo[4 * g4 + 1] * inv),
                                   pack2_hw(oo[4 * g4 + 2] * inv, oo[4 * g4 + 3] * inv));
                }
            wave_sync();
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int r = er + 8 * k, q = row_q(r);
                const uint4 y = *reinterpret_cast<const uint4*>(ew + r * ER + 8 * ec);
                const uint4 g = graw[ps][k];
                const uint32_t yw[4] = {y.x, y.y, y.z, y.w}, gw[4] = {g.x, g.y, g.z, g.w};
                uint32_t ow[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    ow[j] = pack2_hw(gated_div(bf_lo(yw[j]), 1.f + __expf(-bf_lo(gw[j]))),
                                     gated_div(bf_hi(yw[j]), 1.f + __expf(-bf_hi(gw[j]))));
                if (q < nb)
                    *reinterpret_cast<uint4*>(p.out + (((size_t)tb + q) * p.Hq + row_h(r)) * HEAD_DIM + 64 * ps +
                                              8 * ec) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
            }
            wave_sync();  // the region is rewritten by the next pass
        }
    }
}

template <int G, int BQ, int NQB, bool F8 = false, int NST = PF_NST, int VP = PF_VPAIR>
__device__ __forceinline__ void prefill_body(const PrefillParams& p, uint16_t* pf_smem) {
    int s, tb, nb;
    if (!find_prefill_tile<BQ>(p, blockIdx.x, s, tb, nb)) return;
    const int kvh = blockIdx.y;
    // bf16 with pages of 16 keys or more: tiles by LDS DMA; otherwise
    // through registers, with uniform page ids per chunk when pages hold at
    // least (loading threads) / 32 keys.
    constexpr bool DMA = !F8;
    if (DMA && p.bs_log2 >= 4)
        prefill_tile<G, BQ, NQB, F8, true, NST, DMA, VP>(p, pf_smem, s, tb, nb, kvh, 0);
    else if (p.bs_log2 >= pf_upage_log2(pf_threads(BQ, NQB, G)))
        prefill_tile<G, BQ, NQB, F8, true, NST, false, VP>(p, pf_smem, s, tb, nb, kvh, 0);
    else
        prefill_tile<G, BQ, NQB, F8, false, NST, false, VP>(p, pf_smem, s, tb, nb, kvh, 0);
}

// The library's prompt kernels for G query heads per kv head (shapes above).
template <int G>
__global__ void __launch_bounds__(pf_lib_threads(G), 1) prefill_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint16_t pf_smem[];
    prefill_body<G, pf_lib_bq(G), pf_lib_nqb(G), false, pf_lib_nst(G)>(p, pf_smem);
}

// Few query tiles (the library kernel's grid would not fill four rounds of
// CUs: one prompt, or one sequence's chunk, of a few thousand tokens): half
// the queries per workgroup and two workgroups per CU, so more workgroups
// share out the causal tiles and fill the CUs (a 2,048-token chunk after
// 6,144 keys: 362 against 406 us at G = 4; a 4,096-token prompt at G = 6:
// 383 against 405 us).
template <int G>
__global__ void __launch_bounds__(pf_fine_threads(G), 2) prefill_fine_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint16_t pf_smem[];
    prefill_body<G, pf_fine_bq(G), 1, false, 2, PF_VPAIR_TIGHT>(p, pf_smem);
}

// How prefill_split_kernel splits the prompt's R query tiles (called by
// whole waves, uniform results): parts = pf_split_parts(R Hkv, cus) ranges
// per tile when R Hkv < cus (each tile's keys cut evenly), else, or when
// the grid would exceed the workspace (split_cap workgroups), 1.
__device__ __forceinline__ int pf_split_plan(const PrefillParams& p, int R) {
    const int w = R * p.Hkv, parts = pf_split_parts(w, p.cus);
    return (long)parts * w > p.split_cap ? 1 : parts;
}

// Index b (< n) of a grid of n workgroups in an order where consecutive
// indices share an XCD: the dispatcher hands workgroup ids to the 8 XCDs in
// turn, and id b becomes index b / 8 of its XCD's contiguous share of the
// grid (the first n % 8 XCDs take one more).
__device__ __forceinline__ int xcd_major(int b, int n) {
    const int q = n >> 3, r = n & 7, xcd = b & 7, slot = b >> 3;
    return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

// Split keys (pkv_attn_prefill_split / _e4m3_split): a 1-D grid of at least
// max(host tile bound x kv heads, 2 cus) workgroups. The kernel counts the
// prompt's R query tiles from cu (the host only bounds them) and takes
// parts = pf_split_plan ranges per tile: workgroup l = x + R (kvh + Hkv
// part) is tile x, kv head kvh, key range part, and the rest of the grid
// returns. With parts > 1 (one or two rounds over the CUs) the tiles of one
// (kv head, range) go to one XCD, which then reads those keys through one
// L2; a tile that takes more than one range leaves records for
// prefill_merge_kernel, a tile with one range writes its gated rows. With
// parts = 1 (a grid that fills the CUs) it is the library kernel's launch,
// longest tiles first, rows written directly. The plan goes to
// p.split_plan for the merge.
template <int G, bool F8 = false>
__global__ void __launch_bounds__(pf_lib_threads(G), 1) prefill_split_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint16_t pf_smem[];
    constexpr int BQ = pf_lib_bq(G), NQB = pf_lib_nqb(G);
    // (uniform values: readfirstlane keeps them in SGPRs for the DMA bases)
    const int R = __builtin_amdgcn_readfirstlane(prompt_tiles<BQ>(p));
    const int parts = __builtin_amdgcn_readfirstlane(pf_split_plan(p, R));
    const int n = parts * R * p.Hkv, b = blockIdx.x;
    if (b == 0 && threadIdx.x == 0 && p.split_plan) {
        p.split_plan[0] = parts;
        p.split_plan[1] = R;
    }
    if (b >= n) return;
    const int l = parts > 1 ? xcd_major(b, n) : b;
    const int x = __builtin_amdgcn_readfirstlane(l % R), kvh = __builtin_amdgcn_readfirstlane((l / R) % p.Hkv),
              part = __builtin_amdgcn_readfirstlane(l / (R * p.Hkv));
    int s, tb, nb;
    if (!find_prefill_tile<BQ>(p, x, s, tb, nb, R)) return;
    // the tile paths of prefill_body
    constexpr bool DMA = !F8;
    if (DMA && p.bs_log2 >= 4)
        prefill_tile<G, BQ, NQB, F8, true, DMA ? pf_lib_nst(G) : PF_NST, DMA, PF_VPAIR, true>(p, pf_smem, s, tb, nb,
                                                                                           kvh, part, parts, l);
    else if (p.bs_log2 >= pf_upage_log2(pf_threads(BQ, NQB, G)))
        prefill_tile<G, BQ, NQB, F8, true, F8 ? pf_lib_nst_f8(G) : PF_NST, false, PF_VPAIR, true>(p, pf_smem, s, tb, nb,
                                                                                             kvh, part, parts, l);
    else
        prefill_tile<G, BQ, NQB, F8, false, F8 ? pf_lib_nst_f8(G) : PF_NST, false, PF_VPAIR, true>(p, pf_smem, s, tb, nb,
                                                                                              kvh, part, parts, l);
}

// Combines the key ranges of prefill_split_kernel: grid (rows, kv heads),
// a wave per query head of the group; row t of a prompt sequence folds its
// query tile's non-empty ranges (the decode merge's arithmetic, gated
// output); other rows, and every row when the split kernel took one range
// per tile, are left untouched.
template <int G>
__global__ void __launch_bounds__(64 * G) prefill_merge_kernel(PrefillParams p) {
    constexpr int BQ = pf_lib_bq(G);
    const int t = blockIdx.x, kvh = blockIdx.y, hh = threadIdx.x >> 6, h = kvh * G + hh, lane = threadIdx.x & 63;
    // nothing to merge without a split (the split kernel's plan)
    const int parts = p.split_plan[0], total = p.split_plan[1];
    if (parts <= 1) return;
    // the sequence holding row t: the last s with cu[s] <= t
    int lo = 0, hi = p.seqs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (p.cu[mid] <= t) lo = mid;
        else hi = mid - 1;
    }
    const int c0 = p.cu[lo], n = p.cu[lo + 1] - c0;
    if (t < c0 || t >= c0 + n || n <= 1 || is_spec(p.outs, p.spec, lo)) return;
    // the tiles of the prompts before sequence lo
    int before = 0;
    for (int i = lane; i < lo; i += 64) before += seq_tiles<BQ>(p, i);
#pragma unroll
    for (int o = 32; o; o >>= 1) before += __shfl_xor(before, o);
    const int tb = c0 + (t - c0) / BQ * BQ, nb = min(BQ, c0 + n - tb);
    // the split kernel's x of this tile (tiles run last first)
    const int x = total - 1 - (before + (t - c0) / BQ);
    const int nt = (p.pos[tb] + nb + PF_BK - 1) / PF_BK, per = pf_split_per(nt, parts);
    // a tile with one range wrote its rows itself
    if (nt <= per) return;
    auto rec = [&](int z) { return pf_split_rec<BQ, G>(pf_split_index(x, kvh, z, total, p.Hkv), t - tb, hh); };
    merge_rows<1>(
        (nt + per - 1) / per, 1.f, [&](int z) { return p.part_ms + rec(z) * 2; },
        [&](int z) { return p.part_acc + rec(z) * HEAD_DIM; },
        p.qkv + (size_t)t * p.qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM, p.out + ((size_t)t * p.Hq + h) * HEAD_DIM);
}

// The same over an E4M3 cache (p.kscale / p.vscale set).
template <int G>
__global__ void __launch_bounds__(pf_lib_threads(G), 1) prefill_e4m3_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint16_t pf_smem[];
    prefill_body<G, pf_lib_bq(G), pf_lib_nqb(G), true, pf_lib_nst_f8(G)>(p, pf_smem);
}

}  // namespace pkv

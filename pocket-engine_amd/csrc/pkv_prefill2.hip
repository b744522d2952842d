// Chunked-prefill attention, 64 queries per wave (the library's entry point).
// Same results as prefill_kernel (and the reference's attn_mfma_g4_t2 /
// attn_flash_group): causal attention of each prompt row over keys
// 0 .. pos[t], q pre-scaled by scale * log2 e and rounded to bf16, exp2
// softmax, P rounded to bf16 for P.V, gated bf16 output.
//
// Why a second kernel. With one 32-query block per wave every K / V
// fragment read from LDS feeds one MFMA, and the LDS reads take as long as
// the MFMAs (128 B / clk / CU against 4 SIMDs of 32x32x16 bf16). Here a wave
// takes two 32-query blocks of one query head, so each fragment feeds two
// MFMAs: a workgroup is 4 waves (the 4 query heads of a kv head) x 64 query
// positions, q (128 VGPRs) and O^T (256 accumulators) stay in registers, and
// the tiles come into LDS by direct global -> LDS loads (no staging
// registers, no LDS store instructions):
//   K tile (32 keys x 256 dims, 16 KiB) in MFMA fragment order: load
//     instruction kk writes fragment kk (lane l: key l % 32, dims
//     16 kk + 8 (l / 32)), so each fragment read is one contiguous
//     ds_read_b128 per lane;
//   V tile row-major (key, 16-byte chunk), chunk c of key r stored at chunk
//     c ^ 4 (r % 4), read transposed by ds_read_b64_tr_b16 (4 keys x 16 dims
//     per 16 lanes): the XOR keeps the 32 lanes of each read on distinct
//     banks.
// No rescale of the accumulators. Each query's probabilities are taken
// relative to a reference m_ref fixed by the first key tile (it holds key 0,
// which every query attends): P = exp2(s - m_ref), l = sum P, O = sum P V,
// out = O / l, the same quotient as the online form for any reference. Later
// scores above m_ref give P > 1, which f32 and bf16 hold; if a score exceeds
// m_ref + 64 (log2 units: P could reach 2^64) the workgroup reruns its tile
// with m_ref = the maximum it observed, so the accumulators never need the
// per-tile rescale that would take them out of the matrix-core accumulator
// registers (256 per wave here). The rerun is prefill_tile<64, 2> (the same
// 4 waves, online rescaling, register-staged tiles), called out of line so
// the key loop here keeps its register allocation.
// Three LDS stages: tile it + 2 is in flight while tile it is multiplied. The
// only vector-memory instructions in the key loop are the 8 tile loads per
// wave per tile (the sequence's page ids are staged in LDS before the loop),
// so "tile it has
// landed" is an explicit vmcnt(8) wait followed by a plain barrier. Keys at or
// past L are loaded from key L - 1 (finite data; their scores are masked).
#pragma once
#include "pkv_prefill.hip"

namespace pkv {

constexpr int P2_BQ = 64, P2_TILE = PF_BK * HEAD_DIM;  // u16 per K or V tile
constexpr int p2_threads(int nqb) { return 512 / nqb; }  // 4 query heads x 64 / (32 nqb) waves
constexpr int P2_MAX_PAGES = 8192;  // page ids staged in LDS (32 KiB): sequences up to 8192 pages

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// d += a b on the matrix cores with d in VGPRs: the output accumulators
// take all 256 AGPRs, so the scores must not.
__device__ __forceinline__ void mfma_v(f32x16& d, bf16x8 a, bf16x8 b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}

template <int NQB>
__device__ __noinline__ void prefill_rerun_tile(const PrefillParams& p, uint16_t* lds, int s, int tb, int nb) {
    prefill_tile<P2_BQ, NQB>(p, lds, s, tb, nb);
}

template <int NQB>
__device__ __forceinline__ void prefill2_body(const PrefillParams& p, const int* __restrict__ block_table) {
    constexpr int THREADS = p2_threads(NQB), WAVES = THREADS / 64, PER = 16 / WAVES;  // tile loads per wave: 2 PER
    // Six 16 KiB tiles (K and V of three stages); the rerun path reuses them
    // as its 2 x 34.5 KiB of stages.
    static_assert(6 * P2_TILE >= prefill_smem_bytes() / 2, "LDS for the rerun path");
    __shared__ __align__(16) uint16_t p2_lds[6 * P2_TILE];
    uint16_t* const k_s0 = p2_lds;
    uint16_t* const k_s1 = p2_lds + P2_TILE;
    uint16_t* const k_s2 = p2_lds + 2 * P2_TILE;
    uint16_t* const v_s0 = p2_lds + 3 * P2_TILE;
    uint16_t* const v_s1 = p2_lds + 4 * P2_TILE;
    uint16_t* const v_s2 = p2_lds + 5 * P2_TILE;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lq = lane & 31, lh = lane >> 5;
    const int kvh = blockIdx.y, h = kvh * 4 + (wave & 3), qb0 = (wave >> 2) * NQB;  // the wave's first query block
    int s, tb, nb;
    if (!find_prefill_tile<P2_BQ>(p, s, tb, nb)) return;
    s = __builtin_amdgcn_readfirstlane(s);
    tb = __builtin_amdgcn_readfirstlane(tb);
    nb = __builtin_amdgcn_readfirstlane(nb);
    const int qp0 = __builtin_amdgcn_readfirstlane(p.pos[tb]);
    const int L = qp0 + nb;  // keys this tile needs: 0 .. L - 1
    const size_t row = (size_t)p.Hkv * HEAD_DIM;
    const int bs_log2 = p.bs_log2, bs_mask = (1 << bs_log2) - 1;
    // The pages of keys 0 .. L - 1, clamped into the pool, staged in LDS.
    __shared__ int pt[P2_MAX_PAGES];
    {
        const int* bt = block_table + (size_t)s * p.max_blocks;
        const int np = ((L - 1) >> bs_log2) + 1;
        for (int i = tid; i < np; i += THREADS) {
            const long pg = bt[i];
            pt[i] = (int)(pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg);
        }
    }

    bf16x8 qf[NQB][16];
    {
        const float f = p.scale * LOG2E;
#pragma unroll
        for (int qb = 0; qb < NQB; qb++) {
            const int myq = (qb0 + qb) * 32 + lq;
            const bool ok = myq < nb;
            const uint16_t* qrow = p.q + ((size_t)(tb + (ok ? myq : 0)) * p.Hq + h) * HEAD_DIM;
#pragma unroll
            for (int kk = 0; kk < 16; kk++) {
                uint4 raw = ok ? *reinterpret_cast<const uint4*>(qrow + 16 * kk + 8 * lh) : make_uint4(0, 0, 0, 0);
                raw = make_uint4(pack2(bf_lo(raw.x) * f, bf_hi(raw.x) * f), pack2(bf_lo(raw.y) * f, bf_hi(raw.y) * f),
                                 pack2(bf_lo(raw.z) * f, bf_hi(raw.z) * f), pack2(bf_lo(raw.w) * f, bf_hi(raw.w) * f));
                qf[qb][kk] = as_bf16x8(raw);
            }
        }
    }
    f32x16 o[NQB][8];
    float mref[NQB], mall[NQB], l[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[qb][db][r] = 0.f;
        mref[qb] = NQB == 1 ? -INFINITY : 0.f;
        mall[qb] = -INFINITY;
        l[qb] = 0.f;
    }
    bool big = false;  // some score exceeded mref + 64 (this lane)

    // Tile loads. Block size: a power of two >= 16 (checked on the host), so
    // a 32-key tile spans at most two pages.
    auto page_of = [&](int kp) __attribute__((always_inline)) -> long {
        return __builtin_amdgcn_readfirstlane(pt[kp >> bs_log2]);
    };
    auto issue_tile = [&](int k0, uint16_t* ks, uint16_t* vs) __attribute__((always_inline)) {
        const int pi0 = k0 >> bs_log2;
        const long pg0 = page_of(k0), pg1 = page_of(min(k0 + PF_BK, L) - 1);
        auto slot = [&](int kl) __attribute__((always_inline)) -> size_t {
            const int kp = min(k0 + kl, L - 1);
            return (size_t)((((kp >> bs_log2) == pi0 ? pg0 : pg1) << bs_log2) + (kp & bs_mask)) * row +
                   (size_t)kvh * HEAD_DIM;
        };
        const size_t ks_lane = slot(lq) + 8 * lh;  // K: key lq, dims 16 kk + 8 lh
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int kk = PER * wave + u;
            __builtin_amdgcn_global_load_lds(p.kc + ks_lane + 16 * kk, (lds_void*)(ks + kk * 512), 16, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = PER * wave + u, kl = 2 * i + lh;  // V: keys 2i, 2i + 1, stored chunk lq
            const int cg = lq ^ (4 * (kl & 3));
            __builtin_amdgcn_global_load_lds(p.vc + slot(kl) + 8 * cg, (lds_void*)(vs + i * 512), 16, 0, 0);
        }
    };

    const int ntiles = (L + PF_BK - 1) / PF_BK;
    const int lq16 = lq & 15, g16 = lq >> 4;
    // One tile: scores, softmax, P.V for both query blocks.
    auto compute = [&](int k0, const uint16_t* ks, const uint16_t* vs) __attribute__((always_inline)) {
        // S^T = K Q^T. With one query block the 16 steps run as two
        // independent accumulation chains (even / odd kk), added at the end.
        constexpr int NCHAIN = NQB == 1 ? 2 : 1;
        f32x16 st[NQB * NCHAIN];
#pragma unroll
        for (int c = 0; c < NQB * NCHAIN; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) st[c][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(ks + kk * 512 + lane * 8));
#pragma unroll
            for (int qb = 0; qb < NQB; qb++) {
                f32x16& acc = st[qb * NCHAIN + (kk % NCHAIN)];
                if constexpr (NQB == 2)
                    mfma_v(acc, a, qf[qb][kk]);
                else
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb][kk], acc, 0, 0, 0);
            }
        }
        if constexpr (NQB == 2) {
            // ALU reads of matrix-core results in VGPRs need wait states the
            // hardware does not insert (at most 18 passes after a 32x32 op).
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) st[0][r] += st[1][r];
        }
        uint4 pb[NQB][2];
#pragma unroll
        for (int qb = 0; qb < NQB; qb++) {
            f32x16& sq = st[qb * NCHAIN];
            const int qb_first = qp0 + (qb0 + qb) * 32, qp = qb_first + lq;
            if (k0 + PF_BK - 1 > qb_first || k0 + PF_BK > L) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int kp = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (kp > qp || kp >= L) sq[r] = -INFINITY;
                }
            }
            float mx = NQB == 1 ? mref[qb] : -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, sq[r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            if constexpr (NQB == 1) {
                // Online softmax: running max in mref, the accumulators
                // rescaled when it moves (they are plain VGPRs here).
                const float bse = mx == -INFINITY ? 0.f : mx;
                const float corr = __builtin_amdgcn_exp2f(mref[qb] - bse);
                mref[qb] = mx;
                l[qb] *= corr;
                if (__any(corr != 1.f)) {
#pragma unroll
                    for (int db = 0; db < 8; db++)
#pragma unroll
                        for (int r = 0; r < 16; r++) o[qb][db][r] *= corr;
                }
                mx = bse;
            } else {
                mall[qb] = fmaxf(mall[qb], mx);
                if (k0 == 0) mref[qb] = mx == -INFINITY ? 0.f : mx;  // first tile: fixes the reference
                big |= mx > mref[qb] + 64.f;
                mx = mref[qb];
            }
            float sum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                sq[r] = __builtin_amdgcn_exp2f(sq[r] - mx);
                sum += sq[r];
            }
            sum += __shfl_xor(sum, 32, 64);
            l[qb] += sum;
#pragma unroll
            for (int kk = 0; kk < 2; kk++)
                pb[qb][kk] = make_uint4(pack2_hw(sq[8 * kk + 0], sq[8 * kk + 1]),
                                        pack2_hw(sq[8 * kk + 2], sq[8 * kk + 3]),
                                        pack2_hw(sq[8 * kk + 4], sq[8 * kk + 5]),
                                        pack2_hw(sq[8 * kk + 6], sq[8 * kk + 7]));
        }
        // O^T += V^T P^T. Fragment (kk, db): lane l needs V[key][32 db + lq]
        // for keys 16 kk + 4 lh + {0..3} and + 8: two transposed reads. In each
        // 16-lane group source lane j addresses key base + j / 4, dims
        // d0 + 4 (j % 4) (d0 = 32 db + 16 (lq / 16)).
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int db = 0; db < 8; db++) {
                s16x4 half[2];
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const int r = 16 * kk + 8 * hh + 4 * lh + (lq16 >> 2);
                    const int d = 32 * db + 16 * g16 + 4 * (lq16 & 3);
                    const int c = (d >> 3) ^ (4 * (r & 3));
                    half[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4*)(vs + r * HEAD_DIM + 8 * c + (d & 7)));
                }
                const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4,
                                                                                     5, 6, 7));
#pragma unroll
                for (int qb = 0; qb < NQB; qb++)
                    o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_bf16x8(pb[qb][kk]), o[qb][db], 0, 0, 0);
            }
    };
    const int last = qp0 + min(nb, (qb0 + NQB) * 32) - 1;  // the wave's last query position
    // Stage S of tile it: wait for it to land (tile it + 1's 8 loads may still
    // be in flight), barrier, start tile it + 2 into the stage tile it - 1
    // used, multiply tile it.
    auto step = [&](int it, auto S) __attribute__((always_inline)) {
        constexpr int cur = decltype(S)::value, nxt = (cur + 2) % 3;
        uint16_t* kc_ = cur == 0 ? k_s0 : cur == 1 ? k_s1 : k_s2;
        uint16_t* vc_ = cur == 0 ? v_s0 : cur == 1 ? v_s1 : v_s2;
        uint16_t* kn_ = nxt == 0 ? k_s0 : nxt == 1 ? k_s1 : k_s2;
        uint16_t* vn_ = nxt == 0 ? v_s0 : nxt == 1 ? v_s1 : v_s2;
        if (it + 1 < ntiles)
            wait_vmcnt<2 * PER>();
        else
            wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (it + 2 < ntiles) issue_tile((it + 2) * PF_BK, kn_, vn_);
        if (it * PF_BK <= last) compute(it * PF_BK, kc_, vc_);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    __shared__ int sh_rerun;
    if (tid == 0) sh_rerun = 0;
    __syncthreads();  // page ids staged, flag cleared
    issue_tile(0, k_s0, v_s0);
    if (ntiles > 1) issue_tile(PF_BK, k_s1, v_s1);
    for (int it = 0; it < ntiles; it += 3) {
        step(it, S0{});
        if (it + 1 < ntiles) step(it + 1, S1{});
        if (it + 2 < ntiles) step(it + 2, S2{});
    }
    if constexpr (NQB == 2) {
        if (__any(big)) sh_rerun = 1;  // benign race: every writer stores 1
        __syncthreads();
        if (sh_rerun) {
            prefill_rerun_tile<NQB>(p, p2_lds, s, tb, nb);
            return;
        }
    }
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
        const int myq = (qb0 + qb) * 32 + lq;
        if (myq >= nb) continue;
        const float inv = l[qb] > 0.f ? 1.f / l[qb] : 0.f;
        const size_t t = (size_t)tb + myq;
        const uint16_t* gate = p.qkv + t * p.qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM;
        uint16_t* orow = p.out + (t * p.Hq + h) * HEAD_DIM;
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int d = 32 * db + 8 * g4 + 4 * lh;
                const uint2 graw = *reinterpret_cast<const uint2*>(gate + d);
                const f32x16& oo = o[qb][db];
                *reinterpret_cast<uint2*>(orow + d) =
                    make_uint2(pack2(rbf(oo[4 * g4] * inv) / (1.f + __expf(-bf_lo(graw.x))),
                                     rbf(oo[4 * g4 + 1] * inv) / (1.f + __expf(-bf_hi(graw.x)))),
                               pack2(rbf(oo[4 * g4 + 2] * inv) / (1.f + __expf(-bf_lo(graw.y))),
                                     rbf(oo[4 * g4 + 3] * inv) / (1.f + __expf(-bf_hi(graw.y)))));
            }
    }
}

// One 32-query block per wave: 8 waves, two per SIMD.
__global__ void __launch_bounds__(512, 1) prefill2_q1_kernel(PrefillParams p, const int* __restrict__ block_table) {
    prefill2_body<1>(p, block_table);
}

// Two 32-query blocks per wave: 4 waves, 512 registers each.
__global__ void __launch_bounds__(256, 1) prefill2_q2_kernel(PrefillParams p, const int* __restrict__ block_table) {
    prefill2_body<2>(p, block_table);
}

}  // namespace pkv

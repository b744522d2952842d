// Draft-verify attention for gfx950: the decode rows of a sequence that
// feeds several tokens in one step (the target pass of speculative decoding,
// reference is_spec rows, qwen35.cu:94-100, attended by attn_paged_g4 one
// token at a time, qwen35.cu:1146-1334) read each KV page once for all of
// them. Same results per row as paged decode attention: row t attends keys
// [0, pos[t] + 1) (causal among the drafts), online softmax in f32, gated
// bf16 output, split partials merged in key order.
//
// Segments. Up to 4 consecutive rows of one sequence form a segment (rows
// cu[s] + 4i ..); a segment's keys are [0, max over its rows of L_t). The
// key space is the segments' keys laid end to end, cut into equal ranges as
// for decode (one workgroup per range and group of 4 kv heads, a wave per kv
// head); partials go to index (head token + range index) * 4 + row.
//
// Per page (16 keys) a wave computes the 16 x 16 score block of 16 keys
// against 16 query columns (4 rows x the 4 query heads of its kv head) on
// MFMA:
//   S^T[16 keys][16 cols] = K Q^T      8 x v_mfma_f32_16x16x32_bf16
//     A = K straight from HBM: lane (key l % 16, group l / 16) loads 16
//     bytes at dims 32c + 8 (l / 16) for c = 0..7 (each instruction reads 64
//     contiguous bytes of 16 key rows; two consecutive ones a full 128-byte
//     line). B = Q^T with the same dims, held in registers for the piece.
//   O^T[256 dims][16 cols] += V^T P^T  32 x v_mfma_f32_16x16x16_bf16
//     B = P^T is the S^T accumulator itself (lane l holds keys 4 (l / 16) + i
//     of column l % 16 in both layouts), as a bf16 high part and a bf16
//     remainder in two MFMAs (32 per page). A = V^T comes
//     from the page's V staged row-major in LDS (one fully coalesced 512-byte
//     row per half-wave load) through ds_read_b64_tr_b16, which transposes
//     4 x 4 blocks of 16-bit values on the way out of LDS.
// Column softmax: per lane over its 4 keys, then across the 4 lane groups
// (two cross-lane shuffles). The MFMA work per page is ~0.3 us of one SIMD's
// time against the ~2.3 us the page's 16 KiB take at the HBM share of a
// SIMD, so the kernel stays bandwidth-bound with the compute hidden.
#pragma once
#include "pkv_common.h"
#include "pkv_decode8.hip"

#include <type_traits>

namespace pkv {

constexpr int VF_ROWS = 4;                // most query rows per segment (partial records per index)
// Rows per segment for G query heads per kv head: the 16 MFMA columns hold
// rows x heads, so 4 rows up to G = 4 and 2 rows for G = 6 or 8.
__host__ __device__ constexpr int vf_rows(int G) { return G <= 4 ? 4 : 2; }
constexpr int VF_VSTR = HEAD_DIM + 16;    // u16 per staged V row (544 B: conflict-free transposed reads)
constexpr int VF_LDS = PAGE * VF_VSTR;    // u16 per wave

// Keys of the segment headed by token t (segments of NR rows, NR a power of
// two); 0 when t does not head a segment (it is not at offset NR i of its
// sequence) or none of its rows attends.
template <int NR>
__device__ __forceinline__ int seg_len(int t, int T, const int* __restrict__ pos, const int* __restrict__ tok_seq,
                                       const int* __restrict__ cu, int skip, const int* __restrict__ outs, int spec,
                                       int& nrows) {
    const int s = tok_seq[t];
    nrows = 0;
    if ((t - cu[s]) & (NR - 1)) return 0;
    nrows = min(NR, min(cu[s + 1], T) - t);
    int L = 0;
    for (int r = 0; r < nrows; r++) L = max(L, decode_len(t + r, pos, tok_seq, cu, skip, outs, spec));
    return L;
}

// One wave: segment headed by token t (rows t + r, r < vf_rows(G),
// attending Lr[r] keys; Lr = 0 for absent rows), kv head kvh with G query
// heads, keys [j0, j1), bf16 cache (an E4M3 cache runs piece_body8,
// pkv_decode8.hip). MFMA column c is row c / G, head c % G.
// The result goes to epi(r, g, gq, acc, m, l) on the lanes of attending rows:
// row r, query head kvh * G + g, dims 16 db + 4 gq + i in acc[db][i]; m in
// log2 units, l the sum of weights (m = -inf, l = 0 when the piece has no
// key for the row).
// FUSED (the fused decode step): keys at positions [P0, Ls) of the segment,
// the ones the step itself feeds, come from the step's source rows (row
// row0 + position - P0 of k_rows / v_rows) instead of the cache, chosen per
// lane on the pages that hold such keys (from the page of P0 on); earlier
// pages take the plain cache addresses.
template <int G, bool FUSED = false, class Epi>
__device__ __forceinline__ void verify_piece(const DecodeParams& p, const int* __restrict__ bt, uint16_t* vl, int t,
                                             int kvh, int j0, int j1, const int (&Lr)[VF_ROWS], Epi epi,
                                             int P0 = INT_MAX, int row0 = 0) {
    constexpr int NR = vf_rows(G);
    const int lane = threadIdx.x & 63, c16 = lane & 15, gq = lane >> 4;
    const int r_me = c16 / G, g_me = c16 % G;
    const int myL = r_me >= NR ? 0 : r_me == 0 ? Lr[0] : r_me == 1 ? Lr[1] : r_me == 2 ? Lr[2] : Lr[3];
    const float sl2 = p.scale * LOG2E;
    const size_t row_elems = (size_t)p.Hkv * HEAD_DIM;  // slot row, elements

    // q.k over the 256 dims in 8 steps of 32: step c, lane group gq takes
    // dims dim0(c) .. + 7 (the same for q and k).
    auto dim0 = [&](int c) { return 32 * c + 8 * gq; };
    bf16x8 qf[8];
    if (myL > 0) {
        const uint16_t* qrow = p.q + ((size_t)(t + r_me) * p.Hq + kvh * G + g_me) * HEAD_DIM;
#pragma unroll
        for (int c = 0; c < 8; c++) qf[c] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + dim0(c)));
    } else {
#pragma unroll
        for (int c = 0; c < 8; c++) qf[c] = as_bf16x8(make_uint4(0, 0, 0, 0));
    }
    auto page_of = [&](int pi) -> long {
        const long pg = bt[pi];
        return pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg;
    };
    auto page_base = [&](int pi) -> size_t { return (size_t)page_of(pi) * PAGE * row_elems + (size_t)kvh * HEAD_DIM; };
    constexpr int NK = 8, NV = 8;  // 16-byte loads per lane per page
    // One page's loads: K and V rows.
    struct Buf {
        uint4 kb[NK], vb[NV];
    };
    // Address of key `key` of page pi (cache slot row, or with FRESH the
    // source row of a key the step feeds) plus `off` elements.
    auto src = [&](const uint16_t* pool, const uint16_t* rows, int pi, size_t base, int key, int off, auto fresh) {
        const uint16_t* c = pool + base + (size_t)key * row_elems + off;
        if constexpr (!decltype(fresh)::value) {
            return c;
        } else {
            const int kp = pi * PAGE + key;
            const uint16_t* f = rows + (ptrdiff_t)(row0 + kp - P0) * p.row_stride + (size_t)kvh * HEAD_DIM + off;
            return kp >= P0 && kp < j1 ? f : c;
        }
    };
    // Plain pages load by buffer loads: the page's (uniform) base in the
    // descriptor, the lane's byte offsets fixed for the piece.
    const uint32_t k_lane = (uint32_t)(2 * ((size_t)c16 * row_elems + 8 * gq));
    const uint32_t v_lane = (uint32_t)(2 * ((size_t)(lane >> 5) * row_elems + 8 * (lane & 31)));
    const uint32_t row_b = (uint32_t)(2 * row_elems);
    auto load_k = [&](Buf& B, size_t base, int pi, auto fresh) {
        if constexpr (decltype(fresh)::value) {
            const uint16_t* r = src(p.kc, p.k_rows, pi, base, c16, 8 * gq, fresh);
#pragma unroll
            for (int c = 0; c < NK; c++) B.kb[c] = load_nt(r + 32 * c);
        } else {
#pragma unroll
            for (int c = 0; c < NK; c++) B.kb[c] = buf_load16_nt(p.kc + base, k_lane + 64 * c);
        }
    };
    auto load_v = [&](Buf& B, size_t base, int pi, auto fresh) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            if constexpr (decltype(fresh)::value)
                B.vb[k] = load_nt(src(p.vc, p.v_rows, pi, base, 2 * k + (lane >> 5), 8 * (lane & 31), fresh));
            else
                B.vb[k] = buf_load16_nt(p.vc + base, v_lane + 2 * k * row_b);
        }
    };
    // A operand of step c: K dims dim0(c) .. + 7 of key c16
    auto k_frag = [&](const Buf& B, int c) -> bf16x8 {
        return as_bf16x8(B.kb[c]);
    };

    f32x4 acc[16];
#pragma unroll
    for (int db = 0; db < 16; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    // transposed-read address of this lane: key row 4 gq + c16 / 4, dims 4 (c16 % 4) + 16 db
    const uint16_t* tr = vl + (4 * gq + (c16 >> 2)) * VF_VSTR + 4 * (c16 & 3);
    uint16_t* st = vl + (lane >> 5) * VF_VSTR + 8 * (lane & 31);

    // One page from buffer B; with PREFETCH, B is refilled with page nxt as
    // soon as its K and V have been consumed.
    using PLAIN = std::integral_constant<bool, false>;
    using FRESHM = std::integral_constant<bool, true>;
    // prefetch: NONE (last page), PLAIN or FRESHM (the next page's mode)
    struct NONE {};
    auto page = [&](Buf& B, int pi, int nxt, auto prefetch) {
        constexpr bool PREFETCH = !std::is_same_v<decltype(prefetch), NONE>;
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 8; c++) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k_frag(B, c), qf[c], s, 0, 0, 0);
        // rows of keys outside [j0, j1) as zeros: their weight is 0, and
        // a stale slot may hold NaN
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int kp = pi * PAGE + 2 * k + (lane >> 5);
            *reinterpret_cast<uint4*>(st + 2 * k * VF_VSTR) =
                (kp >= j0 && kp < j1) ? B.vb[k] : make_uint4(0, 0, 0, 0);
        }
        if constexpr (PREFETCH) {
            const size_t next = page_base(nxt);
            load_k(B, next, nxt, prefetch);
            load_v(B, next, nxt, prefetch);
        }
        const int k0 = pi * PAGE + 4 * gq;
        float sc[4], mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kp = k0 + i;
            sc[i] = (kp >= j0 && kp < j1 && kp < myL) ? s[i] * sl2 : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        mx = max_xor32(max_xor16(mx));
        const float mn = fmaxf(m, mx);
        const float mref = mn == -INFINITY ? 0.f : mn;  // a column with no key yet keeps zeros
        const float corr = __builtin_amdgcn_exp2f(m - mref);
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pr[i] = __builtin_amdgcn_exp2f(sc[i] - mref);
        // P^T as a bf16 high part plus a bf16 remainder (two MFMAs, ~16
        // mantissa bits): decode rows keep their weights in f32 (the
        // reference's attn_paged_g4), which one bf16 per weight would miss by
        // up to 2^-9 relative; the denominator sums the f32 weights.
        const uint32_t h01 = pack2_hw(pr[0], pr[1]), h23 = pack2_hw(pr[2], pr[3]);
        const uint32_t r01 = pack2_hw(pr[0] - bf_lo(h01), pr[1] - bf_hi(h01));
        const uint32_t r23 = pack2_hw(pr[2] - bf_lo(h23), pr[3] - bf_hi(h23));
        l = l * corr + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
        m = mn;
        if (__any(corr != 1.f)) {
#pragma unroll
            for (int db = 0; db < 16; db++) acc[db] *= corr;
        }
        const s16x4 pb_hi = __builtin_bit_cast(s16x4, make_uint2(h01, h23));
        const s16x4 pb_lo = __builtin_bit_cast(s16x4, make_uint2(r01, r23));
        wave_sync();  // V staged
#pragma unroll
        for (int db = 0; db < 16; db++) {
            const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(tr + 16 * db));
            acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pb_hi, acc[db], 0, 0, 0);
            acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pb_lo, acc[db], 0, 0, 0);
        }
        wave_sync();  // reads done before the next page is staged
    };
    const int pg0 = j0 / PAGE, pg1 = (j1 - 1) / PAGE;
    // first page holding keys the step feeds (none: pg1 + 1)
    const int pf = FUSED ? max(pg0, min(pg1 + 1, P0 / PAGE)) : pg1 + 1;
    Buf A;
    if (pf > pg1) {
        load_k(A, page_base(pg0), pg0, PLAIN{});
        load_v(A, page_base(pg0), pg0, PLAIN{});
        for (int pi = pg0; pi < pg1; pi++) page(A, pi, pi + 1, PLAIN{});
    } else if constexpr (FUSED) {
        if (pf == pg0) {
            load_k(A, page_base(pg0), pg0, FRESHM{});
            load_v(A, page_base(pg0), pg0, FRESHM{});
        } else {
            load_k(A, page_base(pg0), pg0, PLAIN{});
            load_v(A, page_base(pg0), pg0, PLAIN{});
            for (int pi = pg0; pi < pf - 1; pi++) page(A, pi, pi + 1, PLAIN{});
            page(A, pf - 1, pf, FRESHM{});
        }
        for (int pi = pf; pi < pg1; pi++) page(A, pi, pi + 1, FRESHM{});
    }
    page(A, pg1, 0, NONE{});

    l = add_xor32(add_xor16(l));
    if (myL == 0) return;
    epi(r_me, g_me, gq, acc, m, l);
}

// Writes a verify piece's result for the lanes of (row r, head g): the gated
// output when the piece holds all of the segment's keys, else the partial
// record at index idx (vf_rows(G) records per index, one per segment row).
template <int G>
struct VerifyEpi {
    const DecodeParams& p;
    int t, kvh, idx;
    bool direct;
    __device__ __forceinline__ void operator()(int r, int g, int gq, const f32x4 (&acc)[16], float m, float l) const {
        const int h = kvh * G + g, row_t = t + r;
        if (direct) {
            const float inv = 1.f / l;
            const uint16_t* gate = p.qkv + (size_t)row_t * p.qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + 4 * gq;
            uint16_t* o = p.out + ((size_t)row_t * p.Hq + h) * HEAD_DIM + 4 * gq;
#pragma unroll
            for (int db = 0; db < 16; db++) {
                const uint2 graw = *reinterpret_cast<const uint2*>(gate + 16 * db);
                *reinterpret_cast<uint2*>(o + 16 * db) =
                    gate4(acc[db][0], acc[db][1], acc[db][2], acc[db][3], inv, graw);
            }
        } else {
            const size_t row = ((size_t)idx * vf_rows(G) + r) * p.Hq + h;
            float* pa = p.part_acc + row * HEAD_DIM + 4 * gq;
#pragma unroll
            for (int db = 0; db < 16; db++)
                *reinterpret_cast<float4*>(pa + 16 * db) = make_float4(acc[db][0], acc[db][1], acc[db][2], acc[db][3]);
            if (gq == 0) *reinterpret_cast<float2*>(p.part_ms + row * 2) = make_float2(m, l);
        }
    }
};

// Key-range kernel over segments of vf_rows(G) rows; grid (n_wg,
// ceil(Hkv / 4)), 64 * min(Hkv, 4) threads. Same range split as
// decode_range_kernel with segment lengths in place of token lengths; block 0
// writes offs[t] (segment offsets by head token, equal neighbours for other
// tokens), offs[T] = W, offs[T + 1] = R. The bound caps it at 256 VGPRs (no
// spills); it runs one workgroup per CU (two ranges per CU measured slower:
// 856 against 817 us at C5).
// FUSED (the fused decode step for groups other than 4): the kernel also
// appends the step's K/V rows (StepAppend) and reads the keys the step feeds
// from those source rows (verify_piece), so no range waits for a write.
template <int G, bool FUSED = false>
__global__ void __launch_bounds__(256, 2)
    verify_range_kernel(DecodeParams p, const int* __restrict__ pos, const int* __restrict__ tok_seq,
                        const int* __restrict__ block_table, const int* __restrict__ cu,
                        const int* __restrict__ outs, const int* __restrict__ slot_map) {
    constexpr int NR = vf_rows(G);
    __shared__ int sh_scan[16];
    __shared__ int sh_t0[2];
    __shared__ __align__(16) uint16_t sh_v[4][VF_LDS];
    const int T = p.T, nthr = blockDim.x, tid = threadIdx.x, b = blockIdx.x;
    StepAppend app;
    if constexpr (FUSED) app.begin(p, slot_map);
    int nr, start, end, t0, off0;
    const bool any = find_range(
        p, [&](int t) { return seg_len<NR>(t, T, pos, tok_seq, cu, p.skip_prompts, outs, p.spec, nr); }, sh_scan,
        sh_t0, start, end, t0, off0);
    if constexpr (FUSED) app.finish(p, slot_map);
    if (!any) return;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), kvh = blockIdx.y * 4 + wave;
    int t = t0, off = off0;
    while (off < end && t < T) {
        const int Ls =
            __builtin_amdgcn_readfirstlane(seg_len<NR>(t, T, pos, tok_seq, cu, p.skip_prompts, outs, p.spec, nr));
        if (Ls > 0) {
            nr = __builtin_amdgcn_readfirstlane(nr);
            int Lr[VF_ROWS];
#pragma unroll
            for (int r = 0; r < VF_ROWS; r++)
                Lr[r] = r < nr ? __builtin_amdgcn_readfirstlane(
                                     decode_len(t + r, pos, tok_seq, cu, p.skip_prompts, outs, p.spec))
                               : 0;
            const int seq = __builtin_amdgcn_readfirstlane(tok_seq[t]);
            const int j0 = max(start, off) - off, j1 = min(end, off + Ls) - off;
            const VerifyEpi<G> epi{p, t, kvh, t + b, j0 == 0 && j1 == Ls && !p.fo.mode};
            if constexpr (FUSED) {
                // the sequence's first row this step and its position
                const int row0 = __builtin_amdgcn_readfirstlane(cu[seq]);
                const int P0 = __builtin_amdgcn_readfirstlane(pos[row0]);
                verify_piece<G, true>(p, block_table + (size_t)seq * p.max_blocks, sh_v[wave], t, kvh, j0, j1, Lr,
                                      epi, P0, row0);
            } else {
                verify_piece<G>(p, block_table + (size_t)seq * p.max_blocks, sh_v[wave], t, kvh, j0, j1, Lr, epi);
            }
            off += Ls;
        }
        t++;
    }
}

// The same over an E4M3 cache with the E4M3 decode body (two pages per
// step, both products on MFMA, 16 columns = rows x query heads): grid
// (n_wg, ceil(Hkv / 4)) with two workgroups per CU (at most 256 VGPRs).
template <int G>
__global__ void __launch_bounds__(256, 2)
    verify_range8_kernel(DecodeParams p, const int* __restrict__ pos, const int* __restrict__ tok_seq,
                         const int* __restrict__ block_table, const int* __restrict__ cu,
                         const int* __restrict__ outs) {
    constexpr int NR = vf_rows(G);
    __shared__ int sh_scan[16];
    __shared__ int sh_t0[2];
    __shared__ WaveLds8 sh_w8[4];
    const int T = p.T, tid = threadIdx.x, b = blockIdx.x;
    int nr, start, end, t0, off0;
    if (!find_range(
            p, [&](int t) { return seg_len<NR>(t, T, pos, tok_seq, cu, p.skip_prompts, outs, p.spec, nr); }, sh_scan,
            sh_t0, start, end, t0, off0))
        return;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), kvh = blockIdx.y * 4 + wave;
    int t = t0, off = off0;
    while (off < end && t < T) {
        const int Ls =
            __builtin_amdgcn_readfirstlane(seg_len<NR>(t, T, pos, tok_seq, cu, p.skip_prompts, outs, p.spec, nr));
        if (Ls > 0) {
            nr = __builtin_amdgcn_readfirstlane(nr);
            int Lr[VF_ROWS];
#pragma unroll
            for (int r = 0; r < VF_ROWS; r++)
                Lr[r] = r < nr ? __builtin_amdgcn_readfirstlane(
                                     decode_len(t + r, pos, tok_seq, cu, p.skip_prompts, outs, p.spec))
                               : 0;
            const int seq = __builtin_amdgcn_readfirstlane(tok_seq[t]);
            const int j0 = max(start, off) - off, j1 = min(end, off + Ls) - off;
            const VerifyEpi<G> vepi{p, t, kvh, t + b, j0 == 0 && j1 == Ls && !p.fo.mode};
            auto epi = [&](int c, int gq, const f32x4 (&acc)[16], float m, float l) {
                vepi(c / G, c % G, gq, acc, m, l);
            };
            piece_body8<NR, G>(p, block_table + (size_t)seq * p.max_blocks, sh_w8[wave], t, kvh, j0, j1, epi, Lr);
            off += Ls;
        }
        t++;
    }
}

// Merges the split segments: one block of 64 NW threads per (row, query
// head) (NW as decode_merge_kernel's); row t's segment (NR rows) is headed
// by the row at offset NR * floor((t - cu[s]) / NR) of its sequence.
template <int NR, int NW = 4>
__global__ void __launch_bounds__(64 * NW)
    verify_merge_kernel(DecodeParams p, const int* __restrict__ pos, const int* __restrict__ tok_seq,
                        const int* __restrict__ cu, const int* __restrict__ outs) {
    const int t = blockIdx.x, T = p.T;
    if (decode_len(t, pos, tok_seq, cu, p.skip_prompts, outs, p.spec) <= 0) return;
    const int c0 = cu[tok_seq[t]];
    const int r = (t - c0) & (NR - 1), th = t - r;
    if (th < 0) return;
    const int o0 = p.offs[th], o1 = p.offs[th + 1];
    if (o1 <= o0) return;
    const int R = p.offs[T + 1];
    const int b0 = o0 / R, b1 = (o1 - 1) / R;
    if (b0 == b1 && !p.fo.mode) return;
    merge_head<NW>(p, t, (th + b0) * NR + r, NR, b1 - b0 + 1, blockIdx.y);
}

}  // namespace pkv

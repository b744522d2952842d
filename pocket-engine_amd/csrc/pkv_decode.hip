// Paged decode attention for gfx950 (bf16 cache, head_dim 256, GQA group 4,
// 16-slot pages). Same results as the reference's attn_paged_g4 +
// attn_merge (qwen35.cu:1146-1334, 2242-2279; AMD body
// amd/attn_decode.cuh:12-183), computed a different way:
//
// Work split ("flattened key space"). The keys of every decode token are
// laid end to end: token t owns [offs[t], offs[t] + L_t), L_t = pos[t] + 1.
// The W keys are cut into equal ranges of R keys (R >= min_range), one per
// workgroup, whatever the length mix: every workgroup streams the same
// number of bytes, so a batch of 512..8192-token contexts balances without a
// work queue. A range crossing token boundaries handles each token piece in
// turn. A token whose keys all fall in one range is finished in place (gated
// output); otherwise each piece leaves a partial (max, sum, weighted values)
// at index t + b (b = range index; t + b strictly grows along the walk, so it
// is unique and below T + n_wg), combined in key order by decode_merge_kernel
// (the same for the fused step).
//
// Inside a workgroup wave w takes kv head w, so one page read serves the G
// query heads of the group and the workgroup as a whole reads whole slot rows
// (all kv heads, 2 KiB) of each page. Per page (16 keys) a wave:
//   K: lane (row r = lane / 16, sub s = lane % 16) loads 16-byte chunks s and
//      s + 16 of keys 4p + r, p = 0..3: 8 loads, each row of 16 lanes reading
//      256 contiguous bytes. q.k partials (4 keys x 4 heads per lane) use
//      v_dot2c_f32_bf16 on bf16 pairs, then a reduce-scatter over the 16
//      lanes of a row (DPP xor 8 / xor 7 / xor 2 / xor 1) leaves lane s with
//      the full score of (key 4 (s / 4) + r, head s % 4).
//   softmax: running max per head over its 16 lanes (DPP rotates + two
//      cross-row shuffles), probabilities in f32, exp2 domain.
//   V: lane (half h = lane / 32, chunk c = lane % 32) loads keys 8h .. 8h + 7,
//      dims 8c .. 8c + 7 (16 bytes each: a full 512-byte row per half-wave);
//      probabilities reach it through 272 bytes of LDS; 256 FMAs per lane.
// K/V loads are nontemporal (read once): buffer loads with the page's base in
// the descriptor for cache pages, global loads for the step's own rows. The
// next page's K is requested
// right after q.k and its V right after P.V, so one page (16 KiB) is always
// in flight per wave; page ids come through the scalar cache. No MFMA.
//
// Fused append (decode_range_kernel<G, true>): the same kernel also appends
// the step's new K/V rows to their slots and reads every key of the step's
// own tokens (positions >= the first position the sequence feeds this step)
// from those source rows instead of the cache, so no range waits for another
// range's write. (Merging inside the kernel as well would need agent-scope
// release/acquire fences per token piece, an L2 writeback and invalidate on
// this multi-XCD part; measured at +45 us per batch-64 step, so the merge
// stays a second launch.)
#pragma once
#include "pkv_common.h"

#include <climits>
#include <type_traits>

namespace pkv {

struct DecodeParams {
    const uint16_t* q;        // [T][Hq][256]
    uint16_t* kc;             // [pages * 16][Hkv][256]
    uint16_t* vc;
    const uint16_t* qkv;      // gate of head h at row t: qkv[t * qstride + h * 512 + 256 ..]
    int qstride, Hq, Hkv;
    int max_blocks;
    uint16_t* out;            // [T][Hq][256]
    float scale;
    int skip_prompts;
    int spec;
    int T;
    long num_blocks;
    int* offs;                // [T + 2]: key offsets, then W and R
    float* part_ms;           // [(T + n_wg) * Hq][2]: max (log2 units), sum
    float* part_acc;          // [(T + n_wg) * Hq][256]
    int n_wg, min_range;
    // fused step: the step's new rows (k_rows + t * row_stride, Hkv * 256 each)
    const uint16_t* k_rows;
    const uint16_t* v_rows;
    long row_stride;          // elements
    // E4M3 cache (decode_range8_kernel, verify_range8_kernel): f32 scale per (slot, kv head)
    const float* kscale;
    const float* vscale;
    // FP8 copies of the gated outputs (mode != 0): every piece leaves a
    // partial record and the merge finishes every row, writing them
    Fp8Out fo;
};

constexpr int PAGE = 16;

// Exclusive prefix sum over the block; returns the block total in `total`.
__device__ __forceinline__ int block_scan(int v, int* sh, int& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) sh[w] = x;
    __syncthreads();
    int before = 0;
    total = 0;
    for (int k = 0; k < nw; k++) {
        const int s = sh[k];
        if (k < w) before += s;
        total += s;
    }
    __syncthreads();
    return before + x - v;
}

template <int G>
struct WaveLds {
    float p[PAGE * G];  // probabilities [key][head]
    float c[G];         // rescale factor per head
    float ml[2 * G];    // final (max, sum) per head
};

// Gated output of 4 dims: y = bf16(rbf(a * inv) * sigmoid(gate)) (reference
// qwen35.cu:1290-1293).
__device__ __forceinline__ uint2 gate4(float a0, float a1, float a2, float a3, float inv, uint2 graw,
                                       float* y = nullptr) {
    const float y0 = rbf(a0 * inv) / (1.f + __expf(-bf_lo(graw.x)));
    const float y1 = rbf(a1 * inv) / (1.f + __expf(-bf_hi(graw.x)));
    const float y2 = rbf(a2 * inv) / (1.f + __expf(-bf_lo(graw.y)));
    const float y3 = rbf(a3 * inv) / (1.f + __expf(-bf_hi(graw.y)));
    if (y) {
        y[0] = y0;
        y[1] = y1;
        y[2] = y2;
        y[3] = y3;
    }
    return make_uint2(pack2(y0, y1), pack2(y2, y3));
}

// Combines n partial records of one (row, query head) into its gated
// output: record i has its (max, sum) at ms_at(i) and its 256 weighted
// values at acc_at(i); max is in log2 units times mscale (1 for this
// library's records, log2 e for natural-log records). Same combination as
// the reference's attn_merge (qwen35.cu:2255-2273). One block of 64 NW
// threads: wave w folds records w, w + NW, .. into a running (max, sum,
// values) with U records in flight per lane (4 dims per lane; U = 16, or 10
// for NW = 16 within its 128 VGPRs), then the NW waves' results are combined
// through LDS (NW = 1: written straight from the wave). Every thread
// reaches the sync. (NW = 16 folds up to 160 records in one round of loads:
// launches with few (row, head) blocks and many records each.)
// With fo (mode != 0) the gated f32 outputs are also written as an FP8
// copy: row t, columns col .. col + 255 of a K-wide row.
template <int NW = 4, class MsAt, class AccAt>
__device__ __forceinline__ void merge_rows(int n, float mscale, MsAt ms_at, AccAt acc_at, const uint16_t* gate,
                                           uint16_t* out, const Fp8Out* fo = nullptr, int t = 0, int col = 0,
                                           int K = 0) {
    constexpr int U = NW >= 16 ? 10 : 16;
    __shared__ __align__(16) float sh_a[NW][HEAD_DIM + 4];
    // NW = 1: the calling wave alone (other waves of the block may merge
    // other rows)
    const int tid = threadIdx.x, lane = tid & 63, w = NW == 1 ? 0 : tid >> 6, d = 4 * lane;
    float M = -INFINITY, S = 0.f, A0 = 0.f, A1 = 0.f, A2 = 0.f, A3 = 0.f;
    for (int i0 = w; i0 < n; i0 += NW * U) {
        float2 mu[U];
        float4 au[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + NW * u;
            if (i < n) {
                mu[u] = *reinterpret_cast<const float2*>(ms_at(i));
                const float* a = acc_at(i) + d;  // 8-byte aligned
                const float2 lo = *reinterpret_cast<const float2*>(a), hi = *reinterpret_cast<const float2*>(a + 2);
                au[u] = make_float4(lo.x, lo.y, hi.x, hi.y);
                mu[u].x *= mscale;
            } else {
                mu[u] = make_float2(-INFINITY, 0.f);
                au[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float Mn = M;
#pragma unroll
        for (int u = 0; u < U; u++) Mn = fmaxf(Mn, mu[u].x);
        if (Mn == -INFINITY) continue;  // nothing attended yet
        const float c = __builtin_amdgcn_exp2f(M - Mn);  // 0 while M = -inf
        S *= c;
        A0 *= c;
        A1 *= c;
        A2 *= c;
        A3 *= c;
        M = Mn;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float f = __builtin_amdgcn_exp2f(mu[u].x - M);  // 0 for an empty record (-inf)
            S += mu[u].y * f;
            A0 += au[u].x * f;
            A1 += au[u].y * f;
            A2 += au[u].z * f;
            A3 += au[u].w * f;
        }
    }
    if constexpr (NW == 1) {
        // one wave: its own fold is the result (the same arithmetic as the
        // combine below with a single term)
        const float f = M == -INFINITY ? 0.f : 1.f;
        const uint2 graw = *reinterpret_cast<const uint2*>(gate + d);
        float y[4];
        *reinterpret_cast<uint2*>(out + d) = gate4(0.f + A0 * f, 0.f + A1 * f, 0.f + A2 * f, 0.f + A3 * f,
                                                   1.f / (0.f + S * f), graw, y);
        if (fo && fo->mode) fp8_quant4(y[0], y[1], y[2], y[3], t, col + d, K, *fo);
        return;
    }
    *reinterpret_cast<float4*>(&sh_a[w][d]) = make_float4(A0, A1, A2, A3);
    if (lane == 0) {
        sh_a[w][HEAD_DIM] = M;
        sh_a[w][HEAD_DIM + 1] = S;
    }
    __syncthreads();
    if (w == 0) {
        float Mt = -INFINITY;
#pragma unroll
        for (int k = 0; k < NW; k++) Mt = fmaxf(Mt, sh_a[k][HEAD_DIM]);
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < NW; k++) {
            const float mk = sh_a[k][HEAD_DIM];
            const float f = mk == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk - Mt);
            const float4 b = *reinterpret_cast<const float4*>(&sh_a[k][d]);
            a.x += b.x * f;
            a.y += b.y * f;
            a.z += b.z * f;
            a.w += b.w * f;
            s += sh_a[k][HEAD_DIM + 1] * f;
        }
        const uint2 graw = *reinterpret_cast<const uint2*>(gate + d);
        float y[4];
        *reinterpret_cast<uint2*>(out + d) = gate4(a.x, a.y, a.z, a.w, 1.f / s, graw, y);
        if (fo && fo->mode) fp8_quant4(y[0], y[1], y[2], y[3], t, col + d, K, *fo);
    }
}

// Merges this library's partials of token t, query head h: record i is row
// (base + i * stride) * Hq + h of part_ms / part_acc.
template <int NW = 4>
__device__ __forceinline__ void merge_head(const DecodeParams& p, int t, int base, int stride, int n, int h) {
    const Fp8Out* fo = p.fo.mode ? &p.fo : nullptr;
    const size_t r0 = (size_t)base * p.Hq + h, step = (size_t)stride * p.Hq;
    merge_rows<NW>(
        n, 1.f, [&](int i) { return p.part_ms + (r0 + i * step) * 2; },
        [&](int i) { return p.part_acc + (r0 + i * step) * HEAD_DIM; },
        p.qkv + (size_t)t * p.qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM, p.out + ((size_t)t * p.Hq + h) * HEAD_DIM,
        fo, t, h * HEAD_DIM, p.Hq * HEAD_DIM);
}

// One wave: token t, kv head kvh, keys [j0, j1) of its sequence. With FRESH,
// keys at positions [P0, L) come from the step's source rows (row
// row0 + position - P0) instead of the cache. The metadata pointers arrive as
// __restrict__ kernel arguments so the compiler reads them with scalar loads
// (no store of the kernel aliases them).
// FUSED: pages holding keys the step itself feeds (from the page of
// position P0 on) choose every K/V address per lane between the cache and
// the source rows (no branch, so the loads stay pipelined); earlier pages of
// the piece take the plain path.
// The wave's results go to epi(g, acc[8], m, l, ch) on the lanes of the
// first half-wave (ch = lane: dims 8 ch .. 8 ch + 7 of query head
// kvh * G + g; m in log2 units, l the sum of weights; m = -inf, l = 0 when
// no key of the piece is attended).
template <int G, bool FUSED, class Epi>
__device__ __forceinline__ void piece_body(const DecodeParams& p, const int* __restrict__ bt, WaveLds<G>& lds,
                                           int t, int kvh, int j0, int j1, int L, int P0, int row0, Epi epi) {
    static_assert(G == 4, "lane mapping assumes 4 keys x 4 heads per lane");
    const int lane = threadIdx.x & 63, sig = lane & 15, rho = lane >> 4;
    const int hv = lane >> 5, ch = lane & 31;
    const int Hkv = p.Hkv;
    const float sl2 = p.scale * LOG2E;

    uint4 qr[G][2];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const uint16_t* qrow = p.q + ((size_t)t * p.Hq + kvh * G + g) * HEAD_DIM;
        qr[g][0] = *reinterpret_cast<const uint4*>(qrow + 8 * sig);
        qr[g][1] = *reinterpret_cast<const uint4*>(qrow + 128 + 8 * sig);
    }
    const size_t row_elems = (size_t)Hkv * HEAD_DIM;
    auto page_base = [&](int pi) -> size_t {
        long pg = bt[pi];
        pg = pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg;
        return (size_t)pg * PAGE * row_elems + (size_t)kvh * HEAD_DIM;
    };
    // Address of key `key` of page pi (cache slot row, or the source row of
    // a key this step feeds), plus `off` elements.
    auto src = [&](const uint16_t* pool, const uint16_t* rows, int pi, size_t base, int key, int off) {
        const int kp = pi * PAGE + key;
        const uint16_t* c = pool + base + (size_t)key * row_elems + off;
        const uint16_t* f = rows + (ptrdiff_t)(row0 + kp - P0) * p.row_stride + (size_t)kvh * HEAD_DIM + off;
        return (kp >= P0 && kp < L) ? f : c;
    };
    uint4 kb[4][2], vb[8];
    // MODE 1: plain cache addresses; MODE 2: per-lane cache / source rows.
    // PLAIN pages load by buffer loads: the page's (uniform) base in the
    // descriptor, the lane's byte offsets fixed for the piece.
    const uint32_t k_lane = (uint32_t)(2 * (8 * sig + rho * row_elems));
    const uint32_t v_lane = (uint32_t)(2 * (8 * ch + 8 * hv * row_elems));
    const uint32_t row_b = (uint32_t)(2 * row_elems);
    auto load_k = [&](int pi, size_t base, auto mode) {
        constexpr bool FRESH = decltype(mode)::value == 2;
#pragma unroll
        for (int pp = 0; pp < 4; pp++) {
            if constexpr (FRESH) {
                const uint16_t* r = src(p.kc, p.k_rows, pi, base, 4 * pp + rho, 8 * sig);
                kb[pp][0] = load_nt(r);
                kb[pp][1] = load_nt(r + 128);
            } else {
                kb[pp][0] = buf_load16_nt(p.kc + base, k_lane + 4 * pp * row_b);
                kb[pp][1] = buf_load16_nt(p.kc + base, k_lane + 4 * pp * row_b + 256);
            }
        }
    };
    auto load_v = [&](int pi, size_t base, auto mode) {
        constexpr bool FRESH = decltype(mode)::value == 2;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if constexpr (FRESH)
                vb[k] = load_nt(src(p.vc, p.v_rows, pi, base, 8 * hv + k, 8 * ch));
            else
                vb[k] = buf_load16_nt(p.vc + base, v_lane + k * row_b);
        }
    };
    using NONE = std::integral_constant<int, 0>;
    using PLAIN = std::integral_constant<int, 1>;
    using FRESHM = std::integral_constant<int, 2>;

    float m = -INFINITY, l = 0.f;
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;

    const int pg0 = j0 / PAGE, pg1 = (j1 - 1) / PAGE;
    // One page: q.k, softmax, P.V. With PREFETCH the next page's K is
    // requested right after q.k and its V right after P.V; the last page is
    // peeled off so the loop body always prefetches and the compiler keeps
    // the loads in flight across iterations (partial vmcnt waits).
    auto page = [&](int pi, int next_pi, size_t next, auto prefetch) {
        constexpr bool PREFETCH = decltype(prefetch)::value != 0;
        // q . k partials: v[pp * 4 + g] over this lane's 16 dims.
        float v[16];
#pragma unroll
        for (int pp = 0; pp < 4; pp++)
#pragma unroll
            for (int g = 0; g < G; g++) v[pp * 4 + g] = dot8(qr[g][1], kb[pp][1], dot8(qr[g][0], kb[pp][0], 0.f));
        if constexpr (PREFETCH) load_k(next_pi, next, prefetch);
        // Reduce-scatter across the row's 16 lanes: after the step on lane
        // bit b the lane keeps the half of its values selected by that bit.
        {
            const bool b3 = sig & 8;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float keep = b3 ? v[k + 8] : v[k], send = b3 ? v[k] : v[k + 8];
                v[k] = keep + dpp<DPP_ROW_ROR8>(send);
            }
            const bool b2 = sig & 4;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float keep = b2 ? v[k + 4] : v[k], send = b2 ? v[k] : v[k + 4];
                v[k] = keep + dpp<DPP_ROW_HALF_MIRROR>(send);
            }
            const bool b1 = sig & 2;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const float keep = b1 ? v[k + 2] : v[k], send = b1 ? v[k] : v[k + 2];
                v[k] = keep + dpp<DPP_QUAD_XOR2>(send);
            }
            const bool b0 = sig & 1;
            const float keep = b0 ? v[1] : v[0], send = b0 ? v[0] : v[1];
            v[0] = keep + dpp<DPP_QUAD_XOR1>(send);
        }
        // Lane (sig, rho) now holds key 4 (sig / 4) + rho, head sig % 4.
        const int key = 4 * (sig >> 2) + rho, kpos = pi * PAGE + key;
        const float sc = (kpos >= j0 && kpos < j1) ? v[0] * sl2 : -INFINITY;
        float mx = fmaxf(sc, dpp<DPP_ROW_ROR4>(sc));
        mx = fmaxf(mx, dpp<DPP_ROW_ROR8>(mx));
        mx = max_xor32(max_xor16(mx));
        const float mn = fmaxf(m, mx);
        const float corr = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first page (m = -inf)
        const float pr = __builtin_amdgcn_exp2f(sc - mn);
        l = l * corr + pr;
        m = mn;
        lds.p[key * G + (sig & 3)] = pr;
        if (lane < G) lds.c[lane] = corr;
        wave_sync();
        const float4 cr = *reinterpret_cast<const float4*>(lds.c);
        const float cg[4] = {cr.x, cr.y, cr.z, cr.w};
        if (__any(cr.x != 1.f || cr.y != 1.f || cr.z != 1.f || cr.w != 1.f)) {
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] *= cg[g];
        }
        // Keys outside [j0, j1) on a partial page (the piece's first or
        // last) carry weight 0; their V is zeroed too, since a stale slot
        // may hold NaN.
        if (pi * PAGE < j0 || pi * PAGE + PAGE > j1) {
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int kp = pi * PAGE + 8 * hv + k;
                if (kp < j0 || kp >= j1) vb[k] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 pk = *reinterpret_cast<const float4*>(&lds.p[(8 * hv + k) * G]);
            const float pg[4] = {pk.x, pk.y, pk.z, pk.w};
            const uint32_t w[4] = {vb[k].x, vb[k].y, vb[k].z, vb[k].w};
#pragma unroll
            for (int e2 = 0; e2 < 4; e2++) {
                const float x0 = bf_lo(w[e2]), x1 = bf_hi(w[e2]);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    acc[g][2 * e2] = fmaf(pg[g], x0, acc[g][2 * e2]);
                    acc[g][2 * e2 + 1] = fmaf(pg[g], x1, acc[g][2 * e2 + 1]);
                }
            }
        }
        wave_sync();  // lds.p / lds.c are rewritten for the next page
        if constexpr (PREFETCH) load_v(next_pi, next, prefetch);
    };
    // First page holding keys of the step (none: pg1 + 1).
    const int pf = FUSED ? max(pg0, min(pg1 + 1, P0 / PAGE)) : pg1 + 1;
    if (pf > pg1) {
        const size_t base = page_base(pg0);
        load_k(pg0, base, PLAIN{});
        load_v(pg0, base, PLAIN{});
        for (int pi = pg0; pi < pg1; pi++) page(pi, pi + 1, page_base(pi + 1), PLAIN{});
    } else if constexpr (FUSED) {
        const size_t base = page_base(pg0);
        if (pf == pg0) {
            load_k(pg0, base, FRESHM{});
            load_v(pg0, base, FRESHM{});
        } else {
            load_k(pg0, base, PLAIN{});
            load_v(pg0, base, PLAIN{});
            for (int pi = pg0; pi < pf - 1; pi++) page(pi, pi + 1, page_base(pi + 1), PLAIN{});
            page(pf - 1, pf, page_base(pf), FRESHM{});
        }
        for (int pi = pf; pi < pg1; pi++) page(pi, pi + 1, page_base(pi + 1), FRESHM{});
    }
    page(pg1, pg1, 0, NONE{});
    // Totals: the sum over the head's 16 lanes, the two halves' values.
    l += dpp<DPP_ROW_ROR4>(l);
    l += dpp<DPP_ROW_ROR8>(l);
    l = add_xor32(add_xor16(l));
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = add_xor32(acc[g][e]);
    if (lane < G) {
        lds.ml[2 * lane] = m;
        lds.ml[2 * lane + 1] = l;
    }
    wave_sync();
    if (hv != 0) return;
#pragma unroll
    for (int g = 0; g < G; g++) epi(g, acc[g], lds.ml[2 * g], lds.ml[2 * g + 1], ch);
}

// Writes a piece's result: the gated output when the piece holds all of the
// token's keys, else the partial record at index idx.
template <int G>
struct DecodeEpi {
    const DecodeParams& p;
    int t, kvh, idx;
    bool direct;
    __device__ __forceinline__ void operator()(int g, const float (&acc)[8], float m, float l, int ch) const {
        const int h = kvh * G + g;
        if (direct) {
            const float inv = 1.f / l;
            const uint4 graw = *reinterpret_cast<const uint4*>(p.qkv + (size_t)t * p.qstride + (size_t)h * 2 * HEAD_DIM +
                                                               HEAD_DIM + 8 * ch);
            const uint2 lo = gate4(acc[0], acc[1], acc[2], acc[3], inv, make_uint2(graw.x, graw.y));
            const uint2 hi = gate4(acc[4], acc[5], acc[6], acc[7], inv, make_uint2(graw.z, graw.w));
            *reinterpret_cast<uint4*>(p.out + ((size_t)t * p.Hq + h) * HEAD_DIM + 8 * ch) =
                make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else {
            float* pa = p.part_acc + ((size_t)idx * p.Hq + h) * HEAD_DIM + 8 * ch;
            *reinterpret_cast<float4*>(pa) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            *reinterpret_cast<float4*>(pa + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
            if (ch == 0) *reinterpret_cast<float2*>(p.part_ms + ((size_t)idx * p.Hq + h) * 2) = make_float2(m, l);
        }
    }
};

template <int G, bool FUSED>
__device__ __forceinline__ void decode_piece(const DecodeParams& p, const int* __restrict__ block_table, WaveLds<G>& lds,
                                             int t, int seq, int row0, int P0, int kvh, int j0, int j1, int L,
                                             int idx) {
    const int* __restrict__ bt = block_table + (size_t)seq * p.max_blocks;
    const DecodeEpi<G> epi{p, t, kvh, idx, j0 == 0 && j1 == L && !p.fo.mode};
    if constexpr (FUSED)
        piece_body<G, true>(p, bt, lds, t, kvh, j0, j1, L, P0, row0, epi);
    else
        piece_body<G, false>(p, bt, lds, t, kvh, j0, j1, L, INT_MAX, 0, epi);
}

// The fused step's append, shared by the fused key-range kernels: block
// (b, y) writes the step's K and V rows of kv heads 4y .. 4y + 3 for tokens
// b, b + n_wg, .. into their slots (slot_map; -1 or past the pool: skipped).
// No range of the launch reads these slots from the cache: keys the step
// feeds come from the source rows. begin() issues the first token's loads
// before the range search; finish() stores them after it (the latency
// overlaps the search) and appends the block's other tokens. Block: 64
// threads per kv head, one uint4 of K or V per thread and token.
struct StepAppend {
    long slot = -1;
    uint4 val;
    __device__ __forceinline__ const uint4* src(const DecodeParams& p, int t, int i) const {
        const int per_row = (blockDim.x >> 6) * HEAD_DIM / 8;  // uint4 per K (or V) row slice
        const bool is_v = i >= per_row;
        return reinterpret_cast<const uint4*>((is_v ? p.v_rows : p.k_rows) + (size_t)t * p.row_stride +
                                              (size_t)blockIdx.y * 4 * HEAD_DIM) +
               (is_v ? i - per_row : i);
    }
    __device__ __forceinline__ void store(const DecodeParams& p, long s, int i, uint4 v) const {
        const int per_row = (blockDim.x >> 6) * HEAD_DIM / 8;
        const bool is_v = i >= per_row;
        reinterpret_cast<uint4*>((is_v ? p.vc : p.kc) + ((size_t)s * p.Hkv + blockIdx.y * 4) * HEAD_DIM)
            [is_v ? i - per_row : i] = v;
    }
    __device__ __forceinline__ void begin(const DecodeParams& p, const int* __restrict__ slot_map) {
        const int b = blockIdx.x;
        if (b < p.T) {
            slot = slot_map[b];
            val = *src(p, b, threadIdx.x);
        }
    }
    __device__ __forceinline__ void finish(const DecodeParams& p, const int* __restrict__ slot_map) const {
        const int b = blockIdx.x, tid = threadIdx.x;
        const long cap = p.num_blocks * PAGE;
        if (slot >= 0 && slot < cap) store(p, slot, tid, val);
        for (int t = b + p.n_wg; t < p.T; t += p.n_wg) {
            const long s = slot_map[t];
            if (s >= 0 && s < cap) store(p, s, tid, *src(p, t, tid));
        }
    }
};

// The workgroup's key range [start, end) of the flattened key space (keys
// of token t: lenf(t)), cut into equal ranges of R = max(min_range,
// ceil(W / n_wg)) keys, and the token t0 holding key `start` at offset off0.
// Workgroup (0, 0) also writes offs[t] (exclusive offsets), offs[T] = W and
// offs[T + 1] = R for the merge. For T <= block size one scan serves both;
// otherwise a first pass totals W and a second finds the offsets. Returns
// false (for the whole workgroup) when the range is empty.
template <class LenF>
__device__ __forceinline__ bool find_range(const DecodeParams& p, LenF lenf, int* sh_scan, int* sh_t0, int& start,
                                           int& end, int& t0, int& off0) {
    const int T = p.T, nthr = blockDim.x, tid = threadIdx.x, b = blockIdx.x;
    const bool writer = b == 0 && blockIdx.y == 0;
    const bool one = T <= nthr;
    int W = 0, myL = 0, myoff = 0;
    if (one) {
        myL = tid < T ? lenf(tid) : 0;
        myoff = block_scan(myL, sh_scan, W);
    } else {
        for (int base = 0; base < T; base += nthr) {
            const int t = base + tid;
            const int L = t < T ? lenf(t) : 0;
            int tot;
            block_scan(L, sh_scan, tot);
            W += tot;
        }
    }
    W = __builtin_amdgcn_readfirstlane(W);  // block-uniform: keep it in scalar registers
    const int R = max(p.min_range, (W + p.n_wg - 1) / p.n_wg);
    start = b * R;
    end = min(W, start + R);
    if (writer && tid == 0) {
        p.offs[T] = W;
        p.offs[T + 1] = R;
    }
    if (one) {
        if (tid < T) {
            if (writer) p.offs[tid] = myoff;
            if (myL > 0 && myoff <= start && start < myoff + myL) {
                sh_t0[0] = tid;
                sh_t0[1] = myoff;
            }
        }
    } else {
        if (start >= W && b != 0) return false;
        int run = 0;
        for (int base = 0; base < T; base += nthr) {
            const int t = base + tid;
            const int L = t < T ? lenf(t) : 0;
            int tot;
            const int off = run + block_scan(L, sh_scan, tot);
            if (t < T) {
                if (writer) p.offs[t] = off;
                if (L > 0 && off <= start && start < off + L) {
                    sh_t0[0] = t;
                    sh_t0[1] = off;
                }
            }
            run += tot;
            if (b != 0 && run > start) break;  // uniform: every thread has the same run
        }
    }
    if (start >= W) return false;
    __syncthreads();
    t0 = __builtin_amdgcn_readfirstlane(sh_t0[0]);
    off0 = __builtin_amdgcn_readfirstlane(sh_t0[1]);
    return true;
}

// Key-range kernel (FUSED = false) or fused step kernel (FUSED = true): one
// workgroup per key range and group of up to 4 kv heads (blockIdx.y), a wave
// per kv head. Block: 64 * min(Hkv, 4) threads (the host rejects Hkv > 4 that
// is not a multiple of 4).
template <int G, bool FUSED>
__global__ void __launch_bounds__(256, 1)
    decode_range_kernel(DecodeParams p, const int* __restrict__ pos, const int* __restrict__ tok_seq,
                        const int* __restrict__ block_table, const int* __restrict__ cu,
                        const int* __restrict__ outs, const int* __restrict__ slot_map) {
    __shared__ int sh_scan[16];
    __shared__ int sh_t0[2];
    __shared__ WaveLds<G> sh_w[4];
    // pos and tok_seq of every token (T <= block size): a piece's sequence,
    // first row and first position come from LDS, not from dependent global
    // loads at every piece start.
    __shared__ int sh_pos[256], sh_seq[256];
    const int T = p.T, nthr = blockDim.x, tid = threadIdx.x, b = blockIdx.x;
    const bool tab = T <= nthr;
    StepAppend app;
    if constexpr (FUSED) app.begin(p, slot_map);
    int start, end, t0, off0;
    const bool any = find_range(
        p,
        [&](int t) {
            const int L = decode_len(t, pos, tok_seq, cu, p.skip_prompts, outs, p.spec);
            if (tab) {
                sh_pos[t] = pos[t];
                sh_seq[t] = tok_seq[t];
            }
            return L;
        },
        sh_scan, sh_t0, start, end, t0, off0);
    if constexpr (FUSED) app.finish(p, slot_map);
    if (!any) return;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), kvh = blockIdx.y * 4 + wave;
    int t = t0, off = off0;
    while (off < end && t < T) {
        const int L = !tab || p.skip_prompts ? decode_len(t, pos, tok_seq, cu, p.skip_prompts, outs, p.spec)
                                             : sh_pos[t] + 1;
        if (L > 0) {
            const int j0 = max(start, off) - off, j1 = min(end, off + L) - off;
            int seq, row0 = t, P0 = 0;
            if (tab) {
                // the sequence's rows of this step are the run of equal
                // tok_seq around t; its first row's position is P0
                seq = __builtin_amdgcn_readfirstlane(sh_seq[t]);
                if constexpr (FUSED) {
                    while (row0 > 0 && sh_seq[row0 - 1] == seq) row0--;
                    P0 = __builtin_amdgcn_readfirstlane(sh_pos[row0]);
                }
            } else {
                seq = __builtin_amdgcn_readfirstlane(tok_seq[t]);
                if constexpr (FUSED) {
                    row0 = __builtin_amdgcn_readfirstlane(cu[seq]);
                    P0 = __builtin_amdgcn_readfirstlane(pos[row0]);
                }
            }
            decode_piece<G, FUSED>(p, block_table, sh_w[wave], t, seq, row0, P0, kvh, j0, j1, L, t + b);
            off += L;
        }
        t++;
    }
}

// Combines the partials of tokens split over several ranges (after
// decode_range_kernel). One block of 64 NW threads per (token, query head).
template <int NW>
__global__ void __launch_bounds__(64 * NW) decode_merge_kernel(DecodeParams p) {
    const int t = blockIdx.x, T = p.T;
    const int o0 = p.offs[t], o1 = p.offs[t + 1];  // offs[T] = W
    if (o1 <= o0) return;
    const int R = p.offs[T + 1];
    const int b0 = o0 / R, b1 = (o1 - 1) / R;
    if (b0 == b1 && !p.fo.mode) return;  // finished in place by its range
    merge_head<NW>(p, t, t + b0, 1, b1 - b0 + 1, blockIdx.y);
}
template __global__ void decode_merge_kernel<1>(DecodeParams);
template __global__ void decode_merge_kernel<4>(DecodeParams);
template __global__ void decode_merge_kernel<16>(DecodeParams);

template __global__ void decode_range_kernel<4, false>(DecodeParams, const int*, const int*, const int*, const int*,
                                                       const int*, const int*);
template __global__ void decode_range_kernel<4, true>(DecodeParams, const int*, const int*, const int*, const int*,
                                                      const int*, const int*);

}  // namespace pkv

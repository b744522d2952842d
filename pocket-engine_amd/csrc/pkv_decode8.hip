// Paged decode attention over an E4M3 cache (gfx950): the reference's
// attn_paged8_g4 + attn_merge (qwen35.cu:1146-1334 with F8, 2242-2279).
// For key j of token t, kv head h (slot s = bt[j / 16] * 16 + j % 16):
//   score_j = (q . e4m3(K[s][h])) * kscale[s][h],
//   weight_j = exp(score_j - max) (the softmax sum takes weight_j),
//   out += weight_j * vscale[s][h] * e4m3(V[s][h]),
// then out / sum, rounded to bf16 and gated as the bf16 decode.
//
// Work split, ranges, partial records and the merge are decode_range_kernel's
// (pkv_decode.hip). What changes is the inner loop: an E4M3 page holds half
// the bytes of a bf16 page, so a wave walks two pages (32 keys, 8 KiB of K
// and V for its kv head) per step, which keeps the same bytes in flight per
// wave as the bf16 kernel and the same register footprint:
//   K: lane (row r = lane / 16, sub s = lane % 16) loads the 16-byte chunk s
//      (dims 16 s .. 16 s + 15) of keys 4 p + r, p = 0..7 (keys 0..15 from
//      the first page, 16..31 from the second): 8 loads, each row of 16 lanes
//      reading one 256-byte key row. The bytes become bf16 pairs
//      (v_cvt_scalef32_pk_bf16_fp8, exact) and meet q in v_dot2c_f32_bf16.
//      A reduce-scatter over the 16 lanes of a row (xor 8, xor 7, xor 2,
//      xor 1) leaves lane s with the scores of key 4 (s / 2) + r for heads
//      2 (s % 2) and 2 (s % 2) + 1.
//   softmax: per head over the 8 lanes of a row that share s % 2 (DPP row
//      rotates by 2, 4, 8) and the 4 rows (two shuffles); exp2 domain.
//   V: lane (quarter u = lane / 16, chunk c = lane % 16) loads dims
//      16 c .. 16 c + 15 of keys 8 u .. 8 u + 7 (16 bytes each), converts
//      them to f32 (v_cvt_pk_f32_fp8) and accumulates 16 dims x 4 heads;
//      the four quarters are summed at the end of a piece.
// kscale / vscale of the lane's key are loaded with the K bytes (4 bytes
// per lane). Keys outside the piece get score -inf and weight 0 by select,
// and their V bytes are zeroed, so a stale slot (NaN bytes or scales)
// contributes nothing.
#pragma once
#include "pkv_decode.hip"

namespace pkv {

constexpr int DPP_ROW_ROR2 = 0x122;  // lane i <- lane (i + 2) % 16 of its row
constexpr int UNIT8 = 2 * PAGE;      // keys per step of the E4M3 kernel

struct WaveLds8 {
    float p[UNIT8 * 4];  // weight x vscale, [key][head]
    float c[4];          // rescale factor per head
    float ml[8];         // final (max, sum) per head
};

// Sixteen E4M3 bytes to sixteen bf16 (two uint4), exact.
__device__ __forceinline__ void e4m3x16_to_bf16(const uint4& b, uint4& lo, uint4& hi) {
    lo = e4m3x8_to_bf16x8(b.x, b.y);
    hi = e4m3x8_to_bf16x8(b.z, b.w);
}

// One wave: token t, kv head kvh, keys [j0, j1) of its sequence (block
// table row bt), over the E4M3 cache. Results go to epi as in piece_body.
template <class Epi>
__device__ __forceinline__ void piece_body8(const DecodeParams& p, const int* __restrict__ bt, WaveLds8& lds, int t,
                                            int kvh, int j0, int j1, Epi epi) {
    constexpr int G = 4;
    const int lane = threadIdx.x & 63, sig = lane & 15, rho = lane >> 4;
    const int Hkv = p.Hkv;
    const float sl2 = p.scale * LOG2E;
    const uint8_t* kc = reinterpret_cast<const uint8_t*>(p.kc);
    const uint8_t* vc = reinterpret_cast<const uint8_t*>(p.vc);

    uint4 qr[G][2];  // q dims 16 sig .. 16 sig + 15 of the group's heads
#pragma unroll
    for (int g = 0; g < G; g++) {
        const uint16_t* qrow = p.q + ((size_t)t * p.Hq + kvh * G + g) * HEAD_DIM + 16 * sig;
        qr[g][0] = *reinterpret_cast<const uint4*>(qrow);
        qr[g][1] = *reinterpret_cast<const uint4*>(qrow + 8);
    }
    const size_t row_bytes = (size_t)Hkv * HEAD_DIM;  // one slot row (all kv heads), bytes
    auto page_id = [&](int pi) -> long {
        long pg = bt[pi];
        return pg < 0 ? 0 : pg >= p.num_blocks ? p.num_blocks - 1 : pg;
    };
    // Slots of the unit's two pages (the second page of a unit past the
    // piece's last key repeats the first: read, then masked).
    auto unit_pages = [&](int u, long& pg_a, long& pg_b) {
        pg_a = page_id(2 * u);
        pg_b = UNIT8 * u + PAGE < j1 ? page_id(2 * u + 1) : pg_a;
    };
    uint4 kb[8], vb[8];
    float ks, vs;  // scales of this lane's score key
    const int skey = 4 * (sig >> 1) + rho;  // the key whose scores this lane ends with
    auto load_k = [&](long pg_a, long pg_b) {
#pragma unroll
        for (int pp = 0; pp < 8; pp++) {
            const long pg = pp < 4 ? pg_a : pg_b;
            const int key = (4 * pp + rho) & (PAGE - 1);
            kb[pp] = load_nt(kc + ((size_t)pg * PAGE + key) * row_bytes + (size_t)kvh * HEAD_DIM + 16 * sig);
        }
        const size_t at = ((size_t)(skey < PAGE ? pg_a : pg_b) * PAGE + (skey & (PAGE - 1))) * Hkv + kvh;
        ks = p.kscale[at];
        vs = p.vscale[at];
    };
    auto load_v = [&](long pg_a, long pg_b) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int key = 8 * rho + k;  // rho is the quarter u here
            const long pg = key < PAGE ? pg_a : pg_b;
            vb[k] = load_nt(vc + ((size_t)pg * PAGE + (key & (PAGE - 1))) * row_bytes + (size_t)kvh * HEAD_DIM +
                            16 * sig);
        }
    };

    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;  // heads 2 (sig & 1) + e
    float acc[G][16];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[g][e] = 0.f;

    const int u0 = j0 / UNIT8, u1 = (j1 - 1) / UNIT8;
    auto unit = [&](int u, int next_u, auto prefetch) {
        constexpr bool PREFETCH = decltype(prefetch)::value != 0;
        long na = 0, nb = 0;
        if constexpr (PREFETCH) unit_pages(next_u, na, nb);
        // q . k partials: v[pp * 4 + g] over this lane's 16 dims.
        float v[32];
#pragma unroll
        for (int pp = 0; pp < 8; pp++) {
            uint4 lo, hi;
            e4m3x16_to_bf16(kb[pp], lo, hi);
#pragma unroll
            for (int g = 0; g < G; g++) v[pp * 4 + g] = dot8(qr[g][1], hi, dot8(qr[g][0], lo, 0.f));
        }
        const float ks_u = ks, vs_u = vs;
        if constexpr (PREFETCH) load_k(na, nb);
        // Reduce-scatter across the row's 16 lanes: the value index ends up
        // as 2 sig + e (bit 4 from sig bit 3, .., bit 1 from sig bit 0).
        {
            const bool b3 = sig & 8;
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float keep = b3 ? v[k + 16] : v[k], send = b3 ? v[k] : v[k + 16];
                v[k] = keep + dpp<DPP_ROW_ROR8>(send);
            }
            const bool b2 = sig & 4;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float keep = b2 ? v[k + 8] : v[k], send = b2 ? v[k] : v[k + 8];
                v[k] = keep + dpp<DPP_ROW_HALF_MIRROR>(send);
            }
            const bool b1 = sig & 2;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float keep = b1 ? v[k + 4] : v[k], send = b1 ? v[k] : v[k + 4];
                v[k] = keep + dpp<DPP_QUAD_XOR2>(send);
            }
            const bool b0 = sig & 1;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const float keep = b0 ? v[k + 2] : v[k], send = b0 ? v[k] : v[k + 2];
                v[k] = keep + dpp<DPP_QUAD_XOR1>(send);
            }
        }
        // Lane (sig, rho): key skey, heads 2 (sig & 1) + e in v[e].
        const int kpos = UNIT8 * u + skey;
        const bool in = kpos >= j0 && kpos < j1;
        const float f = ks_u * sl2;
        const float sc0 = in ? v[0] * f : -INFINITY, sc1 = in ? v[1] * f : -INFINITY;
        auto rowmax = [&](float x) {
            x = fmaxf(x, dpp<DPP_ROW_ROR2>(x));
            x = fmaxf(x, dpp<DPP_ROW_ROR4>(x));
            x = fmaxf(x, dpp<DPP_ROW_ROR8>(x));
            x = fmaxf(x, shfl_xor(x, 16));
            return fmaxf(x, shfl_xor(x, 32));
        };
        const float mn0 = fmaxf(m0, rowmax(sc0)), mn1 = fmaxf(m1, rowmax(sc1));
        const float c0 = __builtin_amdgcn_exp2f(m0 - mn0), c1 = __builtin_amdgcn_exp2f(m1 - mn1);
        const float p0 = __builtin_amdgcn_exp2f(sc0 - mn0), p1 = __builtin_amdgcn_exp2f(sc1 - mn1);
        l0 = l0 * c0 + p0;
        l1 = l1 * c1 + p1;
        m0 = mn0;
        m1 = mn1;
        const int hb = 2 * (sig & 1);
        lds.p[skey * G + hb] = in ? p0 * vs_u : 0.f;
        lds.p[skey * G + hb + 1] = in ? p1 * vs_u : 0.f;
        if (lane < 2) {
            lds.c[hb] = c0;
            lds.c[hb + 1] = c1;
        }
        wave_sync();
        const float4 cr = *reinterpret_cast<const float4*>(lds.c);
        const float cg[4] = {cr.x, cr.y, cr.z, cr.w};
        if (__any(cr.x != 1.f || cr.y != 1.f || cr.z != 1.f || cr.w != 1.f)) {
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[g][e] *= cg[g];
        }
        // V bytes of keys outside [j0, j1) (a partial unit) are zeroed.
        if (UNIT8 * u < j0 || UNIT8 * u + UNIT8 > j1) {
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int kp = UNIT8 * u + 8 * rho + k;
                if (kp < j0 || kp >= j1) vb[k] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 pk = *reinterpret_cast<const float4*>(&lds.p[(8 * rho + k) * G]);
            const float pg[4] = {pk.x, pk.y, pk.z, pk.w};
            const uint32_t w[4] = {vb[k].x, vb[k].y, vb[k].z, vb[k].w};
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++) {
                const f32x2 x01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[e4], false);
                const f32x2 x23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[e4], true);
                const float x[4] = {x01.x, x01.y, x23.x, x23.y};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int g = 0; g < G; g++) acc[g][4 * e4 + i] = fmaf(pg[g], x[i], acc[g][4 * e4 + i]);
            }
        }
        wave_sync();  // lds.p / lds.c are rewritten for the next unit
        if constexpr (PREFETCH) load_v(na, nb);
    };
    using NONE = std::integral_constant<int, 0>;
    using PF = std::integral_constant<int, 1>;
    {
        long a, b;
        unit_pages(u0, a, b);
        load_k(a, b);
        load_v(a, b);
    }
    for (int u = u0; u < u1; u++) unit(u, u + 1, PF{});
    unit(u1, u1, NONE{});
    // Totals: a head's sum over the 8 lanes of each row sharing sig & 1 and
    // the 4 rows; values over the 4 quarters.
    auto rowsum = [&](float x) {
        x += dpp<DPP_ROW_ROR2>(x);
        x += dpp<DPP_ROW_ROR4>(x);
        x += dpp<DPP_ROW_ROR8>(x);
        x += shfl_xor(x, 16);
        return x + shfl_xor(x, 32);
    };
    l0 = rowsum(l0);
    l1 = rowsum(l1);
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            acc[g][e] += shfl_xor(acc[g][e], 16);
            acc[g][e] += shfl_xor(acc[g][e], 32);
        }
    if (lane < 2) {
        const int hb = 2 * lane;
        lds.ml[2 * hb] = m0;
        lds.ml[2 * hb + 1] = l0;
        lds.ml[2 * hb + 2] = m1;
        lds.ml[2 * hb + 3] = l1;
    }
    wave_sync();
    if (lane >= 16) return;
#pragma unroll
    for (int g = 0; g < G; g++) {
        float a[8], b[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            a[e] = acc[g][e];
            b[e] = acc[g][8 + e];
        }
        epi(g, a, lds.ml[2 * g], lds.ml[2 * g + 1], 2 * sig);
        epi(g, b, lds.ml[2 * g], lds.ml[2 * g + 1], 2 * sig + 1);
    }
}

// Key-range kernel over the E4M3 cache: decode_range_kernel<4, false>'s
// ranges and records with piece_body8 inside. Grid (n_wg, ceil(Hkv / 4)),
// 64 * min(Hkv, 4) threads; two workgroups per CU (at most 256 VGPRs).
__global__ void __launch_bounds__(256, 2)
    decode_range8_kernel(DecodeParams p, const int* __restrict__ pos, const int* __restrict__ tok_seq,
                         const int* __restrict__ block_table, const int* __restrict__ cu,
                         const int* __restrict__ outs) {
    __shared__ int sh_scan[16];
    __shared__ int sh_t0[2];
    __shared__ WaveLds8 sh_w[4];
    __shared__ int sh_pos[256], sh_seq[256];
    const int T = p.T, nthr = blockDim.x, tid = threadIdx.x, b = blockIdx.x;
    const bool tab = T <= nthr;
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
    if (!any) return;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), kvh = blockIdx.y * 4 + wave;
    int t = t0, off = off0;
    while (off < end && t < T) {
        const int L = !tab || p.skip_prompts ? decode_len(t, pos, tok_seq, cu, p.skip_prompts, outs, p.spec)
                                             : sh_pos[t] + 1;
        if (L > 0) {
            const int j0 = max(start, off) - off, j1 = min(end, off + L) - off;
            const int seq = __builtin_amdgcn_readfirstlane(tab ? sh_seq[t] : tok_seq[t]);
            const DecodeEpi<4> epi{p, t, kvh, t + b, j0 == 0 && j1 == L};
            piece_body8(p, block_table + (size_t)seq * p.max_blocks, sh_w[wave], t, kvh, j0, j1, epi);
            off += L;
        }
        t++;
    }
}

}  // namespace pkv

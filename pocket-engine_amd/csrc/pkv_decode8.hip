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
// wave as the bf16 kernel:
//   q.k on MFMA: per page S[16 keys][16 columns] in 8 steps of
//      v_mfma_f32_16x16x32_bf16. Lane (column s = lane % 16, group
//      r = lane / 16) loads 64 contiguous bytes of key s (dims 16 r + 64 c,
//      c = 0..3: 4 loads per page) and converts them to bf16 (exact,
//      v_cvt_scalef32_pk_bf16_fp8) as the A operand; the B operand is query
//      head s (columns 4..15 zero) over the same dims. The lane ends with the
//      scores of keys 4 r .. 4 r + 3 of the page for head s.
//   softmax: per head over the lane's 8 keys and its 4 lane groups (two
//      shuffles); exp2 domain; kscale / vscale of the unit's 32 keys come
//      through 256 bytes of LDS (one 4-byte load per lane).
//   V on VALU: lane (quarter u = lane / 16, chunk c = lane % 16) loads dims
//      16 c .. 16 c + 15 of keys 8 u .. 8 u + 7 (16 bytes each), converts
//      them to f32 (v_cvt_pk_f32_fp8) and accumulates 16 dims x 4 heads with
//      f32 FMAs of weight x vscale (the reference's f32 products); the four
//      quarters are summed at the end of a piece.
// Keys outside the piece get score -inf and weight 0 by select, and their V
// bytes are zeroed, so a stale slot (NaN bytes or scales) contributes
// nothing.
#pragma once
#include "pkv_decode.hip"

namespace pkv {

constexpr int DPP_ROW_ROR2 = 0x122;  // lane i <- lane (i + 2) % 16 of its row
constexpr int UNIT8 = 2 * PAGE;      // keys per step of the E4M3 kernel

struct WaveLds8 {
    float p[UNIT8 * 4];  // weight x vscale, [key][head]
    float sc[64];        // the unit's kscale [key], then vscale [key]
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

    // q.k on MFMA: S[16 keys][16 columns] = K Q^T per page, 8 steps of
    // v_mfma_f32_16x16x32_bf16 over the 256 dims. Lane (column sig, group
    // rho) supplies, in step s = 2 c + h, dims 64 c + 16 rho + 8 h .. + 7 of
    // key sig (A, from the E4M3 bytes) and of query head sig (B; columns
    // 4..15 are zero), and ends with the scores of keys 4 rho .. 4 rho + 3 of
    // the page for head sig.
    bf16x8 qf[8];
    {
        const uint16_t* qrow = p.q + ((size_t)t * p.Hq + kvh * G + (sig & 3)) * HEAD_DIM + 16 * rho;
#pragma unroll
        for (int s = 0; s < 8; s++)
            qf[s] = as_bf16x8(sig < G ? *reinterpret_cast<const uint4*>(qrow + 64 * (s >> 1) + 8 * (s & 1))
                                      : make_uint4(0, 0, 0, 0));
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
    uint4 kb[2][4], vb[8];
    float sc_ld;  // kscale (lanes 0..31) or vscale (lanes 32..63) of unit key lane % 32
    auto load_k = [&](long pg_a, long pg_b) {
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            const uint8_t* r = kc + ((size_t)(pg ? pg_b : pg_a) * PAGE + sig) * row_bytes + (size_t)kvh * HEAD_DIM +
                               16 * rho;
#pragma unroll
            for (int c = 0; c < 4; c++) kb[pg][c] = load_nt(r + 64 * c);
        }
        const int key = lane & 31;
        const size_t at = ((size_t)(key < PAGE ? pg_a : pg_b) * PAGE + (key & (PAGE - 1))) * Hkv + kvh;
        sc_ld = (lane < 32 ? p.kscale : p.vscale)[at];
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

    float m = -INFINITY, l = 0.f;  // head sig (lanes with sig < 4)
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
        f32x4 sacc[2];
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            sacc[pg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const uint4 w = kb[pg][s >> 1];
                const bf16x8 a = as_bf16x8((s & 1) ? e4m3x8_to_bf16x8(w.z, w.w) : e4m3x8_to_bf16x8(w.x, w.y));
                sacc[pg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[s], sacc[pg], 0, 0, 0);
            }
        }
        lds.sc[lane] = sc_ld;  // kscale [0, 32), vscale [32, 64) of the unit's keys
        if constexpr (PREFETCH) load_k(na, nb);
        wave_sync();
        // Lane (sig, rho): keys 16 pg + 4 rho + i of the unit, head sig.
        float sc[8], mx = -INFINITY;
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            const float4 ks4 = *reinterpret_cast<const float4*>(&lds.sc[16 * pg + 4 * rho]);
            const float ks[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kpos = UNIT8 * u + 16 * pg + 4 * rho + i;
                sc[4 * pg + i] = kpos >= j0 && kpos < j1 ? sacc[pg][i] * ks[i] * sl2 : -INFINITY;
                mx = fmaxf(mx, sc[4 * pg + i]);
            }
        }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float cr_me = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first unit (m = -inf)
        float psum = 0.f;
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            const float4 vs4 = *reinterpret_cast<const float4*>(&lds.sc[32 + 16 * pg + 4 * rho]);
            const float vs[4] = {vs4.x, vs4.y, vs4.z, vs4.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = 16 * pg + 4 * rho + i;
                const float pr = __builtin_amdgcn_exp2f(sc[4 * pg + i] - mn);  // 0 for a masked key
                psum += pr;
                // a masked key's weight is 0 by select: its vscale may be NaN
                if (sig < G) lds.p[kk * G + sig] = sc[4 * pg + i] == -INFINITY ? 0.f : pr * vs[i];
            }
        }
        l = l * cr_me + psum;
        m = mn;
        if (rho == 0 && sig < G) lds.c[sig] = cr_me;
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
        wave_sync();  // lds.p / lds.c / lds.sc are rewritten for the next unit
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
    // Totals: a head's sum over its 4 lane groups; values over the 4 quarters.
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            acc[g][e] += shfl_xor(acc[g][e], 16);
            acc[g][e] += shfl_xor(acc[g][e], 32);
        }
    if (lane < G) {
        lds.ml[2 * lane] = m;
        lds.ml[2 * lane + 1] = l;
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

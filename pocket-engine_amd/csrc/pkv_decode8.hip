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
// wave as the bf16 kernel, and both products run on the matrix cores:
//   q.k on MFMA: per page S[16 keys][16 columns] in 8 steps of
//      v_mfma_f32_16x16x32_bf16. Lane (column s = lane % 16, group
//      r = lane / 16) loads 64 contiguous bytes of key s (dims 16 r + 64 c,
//      c = 0..3: 4 loads per page) and converts them to bf16 (exact,
//      v_cvt_scalef32_pk_bf16_fp8) as the A operand; the B operand is
//      column s over the same dims: query head s for decode (columns 4..15
//      zero), row s / 4 and head s % 4 for a verify segment
//      (verify_range8_kernel). The lane ends with the scores of keys
//      4 r .. 4 r + 3 of the page for column s.
//   softmax: per head over the lane's 8 keys and its 4 lane groups (two
//      shuffles); exp2 domain; kscale / vscale of the unit's 32 keys come
//      through 256 bytes of LDS (one 4-byte load per lane).
//   P.V on MFMA: the unit's V bytes are converted to bf16 (exact) into
//      row-major LDS rows (544 bytes apart), and per page and 16-dim block
//      O^T[16 dims][16 columns] += V^T P^T as two v_mfma_f32_16x16x16_bf16:
//      A = V^T through ds_read_b64_tr_b16 (4 x 4 blocks transposed on the
//      read), B = P^T, which is the score accumulator's own lane layout,
//      holding weight x vscale as a bf16 high part and a bf16 remainder
//      (~16 mantissa bits, close to the reference's f32 products).
// Keys outside the piece get score -inf and weight 0 by select, and their V
// bytes are zeroed, so a stale slot (NaN bytes or scales) contributes
// nothing.
#pragma once
#include "pkv_decode.hip"

namespace pkv {

constexpr int UNIT8 = 2 * PAGE;  // keys per step of the E4M3 kernel

constexpr int V8_VSTR = HEAD_DIM + 16;  // u16 per staged V row (544 B: conflict-free transposed reads)

struct WaveLds8 {
    uint16_t v[UNIT8 * V8_VSTR];  // the unit's V rows as bf16, [key][dim]
    float sc[64];                 // the unit's kscale [key], then vscale [key]
};

// One wave: rows t .. t + NR - 1 of one sequence (row r attends keys
// [0, Lr[r]); NR = 1: decode, the piece's bounds alone), kv head kvh, keys
// [j0, j1) of the sequence (block table row bt), over the E4M3 cache, for a
// group of G query heads per kv head (NR * G <= 16). Column c = G r + g of
// the products is row r, query head kvh * G + g. Results go to epi(c, gq,
// acc, m, l) on the lanes of the columns of attending rows (DecodeEpi8 for
// decode; m = -inf, l = 0 for a column with no key in the piece).
template <int NR = 1, int G = 4, class Epi>
__device__ __forceinline__ void piece_body8(const DecodeParams& p, const int* __restrict__ bt, WaveLds8& lds, int t,
                                            int kvh, int j0, int j1, Epi epi, const int* Lr = nullptr) {
    static_assert(NR >= 1 && NR <= 4 && NR * G <= 16, "up to 16 columns of up to 4 rows");
    // wave-uniform bounds (page ids and bases then stay scalar)
    j0 = __builtin_amdgcn_readfirstlane(j0);
    j1 = __builtin_amdgcn_readfirstlane(j1);
    // Decode (one row, G <= 8 columns of 16): columns NCOL .. 2 NCOL - 1
    // repeat columns 0 .. NCOL - 1 (same q, so bit-identical scores, max,
    // sum and rescale) and take the bf16 remainders of the P.V weights while
    // the first NCOL take the high parts: one MFMA per page and 16-dim block
    // instead of two; the two halves are added once at the end.
    constexpr int NCOL = NR * G;
    constexpr bool DUP = NR == 1 && 2 * NCOL <= 16;
    const int lane = threadIdx.x & 63, sig = lane & 15, rho = lane >> 4;
    const int csig = DUP && sig >= NCOL && sig < 2 * NCOL ? sig - NCOL : sig;  // the column this lane computes
    const int col_r = csig / G, col_g = csig % G;
    // this lane's column: its row's key bound (decode: the piece's), and
    // whether the column is a row that attends
    const int myL = NR == 1 ? j1 : col_r == 0 ? Lr[0] : col_r == 1 ? Lr[1] : col_r == 2 ? Lr[2] : col_r == 3 ? Lr[3] : 0;
    const bool active = col_r < NR && myL > 0;
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
        const uint16_t* qrow = p.q + ((size_t)(t + (active ? col_r : 0)) * p.Hq + kvh * G + (active ? col_g : 0)) *
                                         HEAD_DIM + 16 * rho;
#pragma unroll
        for (int s = 0; s < 8; s++)
            qf[s] = as_bf16x8(active ? *reinterpret_cast<const uint4*>(qrow + 64 * (s >> 1) + 8 * (s & 1))
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
    // Buffer loads: the page's (uniform) base in the descriptor and a 32-bit
    // lane offset fixed for the piece (no per-load 64-bit address math). K
    // without the nontemporal hint: each instruction reads 64 bytes of each
    // of 16 keys, half of every 128-byte line, and the next instruction the
    // other half, which then hits in L2 (nontemporal K: C3 over E4M3 118 us
    // per step against 108; V, read in whole 256-byte pieces, keeps the hint:
    // without it 124 us).
    const uint32_t k_lane = (uint32_t)(sig * row_bytes + kvh * HEAD_DIM + 16 * rho);
    auto load_k = [&](long pg_a, long pg_b) {
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            const uint8_t* r = kc + (size_t)(pg ? pg_b : pg_a) * PAGE * row_bytes;
#pragma unroll
            for (int c = 0; c < 4; c++) kb[pg][c] = buf_load16(r, k_lane + 64 * c);
        }
        const int key = lane & 31;
        const size_t at = ((size_t)(key < PAGE ? pg_a : pg_b) * PAGE + (key & (PAGE - 1))) * Hkv + kvh;
        sc_ld = (lane < 32 ? p.kscale : p.vscale)[at];
    };
    // V: load k < 4 reads key 4 rho + k of the first page, k >= 4 key
    // 4 rho + k - 4 of the second (unit key vkey(k)), dims 16 sig .. + 15.
    auto vkey = [&](int k) { return 16 * (k >> 2) + 4 * rho + (k & 3); };
    const uint32_t v_lane = (uint32_t)(4 * rho * row_bytes + kvh * HEAD_DIM + 16 * sig);
    auto load_v = [&](long pg_a, long pg_b) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint8_t* r = vc + (size_t)(k < 4 ? pg_a : pg_b) * PAGE * row_bytes;
            vb[k] = buf_load16_nt(r, v_lane + (uint32_t)((k & 3) * row_bytes));
        }
    };

    float m = -INFINITY, l = 0.f;  // column sig
    // O^T[256 dims][16 columns]: lane (sig, rho) holds dims 16 db + 4 rho + i
    // of column sig in acc[db][i].
    f32x4 acc[16];
#pragma unroll
    for (int db = 0; db < 16; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    // transposed-read address of this lane: key row 4 rho + sig / 4 of a
    // page, dims 4 (sig % 4) + 16 db
    const uint16_t* tr = lds.v + (4 * rho + (sig >> 2)) * V8_VSTR + 4 * (sig & 3);

    const int u0 = j0 / UNIT8, u1 = (j1 - 1) / UNIT8;
    auto unit = [&](int u, int next_u, auto prefetch) {
        constexpr bool PREFETCH = decltype(prefetch)::value != 0;
        long na = 0, nb = 0;
        if constexpr (PREFETCH) unit_pages(next_u, na, nb);
        // V first: the unit's V bytes (requested at the start of the
        // previous unit) go to LDS, and the next unit's V is requested at
        // once, so it has a whole unit to arrive.
        // V rows to LDS as bf16 (exact): row vkey(k), dims 16 sig .. + 15;
        // rows of keys outside [j0, j1) as zeros (a stale slot may hold NaN)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int row = vkey(k), kp = UNIT8 * u + row;
            const bool in = kp >= j0 && kp < j1;
            uint16_t* d = lds.v + row * V8_VSTR + 16 * sig;
            *reinterpret_cast<uint4*>(d) = in ? e4m3x8_to_bf16x8(vb[k].x, vb[k].y) : make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4*>(d + 8) = in ? e4m3x8_to_bf16x8(vb[k].z, vb[k].w) : make_uint4(0, 0, 0, 0);
        }
        if constexpr (PREFETCH) load_v(na, nb);
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
        // Lane (sig, rho): keys 16 pg + 4 rho + i of the unit, column sig.
        float sc[8], mx = -INFINITY;
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            const float4 ks4 = *reinterpret_cast<const float4*>(&lds.sc[16 * pg + 4 * rho]);
            const float ks[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kpos = UNIT8 * u + 16 * pg + 4 * rho + i;
                sc[4 * pg + i] = kpos >= j0 && kpos < j1 && kpos < myL ? sacc[pg][i] * ks[i] * sl2 : -INFINITY;
                mx = fmaxf(mx, sc[4 * pg + i]);
            }
        }
        mx = max_xor32(max_xor16(mx));
        const float mn = fmaxf(m, mx);
        // a column with no key yet subtracts 0 (its weights are all 0)
        const float mref = mn == -INFINITY ? 0.f : mn;
        const float cr_me = __builtin_amdgcn_exp2f(m - mref);  // 0 while m = -inf
        // P^T operands: the lane's own weights times vscale, as a bf16 high
        // part plus a bf16 remainder (two MFMAs: ~16 mantissa bits, where one
        // bf16 would add 2^-9 relative error per weight to products the
        // reference keeps in f32); a masked key's weight is 0 by select.
        float psum = 0.f;
        s16x4 pw_hi[2], pw_lo[2];
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            const float4 vs4 = *reinterpret_cast<const float4*>(&lds.sc[32 + 16 * pg + 4 * rho]);
            const float vs[4] = {vs4.x, vs4.y, vs4.z, vs4.w};
            float w[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pr = __builtin_amdgcn_exp2f(sc[4 * pg + i] - mref);  // 0 for a masked key
                psum += pr;
                w[i] = sc[4 * pg + i] == -INFINITY ? 0.f : pr * vs[i];
            }
            const uint32_t h01 = pack2_hw(w[0], w[1]), h23 = pack2_hw(w[2], w[3]);
            const uint32_t r01 = pack2_hw(w[0] - bf_lo(h01), w[1] - bf_hi(h01));
            const uint32_t r23 = pack2_hw(w[2] - bf_lo(h23), w[3] - bf_hi(h23));
            pw_hi[pg] = __builtin_bit_cast(s16x4, make_uint2(h01, h23));
            pw_lo[pg] = __builtin_bit_cast(s16x4, make_uint2(r01, r23));
        }
        l = l * cr_me + psum;
        m = mn;
        if (__any(cr_me != 1.f)) {
#pragma unroll
            for (int db = 0; db < 16; db++) acc[db] *= cr_me;
        }
        wave_sync();  // V staged
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
#pragma unroll
        for (int pg = 0; pg < 2; pg++) {
            // DUP: the remainder columns' lanes supply their weights' low parts
            const s16x4 pw = DUP && sig >= NCOL ? pw_lo[pg] : pw_hi[pg];
#pragma unroll
            for (int db = 0; db < 16; db++) {
                const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(tr + pg * PAGE * V8_VSTR + 16 * db));
                if constexpr (DUP) {
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pw, acc[db], 0, 0, 0);
                } else {
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pw_hi[pg], acc[db], 0, 0, 0);
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pw_lo[pg], acc[db], 0, 0, 0);
                }
            }
        }
        wave_sync();  // lds.v / lds.sc are rewritten for the next unit
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
    // Totals: a column's sum over its 4 lane groups.
    l = add_xor32(add_xor16(l));
    if constexpr (DUP) {
        // column c (high parts) + column c + NCOL (remainders), same dims
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[db][i] += __shfl_down(acc[db][i], NCOL, 16);
    }
    if (active && sig < NCOL) epi(sig, rho, acc, m, l);
}

// Writes a piece's result for the lanes of head g of the group (dims
// 16 db + 4 gq + i in acc[db][i]): the gated output when the piece holds
// all of the token's keys, else the partial record at index idx.
template <int G = 4>
struct DecodeEpi8 {
    const DecodeParams& p;
    int t, kvh, idx;
    bool direct;
    __device__ __forceinline__ void operator()(int g, int gq, const f32x4 (&acc)[16], float m, float l) const {
        const int h = kvh * G + g;
        if (direct) {
            const float inv = 1.f / l;
            const uint16_t* gate = p.qkv + (size_t)t * p.qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + 4 * gq;
            uint16_t* o = p.out + ((size_t)t * p.Hq + h) * HEAD_DIM + 4 * gq;
#pragma unroll
            for (int db = 0; db < 16; db++) {
                const uint2 graw = *reinterpret_cast<const uint2*>(gate + 16 * db);
                *reinterpret_cast<uint2*>(o + 16 * db) =
                    gate4(acc[db][0], acc[db][1], acc[db][2], acc[db][3], inv, graw);
            }
        } else {
            const size_t row = (size_t)idx * p.Hq + h;
            float* pa = p.part_acc + row * HEAD_DIM + 4 * gq;
#pragma unroll
            for (int db = 0; db < 16; db++)
                *reinterpret_cast<float4*>(pa + 16 * db) = make_float4(acc[db][0], acc[db][1], acc[db][2], acc[db][3]);
            if (gq == 0) *reinterpret_cast<float2*>(p.part_ms + row * 2) = make_float2(m, l);
        }
    }
};

// Key-range kernel over the E4M3 cache: decode_range_kernel<4, false>'s
// ranges and records with piece_body8 inside (G query heads per kv head).
// Grid (n_wg, ceil(Hkv / 4)), 64 * min(Hkv, 4) threads; two workgroups per
// CU (at most 256 VGPRs).
template <int G>
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
            const DecodeEpi8<G> epi{p, t, kvh, t + b, j0 == 0 && j1 == L && !p.fo.mode};
            piece_body8<1, G>(p, block_table + (size_t)seq * p.max_blocks, sh_w[wave], t, kvh, j0, j1, epi);
            off += L;
        }
        t++;
    }
}

}  // namespace pkv

// Attention input preparation on gfx950: the reference's attn_prep
// (qwen35.cu:1067-1128), which is where the reference appends K/V to the
// paged cache. For token t and head hh of the qkv row
// [Hq x (q 256 | gate 256) | k Hkv x 256 | v Hkv x 256]:
//   q / k heads: y = bf16(x * scale * w), scale = 1 / sqrt(sum x^2 / 256 + eps)
//     (RMSNorm with f32 weights), then dims 0..63 rotate as pairs (d, d + 32)
//     with bf16 cos / sin of pos * inv_freq[d]:
//       lo' = bf16(bf16(lo c) - bf16(hi s)),  hi' = bf16(bf16(hi c) + bf16(lo s)),
//     pos = rope[axis * rope_stride + t], axis 1 (height) for d % 3 == 1 below
//     3 sec_h, 2 (width) for d % 3 == 2 below 3 sec_w, else 0 (time);
//     q goes to qout[t][hh], k to kcache[slot][hh - Hq];
//   v heads: copied bit for bit to vcache[slot];
//   k and v are skipped for slot_map[t] < 0 (padding rows); q is always written;
//   with an E4M3 cache (kscale / vscale given) k and v are stored as E4M3
//   bytes with an f32 scale per (slot, kv head) (store_e4m3_wave).
//
// Layout (this build's own): one wave per (token, head), 4 consecutive dims
// per lane (one 8-byte load and store), the squared sum reduced across the
// wave by shuffles, and each rotary pair's partner 8 lanes away inside the
// same 16-lane row (dims 0..31 on lanes 0..7, 32..63 on lanes 8..15), fetched
// with one DPP row rotate: no LDS, no barrier.
#pragma once
#include "pkv_common.h"

namespace pkv {

constexpr int ROPE_DIM = 64;  // rotated leading dims of each head (reference qwen35.cu:23)

struct PrepArgs {
    const uint16_t* qkv;
    int qstride, Hq, Hkv;
    const float* q_norm;
    const float* k_norm;
    const int* rope;
    int rope_stride, sec_h, sec_w;
    const int* slot_map;
    const float* inv_freq;
    uint16_t* qout;
    uint16_t* kcache;
    uint16_t* vcache;
    float* kscale;  // non-null: an E4M3 cache (bytes in kcache / vcache, f32 scale per slot and kv head)
    float* vscale;
    float eps;
    long num_slots;
};

// One head's 256 values (4 per lane) as E4M3 with scale amax / 448 (1 if
// all zero): bytes = e4m3(v * (1 / scale)) (reference store_e4m3,
// qwen35.cu:1055-1065).
__device__ __forceinline__ void store_e4m3_wave(const float (&v)[4], uint8_t* dst, float* scale) {
    const int lane = threadIdx.x & 63;
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float sc = amax > 0.f ? amax / 448.f : 1.f;
    const float inv = 1.f / sc;
    *reinterpret_cast<uint32_t*>(dst + 4 * lane) = f32x4_to_e4m3x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    if (lane == 0) *scale = sc;
}

// One wave: token t, head hh (q heads, then k heads, then v heads).
__device__ __forceinline__ void prep_head(const PrepArgs& a, int t, int hh) {
    const int lane = threadIdx.x & 63;
    const uint16_t* row = a.qkv + (size_t)t * a.qstride;
    const long slot = a.slot_map[t];
    const bool has_slot = slot >= 0 && slot < a.num_slots;
    if (hh >= a.Hq + a.Hkv) {
        if (!has_slot) return;
        const int vh = hh - a.Hq - a.Hkv;
        const uint16_t* src = row + (size_t)a.Hq * 2 * HEAD_DIM + (size_t)(a.Hkv + vh) * HEAD_DIM;
        const size_t at = (size_t)slot * a.Hkv + vh;
        const uint2 raw = *reinterpret_cast<const uint2*>(src + 4 * lane);
        if (a.vscale) {
            const float x[4] = {bf_lo(raw.x), bf_hi(raw.x), bf_lo(raw.y), bf_hi(raw.y)};
            store_e4m3_wave(x, reinterpret_cast<uint8_t*>(a.vcache) + at * HEAD_DIM, a.vscale + at);
        } else {
            *reinterpret_cast<uint2*>(a.vcache + at * HEAD_DIM + 4 * lane) = raw;
        }
        return;
    }
    const bool is_q = hh < a.Hq;
    if (!is_q && !has_slot) return;
    const uint16_t* src = is_q ? row + (size_t)hh * 2 * HEAD_DIM : row + (size_t)a.Hq * 2 * HEAD_DIM +
                                                                     (size_t)(hh - a.Hq) * HEAD_DIM;
    // The row, the norm weights, then the rotary positions and frequencies
    // of the lane's 4 dims, all requested before anything waits (loads
    // return in order: the squared sum waits for the row alone), so the 4
    // cos / sin evaluations below wait on one round trip, not one each.
    const uint2 raw = *reinterpret_cast<const uint2*>(src + 4 * lane);
    const float4 w = *reinterpret_cast<const float4*>((is_q ? a.q_norm : a.k_norm) + 4 * lane);
    // (Every lane loads them, from valid indices: under a lane condition the
    // compiler could not count the loads, and the squared sum would wait
    // for all of them.)
    int rpos[4];
    float rinv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int d = (4 * lane + e) & (ROPE_DIM / 2 - 1);
        const int axis = (d % 3 == 1 && d < 3 * a.sec_h) ? 1 : (d % 3 == 2 && d < 3 * a.sec_w) ? 2 : 0;
        rpos[e] = a.rope[(size_t)axis * a.rope_stride + t];
        rinv[e] = a.inv_freq[d];
    }
    const float x[4] = {bf_lo(raw.x), bf_hi(raw.x), bf_lo(raw.y), bf_hi(raw.y)};
    float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float scale = 1.f / sqrtf(ss / HEAD_DIM + a.eps);
    float y[4] = {rbf(x[0] * scale * w.x), rbf(x[1] * scale * w.y), rbf(x[2] * scale * w.z), rbf(x[3] * scale * w.w)};
    // Rotary: lanes 0..7 hold dims d = 0..31 ("lo"), lanes 8..15 dims d + 32.
    float yp[4];
#pragma unroll
    for (int e = 0; e < 4; e++) yp[e] = dpp<DPP_ROW_ROR8>(y[e]);  // lane i <- lane i ^ 8 of its row
    if (lane < ROPE_DIM / 4) {
        const bool lo_half = lane < ROPE_DIM / 8;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float f = (float)rpos[e] * rinv[e];
            const float c = rbf(cosf(f)), s = rbf(sinf(f));
            const float lo = lo_half ? y[e] : yp[e], hi = lo_half ? yp[e] : y[e];
            y[e] = lo_half ? rbf(rbf(lo * c) - rbf(hi * s)) : rbf(rbf(hi * c) + rbf(lo * s));
        }
    }
    if (!is_q && a.kscale) {
        const size_t at = (size_t)slot * a.Hkv + (hh - a.Hq);
        store_e4m3_wave(y, reinterpret_cast<uint8_t*>(a.kcache) + at * HEAD_DIM, a.kscale + at);
        return;
    }
    uint16_t* dst = is_q ? a.qout + ((size_t)t * a.Hq + hh) * HEAD_DIM
                         : a.kcache + ((size_t)slot * a.Hkv + (hh - a.Hq)) * HEAD_DIM;
    *reinterpret_cast<uint2*>(dst + 4 * lane) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
}

// Grid (T, ceil((Hq + 2 Hkv) / 4)), 256 threads: wave w takes head 4 y + w.
__global__ void __launch_bounds__(256) prep_kernel(PrepArgs a) {
    const int hh = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (hh < a.Hq + 2 * a.Hkv) prep_head(a, blockIdx.x, hh);
}

}  // namespace pkv

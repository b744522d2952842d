// Shared device helpers for the paged KV cache kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pkv {

constexpr int HEAD_DIM = 256;  // attention head width (reference model.rs:14)
constexpr float LOG2E = 1.4426950408889634f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// 16-byte streaming load marked nontemporal: data read once (K/V pages)
// should not displace reusable lines. Measured on MI355X: plain 16-byte
// streaming reads reach ~6.2 TB/s, nontemporal ones ~7.0 TB/s.
__device__ __forceinline__ uint4 load_nt(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes at byte offset `off` of `base` (a uniform address: it goes in the
// buffer descriptor, the offset stays one VGPR), nontemporal.
__device__ __forceinline__ uint4 buf_load16_nt(const void* base, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                                                       0x00020000);
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// The same without the nontemporal hint: for lines read again soon (prompt
// tiles shared by query tiles; E4M3 K pieces, where each instruction reads
// half of every 128-byte line and the next one the other half).
__device__ __forceinline__ uint4 buf_load16(const void* base, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                                                       0x00020000);
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float b2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// f32 -> bf16, round to nearest even; NaN stays NaN (quiet, sign kept).
__device__ __forceinline__ uint32_t f2b_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float rbf(float x) { return __uint_as_float(f2b_bits(x) << 16); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return f2b_bits(lo) | (f2b_bits(hi) << 16); }
// x / y for the gated epilogue (y = 1 + exp(-gate) >= 1): the reciprocal
// and one residual correction (q + (x - y q) / y), which gives IEEE's
// correctly rounded quotient except in rare last-bit cases, before the
// bf16 rounding; x / inf is 0 as in IEEE.
__device__ __forceinline__ float gated_div(float x, float y) {
    const float r = __builtin_amdgcn_rcpf(y), q = x * r;
    const float c = __builtin_fmaf(__builtin_fmaf(-y, q, x), r, q);
    return __builtin_isinf(y) ? 0.f * x : c;
}
// Two finite floats to packed bf16 with the hardware's round-to-nearest-even
// conversion (one v_cvt_pk_bf16_f32); for values that are never NaN.
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_hw(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// E4M3 (OCP E4M3FN on gfx950: bias 7, max 448, NaN 0x7F) conversions.
// Two E4M3 bytes (the low or high half of w) to two bf16 (exact: bf16 holds
// every E4M3 value).
template <bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}
// Eight E4M3 bytes (two words) to eight bf16 (an MFMA operand).
__device__ __forceinline__ uint4 e4m3x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    return make_uint4(e4m3x2_to_bf16x2<false>(w0), e4m3x2_to_bf16x2<true>(w0), e4m3x2_to_bf16x2<false>(w1),
                      e4m3x2_to_bf16x2<true>(w1));
}
// Four floats to four E4M3 bytes, round to nearest even (values within the
// E4M3 range; callers scale to |v| <= 448).
__device__ __forceinline__ uint32_t f32x4_to_e4m3x4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

// Two bf16 products summed into c in f32 (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float c) {
    c = dot2(a.x, b.x, c);
    c = dot2(a.y, b.y, c);
    c = dot2(a.z, b.z, c);
    return dot2(a.w, b.w, c);
}

// DPP lane moves inside 16-lane rows.
enum : int {
    DPP_ROW_MIRROR = 0x140,       // lane i <- lane 15 - i
    DPP_ROW_HALF_MIRROR = 0x141,  // lane i <- lane i ^ 7 (within 8)
    DPP_ROW_ROR4 = 0x124,         // lane i <- lane (i + 4) % 16
    DPP_ROW_ROR8 = 0x128,         // lane i <- lane (i + 8) % 16 == i ^ 8
    DPP_QUAD_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
    DPP_QUAD_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
};
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Reductions with lane i ^ 32 / lane i ^ 16 through v_permlane32_swap /
// v_permlane16_swap (VALU cross-lane moves, no LDS round trip as
// ds_bpermute has): the swap hands every lane its own value and its
// partner's, in the same order on both lanes of a pair, so both end with
// bit-identical results.
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// LDS byte address of a shared-memory pointer (the M0 operand of LDS DMA).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
// LDS DMA (global_load_lds_dwordx4 / _dword): every active lane reads 16
// (4) bytes at its own global address and the data lands at LDS address
// m0 + 16 (4) x lane (m0 must be wave-uniform). Issued from inline assembly so the compiler neither
// waits for it nor counts it: the caller waits on vmcnt itself (the
// compiler's own vmcnt waits stay correct, only stricter, since counts are
// of operations newer than the one awaited).
__device__ __forceinline__ void dma16(const void* src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(m0))
                 : "memory");
}
__device__ __forceinline__ void dma4(const void* src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(m0))
                 : "memory");
}
// s_waitcnt vmcnt(N) (N < 64: bits 3:0 and 15:14) that leaves the other
// counters alone.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt 0..63");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
// The same LDS DMA from a uniform base plus a 32-bit lane byte offset.
__device__ __forceinline__ void dma16_s(const void* base, uint32_t off, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(off), "s"(base), "s"(__builtin_amdgcn_readfirstlane(m0))
                 : "memory");
}
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// FP8 activation copies of the gated attention outputs (the reference's
// Fp8Out / quant8, src/kernels/fp8.cuh:29-85): row t of K values as E4M3
// bytes at q[t * K + e] with mode 1 (Block128) one f32 scale amax / 448 (1
// for an all-zero group) per 128 columns at s[(e / 128) * rows + t], or
// mode 2 (Mx32) one E8M0 exponent 127 + x per 32 columns (the smallest x
// with amax / 2^x <= 448) at the MXFP8 tiled index mx_index; bytes =
// e4m3(v * (1 / scale)), round to nearest even.
struct Fp8Out {
    uint8_t* q;
    void* s;
    int mode;  // 0 none, 1 Block128, 2 Mx32
    int rows;  // row capacity (Block128 scale stride)
};
// Byte offset of the Mx32 scale of (row r, 32-column block kb) among KB
// blocks per row: tiles of 128 rows x 4 blocks (512 bytes), inside a tile
// row r % 32 at 16 r, (r % 128) / 32 at 4 x that, kb % 4 at 1 x that.
__device__ __forceinline__ size_t mx_index(int r, int kb, int KB) {
    const int kt = (KB + 3) / 4;
    return ((size_t)(r / 128) * kt + kb / 4) * 512 + (r % 32) * 16 + ((r % 128) / 32) * 4 + (kb % 4);
}
__device__ __forceinline__ int mx_exp(float amax) {
    if (!(amax > 0.f)) return -127;
    int ex;
    const float m = frexpf(amax / 448.f, &ex);  // amax / 448 = m 2^ex, m in [0.5, 1)
    if (m == 0.5f) ex -= 1;                     // a power of two needs no rounding up
    return max(-127, min(127, ex));
}
// Four consecutive columns e .. e + 3 of row t per lane, the 64 lanes of the
// wave in column order (a 128-column group spans 32 lanes, a 32-column
// group 8); every lane calls.
__device__ __forceinline__ void fp8_quant4(float y0, float y1, float y2, float y3, int t, int e, int K,
                                           const Fp8Out& o) {
    float a = fmaxf(fmaxf(fabsf(y0), fabsf(y1)), fmaxf(fabsf(y2), fabsf(y3)));
    a = fmaxf(a, __shfl_xor(a, 1));
    a = fmaxf(a, __shfl_xor(a, 2));
    a = fmaxf(a, __shfl_xor(a, 4));
    float inv;
    if (o.mode == 1) {
        a = fmaxf(a, __shfl_xor(a, 8));
        a = fmaxf(a, __shfl_xor(a, 16));
        const float sc = a > 0.f ? a / 448.f : 1.f;
        inv = 1.f / sc;
        if (e % 128 == 0) reinterpret_cast<float*>(o.s)[(size_t)(e / 128) * o.rows + t] = sc;
    } else {
        const int ex = mx_exp(a);
        inv = ldexpf(1.f, -ex);
        if (e % 32 == 0) reinterpret_cast<uint8_t*>(o.s)[mx_index(t, e / 32, K / 32)] = (uint8_t)(127 + ex);
    }
    *reinterpret_cast<uint32_t*>(o.q + (size_t)t * K + e) = f32x4_to_e4m3x4(y0 * inv, y1 * inv, y2 * inv, y3 * inv);
}

// Speculative rows verify drafts: outs[s * spec] >= 0 (reference qwen35.cu:94-100).
__device__ __forceinline__ bool is_spec(const int* outs, int spec, int s) {
    return outs && outs[(size_t)s * spec] >= 0;
}

// Keys a token attends to in decode attention: pos + 1, or 0 for tokens of
// prompt sequences when prompts are left to the prefill kernel
// (reference qwen35.cu:1171-1172).
__device__ __forceinline__ int decode_len(int t, const int* pos, const int* tok_seq, const int* cu,
                                          int skip_prompts, const int* outs, int spec) {
    if (skip_prompts) {
        const int sq = tok_seq[t];
        if (cu[sq + 1] - cu[sq] > 1 && !is_spec(outs, spec, sq)) return 0;
    }
    return pos[t] + 1;
}

}  // namespace pkv

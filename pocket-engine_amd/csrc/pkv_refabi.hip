// The reference's kernel ABI for the paged-attention path, as a gfx950 code
// object (pkv_kernels.hsaco). The reference engine loads one code object with
// hipModuleLoadData (src/gpu.rs:434-466), resolves kernels by name
// (src/gpu.rs:552-566) and launches them with its own grids, blocks, dynamic
// shared memory and argument slots (src/gpu.rs:903-930). The kernels below
// carry the reference's names and signatures, accept exactly those launches
// (src/model.rs:2366-2493) and compute the same results with this build's
// kernel bodies:
//
//   attn_prep       (qwen35.cu:1076-1082)  grid (T, Hq + 2 Hkv), 128 threads
//   attn_paged_g<G> (qwen35.cu:1313-1334)  grid (T, Hkv, Z), 256 threads
//                   (G = 1, 2, 4) or 128 (G = 6, 8)
//   attn_paged8_g<G> the same over an E4M3 cache (kscale / vscale)
//   attn_merge      (qwen35.cu:2245-2249)  grid (T, Hq), 256 threads
//   attn_groupr_g4_t2_k32 (qwen35.cu:1600-1616) grid (ceil(T/32) + seqs, Hkv),
//                   256 threads: the prompt kernel a gfx950 device (compute
//                   capability 9.5) selects (fa_shape, src/model.rs:58-79)
//   attn_mfma_g4_t2 (amd/attention.cuh:137-142) the same grid, 512 threads:
//                   the name gfx942 devices select
//   attn_group8_g4_t2_k16 (qwen35.cu:1593-1608) the same grid, 256 threads,
//                   over an E4M3 cache (kscale / vscale): gfx950's choice
//                   for an E4M3 cache
//   the other groups' prompt kernels gfx950 selects (fa_shape), on grids of
//   16 x NT-query tiles with 32 x G x NT threads (qwen35.cu:1593-1616):
//   attn_groupr_g6_t1_k32 (192), attn_group_g1_t8_k16, attn_group_g2_t4_k16,
//   attn_group_g8_t1_k16 (256), and over an E4M3 cache
//   attn_group8_g{1,2,6,8}_t{8,4,1,1}_k16
//
// Split decode follows the reference's contract so its buffer sizing holds:
// range z of nz = split_parts(L, Z, min_chunk) covers keys [z c, z c + c),
// c = ceil(L / nz), and leaves a record [M (natural log), S, A[256]] at
// part[((s * spec + t - cu[s]) * Hq + h) * Z + z]; attn_merge combines the nz
// records. Inside a block the waves take an equal share of the range's pages
// each (G = 4: this build's decode wave body, dot2 + DPP reduce-scatter,
// online softmax, one page in flight; other groups: the verify body with one
// row) and combine through LDS.
//
// FP8 output copies (fq / fs / fmode / frows, the reference's Fp8Out) are
// written by attn_paged_g<G> when it does not split (part null) and by
// attn_merge, as the reference writes them (qwen35.cu:1297-1307, 2269-2279).
//
// Bounds of this ABI: block_size 16 for decode, a
// power of two for prompts; G = Hq / Hkv of the kernel's name (1, 2, 4, 6
// or 8). A launch outside these bounds
// writes nothing. Page ids are not clamped (the reference ABI passes no pool
// size).
#include "pkv_copy.hip"
#include "pkv_decode.hip"
#include "pkv_decode8.hip"
#include "pkv_prefill.hip"
#include "pkv_prep.hip"
#include "pkv_verify.hip"

#include <climits>

namespace pkv {

constexpr float LN2 = 0.69314718055994531f;
constexpr long REF_NO_CLAMP = 1L << 40;  // no pool bound in the reference ABI

// Key ranges of a decode token (reference split_parts, qwen35.cu:1139-1141).
__device__ __forceinline__ int ref_split_parts(int L, int Z, int min_chunk) {
    return max(1, min(Z, (L + min_chunk - 1) / max(1, min_chunk)));
}

__device__ __forceinline__ bool ref_prompt_row(int skip_prompts, const int* cu, int sq, const int* outs, int spec) {
    return skip_prompts && cu[sq + 1] - cu[sq] > 1 && !is_spec(outs, spec, sq);
}

}  // namespace pkv

using pkv::HEAD_DIM;

// One (token, head) per block as the reference launches it; the first wave
// does the work (4 dims per lane), the second has none.
extern "C" __global__ void __launch_bounds__(128)
    attn_prep(const uint16_t* __restrict__ qkv, int qstride, int Hq, int Hkv, const float* __restrict__ q_norm,
              const float* __restrict__ k_norm, const int* __restrict__ rope, int rope_stride, int sec_h, int sec_w,
              const int* __restrict__ slot_map, const float* __restrict__ inv_freq, uint16_t* __restrict__ qout,
              void* __restrict__ kcache, void* __restrict__ vcache, float* __restrict__ kscale,
              float* __restrict__ vscale, float eps) {
    if (threadIdx.x >= 64 || (kscale == nullptr) != (vscale == nullptr)) return;
    pkv::PrepArgs a;
    a.qkv = qkv;
    a.qstride = qstride;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.rope = rope;
    a.rope_stride = rope_stride;
    a.sec_h = sec_h;
    a.sec_w = sec_w;
    a.slot_map = slot_map;
    a.inv_freq = inv_freq;
    a.qout = qout;
    a.kcache = (uint16_t*)kcache;
    a.vcache = (uint16_t*)vcache;
    a.kscale = kscale;
    a.vscale = vscale;
    a.eps = eps;
    a.num_slots = pkv::REF_NO_CLAMP;
    pkv::prep_head(a, blockIdx.x, blockIdx.y);
}

namespace pkv {

// attn_paged_g<G> / attn_paged8_g<G> on the reference's grid (token t, kv
// head, range z) and block (256 threads for G <= 4, 128 for G = 6 and 8,
// model.rs:2374): the range's pages split over the NW waves (bf16: the decode
// wave body for G = 4, the verify body with one row for other groups; E4M3:
// the E4M3 decode body, two pages per step), combined through LDS.
template <int G, bool F8>
__device__ __forceinline__ void paged_ref(const uint16_t* q, const void* kcache, const void* vcache,
                                          const float* kscale, const float* vscale, const uint16_t* qkv, int qstride,
                                          int Hq, int Hkv, const int* __restrict__ pos,
                                          const int* __restrict__ tok_seq, const int* __restrict__ block_table,
                                          int max_blocks, int block_size, uint16_t* out, float scale,
                                          const Fp8Out fo, const int* __restrict__ cu, int skip_prompts,
                                          int min_chunk, float* part, const int* __restrict__ outs, int spec) {
    constexpr int NW = G >= 6 ? 2 : 4;  // waves
    constexpr bool BODY4 = !F8 && G == 4;
    constexpr bool BODYV = !F8 && G != 4;
    static_assert(G * HEAD_DIM * 4 <= (int)sizeof(WaveLds8::v), "E4M3 record fits the V staging rows");
    // bf16: the decode wave body's LDS (or the verify body's V staging) and a
    // separate record per wave. E4M3: the E4M3 decode body's LDS per wave,
    // whose V staging rows also hold the wave's record once its loop is done
    // (72 KB in all at G = 4: two workgroups per CU).
    __shared__ WaveLds<4> sh_w[BODY4 ? NW : 1];
    __shared__ __align__(16) uint16_t sh_v[BODYV ? NW : 1][BODYV ? VF_LDS : 8];
    __shared__ __align__(16) WaveLds8 sh_w8[F8 ? NW : 1];
    __shared__ __align__(16) float sh_acc_bf[F8 ? 1 : NW][G][HEAD_DIM];
    __shared__ float sh_ml[NW][G][2];
    auto rec = [&](int w) -> float (*)[HEAD_DIM] {
        if constexpr (F8) return reinterpret_cast<float (*)[HEAD_DIM]>(sh_w8[w].v);
        else return sh_acc_bf[w];
    };
    if (blockDim.x != 64 * NW || block_size != PAGE || Hq != G * Hkv || (kscale != nullptr) != F8 ||
        (vscale != nullptr) != F8)
        return;
    const int tid = threadIdx.x;
    // Work item of this workgroup. The grid is the reference's (token, kv
    // head, range) and so is each item's result slot, but which workgroup
    // computes which item is free: with up to 256 tokens the k-th workgroup
    // in dispatch order (x fastest, then y, then z) takes the k-th item in
    // order of decreasing context (longest tokens first, each token's
    // ranges and kv heads together), so the long items do not start last.
    int t = blockIdx.x, kvh = blockIdx.y, z = blockIdx.z;
    if (gridDim.x <= 256) {
        __shared__ int sh_len[256], sh_order[256];
        const int T = gridDim.x;
        for (int u = tid; u < T; u += 64 * NW) sh_len[u] = pos[u];
        __syncthreads();
        for (int me = tid; me < T; me += 64 * NW) {
            const int mine = sh_len[me];
            int rank = 0;
            for (int u = 0; u < T; u++) {
                const int o = sh_len[u];
                rank += o > mine || (o == mine && u < me);
            }
            sh_order[rank] = me;
        }
        __syncthreads();
        const int per = gridDim.y * gridDim.z;
        const int k = blockIdx.x + T * (blockIdx.y + gridDim.y * blockIdx.z);
        const int rem = k % per;
        t = sh_order[k / per];
        z = rem / gridDim.y;
        kvh = rem % gridDim.y;
    }
    const int sq = tok_seq[t];
    if (ref_prompt_row(skip_prompts, cu, sq, outs, spec)) return;
    const int L = pos[t] + 1;
    const int parts = part ? ref_split_parts(L, gridDim.z, min_chunk) : 1;
    if (z >= parts) return;
    const int chunk = (L + parts - 1) / parts;
    const int j0 = part ? z * chunk : 0, j1 = part ? min(L, j0 + chunk) : L;

    DecodeParams p = {};
    p.q = q;
    p.kc = (uint16_t*)kcache;  // read only
    p.vc = (uint16_t*)vcache;
    p.qkv = qkv;
    p.qstride = qstride;
    p.Hq = Hq;
    p.Hkv = Hkv;
    p.max_blocks = max_blocks;
    p.out = out;
    p.scale = scale;
    p.num_blocks = REF_NO_CLAMP;
    p.kscale = kscale;
    p.vscale = vscale;

    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int a = j1, b = j1;
    if (j0 < j1) {
        const int pg0 = j0 / PAGE, np = (j1 - 1) / PAGE - pg0 + 1, per = (np + NW - 1) / NW;
        a = max(j0, (pg0 + wave * per) * PAGE);
        b = min(j1, (pg0 + (wave + 1) * per) * PAGE);
    }
    // every lane first clears its wave's record (rows a wave does not reach
    // stay empty), then the wave's piece overwrites it
    {
        const int lane = tid & 63;
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int e = 0; e < 4; e++) rec(wave)[g][4 * lane + e] = 0.f;
            if (lane == 0) {
                sh_ml[wave][g][0] = -INFINITY;
                sh_ml[wave][g][1] = 0.f;
            }
        }
        wave_sync();
    }
    if (a < b) {
        const int* bt = block_table + (size_t)sq * max_blocks;
        if constexpr (F8) {
            auto epi = [&](int g, int gq, const f32x4 (&acc)[16], float m, float l) {
#pragma unroll
                for (int db = 0; db < 16; db++)
#pragma unroll
                    for (int i = 0; i < 4; i++) rec(wave)[g][16 * db + 4 * gq + i] = acc[db][i];
                if (gq == 0) {
                    sh_ml[wave][g][0] = m;
                    sh_ml[wave][g][1] = l;
                }
            };
            piece_body8<1, G>(p, bt, sh_w8[wave], t, kvh, a, b, epi);
        } else if constexpr (BODYV) {
            auto epi = [&](int, int g, int gq, const f32x4 (&acc)[16], float m, float l) {
#pragma unroll
                for (int db = 0; db < 16; db++)
#pragma unroll
                    for (int i = 0; i < 4; i++) rec(wave)[g][16 * db + 4 * gq + i] = acc[db][i];
                if (gq == 0) {
                    sh_ml[wave][g][0] = m;
                    sh_ml[wave][g][1] = l;
                }
            };
            const int Lr[VF_ROWS] = {L, 0, 0, 0};
            verify_piece<G>(p, bt, sh_v[wave], t, kvh, a, b, Lr, epi);
        } else {
            auto epi = [&](int g, const float (&acc)[8], float m, float l, int ch) {
#pragma unroll
                for (int e = 0; e < 8; e++) rec(wave)[g][8 * ch + e] = acc[e];
                if (ch == 0) {
                    sh_ml[wave][g][0] = m;
                    sh_ml[wave][g][1] = l;
                }
            };
            piece_body<4, false>(p, bt, sh_w[wave], t, kvh, a, b, L, INT_MAX, 0, epi);
        }
    }
    __syncthreads();
    // Combine the waves: thread d owns dimensions d, d + 64 NW, .. of every head.
    for (int gd = tid; gd < G * HEAD_DIM; gd += 64 * NW) {
        const int g = gd / HEAD_DIM, d = gd % HEAD_DIM;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sh_ml[w][g][0]);
        float S = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = sh_ml[w][g][0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sh_ml[w][g][0] - M);
            S += sh_ml[w][g][1] * f;
            A += rec(w)[g][d] * f;
        }
        const int h = kvh * G + g;
        if (part) {
            const size_t row = (size_t)sq * spec + (t - cu[sq]);
            float* pp = part + ((row * Hq + h) * gridDim.z + z) * (HEAD_DIM + 2);
            if (d == 0) {
                pp[0] = M * LN2;  // natural-log units, as the reference's records
                pp[1] = S;
            }
            pp[2 + d] = A;
        } else {
            const float gate = b2f(qkv[(size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + d]);
            const float y = rbf(A / S) / (1.f + __expf(-gate));
            out[((size_t)t * Hq + h) * HEAD_DIM + d] = (uint16_t)f2b_bits(y);
            // element (g, d) of wave 0's record is read above by this
            // thread only: it now holds the f32 output for the FP8 copy
            if (fo.mode) rec(0)[g][d] = y;
        }
    }
    if (fo.mode && !part) {
        // each head's 256 gated outputs as FP8, one wave per head, 4 columns
        // per lane (the reference's attn_body epilogue, qwen35.cu:1297-1307)
        __syncthreads();
        const int lane = tid & 63;
        for (int g = wave; g < G; g += NW) {
            const float4 y = *reinterpret_cast<const float4*>(&rec(0)[g][4 * lane]);
            fp8_quant4(y.x, y.y, y.z, y.w, t, (kvh * G + g) * HEAD_DIM + 4 * lane, Hq * HEAD_DIM, fo);
        }
    }
}

}  // namespace pkv

#define PKV_PAGED_ARGS                                                                                           \
    const uint16_t *__restrict__ q, const void *__restrict__ kcache, const void *__restrict__ vcache,            \
        const float *__restrict__ kscale, const float *__restrict__ vscale, const uint16_t *__restrict__ qkv,    \
        int qstride, int Hq, int Hkv, const int *__restrict__ pos, const int *__restrict__ tok_seq,              \
        const int *__restrict__ block_table, int max_blocks, int block_size, uint16_t *__restrict__ out,         \
        float scale, uint8_t *fq, void *fs, int fmode, int frows, const int *__restrict__ cu, int skip_prompts,   \
        int min_chunk, float *part, const int *__restrict__ outs, int spec
#define PKV_PAGED_PASS                                                                                           \
    q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, tok_seq, block_table, max_blocks, block_size, \
        out, scale, pkv::Fp8Out{fq, fs, fmode, frows}, cu, skip_prompts, min_chunk, part, outs, spec

// attn_paged_g<G> over a bf16 cache and attn_paged8_g<G> over an E4M3 cache
// (kscale / vscale given), for the groups the reference instantiates
// (qwen35.cu:1330-1334).
#define PKV_PAGED_KERNELS(G, THREADS)                                                                            \
    extern "C" __global__ void __launch_bounds__(THREADS) attn_paged_g##G(PKV_PAGED_ARGS) {                      \
        pkv::paged_ref<G, false>(PKV_PAGED_PASS);                                                                \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(THREADS, 2) attn_paged8_g##G(PKV_PAGED_ARGS) {                  \
        pkv::paged_ref<G, true>(PKV_PAGED_PASS);                                                                 \
    }
PKV_PAGED_KERNELS(1, 256)
PKV_PAGED_KERNELS(2, 256)
PKV_PAGED_KERNELS(4, 256)
PKV_PAGED_KERNELS(6, 128)
PKV_PAGED_KERNELS(8, 128)

extern "C" __global__ void __launch_bounds__(256)
    attn_merge(const float* __restrict__ part, int Z, int min_chunk, const uint16_t* __restrict__ qkv, int qstride,
               int Hq, const int* __restrict__ pos, const int* __restrict__ tok_seq, const int* __restrict__ cu,
               int skip_prompts, uint16_t* __restrict__ out, uint8_t* fq, void* fs, int fmode, int frows,
               const int* __restrict__ outs, int spec) {
    if (blockDim.x != 256) return;
    const int t = blockIdx.x, h = blockIdx.y;
    const int sq = tok_seq[t];
    if (pkv::ref_prompt_row(skip_prompts, cu, sq, outs, spec)) return;
    const int nz = pkv::ref_split_parts(pos[t] + 1, Z, min_chunk);
    const float* pp = part + (((size_t)sq * spec + (t - cu[sq])) * Hq + h) * Z * (HEAD_DIM + 2);
    const pkv::Fp8Out fo{fq, fs, fmode, frows};
    pkv::merge_rows(
        nz, pkv::LOG2E, [&](int i) { return pp + (size_t)i * (HEAD_DIM + 2); },
        [&](int i) { return pp + (size_t)i * (HEAD_DIM + 2) + 2; },
        qkv + (size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM, out + ((size_t)t * Hq + h) * HEAD_DIM,
        &fo, t, h * HEAD_DIM, Hq * HEAD_DIM);
}

#define PKV_FLASH_ARGS                                                                                            \
    const uint16_t *__restrict__ q, const void *__restrict__ kcache, const void *__restrict__ vcache,             \
        const float *__restrict__ kscale, const float *__restrict__ vscale, const uint16_t *__restrict__ qkv,     \
        int qstride, int Hq, int Hkv, const int *__restrict__ pos, const int *__restrict__ cu, int seqs,          \
        const int *__restrict__ block_table, int max_blocks, int block_size, uint16_t *__restrict__ out,          \
        float scale, const int *__restrict__ outs, int spec

namespace pkv {

// The prompt kernels on the engine's grid of BQ-query tiles (attn_mfma:
// one workgroup per two 32-query tiles, the other blocks of the grid exit).
// Tiles load by LDS DMA (bf16) or through registers (E4M3) into two stages
// (one tile of lead) with the DMA waves' page-id rings after them.
// attn_groupr (4 or 3 waves): the stages and rings live in the launch's
// dynamic shared memory (the engine asks for 67,584 bytes; two stages with
// V pairs 1,056 bytes apart and the rings take 67,328 at G = 4, 67,200 at
// G = 6) and nothing is static, so two workgroups fit a CU at up to 256
// VGPRs. attn_mfma (8 waves): two stages of the default layout and 8 rings
// in static LDS (68,608 bytes beside the launch's 37,376 dynamic ones).
constexpr int REF_VP32 = PF_VPAIR_TIGHT;  // V pair stride of the attn_groupr stages (elements)

// G heads per kv head, BQ queries per workgroup (16 x the name's tiles),
// F8: E4M3 cache, VP: V pair stride of the NST stages, DYN: stages in the
// launch's dynamic shared memory (checked against the dispatch packet's
// group segment size, byte offset 28: a launch with too little does
// nothing), else in static LDS.
template <int G, int BQ, bool F8, int VP, bool DYN, int NST = 2>
__device__ __forceinline__ void flash_ref(PKV_FLASH_ARGS) {
    constexpr int THREADS = pf_threads(BQ, 1, G);
    uint16_t* sm;
    if constexpr (DYN) {
        extern __shared__ __align__(16) uint16_t dyn_sm[];
        sm = dyn_sm;
        constexpr uint32_t need = (uint32_t)NST * pf_stage(VP) * 2u + (F8 ? 0u : (uint32_t)pf_ids_bytes(THREADS));
        const uint32_t group_bytes = reinterpret_cast<const uint32_t*>(__builtin_amdgcn_dispatch_ptr())[7];
        if (group_bytes < need) return;
    } else {
        __shared__ __align__(16) uint16_t st_sm[2 * pf_stage(VP) + pf_ids_bytes(THREADS) / 2];
        sm = st_sm;
    }
    if ((int)blockDim.x != THREADS || Hq != G * Hkv || (kscale != nullptr) != F8 || (vscale != nullptr) != F8 ||
        block_size <= 0 || (block_size & (block_size - 1)))
        return;
    PrefillParams p;
    p.q = q;
    p.kc = (const uint16_t*)kcache;
    p.vc = (const uint16_t*)vcache;
    p.qkv = qkv;
    p.qstride = qstride;
    p.Hq = Hq;
    p.Hkv = Hkv;
    p.pos = pos;
    p.cu = cu;
    p.seqs = seqs;
    p.block_table = block_table;
    p.max_blocks = max_blocks;
    p.block_size = block_size;
    p.bs_log2 = __builtin_ctz((unsigned)block_size);
    p.out = out;
    p.scale = scale;
    p.outs = outs;
    p.spec = spec;
    p.num_blocks = REF_NO_CLAMP;
    p.kscale = kscale;
    p.vscale = vscale;
    prefill_body<G, BQ, 1, F8, NST, VP>(p, sm);
}

}  // namespace pkv

#define PKV_FLASH_PASS                                                                                           \
    q, kcache, vcache, kscale, vscale, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks, block_size, \
        out, scale, outs, spec

// bf16 cache, queries in registers (what gfx950 selects for G = 4 and 6):
// stages with V pairs REF_VP32 apart fit the engine's 67,584 bytes, two
// workgroups per CU.
extern "C" __global__ void __launch_bounds__(256, 2) attn_groupr_g4_t2_k32(PKV_FLASH_ARGS) {
    pkv::flash_ref<4, 32, false, pkv::REF_VP32, true>(PKV_FLASH_PASS);
}
extern "C" __global__ void __launch_bounds__(192, 2) attn_groupr_g6_t1_k32(PKV_FLASH_ARGS) {
    pkv::flash_ref<6, 16, false, pkv::REF_VP32, true>(PKV_FLASH_PASS);
}

// bf16 cache, G = 1, 2, 8 (fa_shape's 16-key default: 128 queries x 1
// head, 64 x 2, 16 x 8 per workgroup, 256 threads, 101,376 bytes of dynamic
// shared memory from the engine), and every group over an E4M3 cache
// (attn_group8_*; 84,480 bytes for G = 6, 101,376 otherwise). Two stages of
// the default layout; one workgroup per CU.
#define PKV_FLASH_K16(NAME, G, BQ, F8, NST, VP)                                                                  \
    extern "C" __global__ void __launch_bounds__(pkv::pf_threads(BQ, 1, G), 1) NAME(PKV_FLASH_ARGS) {            \
        pkv::flash_ref<G, BQ, F8, VP, true, NST>(PKV_FLASH_PASS);                                                \
    }
// 101,376 bytes hold three stages with V pairs 1,056 bytes apart (100,608
// bytes, plus 256 of page-id rings for bf16): tiles requested two ahead;
// G = 6's 84,480 hold two stages.
PKV_FLASH_K16(attn_group_g1_t8_k16, 1, 128, false, 3, pkv::REF_VP32)
PKV_FLASH_K16(attn_group_g2_t4_k16, 2, 64, false, 3, pkv::REF_VP32)
PKV_FLASH_K16(attn_group_g8_t1_k16, 8, 16, false, 3, pkv::REF_VP32)
PKV_FLASH_K16(attn_group8_g1_t8_k16, 1, 128, true, 3, pkv::REF_VP32)
PKV_FLASH_K16(attn_group8_g2_t4_k16, 2, 64, true, 3, pkv::REF_VP32)
PKV_FLASH_K16(attn_group8_g4_t2_k16, 4, 32, true, 3, pkv::REF_VP32)
PKV_FLASH_K16(attn_group8_g6_t1_k16, 6, 16, true, 2, pkv::PF_VPAIR)
PKV_FLASH_K16(attn_group8_g8_t1_k16, 8, 16, true, 3, pkv::REF_VP32)

// gfx942's name for G = 4 (attn_mfma_g4_t2, 512 threads): 64 queries per
// workgroup, stages in static LDS beside the launch's 37,376 dynamic bytes.
extern "C" __global__ void __launch_bounds__(512, 1) attn_mfma_g4_t2(PKV_FLASH_ARGS) {
    pkv::flash_ref<4, 64, false, pkv::PF_VPAIR, false>(PKV_FLASH_PASS);
}

// The draft passes' slot mapping under the reference's name and signature
// (qwen35.cu:2633-2650; grid ceil(S / 128) x 128 threads).
extern "C" __global__ void __launch_bounds__(256)
    mtp_next(const int* __restrict__ rows, const int* __restrict__ pos, const int* __restrict__ rope, int rope_stride,
             const int* __restrict__ block_table, int max_blocks, int block_size, const int* __restrict__ limits, int k,
             int* __restrict__ dpos, int* __restrict__ dslot, int* __restrict__ drope, int S) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s < S && block_size > 0)
        pkv::mtp_next_one(s, rows, pos, rope, rope_stride, block_table, max_blocks, block_size, limits, k, dpos,
                          dslot, drope, S);
}

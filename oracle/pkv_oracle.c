/*
 * CPU oracle for the paged KV cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * or the timed CPU baseline. The product path (libpkv.so) never calls it.
 *
 * A scalar restatement, written from the reference's semantics, of:
 *   - the KV append scatter        (reference src/kernels/qwen35.cu:1086-1100, 1120-1127)
 *   - the gather through the block table (qwen35.cu:1204, amd/attn_decode.cuh:56-74)
 *   - paged decode attention + gate (qwen35.cu:1146-1309, amd/attn_decode.cuh:12-183)
 *   - split-K partials and merge    (qwen35.cu:1137-1141, 1264-1288, 2242-2279)
 *   - chunked-prefill causal attention (qwen35.cu:1364-1585, amd/attention.cuh:12-136)
 *   - page copy (copy-on-write; build-defined: the reference has no CoW)
 *   - attention input preparation: q/k RMSNorm, interleaved multimodal
 *     rotary, q out, k/v to their cache slots (attn_prep, qwen35.cu:1067-1128)
 *   - the E4M3 cache: per-(slot, head) scale amax / 448 and saturating
 *     round-to-nearest-even E4M3 (OCP "E4M3FN": bias 7, max 448, NaN 0x7F /
 *     0xFF, no infinities) bytes (store_e4m3, qwen35.cu:1055-1065), and
 *     decode attention over it (attn_paged8_g*, qwen35.cu:1146-1309 with F8)
 *   - FP8 activation copies of the gated outputs (Fp8Out / quant8,
 *     src/kernels/fp8.cuh:29-85, written at qwen35.cu:1297-1307, 2269-2279):
 *     mode 1 Block128 f32 scales, mode 2 Mx32 E8M0 exponents in the MXFP8
 *     tiled layout
 *
 * Pinning (what each function is checked against, in tests/test_oracle.py):
 *   append/gather/page_copy: closed forms, gather(append(x)) == x under
 *       random permutation block tables, brute-force on tiny pools.
 *   attention: torch fp64 scaled_dot_product_attention golden fixtures
 *       (tests/golden/), closed forms (one key -> v; equal keys -> mean of v;
 *       a dominant key -> its v), split+merge == unsplit.
 *   E4M3: decoding of all 256 codes and rounding of random and tie values
 *       against torch.float8_e4m3fn (which agrees in range; the reference
 *       saturates where torch gives NaN: closed-form checks at +-448);
 *       decode8 closed forms (one key -> its scaled value, equal keys -> the
 *       mean) and decode8 == bf16 decode on values the E4M3 grid holds.
 *   attn_prep: closed forms (constant rows normalise to the weights; position
 *       0 leaves rows unrotated; a rotation keeps each pair's norm; the axis
 *       rule picks height/width positions for exactly the frequencies
 *       d % 3 == 1 / 2 below 3 sec_h / 3 sec_w), v copied bit for bit.
 *   prefill with the reference's P rounding (p_tile = 32): a 3-key closed
 *       form where a new fractional max in the second tile moves the anchor
 *       (any other anchoring or rounding point gives other bits), and exact
 *       equality with the textbook softmax when every p is a power of two.
 *   FP8 copies: the Mx32 exponent is the smallest e with amax / 2^e <= 448
 *       (checked by brute force over a range of amax, powers of two included);
 *       the tiled index is a bijection onto [0, tiles x 512) and puts rows
 *       r, r + 32, r + 64, r + 96 of a 128-row tile 4 bytes apart inside the
 *       same 16 bytes (cuBLASLt's 128 x 4 block-scale tile); bytes dequantise
 *       to within half an E4M3 step of v, and values on the E4M3 grid times a
 *       power-of-two scale come back exactly.
 *   Parity unpinned beyond the stated tolerance: expf vs exp2f last bits
 *   (the reference's fast_exp2 against exp2 in double), f32 against double
 *   accumulation order; in attn_prep the f32 order of the squared sum and
 *   the last bits of cosf/sinf (1 bf16 ulp).
 *
 * Arithmetic: softmax and weighted sums in double; the epilogue follows the
 * reference exactly in f32: o = bf16_round(A / S); y = o / (1 + expf(-gate));
 * out = bf16_rne(y)  (qwen35.cu:1290-1293, 2270-2273).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define HEAD_DIM 256

/* ---- bf16 helpers (reference b2f/f2b/rbf, qwen35.cu:26-28; RNE like
 * __float2bfloat16_rn) ---- */
float orc_b2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f2b(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) /* NaN: keep sign, quiet */
        return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float rbf(float x) { return orc_b2f(orc_f2b(x)); }

/* Speculative rows: outs[s * spec] >= 0 (qwen35.cu:94-100). */
static int is_spec(const int* outs, int spec, int s) { return outs && outs[(size_t)s * spec] >= 0; }

/* ---- slot of key position p through a block-table row (sched.rs:1113-1114,
 * qwen35.cu:1204) ---- */
long orc_slot(const int* bt_row, int p, int block_size) {
    return (long)bt_row[p / block_size] * block_size + p % block_size;
}

/* ---- KV append: cache[(slot * Hkv + h) * row] = src[t][h]; slot < 0 skips
 * (qwen35.cu:1090-1100 for V, 1120-1127 for K after norm/rope, which callers
 * of this path have already applied). Byte-exact copy. `row_stride` is in
 * bytes between consecutive tokens' rows; head rows are contiguous. ---- */
void orc_append(const uint8_t* k_src, const uint8_t* v_src, long row_stride, const int* slot_map, int T,
                int Hkv, int head_bytes, uint8_t* kcache, uint8_t* vcache) {
    for (int t = 0; t < T; t++) {
        const int slot = slot_map[t];
        if (slot < 0) continue;
        for (int h = 0; h < Hkv; h++) {
            const size_t at = ((size_t)slot * Hkv + h) * head_bytes;
            memcpy(kcache + at, k_src + (size_t)t * row_stride + (size_t)h * head_bytes, head_bytes);
            memcpy(vcache + at, v_src + (size_t)t * row_stride + (size_t)h * head_bytes, head_bytes);
        }
    }
}

/* ---- gather: dense[j][h] = cache[slot(j)][h] for j < L (implicit in every
 * reference attention read: qwen35.cu:1203-1205). ---- */
void orc_gather(const uint8_t* kcache, const uint8_t* vcache, const int* bt_row, int L, int block_size, int Hkv,
                int head_bytes, uint8_t* k_out, uint8_t* v_out) {
    const size_t rb = (size_t)Hkv * head_bytes;
    for (int j = 0; j < L; j++) {
        const size_t slot = (size_t)orc_slot(bt_row, j, block_size);
        memcpy(k_out + j * rb, kcache + slot * rb, rb);
        memcpy(v_out + j * rb, vcache + slot * rb, rb);
    }
}

/* ---- page copy (copy-on-write): page dst := page src for K and V, all
 * block_size slots and all kv heads, byte-exact. ---- */
void orc_page_copy(uint8_t* kcache, uint8_t* vcache, const int* src, const int* dst, int n, long page_bytes) {
    for (int i = 0; i < n; i++) {
        memmove(kcache + (size_t)dst[i] * page_bytes, kcache + (size_t)src[i] * page_bytes, page_bytes);
        memmove(vcache + (size_t)dst[i] * page_bytes, vcache + (size_t)src[i] * page_bytes, page_bytes);
    }
}

/* One (token, q head) over keys [j0, j1): natural-log softmax partial
 * (M = max score, S = sum e^(s-M), A[d] = sum e^(s-M) v[d]) in double.
 * Scores are (q . k) * scale (qwen35.cu:1188-1190 scales q by `scale`).
 * dtype 0: bf16 cache and q; 1: f32. */
static void partial(const void* q, const void* kc, const void* vc, int dtype, int D, int Hq, int Hkv, int t, int h,
                    const int* bt, int block_size, int j0, int j1, float scale, double* M, double* S, double* A) {
    const int G = Hq / Hkv, kvh = h / G;
    double qd[HEAD_DIM];
    for (int d = 0; d < D; d++)
        qd[d] = dtype ? ((const float*)q)[((size_t)t * Hq + h) * D + d]
                      : orc_b2f(((const uint16_t*)q)[((size_t)t * Hq + h) * D + d]);
    double m = -INFINITY;
    double* s = (double*)malloc(sizeof(double) * (size_t)(j1 > j0 ? j1 - j0 : 1));
    for (int j = j0; j < j1; j++) {
        const size_t at = ((size_t)orc_slot(bt, j, block_size) * Hkv + kvh) * D;
        double dot = 0.0;
        for (int d = 0; d < D; d++)
            dot += qd[d] * (dtype ? ((const float*)kc)[at + d] : orc_b2f(((const uint16_t*)kc)[at + d]));
        s[j - j0] = dot * (double)scale;
        if (s[j - j0] > m) m = s[j - j0];
    }
    double sum = 0.0;
    for (int d = 0; d < D; d++) A[d] = 0.0;
    for (int j = j0; j < j1; j++) {
        const double p = exp(s[j - j0] - m);
        sum += p;
        const size_t at = ((size_t)orc_slot(bt, j, block_size) * Hkv + kvh) * D;
        for (int d = 0; d < D; d++)
            A[d] += p * (dtype ? ((const float*)vc)[at + d] : orc_b2f(((const uint16_t*)vc)[at + d]));
    }
    free(s);
    *M = m;
    *S = sum;
}

/* Gated epilogue (qwen35.cu:1290-1293): y = rbf(o) * sigmoid(gate), in f32. */
static uint16_t gated(double o, float gate) {
    const float ov = rbf((float)o);
    const float y = ov / (1.f + expf(-gate));
    return orc_f2b(y);
}

/* ---- paged decode attention, bf16 cache (attn_paged_g<G> semantics,
 * qwen35.cu:1146-1309): for every decode token t (prompt rows skipped when
 * skip_prompts, qwen35.cu:1171-1172), every q head h: attention over keys
 * 0 .. pos[t] of its sequence's pages, gated output bf16 into out[t][h][256].
 * Rows that are skipped are left untouched. Returns the number of rows
 * written. Optional o_raw (may be NULL) receives the ungated f32 A/S. ---- */
int orc_attn_decode(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, const uint16_t* qkv,
                    int qstride, int Hq, int Hkv, const int* pos, const int* tok_seq, const int* block_table,
                    int max_blocks, int block_size, uint16_t* out, float scale, const int* cu, int skip_prompts,
                    const int* outs, int spec, int T, float* o_raw) {
    int rows = 0;
    double A[HEAD_DIM];
    for (int t = 0; t < T; t++) {
        const int sq = tok_seq[t];
        if (skip_prompts && cu[sq + 1] - cu[sq] > 1 && !is_spec(outs, spec, sq)) continue;
        const int L = pos[t] + 1;
        const int* bt = block_table + (size_t)sq * max_blocks;
        for (int h = 0; h < Hq; h++) {
            double M, S;
            partial(q, kcache, vcache, 0, HEAD_DIM, Hq, Hkv, t, h, bt, block_size, 0, L, scale, &M, &S, A);
            for (int d = 0; d < HEAD_DIM; d++) {
                const double o = A[d] / S;
                const float gate = orc_b2f(qkv[(size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + d]);
                out[((size_t)t * Hq + h) * HEAD_DIM + d] = gated(o, gate);
                if (o_raw) o_raw[((size_t)t * Hq + h) * HEAD_DIM + d] = (float)o;
            }
        }
        rows++;
    }
    return rows;
}

/* ---- the same decode attention as a one-pass scalar f32 implementation
 * (the CPU baseline's second leg, not a checker): per (token, kv head) each
 * key's K and V rows are read once for the G query heads of the group, the
 * scores and the online softmax (running max, rescale on a new max) and the
 * weighted sums are f32, as a plain CPU port of attn_paged_g<G>
 * (qwen35.cu:1146-1309) would keep them. Same rows, skipping and gated
 * epilogue as orc_attn_decode. Returns the number of rows written. ---- */
int orc_attn_decode_f32(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, const uint16_t* qkv,
                        int qstride, int Hq, int Hkv, const int* pos, const int* tok_seq, const int* block_table,
                        int max_blocks, int block_size, uint16_t* out, float scale, const int* cu, int skip_prompts,
                        const int* outs, int spec, int T) {
    const int G = Hq / Hkv;
    if (G > 16) return -1;
    int rows = 0;
    float qf[16][HEAD_DIM], A[16][HEAD_DIM], kr[HEAD_DIM], vr[HEAD_DIM], m[16], l[16];
    for (int t = 0; t < T; t++) {
        const int sq = tok_seq[t];
        if (skip_prompts && cu[sq + 1] - cu[sq] > 1 && !is_spec(outs, spec, sq)) continue;
        const int L = pos[t] + 1;
        const int* bt = block_table + (size_t)sq * max_blocks;
        for (int kvh = 0; kvh < Hkv; kvh++) {
            for (int g = 0; g < G; g++) {
                const int h = kvh * G + g;
                for (int d = 0; d < HEAD_DIM; d++) {
                    qf[g][d] = orc_b2f(q[((size_t)t * Hq + h) * HEAD_DIM + d]) * scale;
                    A[g][d] = 0.f;
                }
                m[g] = -INFINITY;
                l[g] = 0.f;
            }
            for (int j = 0; j < L; j++) {
                const size_t at = ((size_t)orc_slot(bt, j, block_size) * Hkv + kvh) * HEAD_DIM;
                for (int d = 0; d < HEAD_DIM; d++) {
                    kr[d] = orc_b2f(kcache[at + d]);
                    vr[d] = orc_b2f(vcache[at + d]);
                }
                for (int g = 0; g < G; g++) {
                    float sc = 0.f;
                    for (int d = 0; d < HEAD_DIM; d++) sc += qf[g][d] * kr[d];
                    if (sc > m[g]) {
                        const float c = expf(m[g] - sc); /* 0 on the first key */
                        l[g] *= c;
                        for (int d = 0; d < HEAD_DIM; d++) A[g][d] *= c;
                        m[g] = sc;
                    }
                    const float p = expf(sc - m[g]);
                    l[g] += p;
                    for (int d = 0; d < HEAD_DIM; d++) A[g][d] += p * vr[d];
                }
            }
            for (int g = 0; g < G; g++) {
                const int h = kvh * G + g;
                for (int d = 0; d < HEAD_DIM; d++) {
                    const float gate = orc_b2f(qkv[(size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + d]);
                    out[((size_t)t * Hq + h) * HEAD_DIM + d] = gated((double)(A[g][d] / l[g]), gate);
                }
            }
        }
        rows++;
    }
    return rows;
}

/* ---- generic single-query attention (f32 or bf16 cache, any head dim) for
 * the CPU plumbing config: o[h][d] = softmax(q . k * scale) v over keys
 * 0..L-1 of one sequence, ungated, f32 output. ---- */
void orc_attn_single(const void* q, const void* kcache, const void* vcache, int dtype, int D, int Hq, int Hkv,
                     const int* bt_row, int L, int block_size, float scale, float* o) {
    double A[1024];
    for (int h = 0; h < Hq; h++) {
        double M, S;
        partial(q, kcache, vcache, dtype, D, Hq, Hkv, 0, h, bt_row, block_size, 0, L, scale, &M, &S, A);
        for (int d = 0; d < D; d++) o[(size_t)h * D + d] = (float)(A[d] / S);
    }
}

/* ---- split-K semantics (flash decoding): the reference splits a token's L
 * keys into parts = max(1, min(Z, ceil(L / min_chunk))) ranges of
 * chunk = ceil(L / parts) keys (qwen35.cu:1137-1141, 1176-1181); each range
 * yields (M, S, A[256]) and attn_merge combines them in range order
 * (qwen35.cu:2255-2273). Partials here are natural-log domain doubles. ---- */
int orc_split_parts(int L, int Z, int min_chunk) {
    int p = (L + min_chunk - 1) / min_chunk;
    if (p > Z) p = Z;
    return p < 1 ? 1 : p;
}

void orc_attn_partial(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, int Hq, int Hkv, int t,
                      int h, const int* bt_row, int block_size, int j0, int j1, float scale, double* M, double* S,
                      double* A) {
    partial(q, kcache, vcache, 0, HEAD_DIM, Hq, Hkv, t, h, bt_row, block_size, j0, j1, scale, M, S, A);
}

/* Merge n partials: M* = max M, S* = sum S e^(M-M*), A* likewise; ranges
 * with M = -inf contribute 0 (qwen35.cu:2258-2266). Writes A* / S* to o. */
void orc_merge(const double* M, const double* S, const double* A, int n, double* o) {
    double Mx = -INFINITY;
    for (int z = 0; z < n; z++)
        if (M[z] > Mx) Mx = M[z];
    double St = 0.0;
    for (int d = 0; d < HEAD_DIM; d++) o[d] = 0.0;
    for (int z = 0; z < n; z++) {
        const double f = M[z] == -INFINITY ? 0.0 : exp(M[z] - Mx);
        St += S[z] * f;
        for (int d = 0; d < HEAD_DIM; d++) o[d] += A[(size_t)z * HEAD_DIM + d] * f;
    }
    for (int d = 0; d < HEAD_DIM; d++) o[d] /= St;
}

/* ---- chunked-prefill attention over paged context (attn_mfma_g<G>_t<NT> /
 * attn_flash_group semantics, amd/attention.cuh:12-136, qwen35.cu:1364-1585):
 * for every prompt sequence s (more than one token and not verifying drafts,
 * amd/attention.cuh:22-24), every token t of it at position pos[t], every q
 * head: causal attention over keys 0..pos[t] (a key kp is visible iff
 * kp <= qp and kp < L, attention.cuh:81-89; with positions contiguous within
 * the chunk that is kp <= pos[t]). The query is rounded to bf16 after scaling
 * by scale * log2(e) as the reference does (amd/attention.cuh:37-44); scores
 * are exp2-domain. Gated epilogue as decode.
 * p_tile = 0 keeps P in double (textbook softmax: the form the torch SDPA
 * goldens pin). p_tile = 32 restates the reference's tiled online softmax
 * (attention.cuh:55-121 with AM_BN = 32, attention.cuh:10): keys in tiles
 * [k0, k0 + 32) from key 0; after each tile the anchor b = running max
 * (over keys seen so far), p = exp2(s - b); the denominator adds p
 * unrounded (attention.cuh:101-107), P.V takes p rounded to bf16
 * (pack4, attention.cuh:115), and earlier sums are rescaled by
 * exp2(b_old - b) (attention.cuh:108-110). Returns the number of token rows
 * written. ---- */
/* orc_attn_prefill_part: the same over token rows [t0, t1) and query heads
 * [h0, h1) only (each (row, head) output is independent of the others; the
 * tests split one prefill over threads this way). */
int orc_attn_prefill_part(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, const uint16_t* qkv,
                          int qstride, int Hq, int Hkv, const int* pos, const int* cu, int seqs,
                          const int* block_table, int max_blocks, int block_size, uint16_t* out, float scale,
                          const int* outs, int spec, int p_tile, int t0, int t1, int h0, int h1) {
    const double LOG2E = 1.4426950408889634;
    const int G = Hq / Hkv;
    int rows = 0;
    double A[HEAD_DIM], qd[HEAD_DIM];
    for (int s = 0; s < seqs; s++) {
        const int n = cu[s + 1] - cu[s];
        if (n <= 1 || is_spec(outs, spec, s)) continue;
        const int* bt = block_table + (size_t)s * max_blocks;
        const int ta = cu[s] > t0 ? cu[s] : t0, tb = cu[s + 1] < t1 ? cu[s + 1] : t1;
        for (int t = ta; t < tb; t++) {
            const int L = pos[t] + 1;
            double* sc = (double*)malloc(sizeof(double) * (size_t)L);
            for (int h = h0; h < h1; h++) {
                const int kvh = h / G;
                for (int d = 0; d < HEAD_DIM; d++)
                    qd[d] = rbf(orc_b2f(q[((size_t)t * Hq + h) * HEAD_DIM + d]) * (scale * (float)LOG2E));
                double m = -INFINITY;
                for (int j = 0; j < L; j++) {
                    const size_t at = ((size_t)orc_slot(bt, j, block_size) * Hkv + kvh) * HEAD_DIM;
                    double dot = 0.0;
                    for (int d = 0; d < HEAD_DIM; d++) dot += qd[d] * orc_b2f(kcache[at + d]);
                    sc[j] = dot;
                    if (dot > m) m = dot;
                }
                double S = 0.0;
                for (int d = 0; d < HEAD_DIM; d++) A[d] = 0.0;
                if (p_tile > 0) {
                    /* the reference's tiles: anchor b after each tile, bf16 P in P.V */
                    double b = -INFINITY;
                    for (int k0 = 0; k0 < L; k0 += p_tile) {
                        const int k1 = k0 + p_tile < L ? k0 + p_tile : L;
                        double bn = b;
                        for (int j = k0; j < k1; j++)
                            if (sc[j] > bn) bn = sc[j];
                        const double c = exp2(b - bn); /* 0 on the first tile (b = -inf) */
                        S *= c;
                        for (int d = 0; d < HEAD_DIM; d++) A[d] *= c;
                        b = bn;
                        for (int j = k0; j < k1; j++) {
                            const double p = exp2(sc[j] - b);
                            S += p;
                            const double pb = orc_b2f(orc_f2b((float)p));
                            const size_t at = ((size_t)orc_slot(bt, j, block_size) * Hkv + kvh) * HEAD_DIM;
                            for (int d = 0; d < HEAD_DIM; d++) A[d] += pb * orc_b2f(vcache[at + d]);
                        }
                    }
                } else {
                    for (int j = 0; j < L; j++) {
                        const double p = exp2(sc[j] - m);
                        S += p;
                        const size_t at = ((size_t)orc_slot(bt, j, block_size) * Hkv + kvh) * HEAD_DIM;
                        for (int d = 0; d < HEAD_DIM; d++) A[d] += p * orc_b2f(vcache[at + d]);
                    }
                }
                for (int d = 0; d < HEAD_DIM; d++) {
                    const float gate = orc_b2f(qkv[(size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + d]);
                    out[((size_t)t * Hq + h) * HEAD_DIM + d] = gated(A[d] / S, gate);
                }
            }
            free(sc);
            rows++;
        }
    }
    return rows;
}

int orc_attn_prefill_t(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, const uint16_t* qkv,
                       int qstride, int Hq, int Hkv, const int* pos, const int* cu, int seqs, const int* block_table,
                       int max_blocks, int block_size, uint16_t* out, float scale, const int* outs, int spec,
                       int p_tile) {
    return orc_attn_prefill_part(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks,
                                 block_size, out, scale, outs, spec, p_tile, 0, cu[seqs], 0, Hq);
}

int orc_attn_prefill(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache, const uint16_t* qkv,
                     int qstride, int Hq, int Hkv, const int* pos, const int* cu, int seqs, const int* block_table,
                     int max_blocks, int block_size, uint16_t* out, float scale, const int* outs, int spec) {
    return orc_attn_prefill_t(q, kcache, vcache, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks,
                              block_size, out, scale, outs, spec, 0);
}

/* ---- draft-token (speculative verify) metadata (mtp_next, qwen35.cu:2633-2650):
 * dslot = p <= limits[s] ? bt[p / bs] * bs + p % bs : -1. ---- */
void orc_mtp_slots(const int* rows, const int* pos, const int* block_table, int max_blocks, int block_size,
                   const int* limits, int k, int* dpos, int* dslot, int S) {
    for (int s = 0; s < S; s++) {
        const int p = pos[rows[s]] + k;
        dpos[s] = p;
        dslot[s] = p <= limits[s] ? block_table[(size_t)s * max_blocks + p / block_size] * block_size + p % block_size
                                  : -1;
    }
}

/* mtp_next in full (qwen35.cu:2633-2650): the slots above plus the three
 * rotary position rows of the draft pass, drope[axis * S + s] =
 * rope[axis * rope_stride + rows[s]] + k. */
void orc_mtp_next(const int* rows, const int* pos, const int* rope, int rope_stride, const int* block_table,
                  int max_blocks, int block_size, const int* limits, int k, int* dpos, int* dslot, int* drope, int S) {
    orc_mtp_slots(rows, pos, block_table, max_blocks, block_size, limits, k, dpos, dslot, S);
    for (int s = 0; s < S; s++)
        for (int axis = 0; axis < 3; axis++) drope[axis * S + s] = rope[(size_t)axis * rope_stride + rows[s]] + k;
}

/* ---- attention input preparation (reference attn_prep, qwen35.cu:1067-1128):
 * per token t and head: q heads (and k heads) are RMS-normalised with their
 * f32 weights, y = bf16(x * scale * w), scale = 1 / sqrt(sum x^2 / 256 + eps)
 * (sum in double here, rounded to f32), then dims 0..63 are rotated as pairs
 * (d, d + 32) with bf16-rounded cos/sin of position * inv_freq[d]: lo' =
 * bf16(bf16(lo c) - bf16(hi s)), hi' = bf16(bf16(hi c) + bf16(lo s)). The
 * position of frequency d is rope[axis * rope_stride + t], axis = 1 (height)
 * when d % 3 == 1 and d < 3 sec_h, 2 (width) when d % 3 == 2 and d < 3 sec_w,
 * else 0 (time). q -> qout[t][h]; k -> kcache[slot][h]; v copied to
 * vcache[slot][h]; k and v are skipped for slot < 0 (or >= num_slots). */
#define ROPE_DIM 64
void orc_attn_prep(const uint16_t* qkv, int qstride, int Hq, int Hkv, const float* q_norm, const float* k_norm,
                   const int* rope, int rope_stride, int sec_h, int sec_w, const int* slot_map,
                   const float* inv_freq, float eps, int T, long num_slots, uint16_t* qout, uint16_t* kcache,
                   uint16_t* vcache) {
    for (int t = 0; t < T; t++) {
        const uint16_t* row = qkv + (size_t)t * qstride;
        const long slot = slot_map[t];
        const int has_slot = slot >= 0 && slot < num_slots;
        for (int hh = 0; hh < Hq + 2 * Hkv; hh++) {
            if (hh >= Hq + Hkv) {
                if (!has_slot) continue;
                const int vh = hh - Hq - Hkv;
                memcpy(vcache + ((size_t)slot * Hkv + vh) * HEAD_DIM, row + (size_t)Hq * 2 * HEAD_DIM +
                       (size_t)Hkv * HEAD_DIM + (size_t)vh * HEAD_DIM, HEAD_DIM * 2);
                continue;
            }
            const int is_q = hh < Hq;
            if (!is_q && !has_slot) continue;
            const uint16_t* src = is_q ? row + (size_t)hh * 2 * HEAD_DIM : row + (size_t)Hq * 2 * HEAD_DIM +
                                                                             (size_t)(hh - Hq) * HEAD_DIM;
            const float* w = is_q ? q_norm : k_norm;
            double ss = 0.0;
            for (int d = 0; d < HEAD_DIM; d++) {
                const double x = orc_b2f(src[d]);
                ss += x * x;
            }
            const float scale = 1.f / sqrtf((float)ss / HEAD_DIM + eps);
            float y[HEAD_DIM];
            for (int d = 0; d < HEAD_DIM; d++) y[d] = rbf(orc_b2f(src[d]) * scale * w[d]);
            float r[ROPE_DIM];
            for (int d = 0; d < ROPE_DIM / 2; d++) {
                const int axis = (d % 3 == 1 && d < 3 * sec_h) ? 1 : (d % 3 == 2 && d < 3 * sec_w) ? 2 : 0;
                const float f = (float)rope[(size_t)axis * rope_stride + t] * inv_freq[d];
                const float c = rbf(cosf(f)), sn = rbf(sinf(f));
                const float lo = y[d], hi = y[d + ROPE_DIM / 2];
                r[d] = rbf(rbf(lo * c) - rbf(hi * sn));
                r[d + ROPE_DIM / 2] = rbf(rbf(hi * c) + rbf(lo * sn));
            }
            for (int d = 0; d < ROPE_DIM; d++) y[d] = r[d];
            uint16_t* dst = is_q ? qout + ((size_t)t * Hq + hh) * HEAD_DIM
                                 : kcache + ((size_t)slot * Hkv + (hh - Hq)) * HEAD_DIM;
            for (int d = 0; d < HEAD_DIM; d++) dst[d] = orc_f2b(y[d]);
        }
    }
}

/* ---- E4M3 (OCP E4M3FN) ---- */
float orc_e4m3_to_f(uint8_t b) {
    const int sign = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0)
        v = ldexpf((float)m, -9);  /* subnormal: m / 8 * 2^-6 */
    else
        v = ldexpf(1.f + m / 8.f, e - 7);
    return sign ? -v : v;
}

/* Round to nearest, ties to even, saturating to +-448; NaN -> 0x7F. */
uint8_t orc_f_to_e4m3(float x) {
    if (isnan(x)) return 0x7F;
    const uint8_t sign = signbit(x) ? 0x80 : 0;
    double a = fabs((double)x);
    if (a >= 448.0) return sign | 0x7E;
    /* the E4M3 grid below 448: exhaustive nearest search with ties to even */
    int best = 0;
    double bd = a;
    for (int c = 1; c <= 0x7E; c++) {
        const double v = orc_e4m3_to_f((uint8_t)c);
        const double d = fabs(v - a);
        if (d < bd || (d == bd && (c & 1) == 0 && (best & 1) == 1)) {
            bd = d;
            best = c;
        }
    }
    return sign | (uint8_t)best;
}

/* One head's 256 values as E4M3 with scale amax / 448 (1 if all zero):
 * bytes = e4m3(v * (1 / scale)) (reference store_e4m3, qwen35.cu:1055-1065). */
void orc_store_e4m3(const float* v, uint8_t* dst, float* scale) {
    float amax = 0.f;
    for (int d = 0; d < HEAD_DIM; d++) amax = fmaxf(amax, fabsf(v[d]));
    const float sc = amax > 0.f ? amax / 448.f : 1.f;
    const float inv = 1.f / sc;
    for (int d = 0; d < HEAD_DIM; d++) dst[d] = orc_f_to_e4m3(v[d] * inv);
    *scale = sc;
}

/* ---- FP8 activation copies (reference Fp8Out / quant8, fp8.cuh:29-85) ---- */
/* Byte offset of the Mx32 scale of (row r, 32-column block kb), KB blocks per
 * row (fp8.cuh:29-33). */
size_t orc_mx_index(int r, int kb, int KB) {
    const size_t kt = (size_t)(KB + 3) / 4;
    return ((size_t)(r / 128) * kt + (size_t)(kb / 4)) * 512 + (size_t)(r % 32) * 16 + (size_t)((r % 128) / 32) * 4 +
           (size_t)(kb % 4);
}
/* Smallest e with amax / 2^e <= 448, clamped to [-127, 127]; -127 for
 * amax <= 0 (fp8.cuh:35-42). */
int orc_mx_exp(float amax) {
    if (!(amax > 0.f)) return -127;
    int ex;
    const float m = frexpf(amax / 448.f, &ex);
    if (m == 0.5f) ex -= 1;
    return ex < -127 ? -127 : ex > 127 ? 127 : ex;
}
/* Rows [T][K] of f32 values y to E4M3 bytes q [T][K] and scales s: mode 1
 * f32 amax / 448 (1 if zero) per 128 columns at s[(e / 128) * rows + t];
 * mode 2 the byte 127 + orc_mx_exp(amax) per 32 columns at orc_mx_index.
 * bytes = e4m3(v * (1 / scale)) (fp8.cuh:61-85). */
void orc_fp8_rows(const float* y, int T, int K, int mode, int rows, uint8_t* q, void* s) {
    const int gw = mode == 1 ? 128 : 32;
    for (int t = 0; t < T; t++)
        for (int e = 0; e < K; e += gw) {
            const float* v = y + (size_t)t * K + e;
            float a = 0.f;
            for (int i = 0; i < gw; i++) a = fmaxf(a, fabsf(v[i]));
            float inv;
            if (mode == 1) {
                const float sc = a > 0.f ? a / 448.f : 1.f;
                inv = 1.f / sc;
                ((float*)s)[(size_t)(e / 128) * rows + t] = sc;
            } else {
                const int ex = orc_mx_exp(a);
                inv = ldexpf(1.f, -ex);
                ((uint8_t*)s)[orc_mx_index(t, e / 32, K / 32)] = (uint8_t)(127 + ex);
            }
            for (int i = 0; i < gw; i++) q[(size_t)t * K + e + i] = orc_f_to_e4m3(v[i] * inv);
        }
}
/* The gated f32 outputs y = rbf(o) / (1 + expf(-gate)) of raw attention
 * outputs o [T][Hq][256] (qwen35.cu:1290-1292, 2270-2272), gate from qkv. */
void orc_gate_rows(const float* raw, const uint16_t* qkv, int qstride, int T, int Hq, float* y) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < Hq; h++)
            for (int d = 0; d < HEAD_DIM; d++) {
                const size_t i = ((size_t)t * Hq + h) * HEAD_DIM + d;
                const float gate = orc_b2f(qkv[(size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + d]);
                y[i] = rbf(raw[i]) / (1.f + expf(-gate));
            }
}

/* attn_prep with an E4M3 cache: as orc_attn_prep, but k (normed, rotated,
 * bf16-rounded) and v (as read) go to kcache8 / vcache8 bytes with their
 * per-(slot, head) scales in kscale / vscale. */
void orc_attn_prep8(const uint16_t* qkv, int qstride, int Hq, int Hkv, const float* q_norm, const float* k_norm,
                    const int* rope, int rope_stride, int sec_h, int sec_w, const int* slot_map,
                    const float* inv_freq, float eps, int T, long num_slots, uint16_t* qout, uint8_t* kcache8,
                    uint8_t* vcache8, float* kscale, float* vscale) {
    uint16_t* kbf = (uint16_t*)malloc((size_t)(num_slots > 0 ? num_slots : 1) * Hkv * HEAD_DIM * 2);
    uint16_t* vbf = (uint16_t*)malloc((size_t)(num_slots > 0 ? num_slots : 1) * Hkv * HEAD_DIM * 2);
    orc_attn_prep(qkv, qstride, Hq, Hkv, q_norm, k_norm, rope, rope_stride, sec_h, sec_w, slot_map, inv_freq, eps, T,
                  num_slots, qout, kbf, vbf);
    for (int t = 0; t < T; t++) {
        const long slot = slot_map[t];
        if (slot < 0 || slot >= num_slots) continue;
        for (int h = 0; h < Hkv; h++) {
            const size_t at = (size_t)slot * Hkv + h;
            float kv[HEAD_DIM], vv[HEAD_DIM];
            for (int d = 0; d < HEAD_DIM; d++) {
                kv[d] = orc_b2f(kbf[at * HEAD_DIM + d]);
                vv[d] = orc_b2f(vbf[at * HEAD_DIM + d]);
            }
            orc_store_e4m3(kv, kcache8 + at * HEAD_DIM, kscale + at);
            orc_store_e4m3(vv, vcache8 + at * HEAD_DIM, vscale + at);
        }
    }
    free(kbf);
    free(vbf);
}

/* Paged decode attention over an E4M3 cache (reference attn_body<F8>,
 * qwen35.cu:1146-1309): s_j = (q * scale) . k8_j * kscale_j, p_j = e^(s_j -
 * max), out = bf16(bf16(sum p_j vscale_j v8_j / sum p_j) * sigmoid(gate));
 * softmax and sums in double. Same metadata rules as orc_attn_decode. */
int orc_attn_decode8(const uint16_t* q, const uint8_t* kcache8, const uint8_t* vcache8, const float* kscale,
                     const float* vscale, const uint16_t* qkv, int qstride, int Hq, int Hkv, const int* pos,
                     const int* tok_seq, const int* block_table, int max_blocks, int block_size, uint16_t* out,
                     float scale, const int* cu, int skip_prompts, const int* outs, int spec, int T,
                     float* o_raw) {
    const int G = Hq / Hkv;
    double* s = NULL;
    size_t cap = 0;
    for (int t = 0; t < T; t++) {
        const int sq = tok_seq[t];
        if (skip_prompts && cu[sq + 1] - cu[sq] > 1 && !is_spec(outs, spec, sq)) continue;
        const int L = pos[t] + 1;
        if ((size_t)L > cap) {
            cap = (size_t)L;
            s = (double*)realloc(s, cap * sizeof(double));
        }
        const int* bt = block_table + (size_t)sq * max_blocks;
        for (int h = 0; h < Hq; h++) {
            const int kvh = h / G;
            double mx = -INFINITY;
            for (int j = 0; j < L; j++) {
                const size_t at = ((size_t)bt[j / block_size] * block_size + j % block_size) * Hkv + kvh;
                double d = 0.0;
                for (int e = 0; e < HEAD_DIM; e++)
                    d += (double)orc_b2f(q[((size_t)t * Hq + h) * HEAD_DIM + e]) * scale *
                         orc_e4m3_to_f(kcache8[at * HEAD_DIM + e]);
                s[j] = d * kscale[at];
                if (s[j] > mx) mx = s[j];
            }
            double S = 0.0, A[HEAD_DIM];
            for (int e = 0; e < HEAD_DIM; e++) A[e] = 0.0;
            for (int j = 0; j < L; j++) {
                const size_t at = ((size_t)bt[j / block_size] * block_size + j % block_size) * Hkv + kvh;
                const double p = exp(s[j] - mx);
                S += p;
                for (int e = 0; e < HEAD_DIM; e++) A[e] += p * vscale[at] * orc_e4m3_to_f(vcache8[at * HEAD_DIM + e]);
            }
            for (int e = 0; e < HEAD_DIM; e++) {
                const float gate = orc_b2f(qkv[(size_t)t * qstride + (size_t)h * 2 * HEAD_DIM + HEAD_DIM + e]);
                out[((size_t)t * Hq + h) * HEAD_DIM + e] = gated(A[e] / S, gate);
                if (o_raw) o_raw[((size_t)t * Hq + h) * HEAD_DIM + e] = (float)(A[e] / S);
            }
        }
    }
    free(s);
    return 0;
}

/* Chunked-prefill attention over an E4M3 cache (reference attn_group8,
 * qwen35.cu:1364-1585 with F8): every K / V row is dequantised to
 * bf16(e4m3 * scale) as the reference loads its tiles (qwen35.cu:1424-1436),
 * then orc_attn_prefill. num_slots rows of Hkv heads. */
/* E4M3 rows to bf16(e4m3 * scale), the dequantisation orc_attn_prefill8
 * applies (n rows of 256, one scale per row). */
void orc_dequant_e4m3(const uint8_t* c8, const float* scale, long n, uint16_t* out) {
    for (long r = 0; r < n; r++)
        for (int d = 0; d < HEAD_DIM; d++)
            out[r * HEAD_DIM + d] = orc_f2b(orc_e4m3_to_f(c8[r * HEAD_DIM + d]) * scale[r]);
}

int orc_attn_prefill8(const uint16_t* q, const uint8_t* kcache8, const uint8_t* vcache8, const float* kscale,
                      const float* vscale, long num_slots, const uint16_t* qkv, int qstride, int Hq, int Hkv,
                      const int* pos, const int* cu, int seqs, const int* block_table, int max_blocks,
                      int block_size, uint16_t* out, float scale, int p_tile) {
    const size_t n = (size_t)num_slots * Hkv;
    uint16_t* kb = (uint16_t*)malloc(n * HEAD_DIM * 2);
    uint16_t* vb = (uint16_t*)malloc(n * HEAD_DIM * 2);
    for (size_t r = 0; r < n; r++)
        for (int d = 0; d < HEAD_DIM; d++) {
            kb[r * HEAD_DIM + d] = orc_f2b(orc_e4m3_to_f(kcache8[r * HEAD_DIM + d]) * kscale[r]);
            vb[r * HEAD_DIM + d] = orc_f2b(orc_e4m3_to_f(vcache8[r * HEAD_DIM + d]) * vscale[r]);
        }
    const int rc = orc_attn_prefill_t(q, kb, vb, qkv, qstride, Hq, Hkv, pos, cu, seqs, block_table, max_blocks,
                                      block_size, out, scale, NULL, 1, p_tile);
    free(kb);
    free(vb);
    return rc;
}

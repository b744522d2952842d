/*
 * A plain C99 consumer of libpkv.so: it includes only include/pkv.h and the
 * HIP runtime's C API, and drives the library the way an engine's FFI
 * binding would (the reference binds its kernels from Rust through a C ABI,
 * src/hip.rs:134-181, and runs them from Model::layer, src/model.rs:2340-2493).
 *
 *   pkv_c_consumer host   host entry points only (no GPU): status codes, the
 *                         block allocator, the KV manager, argument checks
 *   pkv_c_consumer gpu    an engine step sequence on device 0:
 *     1. three prompts admitted by the KV manager, their step metadata from
 *        pkv_kv_fill, K/V rows stored with pkv_append;
 *     2. pkv_gather returns every appended row byte for byte;
 *     3. one decode step per sequence (the token after its prompt): the
 *        fused pkv_attn_decode_step, pkv_append + pkv_attn_decode and
 *        pkv_attn_decode_step_noalloc give identical bytes;
 *     4. the decode output equals the last row of pkv_attn_prefill over the
 *        prompt plus that token (same keys) within the attention tolerance
 *        |got - want| <= 2e-3 + 1e-2 |want| — the reference's decode-vs-
 *        prefill check (bench-attn --check, src/main.rs:843-938);
 *     5. pkv_attn_prefill_split over the same prompts matches it within the
 *        same tolerance.
 * Prints one line per check and "ok" at the end; exits non-zero on failure.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pkv.h"

#define D 256
#define BS 16
#define HQ 16
#define HKV 4
#define NSEQ 3
#define NBLOCKS 512

static int failures = 0;

static void check(int cond, const char* what) {
    printf("%s: %s\n", cond ? "pass" : "FAIL", what);
    fflush(stdout);
    if (!cond) failures++;
}

#define HIP_OK(x)                                                               \
    do {                                                                        \
        hipError_t e_ = (x);                                                    \
        if (e_ != hipSuccess) {                                                 \
            printf("FAIL: %s -> hip error %d\n", #x, (int)e_);                  \
            exit(2);                                                            \
        }                                                                       \
    } while (0)
#define PKV_OK_(x)                                                              \
    do {                                                                        \
        int s_ = (x);                                                           \
        if (s_ != PKV_OK) {                                                     \
            printf("FAIL: %s -> %d (%s)\n", #x, s_, pkv_strerror(s_));          \
            exit(2);                                                            \
        }                                                                       \
    } while (0)

/* xorshift64*: seeded, portable */
static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static double urand(void) {
    rng_state ^= rng_state >> 12;
    rng_state ^= rng_state << 25;
    rng_state ^= rng_state >> 27;
    return (double)((rng_state * 2685821657736338717ull) >> 11) / 9007199254740992.0;
}
/* bf16 bits of a float (round to nearest even; the values here are finite) */
static uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFF + ((u >> 16) & 1);
    return (uint16_t)(u >> 16);
}
static float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static void fill_bf16(uint16_t* x, size_t n, float amp) {
    for (size_t i = 0; i < n; i++) x[i] = f2bf((float)((urand() * 2.0 - 1.0) * amp));
}

static int run_host(void) {
    check(pkv_version() >= 1, "pkv_version");
    check(strlen(pkv_strerror(PKV_ERR_UNSUPPORTED)) > 0, "pkv_strerror names 801");

    /* block allocator: free list [n-1 .. 0]; a take splits off its tail
     * (sched.rs:515, 801-807), so a fresh pool's first 8 are 7, 6, .., 0 */
    pkv_pool* pool = pkv_pool_create(64);
    uint32_t ids[8];
    PKV_OK_(pkv_pool_take(pool, 8, ids));
    check(ids[0] == 7 && ids[7] == 0 && pkv_pool_free_count(pool) == 56, "pool take: ids 7..0, 56 free");
    PKV_OK_(pkv_pool_ref(pool, ids, 1));
    check(pkv_pool_refs(pool, ids[0]) == 2, "pool ref");
    PKV_OK_(pkv_pool_unref(pool, ids, 8));
    check(pkv_pool_free_count(pool) == 63 && pkv_pool_refs(pool, ids[0]) == 1, "pool unref");
    check(pkv_pool_take(pool, 64, ids) == PKV_ERR_NO_BLOCKS, "pool exhaustion is PKV_ERR_NO_BLOCKS");
    pkv_pool_destroy(pool);

    /* KV manager: admission reserves prompt + max_new, a cached 64-token unit is shared */
    pkv_kv* kv = pkv_kv_create(64, BS, 0);
    uint32_t prompt[130];
    for (int i = 0; i < 130; i++) prompt[i] = 1000 + i;
    int s0, s1;
    int64_t cached = -1;
    PKV_OK_(pkv_kv_admit(kv, 0, prompt, 130, 30, 1, &s0, &cached));
    check(cached == 0 && pkv_pool_free_count(pkv_kv_pool(kv)) == 64 - 10, "admit reserves ceil(160 / 16) blocks");
    PKV_OK_(pkv_kv_set_len(kv, s0, 130));
    PKV_OK_(pkv_kv_cache_add(kv, s0, 0, prompt, 128));
    PKV_OK_(pkv_kv_admit(kv, 0, prompt, 130, 30, 1, &s1, &cached));
    uint32_t b0[16], b1[16];
    const int64_t n0 = pkv_kv_blocks(kv, s0, b0, 16), n1 = pkv_kv_blocks(kv, s1, b1, 16);
    check(cached == 128 && n0 == 10 && n1 == 10 && memcmp(b0, b1, 8 * sizeof(uint32_t)) == 0 &&
              pkv_pool_refs(pkv_kv_pool(kv), b0[0]) == 3,
          "a cached 128-token prefix shares 8 pages (refs 3: two tables + the entry)");
    PKV_OK_(pkv_kv_release(kv, s0));
    PKV_OK_(pkv_kv_release(kv, s1));
    check(pkv_kv_evict_one(kv) == 1 && pkv_pool_free_count(pkv_kv_pool(kv)) == 64, "release + evict frees all");
    pkv_kv_destroy(kv);

    /* argument checks happen before any device work */
    check(pkv_attn_decode(NULL, NULL, NULL, NULL, 0, HQ, HKV, NULL, NULL, NULL, 1, 32, NULL, 1.f, NULL, 0, NULL, 1, 1,
                          1, NULL, 0, NULL) == PKV_ERR_UNSUPPORTED,
          "decode with block size 32 is PKV_ERR_UNSUPPORTED");
    check(pkv_attn_decode(NULL, NULL, NULL, NULL, 0, HQ, HKV, NULL, NULL, NULL, 1, BS, NULL, 1.f, NULL, 0, NULL, 1, 1,
                          1, NULL, 0, NULL) == PKV_ERR_INVALID,
          "decode with null buffers is PKV_ERR_INVALID");
    size_t ws = 0;
    check(pkv_attn_decode_workspace(-1, HQ, &ws) == PKV_ERR_INVALID, "workspace of T < 0 is PKV_ERR_INVALID");
    return failures;
}

static void* dmalloc(size_t n) {
    void* p = NULL;
    HIP_OK(hipMalloc(&p, n));
    return p;
}
static void* dcopy(const void* h, size_t n) {
    void* p = dmalloc(n);
    HIP_OK(hipMemcpy(p, h, n, hipMemcpyHostToDevice));
    return p;
}

static int run_gpu(void) {
    const int L[NSEQ] = {700, 101, 1500};
    const int qstride = (2 * HQ + 2 * HKV) * D; /* q | gate per head, then K, V (elements) */
    const int max_blocks = 128;
    const float scale = 1.0f / 16.0f;
    const int64_t nslots = (int64_t)NBLOCKS * BS;
    const size_t pool_bytes = (size_t)nslots * HKV * D * 2;

    pkv_kv* kv = pkv_kv_create(NBLOCKS, BS, 0);
    int seq[NSEQ];
    for (int s = 0; s < NSEQ; s++) {
        uint32_t* p = malloc(sizeof(uint32_t) * L[s]);
        for (int i = 0; i < L[s]; i++) p[i] = (uint32_t)(s * 100000 + i);
        int64_t cached;
        PKV_OK_(pkv_kv_admit(kv, 0, p, L[s], 8, 0, &seq[s], &cached));
        free(p);
    }

    void* kc = dmalloc(pool_bytes);
    void* vc = dmalloc(pool_bytes);
    HIP_OK(hipMemset(kc, 0, pool_bytes));
    HIP_OK(hipMemset(vc, 0, pool_bytes));

    /* 1. prompt step: metadata from the manager, K/V rows appended */
    int T = 0;
    for (int s = 0; s < NSEQ; s++) T += L[s];
    int32_t *pos = malloc(4 * T), *slot = malloc(4 * T), *tseq = malloc(4 * T), cu[NSEQ + 1], lim[NSEQ];
    int32_t* bt = calloc((size_t)NSEQ * max_blocks, 4);
    PKV_OK_(pkv_kv_fill(kv, seq, L, NSEQ, T, max_blocks, pos, slot, tseq, cu, lim, bt));
    uint16_t* qkv = malloc((size_t)T * qstride * 2);
    fill_bf16(qkv, (size_t)T * qstride, 1.0f);
    uint16_t* q = malloc((size_t)T * HQ * D * 2);
    fill_bf16(q, (size_t)T * HQ * D, 0.5f);
    void* qkv_d = dcopy(qkv, (size_t)T * qstride * 2);
    void* slot_d = dcopy(slot, 4 * (size_t)T);
    const uint16_t* k_rows = (const uint16_t*)qkv_d + 2 * HQ * D;
    const uint16_t* v_rows = k_rows + HKV * D;
    PKV_OK_(pkv_append(k_rows, v_rows, (int64_t)qstride * 2, slot_d, T, HKV, D * 2, kc, vc, nslots, NULL));

    /* 2. gather returns the appended rows */
    int gather_ok = 1;
    for (int s = 0; s < NSEQ; s++) {
        const size_t row = (size_t)HKV * D * 2;
        void* bt_row = dcopy(bt + (size_t)s * max_blocks, 4 * (size_t)max_blocks);
        void* ko = dmalloc(row * L[s]);
        void* vo = dmalloc(row * L[s]);
        PKV_OK_(pkv_gather(kc, vc, bt_row, L[s], BS, HKV, D * 2, NBLOCKS, ko, vo, NULL));
        uint8_t* kh = malloc(row * L[s]);
        uint8_t* vh = malloc(row * L[s]);
        HIP_OK(hipMemcpy(kh, ko, row * L[s], hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(vh, vo, row * L[s], hipMemcpyDeviceToHost));
        for (int j = 0; j < L[s]; j++) {
            const uint16_t* src = qkv + (size_t)(cu[s] + j) * qstride + 2 * HQ * D;
            gather_ok &= memcmp(kh + row * j, src, row) == 0 && memcmp(vh + row * j, src + HKV * D, row) == 0;
        }
        free(kh);
        free(vh);
        HIP_OK(hipFree(bt_row));
        HIP_OK(hipFree(ko));
        HIP_OK(hipFree(vo));
    }
    check(gather_ok, "gather(append(rows)) == rows, byte for byte, 3 sequences through the manager's tables");
    for (int s = 0; s < NSEQ; s++) PKV_OK_(pkv_kv_set_len(kv, seq[s], L[s]));

    /* 3. decode step: one new token per sequence at position L[s] */
    const int one[NSEQ] = {1, 1, 1};
    int32_t dpos[NSEQ], dslot[NSEQ], dts[NSEQ], dcu[NSEQ + 1], dlim[NSEQ];
    int32_t* dbt = calloc((size_t)NSEQ * max_blocks, 4);
    PKV_OK_(pkv_kv_fill(kv, seq, one, NSEQ, NSEQ, max_blocks, dpos, dslot, dts, dcu, dlim, dbt));
    check(dpos[0] == L[0] && dpos[2] == L[2] && memcmp(dbt, bt, 4 * (size_t)NSEQ * max_blocks) == 0,
          "decode metadata: positions after the prompts, same block tables");
    uint16_t* dqkv = malloc((size_t)NSEQ * qstride * 2);
    fill_bf16(dqkv, (size_t)NSEQ * qstride, 1.0f);
    uint16_t* dq = malloc((size_t)NSEQ * HQ * D * 2);
    fill_bf16(dq, (size_t)NSEQ * HQ * D, 0.5f);
    void* dqkv_d = dcopy(dqkv, (size_t)NSEQ * qstride * 2);
    void* dq_d = dcopy(dq, (size_t)NSEQ * HQ * D * 2);
    void* dpos_d = dcopy(dpos, sizeof dpos);
    void* dslot_d = dcopy(dslot, sizeof dslot);
    void* dts_d = dcopy(dts, sizeof dts);
    void* dcu_d = dcopy(dcu, sizeof dcu);
    void* dbt_d = dcopy(dbt, 4 * (size_t)NSEQ * max_blocks);
    const uint16_t* dk_rows = (const uint16_t*)dqkv_d + 2 * HQ * D;
    const uint16_t* dv_rows = dk_rows + HKV * D;
    size_t wsb = 0;
    PKV_OK_(pkv_attn_decode_workspace(NSEQ, HQ, &wsb));
    void* ws = dmalloc(wsb);
    const size_t out_bytes = (size_t)NSEQ * HQ * D * 2;
    void* out_f = dmalloc(out_bytes);
    void* out_u = dmalloc(out_bytes);
    void* out_n = dmalloc(out_bytes);
    PKV_OK_(pkv_attn_decode_step(dk_rows, dv_rows, (int64_t)qstride * 2, dslot_d, dq_d, kc, vc, dqkv_d, qstride, HQ,
                                 HKV, dpos_d, dts_d, dbt_d, max_blocks, BS, out_f, scale, dcu_d, 0, NULL, 1, NSEQ,
                                 NBLOCKS, ws, wsb, NULL));
    /* the same step unfused (re-appending the same rows leaves the cache as it is) */
    PKV_OK_(pkv_append(dk_rows, dv_rows, (int64_t)qstride * 2, dslot_d, NSEQ, HKV, D * 2, kc, vc, nslots, NULL));
    PKV_OK_(pkv_attn_decode(dq_d, kc, vc, dqkv_d, qstride, HQ, HKV, dpos_d, dts_d, dbt_d, max_blocks, BS, out_u, scale,
                            dcu_d, 0, NULL, 1, NSEQ, NBLOCKS, ws, wsb, NULL));
    PKV_OK_(pkv_attn_decode_step_noalloc(dk_rows, dv_rows, (int64_t)qstride * 2, dslot_d, dq_d, kc, vc, dqkv_d,
                                         qstride, HQ, HKV, dpos_d, dts_d, dbt_d, max_blocks, BS, out_n, scale, dcu_d, 0,
                                         NULL, 1, NSEQ, NBLOCKS, NULL));
    HIP_OK(hipDeviceSynchronize());
    uint16_t *hf = malloc(out_bytes), *hu = malloc(out_bytes), *hn = malloc(out_bytes);
    HIP_OK(hipMemcpy(hf, out_f, out_bytes, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hu, out_u, out_bytes, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hn, out_n, out_bytes, hipMemcpyDeviceToHost));
    check(memcmp(hf, hu, out_bytes) == 0, "fused decode step == append + decode, bit for bit");
    check(memcmp(hf, hn, out_bytes) == 0, "decode_step_noalloc == decode_step, bit for bit");

    /* 4. prefill over prompt + new token: its last row per sequence is the decode row */
    const int T2 = T + NSEQ;
    int32_t *pos2 = malloc(4 * T2), cu2[NSEQ + 1];
    uint16_t* q2 = malloc((size_t)T2 * HQ * D * 2);
    uint16_t* qkv2 = malloc((size_t)T2 * qstride * 2);
    int r = 0;
    cu2[0] = 0;
    for (int s = 0; s < NSEQ; s++) {
        memcpy(q2 + (size_t)r * HQ * D, q + (size_t)cu[s] * HQ * D, (size_t)L[s] * HQ * D * 2);
        memcpy(qkv2 + (size_t)r * qstride, qkv + (size_t)cu[s] * qstride, (size_t)L[s] * qstride * 2);
        memcpy(q2 + (size_t)(r + L[s]) * HQ * D, dq + (size_t)s * HQ * D, (size_t)HQ * D * 2);
        memcpy(qkv2 + (size_t)(r + L[s]) * qstride, dqkv + (size_t)s * qstride, (size_t)qstride * 2);
        for (int j = 0; j <= L[s]; j++) pos2[r + j] = j;
        r += L[s] + 1;
        cu2[s + 1] = r;
    }
    void* q2_d = dcopy(q2, (size_t)T2 * HQ * D * 2);
    void* qkv2_d = dcopy(qkv2, (size_t)T2 * qstride * 2);
    void* pos2_d = dcopy(pos2, 4 * (size_t)T2);
    void* cu2_d = dcopy(cu2, sizeof cu2);
    void* out_p = dmalloc((size_t)T2 * HQ * D * 2);
    PKV_OK_(pkv_attn_prefill(q2_d, kc, vc, qkv2_d, qstride, HQ, HKV, pos2_d, cu2_d, NSEQ, dbt_d, max_blocks, BS, out_p,
                             scale, NULL, 1, T2, NBLOCKS, NULL));
    HIP_OK(hipDeviceSynchronize());
    uint16_t* hp = malloc((size_t)T2 * HQ * D * 2);
    HIP_OK(hipMemcpy(hp, out_p, (size_t)T2 * HQ * D * 2, hipMemcpyDeviceToHost));
    int within = 1;
    double worst = 0;
    for (int s = 0; s < NSEQ; s++) {
        const uint16_t* pr = hp + (size_t)(cu2[s + 1] - 1) * HQ * D;
        const uint16_t* dr = hf + (size_t)s * HQ * D;
        for (int i = 0; i < HQ * D; i++) {
            const double want = bf2f(pr[i]), got = bf2f(dr[i]), err = fabs(got - want);
            if (!(err <= 2e-3 + 1e-2 * fabs(want))) within = 0;
            if (err > worst) worst = err;
        }
    }
    printf("decode vs prefill last rows: max |diff| %.3g\n", worst);
    check(within, "decode row == prefill's last row within 2e-3 + 1e-2 |want|");

    /* 5. the same prompts with split keys (this grid is smaller than the CUs) */
    size_t pws = 0;
    PKV_OK_(pkv_attn_prefill_workspace(T2, HQ, HKV, NSEQ, &pws));
    check(pws > 0, "pkv_attn_prefill_workspace: room for the split records");
    void* pws_d = dmalloc(pws);
    void* out_s = dmalloc((size_t)T2 * HQ * D * 2);
    PKV_OK_(pkv_attn_prefill_split(q2_d, kc, vc, qkv2_d, qstride, HQ, HKV, pos2_d, cu2_d, NSEQ, dbt_d, max_blocks, BS,
                                   out_s, scale, NULL, 1, T2, NBLOCKS, pws_d, pws, NULL));
    HIP_OK(hipDeviceSynchronize());
    uint16_t* hs = malloc((size_t)T2 * HQ * D * 2);
    HIP_OK(hipMemcpy(hs, out_s, (size_t)T2 * HQ * D * 2, hipMemcpyDeviceToHost));
    int split_ok = 1;
    for (size_t i = 0; i < (size_t)T2 * HQ * D; i++) {
        const double want = bf2f(hp[i]), got = bf2f(hs[i]);
        if (!(fabs(got - want) <= 2e-3 + 1e-2 * fabs(want))) split_ok = 0;
    }
    check(split_ok, "pkv_attn_prefill_split == pkv_attn_prefill within 2e-3 + 1e-2 |want|, every row");
    free(hs);
    HIP_OK(hipFree(pws_d));
    HIP_OK(hipFree(out_s));

    free(pos); free(slot); free(tseq); free(bt); free(qkv); free(q); free(dbt); free(dqkv); free(dq);
    free(hf); free(hu); free(hn); free(pos2); free(q2); free(qkv2); free(hp);
    void* dev[] = {kc, vc, qkv_d, slot_d, dqkv_d, dq_d, dpos_d, dslot_d, dts_d, dcu_d, dbt_d, ws, out_f, out_u,
                   out_n, q2_d, qkv2_d, pos2_d, cu2_d, out_p};
    for (size_t i = 0; i < sizeof dev / sizeof dev[0]; i++) HIP_OK(hipFree(dev[i]));
    pkv_kv_destroy(kv);
    return failures;
}

int main(int argc, char** argv) {
    if (argc != 2 || (strcmp(argv[1], "host") != 0 && strcmp(argv[1], "gpu") != 0)) {
        fprintf(stderr, "usage: %s host|gpu\n", argv[0]);
        return 2;
    }
    const int f = strcmp(argv[1], "host") == 0 ? run_host() : run_gpu();
    printf("%s\n", f ? "FAILED" : "ok");
    return f ? 1 : 0;
}

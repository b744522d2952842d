/*
 * pkv — MI355X (gfx950) paged KV cache: the C-ABI boundary of libpkv.so.
 *
 * Every entry point returns an int status: 0 on success, a HIP error code
 * (hipError_t, passed through) when a HIP call fails, PKV_ERR_INVALID for
 * arguments that fail validation, PKV_ERR_UNSUPPORTED (801, the reference's
 * CUDA_ERROR_NOT_SUPPORTED convention, reference src/hip.rs:17-18, 61-66) for
 * shapes the kernels do not implement. Nothing aborts. pkv_strerror() names
 * a status.
 *
 * Device entry points are asynchronous on the caller's stream (`stream` is a
 * hipStream_t; NULL = the null stream), never allocate and never synchronize,
 * so they can be captured into HIP graphs (the reference's forward pass makes
 * the same promise, model.rs:1739-1741). Device pointers are plain device
 * addresses; the caller owns every buffer (reference gpu.rs:46-58).
 *
 * Cache layout (reference model.rs:1166-1197): one K and one V pool per
 * attention layer of [pages * block_size][Hkv][head_dim] elements; the slot
 * of key position p of a sequence is block_table[p / block_size] *
 * block_size + p % block_size (reference sched.rs:1113-1114).
 *
 * Host allocator entry points (pkv_pool_*, pkv_kv_*) are single-threaded like
 * the reference's Scheduler, which owns them on the engine thread.
 */
#ifndef PKV_H
#define PKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_OK 0
#define PKV_ERR_INVALID 1      /* same value as hipErrorInvalidValue */
#define PKV_ERR_UNSUPPORTED 801
#define PKV_ERR_NO_BLOCKS 802  /* the pool cannot satisfy a request */

const char* pkv_strerror(int status);
/* ABI version: bumps when a signature changes. */
int pkv_version(void);

/* ---------------------------------------------------------------------------
 * Device: data movement (byte-exact)
 * ------------------------------------------------------------------------- */

/* KV append: for each token t < T with slot = slot_map[t] in [0, num_slots),
 * copies the Hkv * head_bytes bytes at k_rows + t * row_stride to the K pool
 * slot row and likewise V. Slots < 0 are padding and skipped.
 * Replaces the cache stores of the reference's attn_prep kernel
 * (src/kernels/qwen35.cu:1076-1128, launched at src/model.rs:2340-2365); the
 * rows are the already normed/rotated K and the V of the qkv projection row,
 * so for the reference's qkv layout k_rows = qkv + Hq * 512 elements,
 * v_rows = k_rows + Hkv * 256 elements, row_stride = qstride * 2 bytes. */
int pkv_append(const void* k_rows, const void* v_rows, int64_t row_stride, const int32_t* slot_map, int T, int Hkv,
               int head_bytes, void* kcache, void* vcache, int64_t num_slots, void* stream);

/* Gather: k_out[j] = K pool slot row of key j, j < L, through one block-table
 * row (bt_row, device); likewise V. Rows are Hkv * head_bytes bytes.
 * The reference reads its cache this way inside every attention kernel
 * (qwen35.cu:1203-1205, amd/attn_decode.cuh:56-74); it is a separate entry
 * point here for checks and for exporting a sequence's KV. */
int pkv_gather(const void* kcache, const void* vcache, const int32_t* bt_row, int L, int block_size, int Hkv,
               int head_bytes, int64_t num_blocks, void* k_out, void* v_out, void* stream);

/* Single-query attention over dense f32 K/V rows, for checks of gathered
 * sequences (the reference's CPU plumbing configuration: gather to
 * [len][Hkv][D] f32, attention of the last token's query, compared in
 * fp64). For s < S: rows off[s] .. off[s] + len[s] - 1 of k / v ([rows][Hkv]
 * [D] f32, device), query q[s] ([Hq][D] f32), out[s][h] ([Hq][D] f32) =
 * softmax_j(scale * q[s][h] . k_j) . v_j with kv head h / (Hq / Hkv), ungated.
 * D <= 256. No reference kernel (the reference checks this case on the
 * CPU). off / len are device arrays. */
int pkv_attn_dense_f32(const float* q, const float* k, const float* v, const int32_t* off, const int32_t* len,
                       int S, int Hq, int Hkv, int D, float scale, float* out, void* stream);

/* Page copy (copy-on-write): for i < n, page dst[i] := page src[i] in both
 * pools; page_bytes = block_size * Hkv * head_bytes (a multiple of 16).
 * src/dst are device arrays. Destinations must be distinct and not sources.
 * No reference counterpart: the reference never writes into a shared page
 * (prefix entries cover whole 64-token units, sched.rs:322, 1044-1067); this
 * is the device half of pkv_kv_prepare_append's copy-on-write. */
int pkv_page_copy(void* kcache, void* vcache, const int32_t* src, const int32_t* dst, int n, int64_t page_bytes,
                  int64_t num_blocks, void* stream);

/* Draft-pass metadata: replaces mtp_next (qwen35.cu:2633-2650, launched per
 * MTP draft pass k >= 1). For sequence s < S with step row rows[s]:
 * dpos[s] = pos[rows[s]] + k; dslot[s] = block_table[s * max_blocks +
 * dpos / block_size] * block_size + dpos % block_size while dpos[s] <=
 * limits[s], else -1 (also -1 when the page index reaches max_blocks);
 * drope[axis * S + s] = rope[axis * rope_stride + rows[s]] + k for the 3
 * rotary axes. All arrays are device int32. */
int pkv_mtp_next(const int32_t* rows, const int32_t* pos, const int32_t* rope, int rope_stride,
                 const int32_t* block_table, int max_blocks, int block_size, const int32_t* limits, int k,
                 int32_t* dpos, int32_t* dslot, int32_t* drope, int S, void* stream);

/* ---------------------------------------------------------------------------
 * Device: paged decode attention (bf16, head_dim 256, block_size 16,
 * G = Hq / Hkv in {1, 2, 4, 6, 8})
 * ------------------------------------------------------------------------- */

/* Workspace bytes pkv_attn_decode needs for T tokens and Hq query heads on
 * the current device. */
int pkv_attn_decode_workspace(int T, int Hq, size_t* bytes);

/* Paged decode attention with the reference's semantics and arguments
 * (attn_paged_g<G> + attn_merge, src/kernels/qwen35.cu:1313-1334 and
 * 2245-2279, launched at src/model.rs:2366-2437; AMD body
 * src/kernels/amd/attn_decode.cuh:12-183): for each token t < T that is a
 * decode token (prompt rows are skipped when skip_prompts, as the reference
 * leaves them to flash attention), each query head h, attention of
 * q[t][h] * scale over keys 0..pos[t] of sequence tok_seq[t] through
 * block_table[tok_seq[t] * max_blocks ..], then
 * out[t][h] = bf16(bf16(A / S) * sigmoid(gate)), gate = qkv[t * qstride +
 * h * 512 + 256 ..]. Same pointer meanings as the reference; kscale/vscale
 * (E4M3 cache) are pkv_attn_decode_e4m3's, fq/fs/fmode/frows (FP8 output
 * copies) come from pkv_attn_fp8_next.
 * The key-range split is the library's own (the reference's part/min_chunk
 * pair is replaced by `workspace`, of pkv_attn_decode_workspace bytes).
 * num_blocks bounds page ids (ids outside the pool are clamped, never read
 * out of bounds). G = Hq / Hkv is one of the reference's groups 1, 2, 4, 6, 8
 * (qwen35.cu:1330-1334); for G other than 4 the call runs the verify kernels
 * (one row per segment) and `cu` is required. Returns PKV_ERR_UNSUPPORTED for
 * another G or block_size != 16. */
int pkv_attn_decode(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                    int Hkv, const int32_t* pos, const int32_t* tok_seq, const int32_t* block_table, int max_blocks,
                    int block_size, void* out, float scale, const int32_t* cu, int skip_prompts,
                    const int32_t* outs, int spec, int T, int64_t num_blocks, void* workspace,
                    size_t workspace_bytes, void* stream);

/* The two launches of pkv_attn_decode, for callers that time or schedule
 * them apart (the reference likewise launches attn_paged_g<G> and then
 * attn_merge, src/model.rs:2371-2437): _split runs the key-range kernel,
 * _merge combines its partials and gates. Same arguments; _merge must follow
 * _split on the same stream with the same workspace and metadata. */
int pkv_attn_decode_split(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                          int Hkv, const int32_t* pos, const int32_t* tok_seq, const int32_t* block_table,
                          int max_blocks, int block_size, void* out, float scale, const int32_t* cu,
                          int skip_prompts, const int32_t* outs, int spec, int T, int64_t num_blocks,
                          void* workspace, size_t workspace_bytes, void* stream);
int pkv_attn_decode_merge(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                          int Hkv, const int32_t* pos, const int32_t* tok_seq, const int32_t* block_table,
                          int max_blocks, int block_size, void* out, float scale, const int32_t* cu,
                          int skip_prompts, const int32_t* outs, int spec, int T, int64_t num_blocks,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Fused decode step: KV append + paged decode attention in two launches
 * (the key-range kernel appends the step's rows itself, then the merge).
 * Same result as pkv_append(k_rows, v_rows, row_stride, slot_map, T, Hkv,
 * 512, kcache, vcache, num_blocks * 16) followed by pkv_attn_decode(...) —
 * the reference's attn_prep cache stores followed by attn_paged_g<G> +
 * attn_merge (src/model.rs:2340-2437) — provided the step's metadata is the
 * scheduler's (src/sched.rs:1105-1115): each sequence's tokens of the step
 * are consecutive rows cu[s] .. cu[s+1]-1 at consecutive positions and
 * slot_map[t] is the slot of pos[t]. Keys at positions the step itself feeds
 * are read from k_rows/v_rows; the step's rows are written to the pools.
 * `cu` is required; G = Hq / Hkv in {1, 2, 4, 6, 8} (G = 4: the decode
 * key-range kernel; other groups: the verify kernel, rows of a sequence in
 * segments as pkv_attn_verify, with the append fused in). row_stride is in
 * bytes (a multiple of 16). No
 * reference counterpart as one call: it saves the append launch. */
int pkv_attn_decode_step(const void* k_rows, const void* v_rows, int64_t row_stride, const int32_t* slot_map,
                         const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                         int Hkv, const int32_t* pos, const int32_t* tok_seq, const int32_t* block_table,
                         int max_blocks, int block_size, void* out, float scale, const int32_t* cu,
                         int skip_prompts, const int32_t* outs, int spec, int T, int64_t num_blocks,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the device array pkv_attn_decode_step_noalloc uses as its
 * workspace (one copy per GPU, held until the process ends). */
#define PKV_NOALLOC_SCRATCH_BYTES (16u << 20)

/* pkv_attn_decode_step without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). It has no counterpart in the reference. The workspace is a
 * file-scope device array of PKV_NOALLOC_SCRATCH_BYTES per GPU; the call
 * allocates nothing (no hipMalloc / hipFree, no allocating library routine).
 * Same arguments and results as pkv_attn_decode_step otherwise. Returns
 * PKV_ERR_UNSUPPORTED when the step's workspace exceeds the array:
 * 256-aligned (T + 2) int32 offsets, then (T + R) * Hq * n partial rows of
 * 2 + 256 f32 (R = key ranges = CUs x pkv_attn_decode_config's wg_per_cu;
 * n = 1 for G = 4, else the verify kernel's rows per segment: 4 for G <= 4,
 * 2 for G = 6 or 8); on a 256-CU device T <= 759 at Hq = 16 (G = 4) and
 * T <= 82 at Hq = 24 (G = 6). Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (different streams, or host threads) race; calls in
 * order on one stream are safe. */
int pkv_attn_decode_step_noalloc(const void* k_rows, const void* v_rows, int64_t row_stride, const int32_t* slot_map,
                                 const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride,
                                 int Hq, int Hkv, const int32_t* pos, const int32_t* tok_seq,
                                 const int32_t* block_table, int max_blocks, int block_size, void* out, float scale,
                                 const int32_t* cu, int skip_prompts, const int32_t* outs, int spec, int T,
                                 int64_t num_blocks, void* stream);

/* Draft-verify attention: the same results as pkv_attn_decode (every
 * decode row t attends keys 0..pos[t] of its sequence, gated output), for
 * batches whose sequences feed several rows at once — the reference's
 * speculative rows (is_spec, src/kernels/qwen35.cu:94-100), which its
 * attn_paged_g<G> serves one token per block, each re-reading the
 * sequence's pages (launched at src/model.rs:2366-2437). Here up to 4
 * (G <= 4) or 2 (G = 6, 8) consecutive rows of a sequence share one pass
 * over its pages. `cu` is
 * required and each sequence's rows must be consecutive (cu[s] ..
 * cu[s+1]-1, as Scheduler::fill writes them, src/sched.rs:1105-1115).
 * Segments hold 4 rows for G <= 4 and 2 rows for G = 6 or 8 (the 16 MFMA
 * columns are rows x query heads).
 * Workspace: pkv_attn_verify_workspace bytes. Shapes as pkv_attn_decode. */
int pkv_attn_verify_workspace(int T, int Hq, size_t* bytes);
int pkv_attn_verify(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                    int Hkv, const int32_t* pos, const int32_t* tok_seq, const int32_t* block_table, int max_blocks,
                    int block_size, void* out, float scale, const int32_t* cu, int skip_prompts,
                    const int32_t* outs, int spec, int T, int64_t num_blocks, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Decode attention over an E4M3 cache: the reference's attn_paged8_g<G>
 * + attn_merge (src/kernels/qwen35.cu:1313-1334 with F8, kscale / vscale
 * given; launched as attn_paged_g<G> at src/model.rs:2366-2437) with the
 * arguments of pkv_attn_decode plus the scales. kcache / vcache hold E4M3
 * bytes [blocks * 16][Hkv][256] and kscale / vscale one f32 per [slot][kv
 * head] (written by pkv_attn_prep with scales): s_j = (q * scale) . k_j *
 * kscale_j, out = bf16(bf16(sum_j p_j vscale_j v_j / sum_j p_j) *
 * sigmoid(gate)). Rows and groups as pkv_attn_decode (`cu` only with
 * skip_prompts, for every G); workspace: pkv_attn_decode_workspace bytes. */
int pkv_attn_decode_e4m3(const void* q, const void* kcache, const void* vcache, const float* kscale,
                         const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                         const int32_t* tok_seq, const int32_t* block_table, int max_blocks, int block_size,
                         void* out, float scale, const int32_t* cu, int skip_prompts, const int32_t* outs, int spec,
                         int T, int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream);

/* The same over an E4M3 cache with the rows of a sequence grouped as in
 * pkv_attn_verify (`cu` required; workspace: pkv_attn_verify_workspace):
 * the reference's attn_paged8_g<G> for speculative rows. */
int pkv_attn_verify_e4m3(const void* q, const void* kcache, const void* vcache, const float* kscale,
                         const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                         const int32_t* tok_seq, const int32_t* block_table, int max_blocks, int block_size,
                         void* out, float scale, const int32_t* cu, int skip_prompts, const int32_t* outs, int spec,
                         int T, int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream);

/* Measurement: the next key-range kernel this thread launches (the dominant
 * kernel of pkv_attn_decode / _split / _step / _e4m3 / pkv_attn_verify) records start_event when it
 * starts executing and stop_event when it ends (hipExtLaunchKernelGGL), so
 * hipEventElapsedTime gives its own duration without dispatch gaps, like the
 * reference's Gpu::time_us event timing (src/gpu.rs:1461-1510). Events are
 * hipEvent_t created with timing enabled; NULL clears. */
int pkv_time_next_range_kernel(void* start_event, void* stop_event);
/* The same for the next pkv_attn_prefill kernel of this thread. */
int pkv_time_next_prefill_kernel(void* start_event, void* stop_event);

/* FP8 output copies for this thread's next decode / verify call (the
 * reference's fq / fs / fmode / frows arguments of attn_paged_g<G> and
 * attn_merge, written for its --fp8 output projection: Fp8Out / quant8,
 * src/kernels/fp8.cuh:29-85, qwen35.cu:1297-1307, 2269-2279). With fmode 1
 * (Block128) or 2 (Mx32) the next pkv_attn_decode, _merge, _step, _verify,
 * _decode_e4m3, _verify_e4m3 or _step_noalloc call also writes every row's
 * gated f32 outputs as E4M3 bytes fq[t][Hq * 256] with scales fs: mode 1 one
 * f32 amax / 448 per 128 columns at fs[(col / 128) * frows + t], mode 2 one
 * E8M0 byte per 32 columns in the 128-row x 4-block tiles of MXFP8. Rows the
 * call skips get none. frows (the engine's row capacity) must be >= T. The
 * request is cleared by the next call that runs the merge (a _split call
 * keeps it for its _merge), also when that call fails its argument checks
 * and writes nothing; fmode 0 clears it. While it is set, every row is
 * finished by the merge kernel (the key-range kernel leaves a partial record
 * for every piece), which costs a little time. */
int pkv_attn_fp8_next(void* fq, void* fs, int fmode, int frows);

/* Tuning: key-range workgroups per CU (default 1) and fewest keys per range
 * (default 32). Process-wide; takes effect for later calls (workspace sizes
 * follow). */
int pkv_attn_decode_config(int wg_per_cu, int min_range);


/* ---------------------------------------------------------------------------
 * Device: chunked-prefill attention over paged context (MFMA bf16)
 * ------------------------------------------------------------------------- */

/* Causal attention for prompt rows with the reference's semantics and
 * arguments (attn_mfma_g<G>_t<NT> / attn_flash_group: ATTN_FLASH_ARGS at
 * src/kernels/qwen35.cu:1351-1356, amd/attention.cuh:12-136, launched at
 * src/model.rs:2438-2493): for every sequence s < seqs with more than one
 * token in cu[s] .. cu[s+1]-1 that is not verifying drafts (outs), each of
 * its tokens t attends over keys 0 .. pos[t] of its pages (positions within
 * a sequence's chunk are consecutive), q scaled by scale * log2(e) and
 * rounded to bf16, exp2 softmax, P rounded to bf16 for P.V, output
 * bf16(bf16(O / l) * sigmoid(gate)). Other rows are left untouched. The
 * chunk's own K/V must already be in the cache (pkv_append first). T is the
 * number of token rows. bf16, head_dim 256, G = Hq / Hkv in {1, 2, 4, 6, 8}
 * (PKV_ERR_UNSUPPORTED otherwise), block size a power of two. kscale/vscale
 * (E4M3 cache) are not part of this path. */
int pkv_attn_prefill(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                     int Hkv, const int32_t* pos, const int32_t* cu, int seqs, const int32_t* block_table,
                     int max_blocks, int block_size, void* out, float scale, const int32_t* outs, int spec, int T,
                     int64_t num_blocks, void* stream);

/* The same with a workspace, for prompts whose query tiles would leave CUs
 * idle (one sequence's prompt chunk of a few thousand tokens, above all
 * after a long context, also beside many one-token decode rows): the kernel
 * counts the prompt's query tiles from cu and, when their workgroups do not
 * fill the CUs, splits each tile's keys over max(2, CUs / workgroups)
 * workgroups (ranges of at least 128 keys), which leave (max, sum, weighted
 * values) records in the workspace; a second launch folds them into the
 * gated rows (the split-K decode's merge, reference attn_merge
 * qwen35.cu:2242-2279). Otherwise the rows are written directly, as
 * pkv_attn_prefill (G = 6 / 8 grids whose tile bound fills the CUs but not
 * four rounds run pkv_attn_prefill's kernel). No counterpart in the
 * reference's prompt kernels (attn_mfma / attn_flash_group have no split).
 * pkv_attn_prefill_workspace gives the bytes for these shapes: 256 bytes
 * where the split launch leaves its plan for the merge launch, then records
 * for at most max(2 min((ceil(T / BQ) + seqs) Hkv, CUs - 1), CUs) workgroups
 * of BQ x G rows of 1,032 bytes (BQ = 256 / G queries, 32 for G = 6 / 8),
 * 68 MB at G = 4 on 256 CUs while that bound is 128 workgroups or fewer. Results
 * within the attention tolerance of pkv_attn_prefill (only the points where
 * P is rounded differ); with no split, its bytes. */
int pkv_attn_prefill_workspace(int T, int Hq, int Hkv, int seqs, size_t* bytes);
int pkv_attn_prefill_split(const void* q, const void* kcache, const void* vcache, const void* qkv, int qstride, int Hq,
                           int Hkv, const int32_t* pos, const int32_t* cu, int seqs, const int32_t* block_table,
                           int max_blocks, int block_size, void* out, float scale, const int32_t* outs, int spec,
                           int T, int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream);

/* Chunked-prefill attention over an E4M3 cache: the reference's
 * attn_group8_g<G> (src/kernels/qwen35.cu:1364-1585 with F8, selected for
 * st.kv_fp8 at src/model.rs:2441-2446): the arguments of pkv_attn_prefill
 * plus kscale / vscale; each loaded K / V row is dequantised to
 * bf16(v * scale) (qwen35.cu:1424-1436), the rest as pkv_attn_prefill. */
int pkv_attn_prefill_e4m3(const void* q, const void* kcache, const void* vcache, const float* kscale,
                          const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                          const int32_t* cu, int seqs, const int32_t* block_table, int max_blocks, int block_size,
                          void* out, float scale, const int32_t* outs, int spec, int T, int64_t num_blocks,
                          void* stream);
/* pkv_attn_prefill_e4m3 with split keys for small grids, as
 * pkv_attn_prefill_split (workspace: pkv_attn_prefill_workspace bytes). */
int pkv_attn_prefill_e4m3_split(const void* q, const void* kcache, const void* vcache, const float* kscale,
                                const float* vscale, const void* qkv, int qstride, int Hq, int Hkv, const int32_t* pos,
                                const int32_t* cu, int seqs, const int32_t* block_table, int max_blocks,
                                int block_size, void* out, float scale, const int32_t* outs, int spec, int T,
                                int64_t num_blocks, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Device: attention input preparation (the reference's append site)
 * ------------------------------------------------------------------------- */

/* The reference's attn_prep (src/kernels/qwen35.cu:1067-1128, launched at
 * src/model.rs:2340-2365; same arguments plus T, num_slots and stream): for
 * each token t < T and head of the qkv row [Hq x (q | gate) | k Hkv | v Hkv]
 * (256 wide): q and k heads are RMS-normalised with the f32 weights q_norm /
 * k_norm [256] (bf16(x * scale * w), scale = 1 / sqrt(sum x^2 / 256 + eps))
 * and their dims 0..63 rotated as pairs (d, d + 32) by
 * rope[axis * rope_stride + t] * inv_freq[d] (axis: height for d % 3 == 1
 * below 3 sec_h, width for d % 3 == 2 below 3 sec_w, else time; bf16 cos/sin);
 * q goes to qout [T][Hq][256], k to kcache and v (copied) to vcache at slot
 * slot_map[t] (rows [slot][Hkv][256]); k/v are skipped for slots outside
 * [0, num_slots). With kscale / vscale (both or neither) the cache is E4M3:
 * kcache / vcache hold bytes [slot][Hkv][256] and each k / v head row is
 * stored as e4m3(v / s), s = amax / 448 (1 for an all-zero row) written to
 * kscale / vscale [slot][Hkv] (the reference's store_e4m3,
 * qwen35.cu:1055-1065). */
int pkv_attn_prep(const void* qkv, int qstride, int Hq, int Hkv, const float* q_norm, const float* k_norm,
                  const int32_t* rope, int rope_stride, int sec_h, int sec_w, const int32_t* slot_map,
                  const float* inv_freq, void* qout, void* kcache, void* vcache, const float* kscale,
                  const float* vscale, float eps, int T, int64_t num_slots, void* stream);

/* ---------------------------------------------------------------------------
 * Host: block allocator (reference Scheduler.free_blocks / block_refs,
 * src/sched.rs:461-465, 515, 801-817)
 * ------------------------------------------------------------------------- */

typedef struct pkv_pool pkv_pool;

/* A pool of n_blocks pages, free list [n-1, ..., 1, 0] like sched.rs:515. */
pkv_pool* pkv_pool_create(int64_t n_blocks);
void pkv_pool_destroy(pkv_pool* pool);
/* take_blocks (sched.rs:801-807): the last n free ids in free-list order,
 * each with one reference. PKV_ERR_NO_BLOCKS if fewer are free. */
int pkv_pool_take(pkv_pool* pool, int n, uint32_t* ids);
/* unref_blocks (sched.rs:809-817): one reference less each; a page reaching
 * zero returns to the end of the free list. Underflow is PKV_ERR_INVALID. */
int pkv_pool_unref(pkv_pool* pool, const uint32_t* ids, int n);
/* One reference more each (prefix sharing, sched.rs:758-760, 1054-1056).
 * Refcounts are u16 like the reference's. */
int pkv_pool_ref(pkv_pool* pool, const uint32_t* ids, int n);
int64_t pkv_pool_free_count(const pkv_pool* pool);
int64_t pkv_pool_total(const pkv_pool* pool);
int pkv_pool_refs(const pkv_pool* pool, uint32_t id);
/* Copies the free list (bottom to top) into out (capacity cap); returns its
 * length or a negative status. */
int64_t pkv_pool_free_list(const pkv_pool* pool, uint32_t* out, int64_t cap);

/* ---------------------------------------------------------------------------
 * Host: KV manager — sequences' block tables over a pool, the prefix cache,
 * step metadata, copy-on-write and truncation (the KV bookkeeping of the
 * reference Scheduler, src/sched.rs). Sequence ids are small ints.
 * ------------------------------------------------------------------------- */

typedef struct pkv_kv pkv_kv;

/* A manager over n_blocks pages of block_size slots; max_entries bounds the
 * prefix cache (0 = unbounded; the reference bounds it by its snapshot
 * slots, sched.rs:530-560). */
pkv_kv* pkv_kv_create(int64_t n_blocks, int block_size, int64_t max_entries);
void pkv_kv_destroy(pkv_kv* kv);
/* The manager's block allocator (for pkv_pool_free_count / _refs). */
pkv_pool* pkv_kv_pool(pkv_kv* kv);

/* Admission (Scheduler::admit's KV part, sched.rs:669-799): reserves
 * ceil((prompt_len + max_new) / block_size) blocks; with use_cache, the
 * longest cached whole-64-token-unit prefix of prompt[..prompt_len-1] is
 * shared (its blocks gain a reference, *cached = its length, the sequence's
 * length starts there) and least recently used entries are evicted while
 * blocks are short. PKV_ERR_NO_BLOCKS leaves the request waiting (entries
 * already evicted stay evicted, as in the reference). */
int pkv_kv_admit(pkv_kv* kv, uint32_t adapter, const uint32_t* prompt, int64_t prompt_len, int64_t max_new,
                 int use_cache, int* seq_id, int64_t* cached);
/* Longest cached whole-unit prefix leaving one token (sched.rs:832-842). */
int pkv_kv_lookup(pkv_kv* kv, uint32_t adapter, const uint32_t* prompt, int64_t prompt_len, int64_t* hit_len);
/* Makes tokens[..len] (len a multiple of 64) of sequence seq_id a cache
 * entry holding a reference on its len / block_size blocks (add_entry,
 * sched.rs:1044-1067); evicts the oldest entry first when the cache is full. */
int pkv_kv_cache_add(pkv_kv* kv, int seq_id, uint32_t adapter, const uint32_t* tokens, int64_t len);
/* Evicts the least recently used entry (sched.rs:820-828); returns 1 if one was. */
int pkv_kv_evict_one(pkv_kv* kv);
int64_t pkv_kv_cache_entries(const pkv_kv* kv);
/* Drops a sequence and its block references (release, sched.rs:844-854). */
int pkv_kv_release(pkv_kv* kv, int seq_id);

/* An empty sequence (no blocks) for on-demand growth or sharing. */
int pkv_kv_new_seq(pkv_kv* kv, int* seq_id);
/* Ensures blocks for n_tokens positions (take_blocks order, LIFO). */
int pkv_kv_reserve(pkv_kv* kv, int seq_id, int64_t n_tokens);
/* Empty sequence dst shares src's first n_tokens (ceil(n / block_size)
 * pages, a partial last page included): each page gains a reference. */
int pkv_kv_share(pkv_kv* kv, int dst_id, int src_id, int64_t n_tokens);
/* Before writing positions [pos, pos + n): grows the table as needed and
 * copies on write every page in range that another sequence or entry also
 * references — a fresh page replaces it in this table, its old reference is
 * dropped, and (cow_src[i], cow_dst[i]) lists the device page copies to run
 * with pkv_page_copy before the write (*n_copies of them, at most cap). No
 * reference counterpart: the reference never writes into a shared page. */
int pkv_kv_prepare_write(pkv_kv* kv, int seq_id, int64_t pos, int n, int32_t* cow_src, int32_t* cow_dst, int cap,
                         int* n_copies);
/* Sets the number of positions whose K/V are written ("fed"). */
int pkv_kv_set_len(pkv_kv* kv, int seq_id, int64_t len);
/* Speculative rollback: the sequence keeps new_len (<= its length)
 * positions. free_pages = 0 keeps every reserved page, as the reference does
 * after rejected drafts (sched.rs:1297-1327); 1 also returns pages wholly
 * past ceil(new_len / block_size) to the pool (on-demand mode). The kept
 * positions' bytes are untouched either way. */
int pkv_kv_truncate(pkv_kv* kv, int seq_id, int64_t new_len, int free_pages);
int64_t pkv_kv_len(pkv_kv* kv, int seq_id);
/* Copies the sequence's block table into out (capacity cap); returns its length. */
int64_t pkv_kv_blocks(pkv_kv* kv, int seq_id, uint32_t* out, int64_t cap);

/* Step metadata (Scheduler::fill's KV arrays, sched.rs:1105-1187): rows
 * si < nrows feed ntok[si] tokens of sequence seq_ids[si] at positions
 * len .. len + ntok - 1. Writes pos, slot_map (bt[p / bs] * bs + p % bs),
 * tok_seq, cu[nrows + 1], limits (blocks * bs - 1) and block_table
 * [nrows][max_blocks] (unused entries 0), host arrays. */
int pkv_kv_fill(pkv_kv* kv, const int* seq_ids, const int* ntok, int nrows, int max_tokens, int max_blocks,
                int32_t* pos, int32_t* slot_map, int32_t* tok_seq, int32_t* cu, int32_t* limits,
                int32_t* block_table);
/* The reference's per-step metadata buffer (Meta, model.rs:1245-1354): one
 * int32 device buffer holding every per-step array at a fixed offset, so a
 * step captured into a HIP graph replays against fixed pointers while the
 * host rewrites the contents (engine.rs:704-720; Scheduler::fill / pad write
 * it). Offsets in int32 words for capacities max_tokens (a multiple of 4 in
 * the engine), max_seqs, max_blocks and spec (tokens a verifying sequence
 * feeds; 1 without drafts); words is the buffer's length. This path reads
 * pos, slot_map, tok_seq, rope, cu, outs, limits and block_table: pass
 * buffer + offset to pkv_kv_fill / pkv_kv_pad and to the device entry
 * points. */
typedef struct {
    int64_t ids, pos, slot_map, tok_seq, emb_src, rope, mtp_ids, mtp_src, cu, slots, fresh, outs, ocu, last, temps,
        seeds, top_ks, top_ps, min_ps, pen_cu, limits, snaps, block_table, lora, masks, words;
} pkv_meta;
int pkv_meta_layout(int64_t max_tokens, int64_t max_seqs, int64_t max_blocks, int64_t spec, pkv_meta* out);

/* Padding rows [from, to) of n tokens each for a graph bucket (Scheduler::pad,
 * sched.rs:1219-1261): pos = k, slot_map = -1 (no KV write), tok_seq = row,
 * cu advancing by n, limits = -1, block_table rows 0. Arrays hold max_rows
 * rows (cu: max_rows + 1) and max_tokens tokens; to * n must fit. */
int pkv_kv_pad(int from, int to, int n, int max_rows, int max_tokens, int max_blocks, int32_t* pos,
               int32_t* slot_map, int32_t* tok_seq, int32_t* cu, int32_t* limits, int32_t* block_table);

#ifdef __cplusplus
}
#endif
#endif /* PKV_H */

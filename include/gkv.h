/* gkv: the gpt-oss KV-cache hot path on MI355X (gfx950), C ABI.
 *
 * Paged bf16 KV cache, KV append with RoPE on K, split-K GQA flash-decoding
 * with per-head sink logits and a sliding window, the cross-split combine, and
 * a causal prefill-chunk attention. Plain pointers and sizes only; every call
 * returns a gkv_status; nothing here exits or throws. Kernel entry points
 * enqueue on the given HIP stream (hipStream_t passed as void*; NULL = the
 * null stream) and never allocate device memory.
 *
 * Reference interfaces replaced (n30nd/Optimize_Inference_GPT-OSS):
 *   gkv_rope_table        <- compute_cos_sin host table, getp-csrc/engine/gpu_engine.hpp:388-396
 *                            (run.cpp:422-504)
 *   gkv_kv_append         <- rope_kv_bf16, getp-csrc/kernels/fast_misc.hpp:112-127
 *                            (and rope_exact + kv_write_kernel, kernels/misc.hpp:55-85)
 *   gkv_qkv_append        <- the pair gemm_bf16 (getp-csrc/kernels/fast_gemm.hpp:888-899)
 *                            + rope_kv_bf16 in layer_attention, gpu_engine.hpp:493-496
 *                            (one launch: the append in the projection's epilogue)
 *   gkv_decode_attention  <- attention_q8v_chunk64 / attention_bf16_chunk64 / attention_bf16,
 *                            getp-csrc/kernels/fast_attention.hpp:604-622, 566-580, 525-547
 *   gkv_decode_layer      <- the pair rope_kv_bf16 + attention_q8v_chunk64 in layer_attention,
 *                            getp-csrc/engine/gpu_engine.hpp:495-498 (one call, fused first launch)
 *   gkv_decode_prepare, gkv_decode_split, gkv_decode_combine
 *                         <- the per-wave split and the LDS merge inside
 *                            attention_gqa8_kernel, fast_attention.hpp:164-425 (a7: 383-424)
 *   gkv_prefill_attention, gkv_prefill_paged
 *                         <- no reference kernel; the reference feeds prompts one
 *                            token at a time through the decode step, each
 *                            attending to the cache (gpu_engine.hpp:805-823); same
 *                            semantics per position
 *   gkv_pool_*            <- KV allocation in gpu_alloc_state, gpu_engine.hpp:306-334,
 *                            and its sizing/regrow (gpu_fit_batch :425-433, :921-927)
 *
 * Layouts (device memory):
 *   qkv rows     fp32 [Q (Hq*64) | K (Hkv*64) | V (Hkv*64)], row stride in floats
 *                (fast_misc.hpp:57-58)
 *   K cache      bf16 [num_blocks][Hkv][1024]: token t, dim d of a 16-token block at
 *                element (d/32)*512 + ((d%32)/8*16 + t)*8 + d%8
 *   V cache      bf16 [num_blocks][Hkv][1024]: token t, dim d at element
 *                (d/32)*512 + ((t/4)*16 + d%16)*8 + ((d/16)%2)*4 + t%4
 *                (both put each lane's matrix-core operand in 16 contiguous bytes,
 *                in lane order; gkv.py block_offsets() tabulates them)
 *   block table  int32 [B][table_stride]: logical block j of sequence b -> physical block
 *   ring layers  (sliding window W, W % 16 == 0): position p lives in slot p % W, the
 *                table row holds W/16 blocks (gpu_engine.hpp:477, misc.hpp:72-85)
 */
#ifndef GKV_H
#define GKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  GKV_OK = 0,
  GKV_ERR_ARG = -1,         /* bad argument (null pointer, negative size, ...) */
  GKV_ERR_UNSUPPORTED = -2, /* shape the kernels do not implement (head_dim != 64, ...) */
  GKV_ERR_CAPACITY = -3,    /* pool out of blocks, or a length beyond a table's capacity */
  GKV_ERR_BLOCK = -4,       /* invalid block id / sequence id */
  GKV_ERR_HIP = -5,         /* a HIP runtime call failed */
  GKV_ERR_WORKSPACE = -6    /* workspace smaller than gkv_decode_workspace_bytes() */
} gkv_status;

/* Bits of the device error word that kernels OR in when they meet bad data
 * (they never fault on it: the token is treated as absent). */
#define GKV_DEVERR_BLOCK_ID 1u /* a table entry outside [0, num_blocks) */
#define GKV_DEVERR_LENGTH 2u   /* a sequence length beyond the table's capacity */
#define GKV_DEVERR_ALIGN 4u    /* a prefill start position that is not a multiple of 16 */
#define GKV_DEVERR_RANGE 8u    /* a V beyond the prefill's range (|v| >= 2^26: the output
                                  holds inf there) */
#define GKV_DEVERR_PLAN 16u    /* gkv_decode_layer_planned was asked to reuse a plan the
                                  workspace does not hold for this call (it planned afresh) */

typedef enum { GKV_F32 = 0, GKV_BF16 = 1 } gkv_dtype;

/* Storage of the cache. GKV_V_INT8 is the reference's int8-V cache
 * (getp-csrc/kernels/fast_misc.hpp:74-84): per token and head, 64 int8 codes
 * and one fp32 scale = max|v| / 127, code = rint(v * 127 / max|v|).
 * GKV_KV_FP8 stores K and V as OCP e4m3 codes (the FP8 type of the CDNA4
 * matrix cores: 1 sign, 4 exponent bits with bias 7, 3 mantissa bits, largest
 * finite 448, no infinities): per token and head, 64 codes of K (after RoPE)
 * and 64 of V, each with one fp32 scale = max|x| / 448, code = the nearest
 * e4m3 value (ties to even) of min(max(x * (448 / max|x|), -448), 448); an
 * all-zero head has scale 0 and codes 0. No counterpart in the reference,
 * which names FP8 K/V as its next step after int8 V. */
typedef enum { GKV_V_BF16 = 0, GKV_V_INT8 = 1, GKV_KV_FP8 = 2 } gkv_v_format;

/* A paged cache of one layer as the kernels see it. */
typedef struct {
  void *k;                     /* bf16 [num_blocks][n_kv_heads][1024] (K block layout);
                                  GKV_KV_FP8: e4m3 [num_blocks][n_kv_heads][1024], code of
                                  token t, dim d at ((d % 32) / 8 * 16 + t) * 16 + (d / 32) * 8
                                  + d % 8 */
  void *v;                     /* GKV_V_BF16: bf16 [num_blocks][n_kv_heads][1024] (V block
                                  layout);
                                  GKV_V_INT8 / GKV_KV_FP8: int8 / e4m3
                                  [num_blocks][n_kv_heads][1024], code of dim d, token t at
                                  ((d % 16) * 4 + t / 4) * 16 + (d / 16) * 4 + t % 4 */
  const int32_t *block_table;  /* int32 [B][table_stride] (device) */
  int32_t table_stride;        /* entries per table row */
  int32_t num_blocks;          /* physical blocks in k / v (ids are checked against it) */
  int32_t n_kv_heads;
  int32_t ring;                /* 0: slot = position; W > 0: slot = position % W */
  void *v_scale;               /* GKV_V_INT8: fp32 [num_blocks][n_kv_heads][16] (V scale of
                                  token t at t); GKV_KV_FP8: fp32 [num_blocks][n_kv_heads][32]
                                  (K scale of token t at t, V scale at 16 + t); else NULL */
  int32_t v_format;            /* gkv_v_format (0: bf16) */
} gkv_cache_view;

const char *gkv_status_string(int status);
/* Text of the last HIP error a gkv call on this thread met ("" if none). */
const char *gkv_last_error(void);
/* Library version, "major.minor.patch". */
const char *gkv_version(void);

/* ---- RoPE angles (host) ------------------------------------------------- */

typedef struct {
  float base;                   /* rope_theta (150000) */
  int32_t head_dim;             /* 64 */
  float scaling_factor;         /* 32 */
  float initial_context_length; /* 4096 */
  float ntk_beta;               /* 32 */
  float ntk_alpha;              /* 1 */
} gkv_rope_config;

/* Host table [n_pos][head_dim/2] of cos and sin, bit-identical to the
 * reference's compute_cos_sin(pos, ...) for pos = 0..n_pos-1. */
int gkv_rope_table(const gkv_rope_config *cfg, int32_t n_pos, float *cos_tab, float *sin_tab);

/* ---- KV append ----------------------------------------------------------- */

/* RoPE on K of each row, then bf16 (round to nearest even) K and V stored into
 * the paged cache at the row's slot. One row per token:
 *   row_pos[r]   position of row r's token (device int32)
 *   row_seq[r]   its sequence (device int32; NULL: row r is sequence r)
 *   seq_lens[s]  tokens of sequence s after this append (device int32;
 *                required on ring layers, GKV_ERR_ARG if NULL there; unused
 *                otherwise). A row whose ring slot a later row of this same
 *                call overwrites (pos + ring < seq_len) is not stored, so the
 *                ring ends up holding the last W positions.
 *   q_out        NULL, or fp32 [rows][q_out_stride] receiving the rotated Q
 *                (may equal qkv with q_out_stride = row_stride: in place)
 *   k_pack/v_pack NULL, or bf16 [rows][Hkv][64] receiving the same bf16 K, V
 *                (the packed operands of gkv_prefill_attention)
 *   dev_err      NULL, or a device uint32 that gets GKV_DEVERR_* bits
 * cos_tab/sin_tab: device copies of gkv_rope_table rows. qkv, the tables and
 * the packed rows are 16-byte aligned and row_stride is a multiple of 4
 * (GKV_ERR_ARG otherwise). */
int gkv_kv_append(void *stream, int32_t n_rows, const float *qkv, int64_t row_stride,
                  int32_t n_q_heads, const float *cos_tab, const float *sin_tab,
                  const int32_t *row_pos, const int32_t *row_seq, const int32_t *seq_lens,
                  gkv_cache_view cache, float *q_out, int64_t q_out_stride, void *k_pack,
                  void *v_pack, uint32_t *dev_err);

/* QKV projection with the append in its epilogue: for each row r,
 *   qkv[r][i] = sum_j x[r][j] * w_qkv[i][j] + b_qkv[i]
 * (fp32 accumulation of bf16 products, the bias added to the finished sum, as
 * gemm_bf16 computes it; i < (Hq + 2 Hkv) * 64), written to qkv_out (fp32
 * [rows][out_stride], NULL: not written), and the row's K part rotated and its
 * K and V parts stored into the paged cache exactly as gkv_kv_append stores
 * the same qkv row (cache.k == cache.v == NULL: no append). Row placement
 * (row_pos, row_seq, seq_lens, the ring rule, dev_err) is gkv_kv_append's;
 * with row_pos NULL, row r sits at position seq_lens[seq]-1 (a decode step).
 *   x      bf16 [rows][x_stride], x_stride a multiple of 8, 16-byte aligned
 *   w_qkv  bf16 [(Hq + 2 Hkv) * 64][hidden] row-major, 16-byte aligned
 *   b_qkv  fp32 [(Hq + 2 Hkv) * 64] or NULL
 * hidden is a multiple of 64 (GKV_ERR_UNSUPPORTED otherwise). For decode
 * steps (hundreds of rows); at prompt sizes (thousands of rows) a library
 * GEMM followed by gkv_kv_append is faster. */
int gkv_qkv_append(void *stream, int32_t n_rows, const void *x, int64_t x_stride,
                   int32_t hidden, const void *w_qkv, const float *b_qkv, int32_t n_q_heads,
                   const float *cos_tab, const float *sin_tab, const int32_t *row_pos,
                   const int32_t *row_seq, const int32_t *seq_lens, gkv_cache_view cache,
                   float *qkv_out, int64_t out_stride, uint32_t *dev_err);

/* ---- Decode attention ---------------------------------------------------- */

/* Bytes of workspace gkv_decode_attention / gkv_decode_split need. */
size_t gkv_decode_workspace_bytes(int32_t B, int32_t n_kv_heads, int32_t max_seq_len,
                                  int32_t window, int32_t split_tokens);

/* One query token per sequence against its cached keys/values plus the head's
 * sink logit (run.cpp:597-642 semantics):
 *   q         fp32 [B][q_stride], heads at h*64; not yet rotated if cos_tab is
 *             given (rotated on load with row seq_lens[b]-1, bit-identical to
 *             the append's rotation), already rotated if cos_tab is NULL
 *   seq_lens  device int32 [B]: tokens in the cache (the new one included)
 *   window    0: full attention over all seq_len tokens; W > 0: the last
 *             min(seq_len, W) tokens (cache.ring must be W or 0)
 *   sinks     fp32 [Hq]
 *   split_tokens  0: balanced (the total is cut into equal ranges, one per
 *             workgroup the GPU holds at once); > 0: ranges of this many tokens
 *             (a multiple of 32, at most 16384)
 *   max_seq_len   host upper bound of seq_lens (sizes the grid)
 *   out       [B][out_stride] of out_dtype, heads at h*64
 * Two launches: a split that plans the ranges in its prologue and streams
 * them, then the combine of the sequences that cross a range boundary. On a
 * window layer with split_tokens 0 the ranges hold whole sequences (a range
 * ends at most one window past its share of the stream) and the split
 * finishes every sequence: no combine is launched. */
int gkv_decode_attention(void *stream, int32_t B, int32_t n_q_heads, const float *q,
                         int64_t q_stride, const float *cos_tab, const float *sin_tab,
                         const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                         int32_t window, const float *sinks, int32_t split_tokens,
                         void *workspace, size_t workspace_bytes, void *out, int64_t out_stride,
                         int32_t out_dtype, uint32_t *dev_err);

/* 1 if gkv_decode_attention / gkv_decode_layer / gkv_decode_layer_noalloc
 * launch the combine after the split for these sizes, 0 if the split
 * finishes every sequence (window layers with split_tokens 0), < 0 on a bad
 * argument. A caller of gkv_decode_layer_split may skip gkv_decode_combine
 * when it returns 0 (the combine then returns at once anyway). No
 * counterpart in the reference. */
int gkv_decode_layer_combines(int32_t B, int32_t n_kv_heads, int32_t max_seq_len,
                              int32_t window, int32_t split_tokens);

/* The staged launches, for callers that time or schedule them separately;
 * same arguments, run in this order on one stream with the same workspace. gkv_decode_prepare lays the sequences out as one
 * token stream cut into equal ranges (block ids checked against the pool,
 * per-step records) and prepares the rotated, scaled query operands;
 * gkv_decode_split streams every range, writes the final output of each
 * sequence that lies in one range and partial results of the others into the
 * workspace; gkv_decode_combine merges those with the sink. */
int gkv_decode_prepare(void *stream, int32_t B, int32_t n_q_heads, const float *q,
                       int64_t q_stride, const float *cos_tab, const float *sin_tab,
                       const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                       int32_t window, const float *sinks, int32_t split_tokens, void *workspace,
                       size_t workspace_bytes, void *out, int64_t out_stride, int32_t out_dtype,
                       uint32_t *dev_err);
int gkv_decode_split(void *stream, int32_t B, int32_t n_q_heads, const float *q,
                     int64_t q_stride, const float *cos_tab, const float *sin_tab,
                     const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                     int32_t window, const float *sinks, int32_t split_tokens, void *workspace,
                     size_t workspace_bytes, void *out, int64_t out_stride, int32_t out_dtype,
                     uint32_t *dev_err);
int gkv_decode_combine(void *stream, int32_t B, int32_t n_q_heads, int32_t n_kv_heads,
                       const int32_t *seq_lens, int32_t max_seq_len, int32_t window,
                       const float *sinks, int32_t split_tokens, const void *workspace,
                       size_t workspace_bytes, void *out, int64_t out_stride, int32_t out_dtype);

/* One decode layer in one call: the append of every sequence's new token
 * and the attention, replacing the pair rope_kv_bf16 + attention_q8v_chunk64
 * of layer_attention (getp-csrc/engine/gpu_engine.hpp:495-498). Row b of qkv
 * ([Q | K | V] fp32, not rotated) is the new token of sequence b at position
 * seq_lens[b] - 1; its K (rotated) and V go into the cache, then the
 * attention runs as gkv_decode_attention with q = qkv, q_stride = row_stride
 * (cos_tab/sin_tab required): the split launch appends the new tokens of
 * its range in its prologue, then streams it; the combine follows unless the
 * ranges hold whole sequences (gkv_decode_layer_combines).
 * gkv_decode_layer_split is that first launch alone (gkv_decode_combine with
 * the same arguments, q = qkv, completes it). gkv_decode_layer_prepare is the
 * staged form's first launch (the append fused with gkv_decode_prepare);
 * gkv_decode_split and gkv_decode_combine complete it. */
int gkv_decode_layer(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                     int64_t row_stride, const float *cos_tab, const float *sin_tab,
                     const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                     int32_t window, const float *sinks, int32_t split_tokens, void *workspace,
                     size_t workspace_bytes, void *out, int64_t out_stride, int32_t out_dtype,
                     uint32_t *dev_err);
int gkv_decode_layer_split(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                           int64_t row_stride, const float *cos_tab, const float *sin_tab,
                           const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                           int32_t window, const float *sinks, int32_t split_tokens,
                           void *workspace, size_t workspace_bytes, void *out,
                           int64_t out_stride, int32_t out_dtype, uint32_t *dev_err);
int gkv_decode_layer_prepare(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                             int64_t row_stride, const float *cos_tab, const float *sin_tab,
                             const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                             int32_t window, const float *sinks, int32_t split_tokens,
                             void *workspace, size_t workspace_bytes, void *out,
                             int64_t out_stride, int32_t out_dtype, uint32_t *dev_err);

/* gkv_decode_layer for the engine's loop over layers
 * (getp-csrc/engine/gpu_engine.hpp:652, layer_attention per layer at :495-498):
 * the layers of one kind (full, or sliding window) in one decode step share
 * the lengths and the block table, so the split launch's plan (the ranges,
 * the step records and block ids) is the same for all of them. plan =
 * GKV_PLAN_KEEP plans as gkv_decode_layer does and keeps the plan in the
 * workspace; GKV_PLAN_REUSE takes the kept plan instead of planning (the
 * prologue then only loads it and appends). GKV_PLAN_NONE is gkv_decode_layer.
 * Results are bit-identical to gkv_decode_layer's. Reuse needs the same
 * workspace, seq_lens and block_table pointers, B, window, split_tokens,
 * max_seq_len and pool shape as the keeping call, and the same lengths; a
 * launch that plans afresh on the workspace (any other decode entry point)
 * drops the kept plan. A key in the workspace checks the shape, the pointers
 * and a 64-bit hash of the lengths' contents: on a mismatch the call plans
 * afresh (so its results are gkv_decode_layer's) and sets GKV_DEVERR_PLAN.
 * The kept plan holds table positions, not block ids: a reusing call reads
 * the ids from the table as it is at the call, so a changed table entry is
 * used, not a stale one. Length errors
 * (GKV_DEVERR_LENGTH) are reported by the keeping call. Each kind needs a
 * workspace of its own (gkv_decode_workspace_bytes). */
typedef enum { GKV_PLAN_NONE = 0, GKV_PLAN_KEEP = 1, GKV_PLAN_REUSE = 2 } gkv_plan_mode;
int gkv_decode_layer_planned(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                             int64_t row_stride, const float *cos_tab, const float *sin_tab,
                             const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                             int32_t window, const float *sinks, int32_t split_tokens,
                             void *workspace, size_t workspace_bytes, void *out,
                             int64_t out_stride, int32_t out_dtype, uint32_t *dev_err,
                             int32_t plan);
/* Its first launch alone, as gkv_decode_layer_split is gkv_decode_layer's
 * (gkv_decode_combine with the same arguments completes it). */
int gkv_decode_layer_split_planned(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                                   int64_t row_stride, const float *cos_tab,
                                   const float *sin_tab, const int32_t *seq_lens,
                                   int32_t max_seq_len, gkv_cache_view cache, int32_t window,
                                   const float *sinks, int32_t split_tokens, void *workspace,
                                   size_t workspace_bytes, void *out, int64_t out_stride,
                                   int32_t out_dtype, uint32_t *dev_err, int32_t plan);

/* gkv_decode_layer without a workspace argument and without allocating: the
 * workspace is the library's own device array (one per GPU, about 16.5 MiB,
 * held until the process ends), looked up once per device. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and results as gkv_decode_layer with
 * split_tokens = 0. Limits: at most 8 kv heads, 8192 sequences and 512 split
 * ranges (ranges hold up to 16384 tokens; more: GKV_ERR_CAPACITY). Calls that
 * overlap on one GPU share the array and race: keep them on one stream. */
int gkv_decode_layer_noalloc(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                             int64_t row_stride, const float *cos_tab, const float *sin_tab,
                             const int32_t *seq_lens, int32_t max_seq_len, gkv_cache_view cache,
                             int32_t window, const float *sinks, void *out, int64_t out_stride,
                             int32_t out_dtype, uint32_t *dev_err);

/* ---- Ceiling yardsticks ---------------------------------------------------- */

/* Read-only kernels that measure what the memory system gives the decode
 * kernel's access patterns, as the reference's attention bench does with its
 * read_stream and loads-only kernels (getp-csrc/bench/attn_bench.cpp:66-76,
 * 161-227). Each folds what it reads into an XOR and writes nothing
 * meaningful to sink (device, >= 256 uint32). */
/* Every byte of src (16-byte aligned, n_bytes a multiple of 16) once,
 * nontemporal, 1 KB per wave instruction, over n_workgroups x 256 threads. */
int gkv_yardstick_stream(void *stream, const void *src, int64_t n_bytes, int32_t n_workgroups,
                         uint32_t *sink);
/* The 2 KB blocks base + id * 2048 for the n_ids ids of block_ids (device;
 * ids are clamped into the n_bytes of base), in steps of 4 blocks per wave,
 * one wave per SIMD (n_workgroups x 4 waves), as the decode kernel reads one
 * (block, kv head) of the paged cache. */
int gkv_yardstick_gather(void *stream, const void *base, int64_t n_bytes,
                         const int32_t *block_ids, int32_t n_ids, int32_t n_workgroups,
                         uint32_t *sink);
/* gkv_decode_layer's split launch (bf16 K/V only, else GKV_ERR_UNSUPPORTED)
 * with the attention math replaced by an XOR of the loaded data: the same
 * plan, appends and load stream (the appends are real; out is not written).
 * No combine. */
int gkv_yardstick_decode_loads(void *stream, int32_t B, int32_t n_q_heads, const float *qkv,
                               int64_t row_stride, const float *cos_tab, const float *sin_tab,
                               const int32_t *seq_lens, int32_t max_seq_len,
                               gkv_cache_view cache, int32_t window, const float *sinks,
                               int32_t split_tokens, void *workspace, size_t workspace_bytes,
                               void *out, int64_t out_stride, int32_t out_dtype,
                               uint32_t *dev_err);

/* ---- Prefill (causal) attention ----------------------------------------- */

/* Causal attention of packed prompts with sinks: row j of prompt b (rows
 * cu_seqlens[b] .. cu_seqlens[b+1]-1, positions 0..L_b-1) attends to rows
 * 0..j of its prompt (window W: j-W+1..j):
 *   q        fp32 [rows][q_stride]: rotated (gkv_kv_append's q_out) if cos_tab
 *            is NULL; else not rotated (the qkv rows themselves, q_stride =
 *            their row stride) and rotated on load at position j, bit-identical
 *            to gkv_kv_append's q_out
 *   cos_tab/sin_tab  NULL (both), or device copies of gkv_rope_table rows
 *   k, v     bf16 [rows][Hkv][64] (gkv_kv_append's k_pack, v_pack)
 *   cu_seqlens device int32 [B+1]; max_len = host bound of the prompt lengths
 *   out      [rows][out_stride] of out_dtype
 * q, k, v and the tables are 16-byte aligned, q_stride a multiple of 4
 * (GKV_ERR_ARG otherwise). V enters an fp16 matrix core as v * 2^-10: exact
 * for bf16 magnitudes 2^-4 .. 2^26, an absolute error of at most 2^-15 below,
 * inf above (which the output shows; gkv_prefill_paged also flags it). */
int gkv_prefill_attention(void *stream, int32_t B, const int32_t *cu_seqlens, int32_t max_len,
                          int32_t n_q_heads, int32_t n_kv_heads, const float *q,
                          int64_t q_stride, const float *cos_tab, const float *sin_tab,
                          const void *k, const void *v, const float *sinks, int32_t window,
                          void *out, int64_t out_stride, int32_t out_dtype);

/* Causal attention of prompt chunks that continue sequences already in the
 * paged cache (chunked prefill), same semantics: row j of prompt b is position
 * start_pos[b] + j and attends to positions max(0, p - W + 1) .. p, plus the
 * sink. start_pos: device int32 [B], multiples of 16 (else GKV_DEVERR_ALIGN
 * is set and that prompt's outputs are meaningless, though finite), or NULL
 * (all 0). For a full layer (cache.ring = 0) the positions must stay below
 * cache.table_stride * 16 (the cos/sin tables cover them): a prompt that runs
 * past sets GKV_DEVERR_LENGTH, and its rows beyond take their angles at the
 * last position that fits (meaningless outputs, no read past the tables).
 *   keys before start_pos[b]  from the cache (gkv_cache_view in any format:
 *            a quantized K or V stands for value(code) * scale): the full
 *            layer's table, or a ring of W slots (cache.ring == window), which
 *            must still hold them -- append a ring layer's chunk after this call
 *   keys from start_pos[b] on  from the packed rows k, v (bf16 [rows][Hkv][64],
 *            gkv_kv_append's k_pack/v_pack of this chunk); k = v = NULL: from
 *            the cache as well (a full layer whose chunk was appended first)
 *   dev_err  NULL, or a device uint32 that gets GKV_DEVERR_* bits (block ids
 *            outside the pool, misaligned start positions, positions past a
 *            full layer's table, V out of range)
 * The other arguments are gkv_prefill_attention's; cos/sin rows are taken at
 * the rows' positions. */
int gkv_prefill_paged(void *stream, int32_t B, const int32_t *cu_seqlens,
                      const int32_t *start_pos, int32_t max_len, int32_t n_q_heads,
                      const float *q, int64_t q_stride, const float *cos_tab,
                      const float *sin_tab, const void *k, const void *v, gkv_cache_view cache,
                      const float *sinks, int32_t window, void *out, int64_t out_stride,
                      int32_t out_dtype, uint32_t *dev_err);

/* ---- Exact path (fp32 caches, bit for bit with the CPU forward) ---------- */

/* The reference's GPTOSS_EXACT engine build (getp-csrc/engine/gpu_engine.hpp:
 * 478-488) keeps fp32 caches of layout [B][slots][kv_dim] (a window layer's
 * cache a ring of `window` slots: position t in slot t % window) and runs
 * rope_exact, kv_write_kernel and attention_exact, whose outputs equal the
 * CPU forward's (run.cpp) bit for bit. These three entry points are that
 * path: each result equals the reference CPU code's on the same inputs, bit
 * for bit (the softmax's exp is glibc's expf, as the x86-64 C library with
 * FMA computes it). Positions come either as one `pos` / `slot` for every
 * row, as the reference engine passes them, or per row (`positions`, device
 * int32 [B], the new token's position = length - 1). */

/* rope_exact (getp-csrc/kernels/misc.hpp:55-72; run.cpp:506-526): rotates
 * heads 0..n_heads-1 of each row in place (the query heads followed by the
 * key heads), x1*c - x2*s and x2*c + x1*s with the first product fused.
 * Row b takes cos/sin row positions[b] of the tables; positions NULL: row 0
 * for every row (pass the tables' row at pos, as the reference does). */
int gkv_rope_exact(void *stream, int32_t B, float *qkv, int64_t row_stride,
                   const float *cos_tab, const float *sin_tab, const int32_t *positions,
                   int32_t n_heads);

/* kv_write_kernel (getp-csrc/kernels/misc.hpp:74-85): copies each row's K
 * (kv_dim floats at row + k_off) and V (at row + v_off) into kc / vc at the
 * row's slot: `slot` for every row, or, with positions, positions[b] (full
 * layer, window = 0) or positions[b] % window. A slot outside [0, slots)
 * skips the row and sets GKV_DEVERR_LENGTH in dev_err (NULL: not reported). */
int gkv_kv_write_exact(void *stream, int32_t B, const float *qkv, int64_t row_stride,
                       int32_t k_off, int32_t v_off, float *kc, float *vc, int32_t slots,
                       int32_t kv_dim, int32_t slot, const int32_t *positions, int32_t window,
                       uint32_t *dev_err);

/* attention_exact (getp-csrc/kernels/attention.hpp:18-83; run.cpp:597-641):
 * row b's query heads (q, fp32 [B][q_stride], head h at h * 64) attend to
 * positions t0 .. p of their kv head (p = pos, or positions[b]; t0 = 0, or
 * max(0, p - window + 1) on a window layer) plus the head's sink; out fp32
 * [B][out_stride]. max_pos: host bound of positions[] (ignored without
 * them). A row whose position the cache cannot hold (p >= slots on a full
 * layer, p < 0, p > max_pos) gets zeros and GKV_DEVERR_LENGTH. A head's
 * scores stay in LDS: GKV_ERR_CAPACITY when even one head's do not fit in
 * what the device gives a workgroup (under 4 bytes per position of it).
 * n_q_heads / n_kv_heads <= 16 (GKV_ERR_UNSUPPORTED otherwise). */
int gkv_attention_exact(void *stream, int32_t B, int32_t n_q_heads, int32_t n_kv_heads,
                        const float *q, int64_t q_stride, const float *kc, const float *vc,
                        int32_t slots, const float *sinks, int32_t pos,
                        const int32_t *positions, int32_t max_pos, int32_t window, float *out,
                        int64_t out_stride, uint32_t *dev_err);

/* ---- Paged KV pool (host bookkeeping, device storage) -------------------- */

typedef struct gkv_pool gkv_pool;

typedef struct {
  int32_t n_layers;        /* layers; layer l is a window layer iff window > 0 and l % 2 == 0
                              (run.cpp:617-619, gpu_engine.hpp:318) */
  int32_t n_kv_heads;
  int32_t head_dim;        /* 64 */
  int32_t window;          /* sliding window W (multiple of 16), 0 = none */
  int32_t max_seqs;        /* sequence ids 0 .. max_seqs-1 */
  int32_t max_seq_len;     /* longest sequence (sizes the table rows) */
  int64_t num_blocks;      /* physical 16-token blocks for the full layers; 0: derive from
                              bytes_budget */
  int64_t bytes_budget;    /* used when num_blocks == 0: device bytes for all caches;
                              0: 90% of hipMemGetInfo's free memory */
  uint64_t shuffle_seed;   /* 0: blocks handed out in id order; else a seeded
                              permutation (scattered physical placement) */
  int32_t v_format;        /* gkv_v_format of every layer's V cache (0: bf16) */
} gkv_pool_config;

int gkv_pool_create(const gkv_pool_config *cfg, gkv_pool **out);
int gkv_pool_destroy(gkv_pool *pool);
/* Takes a free sequence id (its length starts at 0). */
int gkv_pool_seq_alloc(gkv_pool *pool, int32_t *seq_id);
/* Makes room for seq_len tokens of seq_id (allocating blocks; never shrinks). */
int gkv_pool_seq_reserve(gkv_pool *pool, int32_t seq_id, int32_t seq_len);
/* Returns the sequence's blocks to the free list. */
int gkv_pool_seq_free(gkv_pool *pool, int32_t seq_id);
/* Brings the device block tables up to date after alloc/reserve/free, on
 * stream, without waiting: only the entries changed since the last sync go,
 * from a pinned staging buffer the pool owns (one of two, each reused only
 * once its copy has completed) through a small scatter kernel, so kernels
 * queued after it on the same stream see the new tables and the host may
 * reserve and free again at once. (The pool's creation uploads both tables
 * whole.) No counterpart in the reference, whose caches are not paged. */
int gkv_pool_sync(gkv_pool *pool, void *stream);
/* Cache view of layer l over the table rows of sequence ids 0 .. max_seqs-1
 * (rows of the batch must be sequence ids: pass row_seq or order the batch by id). */
int gkv_pool_layer_view(const gkv_pool *pool, int32_t layer, gkv_cache_view *view);
/* Table-row view starting at sequence id first_seq (for batches of consecutive ids). */
int gkv_pool_layer_view_from(const gkv_pool *pool, int32_t layer, int32_t first_seq,
                             gkv_cache_view *view);
int64_t gkv_pool_free_blocks(const gkv_pool *pool);
int64_t gkv_pool_num_blocks(const gkv_pool *pool);
/* Device bytes held by the pool's caches and tables. */
int64_t gkv_pool_device_bytes(const gkv_pool *pool);
/* Host copy of a sequence's full-layer table row (n entries at most). */
int gkv_pool_seq_blocks(const gkv_pool *pool, int32_t seq_id, int32_t *blocks, int32_t n,
                        int32_t *n_used);

#ifdef __cplusplus
}
#endif
#endif /* GKV_H */

/* CPU oracle of the gpt-oss KV-cache hot path (test infrastructure only).
 *
 * A plain-C restatement of the reference's CPU attention in run.cpp, extended
 * to a batch of sequences with their own lengths. Only tests, the smoke check
 * and bench.py's CPU-baseline leg may call it; the product never does.
 *
 * Every function names the reference lines it restates. Rounding follows the
 * reference binary built by hipcc -O3 with FMA contraction: the spots where
 * that build fuses a multiply into an add are written as explicit fmaf(), so
 * this file gives the same bits under any compiler flags (it is compiled with
 * -ffp-contract=off).
 */
#ifndef KV_ORACLE_H
#define KV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gpt-oss YaRN settings: run.cpp:582-583 (ntk_beta, ntk_alpha) and the
 * checkpoint config (rope_theta, rope_scaling_factor, initial_context_length). */
typedef struct {
  float base;           /* rope_theta, 150000 */
  int head_dim;         /* 64 */
  float scaling_factor; /* 32 */
  float initial_context_length; /* 4096 */
  float ntk_beta;       /* 32 */
  float ntk_alpha;      /* 1 */
} orc_rope_cfg;

/* run.cpp:422-477 compute_concentration_and_inv_freq. */
void orc_yarn(const orc_rope_cfg *c, float *concentration, float *inv_freq);
/* run.cpp:479-504 compute_cos_sin: head_dim/2 cosines and sines for one position. */
void orc_cos_sin(const orc_rope_cfg *c, int pos, float *cos_out, float *sin_out);
/* Rows 0..n_pos-1 of compute_cos_sin, [n_pos][head_dim/2] each
 * (the host table of gpu_engine.hpp:388-396). */
void orc_rope_table(const orc_rope_cfg *c, int n_pos, float *cos_tab, float *sin_tab);
/* run.cpp:506-526 apply_rotary_emb on n_heads heads of x, in place:
 * o1 = fma(x1, c, -(x2 s)), o2 = fma(x2, c, x1 s). */
void orc_rotate(float *x, const float *cosv, const float *sinv, int n_heads, int head_dim);

/* fp32 -> bf16, round to nearest even, NaN kept quiet (fast_common.hpp:14-20). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float *x, uint16_t *y, long n);

/* run.cpp:335-353 softmax (fp64 max and sum, expf per entry, divide). */
void orc_softmax(float *x, int size);

/* Decode attention of one new token per sequence, run.cpp:597-642, batched.
 *   q[b*q_stride + h*d + i]              rotated query, fp32
 *   kc/vc[b*seq_stride + slot*kv_dim + g*d + i]  the cache, fp32 (pass
 *       bf16-decoded values for the bf16-cache comparison)
 *   pos[b]  position of the new token; positions 0..pos[b] are attended
 *   window  0: every position (full layer); W > 0: positions t with
 *           pos - t >= W get -inf (run.cpp:170-176, 617-619)
 *   ring    0: position t sits in slot t; R > 0: in slot t % R (the ring of
 *           a window layer, gpu_engine.hpp:477; requires window <= ring)
 *   sinks[h] one extra logit per query head (run.cpp:624)
 *   out[b*out_stride + h*d + i]
 * Masked positions contribute exactly zero to the max, the fp64 sum and the
 * fma accumulation, so they are skipped: same bits as visiting them.
 * Returns 0, or -1 on bad arguments. */
int orc_decode_attention(int B, int n_q_heads, int n_kv_heads, int head_dim, const float *q,
                         long q_stride, const float *kc, const float *vc, long seq_stride,
                         const int *pos, const float *sinks, int window, int ring, float *out,
                         long out_stride, int n_threads);

/* Causal prefill attention of a packed batch of prompts: query token j of
 * prompt b (at position j) attends to that prompt's positions 0..j (window W:
 * j-W+1..j), plus the sink. Each query is computed exactly as
 * orc_decode_attention computes a decode token at pos = j (the reference
 * feeds prompts one token at a time through the decode step,
 * gpu_engine.hpp:811-813).
 *   cu_seqlens[B+1] prefix offsets of the prompts in the packed rows
 *   q[row*q_stride + h*d + i], kv[row*kv_stride + g*d + i] (k, v separate)
 *   out[row*out_stride + h*d + i] */
int orc_prefill_attention(int B, int n_q_heads, int n_kv_heads, int head_dim,
                          const int *cu_seqlens, const float *q, long q_stride,
                          const float *k, const float *v, long kv_stride, const float *sinks,
                          int window, float *out, long out_stride, int n_threads);

/* KV append of one token per sequence (run.cpp:573-576 + 588-592, and the
 * bf16 store of fast_misc.hpp:87-99 without the int8 V):
 *   qkv[b*row_stride + ...] rows [Q (Hq*d) | K (Hkv*d) | V (Hkv*d)], fp32
 *   cos_tab/sin_tab [pos][d/2]; pos[b] the token's position
 * Outputs per sequence (kv_dim = Hkv*d): k_rot (fp32 rotated K, may be NULL),
 * k_bf16 and v_bf16 ([b*kv_dim + g*d + i]); q_rot (fp32 rotated Q, may be
 * NULL, [b*Hq*d + h*d + i]). */
void orc_linear(int n_rows, const float *x, long x_stride, const float *w, const float *bias,
                int n_in, int n_out, float *out, long out_stride);
void orc_kv_append(int B, int n_q_heads, int n_kv_heads, int head_dim, const float *qkv,
                   long row_stride, const float *cos_tab, const float *sin_tab, const int *pos,
                   float *q_rot, float *k_rot, uint16_t *k_bf16, uint16_t *v_bf16);

/* int8 V of one token: per head of head_dim values, scale = max|v| / 127 and
 * code = clamp(rint(v * (127 / max|v|)), -127, 127) (0 codes and scale 0 for
 * an all-zero head): the rule of the reference's int8-V cache,
 * getp-csrc/kernels/fast_misc.hpp:74-84, restated on the host in
 * getp-csrc/tests/attn_test.cpp:218-226 (quantize_v).
 *   v[h*head_dim + i] fp32 -> codes[h*head_dim + i], scales[h] */
void orc_quantize_v(const float *v, int n_heads, int head_dim, int8_t *codes, float *scales);
/* e4m3 (OCP FP8 E4M3) cache: the value of a code, and per-head quantization
 * (scale = amax / 448, code = nearest e4m3 of clamp(x * 448 / amax)). */
float orc_fp8_value(uint8_t c);
void orc_quantize_fp8(const float *x, int n_heads, int head_dim, uint8_t *codes,
                      float *scales);

#ifdef __cplusplus
}
#endif
#endif

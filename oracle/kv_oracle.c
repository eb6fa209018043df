/* CPU oracle of the gpt-oss KV-cache hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's CPU path (run.cpp) for a batch of sequences. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this;
 * the product library never links or calls it.
 *
 * Parity pinning (what checks each function; all in tests/):
 *   orc_yarn, orc_cos_sin, orc_rope_table  bit-exact vs the reference's own
 *       compute_cos_sin (oracle/_ref build of run.cpp, and the committed
 *       golden table from it); closed forms: pos 0 gives cos = concentration,
 *       sin = 0; concentration = 0.1 ln 32 + 1; inv_freq monotone.
 *   orc_rotate     bit-exact vs run.cpp apply_rotary_emb (_ref + goldens);
 *       norm preservation of each pair up to concentration^2.
 *   orc_f32_to_bf16  closed-form cases (ties to even, NaN quiet, +-0, inf,
 *       overflow to inf) and exhaustive agreement with a numpy restatement of
 *       round-to-nearest-even over all 2^16 upper halves x sampled lower halves.
 *   orc_softmax    bit-exact vs run.cpp softmax (_ref).
 *   orc_decode_attention  bit-exact vs run.cpp forward() attention output
 *       (_ref + goldens, full and window layers, pos 0..600); closed forms
 *       n = 1 (out = v sigmoid(s - sink)), equal keys, sink -> -inf,
 *       slot-permutation invariance, window >= n equals full.
 *   orc_prefill_attention  equals orc_decode_attention at every prompt
 *       position (it is defined as that); brute force fp64 on tiny prompts.
 *   orc_kv_append  bit-exact vs run.cpp (_ref: the key written into the
 *       cache by forward()) and the bf16 rule above.
 *   orc_linear     bit-exact vs run.cpp matmul + bias add (_ref); closed forms:
 *       a one-hot input row gives W's column plus the bias exactly; products
 *       of bf16 values are exact, so it equals an fp64 sum rounded once to
 *       fp32 (numpy) before the bias.
 *   orc_quantize_v  bit-exact vs the reference's own quantize_v
 *       (getp-csrc/tests/attn_test.cpp, built into oracle/_ref/libref_q8.so)
 *       on random heads; closed forms: exact multiples of the step, the amax
 *       element at +-127, ties to even, the all-zero head.
 *   orc_fp8_value, orc_quantize_fp8  (the e4m3 K/V cache, which the
 *       reference does not implement: it names FP8 K/V as its next step)
 *       pinned by the format's closed forms (1.0 = 0x38, 448 = 0x7e, 2^-6 =
 *       0x08, 2^-9 = 0x01, 0x7f NaN, monotone codes, sign symmetry) and by
 *       brute force: every code equals the nearest table value, ties to the
 *       even code, over random values, all midpoints and the edges.
 */
#include "kv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

/* run.cpp:422-477. The reference build (hipcc -O3, FMA) contracts
 * `interpolation * (1 - mask) + extrapolation * mask` into
 * fma(extrapolation, mask, round(interpolation * (1 - mask))): the right-hand
 * product is the fused one (found by comparing with the reference build at
 * every index of the ramp). `0.1f * logf(s) + 1.0f` gives the same float fused
 * or not for s = 32; it is written fused. */
void orc_yarn(const orc_rope_cfg *c, float *concentration, float *inv_freq) {
  const int d_half = c->head_dim / 2;
  float freq[256];
  for (int i = 0; i < d_half; i++)
    freq[i] = powf(c->base, ((float)(2 * i)) / (float)c->head_dim);
  if (c->scaling_factor > 1.0f) {
    *concentration = fmaf(0.1f, logf(c->scaling_factor), 1.0f);
    /* (ntk_beta * 2.0f) is float, times M_PI is double; logf takes the
     * quotient rounded to float. */
    const double two_pi_beta = (double)(c->ntk_beta * 2.0f) * M_PI;
    const double two_pi_alpha = (double)(c->ntk_alpha * 2.0f) * M_PI;
    const float low = (float)d_half * logf((float)((double)c->initial_context_length / two_pi_beta)) /
                      logf(c->base);
    const float high = (float)d_half *
                       logf((float)((double)c->initial_context_length / two_pi_alpha)) /
                       logf(c->base);
    for (int i = 0; i < d_half; i++) {
      const float interpolation = 1.0f / (c->scaling_factor * freq[i]);
      const float extrapolation = 1.0f / freq[i];
      float ramp = ((float)i - low) / (high - low);
      if (ramp < 0)
        ramp = 0;
      if (ramp > 1)
        ramp = 1;
      const float mask = 1.0f - ramp;
      inv_freq[i] = fmaf(extrapolation, mask, interpolation * (1.0f - mask));
    }
  } else {
    *concentration = 1.0f;
    for (int i = 0; i < d_half; i++)
      inv_freq[i] = 1.0f / freq[i];
  }
}

/* run.cpp:479-504. */
void orc_cos_sin(const orc_rope_cfg *c, int pos, float *cos_out, float *sin_out) {
  float conc, inv_freq[256];
  orc_yarn(c, &conc, inv_freq);
  for (int j = 0; j < c->head_dim / 2; j++) {
    const float val = (float)pos * inv_freq[j];
    cos_out[j] = cosf(val) * conc;
    sin_out[j] = sinf(val) * conc;
  }
}

void orc_rope_table(const orc_rope_cfg *c, int n_pos, float *cos_tab, float *sin_tab) {
  const int half = c->head_dim / 2;
  for (int p = 0; p < n_pos; p++)
    orc_cos_sin(c, p, cos_tab + (long)p * half, sin_tab + (long)p * half);
}

/* run.cpp:506-526; the products x2*s and x1*s are rounded, the others fused
 * (docs/04-bit-exact-gpu-port.md:40). */
void orc_rotate(float *x, const float *cosv, const float *sinv, int n_heads, int head_dim) {
  const int half = head_dim / 2;
  for (int h = 0; h < n_heads; h++)
    for (int i = 0; i < half; i++) {
      const float x1 = x[h * head_dim + i], x2 = x[h * head_dim + half + i];
      const float c = cosv[i], s = sinv[i];
      const float o1 = fmaf(x1, c, -(x2 * s));
      const float o2 = fmaf(x2, c, x1 * s);
      x[h * head_dim + i] = o1;
      x[h * head_dim + half + i] = o2;
    }
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_bf16_n(const float *x, uint16_t *y, long n) {
  for (long i = 0; i < n; i++)
    y[i] = orc_f32_to_bf16(x[i]);
}

/* run.cpp:335-353. */
void orc_softmax(float *x, int size) {
  double max_val = x[0];
  for (int i = 1; i < size; i++)
    if (x[i] > max_val)
      max_val = x[i];
  double sum = 0.0;
  for (int i = 0; i < size; i++) {
    x[i] = expf((float)((double)x[i] - max_val));
    sum += x[i];
  }
  for (int i = 0; i < size; i++)
    x[i] = (float)((double)x[i] / sum);
}

/* One query head over positions t0..pos (run.cpp:601-641). k/v point at the
 * head's element 0 of slot 0; slot s starts at s * slot_stride. att has room
 * for pos - t0 + 2 floats. */
static void attend(const float *q, const float *k, const float *v, long slot_stride, int ring,
                   int t0, int pos, float sink, int d, float *att, float *out) {
  const int n = pos - t0 + 1;
  const double scale = (double)sqrtf((float)d);
  for (int t = t0; t <= pos; t++) {
    const long slot = ring > 0 ? t % ring : t;
    const float *kt = k + slot * slot_stride;
    double score = 0.0;
    for (int i = 0; i < d; i++)
      score += (double)(q[i] * kt[i]);
    score /= scale;
    att[t - t0] = (float)score;
  }
  att[n] = sink;
  orc_softmax(att, n + 1);
  for (int i = 0; i < d; i++)
    out[i] = 0.0f;
  for (int t = t0; t <= pos; t++) {
    const long slot = ring > 0 ? t % ring : t;
    const float *vt = v + slot * slot_stride;
    const float a = att[t - t0];
    for (int i = 0; i < d; i++)
      out[i] = fmaf(a, vt[i], out[i]);
  }
}

int orc_decode_attention(int B, int n_q_heads, int n_kv_heads, int head_dim, const float *q,
                         long q_stride, const float *kc, const float *vc, long seq_stride,
                         const int *pos, const float *sinks, int window, int ring, float *out,
                         long out_stride, int n_threads) {
  if (B < 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0 || head_dim <= 0 ||
      head_dim % 2 != 0 || window < 0 || ring < 0 || (ring > 0 && window > ring))
    return -1;
  int max_pos = 0;
  for (int b = 0; b < B; b++) {
    if (pos[b] < 0 || (ring == 0 && (long)(pos[b] + 1) * n_kv_heads * head_dim > seq_stride))
      return -1;
    if (pos[b] > max_pos)
      max_pos = pos[b];
  }
  const int kv_mul = n_q_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim;
  const long work = (long)B * n_q_heads;
  (void)n_threads;
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : omp_get_max_threads())
  {
    float *att = (float *)malloc(sizeof(float) * (size_t)(max_pos + 2));
#pragma omp for schedule(dynamic, 4)
    for (long w = 0; w < work; w++) {
      const int b = (int)(w / n_q_heads), h = (int)(w % n_q_heads), g = h / kv_mul;
      const int p = pos[b];
      const int t0 = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
      const long base = (long)b * seq_stride + (long)g * head_dim;
      attend(q + (long)b * q_stride + (long)h * head_dim, kc + base, vc + base, kv_dim, ring, t0,
             p, sinks[h], head_dim, att, out + (long)b * out_stride + (long)h * head_dim);
    }
    free(att);
  }
  return 0;
}

int orc_prefill_attention(int B, int n_q_heads, int n_kv_heads, int head_dim,
                          const int *cu_seqlens, const float *q, long q_stride,
                          const float *k, const float *v, long kv_stride, const float *sinks,
                          int window, float *out, long out_stride, int n_threads) {
  if (B < 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0 || head_dim <= 0 || window < 0)
    return -1;
  int max_len = 0;
  for (int b = 0; b < B; b++) {
    const int L = cu_seqlens[b + 1] - cu_seqlens[b];
    if (L < 0)
      return -1;
    if (L > max_len)
      max_len = L;
  }
  const int kv_mul = n_q_heads / n_kv_heads;
  const long rows = cu_seqlens[B];
  (void)n_threads;
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : omp_get_max_threads())
  {
    float *att = (float *)malloc(sizeof(float) * (size_t)(max_len + 2));
#pragma omp for schedule(dynamic, 8)
    for (long w = 0; w < rows * n_q_heads; w++) {
      const long row = w / n_q_heads;
      const int h = (int)(w % n_q_heads), g = h / kv_mul;
      int b = 0;
      while (cu_seqlens[b + 1] <= row)
        b++;
      const long r0 = cu_seqlens[b];
      const int j = (int)(row - r0);
      const int t0 = (window > 0 && j - window + 1 > 0) ? j - window + 1 : 0;
      const long base = r0 * kv_stride + (long)g * head_dim;
      attend(q + row * q_stride + (long)h * head_dim, k + base, v + base, kv_stride, 0, t0, j,
             sinks[h], head_dim, att, out + row * out_stride + (long)h * head_dim);
    }
    free(att);
  }
  return 0;
}

void orc_kv_append(int B, int n_q_heads, int n_kv_heads, int head_dim, const float *qkv,
                   long row_stride, const float *cos_tab, const float *sin_tab, const int *pos,
                   float *q_rot, float *k_rot, uint16_t *k_bf16, uint16_t *v_bf16) {
  const int half = head_dim / 2, kv_dim = n_kv_heads * head_dim, qd = n_q_heads * head_dim;
  float *tmp = (float *)malloc(sizeof(float) * (size_t)(qd > kv_dim ? qd : kv_dim));
  for (int b = 0; b < B; b++) {
    const float *row = qkv + (long)b * row_stride;
    const float *c = cos_tab + (long)pos[b] * half, *s = sin_tab + (long)pos[b] * half;
    if (q_rot) {
      memcpy(tmp, row, sizeof(float) * qd);
      orc_rotate(tmp, c, s, n_q_heads, head_dim);
      memcpy(q_rot + (long)b * qd, tmp, sizeof(float) * qd);
    }
    memcpy(tmp, row + qd, sizeof(float) * kv_dim);
    orc_rotate(tmp, c, s, n_kv_heads, head_dim);
    if (k_rot)
      memcpy(k_rot + (long)b * kv_dim, tmp, sizeof(float) * kv_dim);
    for (int i = 0; i < kv_dim; i++) {
      k_bf16[(long)b * kv_dim + i] = orc_f32_to_bf16(tmp[i]);
      v_bf16[(long)b * kv_dim + i] = orc_f32_to_bf16(row[qd + kv_dim + i]);
    }
  }
  free(tmp);
}

/* fast_misc.hpp:74-84 / attn_test.cpp:218-226: amax over the head, the
 * reciprocal 127/amax rounded once, each value times it rounded, then rint
 * (ties to even) and the clamp. */
void orc_quantize_v(const float *v, int n_heads, int head_dim, int8_t *codes, float *scales) {
  for (int h = 0; h < n_heads; h++) {
    const float *x = v + (long)h * head_dim;
    float amax = 0.0f;
    for (int i = 0; i < head_dim; i++)
      amax = fmaxf(amax, fabsf(x[i]));
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    for (int i = 0; i < head_dim; i++) {
      float c = rintf(x[i] * inv);
      c = fminf(fmaxf(c, -127.0f), 127.0f);
      codes[(long)h * head_dim + i] = (int8_t)c;
    }
    scales[h] = amax / 127.0f;
  }
}

/* qkv rows of the QKV projection: out[r][i] = fp32(sum_j fp32(w[i][j] x[r][j]))
 * in a double accumulator, then + bias[i] in fp32 (run.cpp:355-367 matmul,
 * run.cpp:565-570 bias add), for n_rows input rows. */
void orc_linear(int n_rows, const float *x, long x_stride, const float *w, const float *bias,
                int n_in, int n_out, float *out, long out_stride) {
  long idx;
#pragma omp parallel for private(idx)
  for (idx = 0; idx < (long)n_rows * n_out; idx++) {
    const long r = idx / n_out, i = idx % n_out;
    const float *xr = x + r * x_stride;
    const float *wi = w + i * (long)n_in;
    double val = 0.0;
    for (int j = 0; j < n_in; j++) {
      const float prod = wi[j] * xr[j];
      val += prod;
    }
    float o = (float)val;
    if (bias)
      o += bias[i];
    out[r * out_stride + i] = o;
  }
}

/* ---- e4m3 (OCP FP8 E4M3) K/V cache ----------------------------------------
 * Not in the reference (its next step after int8 V). Format: sign, 4 exponent
 * bits (bias 7), 3 mantissa bits; exponent 0 holds the subnormals m * 2^-9;
 * S.1111.111 is NaN; no infinities; largest finite 448. */
float orc_fp8_value(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7)
    return NAN;
  const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
  return (c & 0x80) ? -v : v;
}

/* The e4m3 code nearest to x (|x| <= 448), ties to the even code. */
static uint8_t fp8_code(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  const uint8_t s = (uint8_t)((b >> 24) & 0x80u);
  const float a = fabsf(x);
  if (a < 0x1p-6f) /* subnormal steps of 2^-9; 8 steps is code 0x08 = 2^-6 */
    return s | (uint8_t)rintf(a * 0x1p9f);
  uint32_t ab = b & 0x7fffffffu;
  ab += 0x7ffffu + ((ab >> 20) & 1u); /* 23 mantissa bits -> 3, ties to even */
  const int e = (int)(ab >> 23) - 127 + 7;
  return s | (uint8_t)((e << 3) | ((ab >> 20) & 7u));
}

/* Per head of head_dim values: amax, the reciprocal 448/amax rounded once,
 * each value times it, clamped to +-448 and rounded to the nearest e4m3 code
 * (ties to even); scale = amax / 448. An all-zero head: scale 0, codes 0. */
void orc_quantize_fp8(const float *x, int n_heads, int head_dim, uint8_t *codes,
                      float *scales) {
  for (int h = 0; h < n_heads; h++) {
    const float *xh = x + (long)h * head_dim;
    float amax = 0.0f;
    for (int i = 0; i < head_dim; i++)
      amax = fmaxf(amax, fabsf(xh[i]));
    const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
    for (int i = 0; i < head_dim; i++) {
      const float c = fminf(fmaxf(xh[i] * inv, -448.0f), 448.0f);
      codes[(long)h * head_dim + i] = fp8_code(c);
    }
    scales[h] = amax / 448.0f;
  }
}

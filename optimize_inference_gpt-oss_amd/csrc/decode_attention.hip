// Split-K GQA flash-decoding over the paged bf16 KV cache, with per-head sink
// logits and the sliding window, plus the cross-split combine.
//
// Semantics: run.cpp:597-642 (score = q.k / sqrt(64), the sink as one more
// logit, softmax, weighted sum of values); window layers attend to the last W
// positions (run.cpp:170-176, 617-619), which a ring of W slots holds exactly
// (the slots in use are 0 .. min(len, W) - 1, and softmax does not depend on
// their order). Replaces attention_q8v_chunk64 / attention_bf16_chunk64
// (getp-csrc/kernels/fast_attention.hpp:566-622) and its in-workgroup merge
// (:383-424) with a paged, variable-length, cross-workgroup design.
//
// Work split. Workgroup (split s, kv head g, sequence b) owns tokens
// [s*split_tokens, (s+1)*split_tokens) of the sequence and reads each of their
// K/V bytes exactly once for all G query heads of the group (GQA sharing). Its
// NW waves take 32-token steps round-robin, each keeping its own online
// softmax; the waves merge through LDS. A sequence with one split is finished
// in place (sink added, output written); otherwise the split's (m, l, o) goes
// to the workspace and decode_combine_kernel merges the splits with the sink.
//
// Matrix cores: v_mfma_f32_16x16x32_bf16, 16x16 output, K = 32.
//   scores  S^T[token][col] = K[token][dims] * Q^T[dims][col]      (2 MFMAs per 16 tokens)
//   output  O^T[dim][col]  += V^T[dim][tokens] * P^T[tokens][col]  (4 MFMAs per 32 tokens)
//   Columns 0..7 carry the bf16 of q (and p) of query head col, columns 8..15
//   the bf16 of what that rounding left over, so q and p keep ~16 bits; the
//   two column halves are added after the MFMA (DPP lane swap).
//   Step token order: output row 4*kg + r of score tile jt (kg = lane / 16) is
//   token 8*kg + 4*jt + r, so lane (kg, col) ends up holding the scores of
//   tokens 8*kg .. 8*kg+7 of its column -- exactly the P^T operand layout,
//   whose matching V^T operand is one 16-byte row piece of the transposed V
//   block. No register transposes, no LDS round trip.
//
// Memory: every load is 16 bytes per lane; one K load instruction covers 16
// half-rows of 64 bytes, one V load 2 x 512 contiguous bytes. The next step's
// 8 KB (per wave) is in flight while the current one is computed.
#include "gkv_device.hpp"

namespace gkv {

constexpr int kStep = 32;       // tokens per wave step
constexpr int kCols = 8;        // query heads per kv head handled (G <= 8)
constexpr int kMlStride = 16;   // floats of (m, l) per split partial: 8 heads x 2

struct DecodeArgs {
  const float *q;
  int64_t q_stride;
  const float *cos_tab, *sin_tab;
  const int32_t *seq_lens;
  const uint16_t *kc, *vc;
  const int32_t *table;
  int table_stride, num_blocks, n_kv_heads, ring, window;
  const float *sinks;
  int G;              // query heads per kv head
  int split_tokens;
  int max_splits;
  float *ws_o;        // [B][Hkv][max_splits][8][64]
  float *ws_ml;       // [B][Hkv][max_splits][8][2]
  void *out;
  int64_t out_stride;
  int out_bf16;
  uint32_t *dev_err;
};

__device__ __forceinline__ int seq_tokens(const DecodeArgs &a, int L) {
  return a.window > 0 ? min(L, a.window) : L;
}

// Tokens a sequence can have here: what its table row holds and what the
// grid and workspace were sized for.
__device__ __forceinline__ int capacity(const DecodeArgs &a) {
  return min(a.table_stride * kBlockTokens, a.max_splits * a.split_tokens);
}

__device__ __forceinline__ void store_out(void *out, int64_t idx, float v, int is_bf16) {
  if (is_bf16)
    ((__bf16 *)out)[idx] = (__bf16)v;
  else
    ((float *)out)[idx] = v;
}

__device__ __forceinline__ bf16x8 pack_pieces(const float (&x)[8], bool lo) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const __bf16 hi = (__bf16)x[i];
    r[i] = lo ? (__bf16)(x[i] - (float)hi) : hi;
  }
  return r;
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void decode_split_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  __shared__ float s_o[NW][kCols][D];
  __shared__ float s_m[NW][kCols], s_l[NW][kCols];

  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int L = a.seq_lens[b];
  int n = seq_tokens(a, L);
  // Capacity: the table row must hold the blocks of n tokens, and the grid /
  // workspace were sized for max_splits splits.
  const int cap = capacity(a);
  if (n > cap) {
    if (threadIdx.x == 0 && split == 0 && a.dev_err)
      atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
    n = cap;
  }
  const int n_splits = max(1, (n + a.split_tokens - 1) / a.split_tokens);
  if (split >= n_splits)
    return;
  const int t_begin = split * a.split_tokens;
  const int t_end = min(n, t_begin + a.split_tokens);
  const int n_steps = (max(t_end - t_begin, 0) + kStep - 1) / kStep;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const bool lo = col >= 8;
  const int head = col & 7;
  const bool head_ok = head < a.G;
  const int hq = g * a.G + head;

  // Query: dims 8*kg + i (first MFMA) and 32 + 8*kg + i (second); the two
  // halves of a RoPE pair sit in the same lane.
  float qa[8], qb[8];
  if (head_ok) {
    const float *qp = a.q + (int64_t)b * a.q_stride + hq * D + 8 * kg;
    const float4 x0 = *(const float4 *)(qp), x1 = *(const float4 *)(qp + 4);
    const float4 y0 = *(const float4 *)(qp + 32), y1 = *(const float4 *)(qp + 36);
    qa[0] = x0.x; qa[1] = x0.y; qa[2] = x0.z; qa[3] = x0.w;
    qa[4] = x1.x; qa[5] = x1.y; qa[6] = x1.z; qa[7] = x1.w;
    qb[0] = y0.x; qb[1] = y0.y; qb[2] = y0.z; qb[3] = y0.w;
    qb[4] = y1.x; qb[5] = y1.y; qb[6] = y1.z; qb[7] = y1.w;
    if (a.cos_tab) {
      const int pos = max(L - 1, 0);
      const float *cp = a.cos_tab + (int64_t)pos * (D / 2) + 8 * kg;
      const float *sp = a.sin_tab + (int64_t)pos * (D / 2) + 8 * kg;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float c = cp[i], s = sp[i];
        const float x1v = qa[i], x2v = qb[i];
        qa[i] = rope_first(x1v, x2v, c, s);
        qb[i] = rope_second(x1v, x2v, c, s);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++)
      qa[i] = qb[i] = 0.0f;
  }
  const float qscale = 0.125f * kLog2e; // 1/sqrt(64), and exp -> exp2
#pragma unroll
  for (int i = 0; i < 8; i++) {
    qa[i] *= qscale;
    qb[i] *= qscale;
  }
  const bf16x8 qop0 = pack_pieces(qa, lo), qop1 = pack_pieces(qb, lo);

  const float sink2 = head_ok ? a.sinks[hq] * kLog2e : 0.0f;
  float m_run = sink2; // running reference max (log2 units) of this column
  float lsum = 0.0f;
  f32x4 o[4];
#pragma unroll
  for (int nn = 0; nn < 4; nn++)
    o[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t head_elems = (int64_t)kBlockTokens * D; // one head of one block
  const int32_t *trow = a.table + (int64_t)b * a.table_stride;
  // Lane roles in the loads.
  const int m = col;                                          // MFMA row
  const int k_blk = m >> 3;                                   // K operand: block of the row's token
  const int k_row0 = 8 * ((m >> 2) & 1) + (m & 3);            // its row in the block (+4*jt)
  const int v_blk = kg >> 1;                                  // V operand: block of tokens 8kg..
  const int v_tok0 = 8 * (kg & 1);

  u32x4 kcur[4], vcur[4], knext[4], vnext[4];
  int valid_cur = 0, valid_next = 0;   // tokens of the step that exist
  int bad_cur = 0, bad_next = 0;       // bit j: block j of the step has an invalid id

  auto load_step = [&](int step, u32x4 (&kr)[4], u32x4 (&vr)[4], int &valid, int &bad) {
    const int t0 = t_begin + step * kStep;
    valid = min(kStep, t_end - t0);
    const int blk0 = t0 / kBlockTokens;
    int p0 = uniform(trow[blk0]);
    int p1 = valid > kBlockTokens ? uniform(trow[blk0 + 1]) : p0;
    bad = 0;
    if (p0 < 0 || p0 >= a.num_blocks) {
      bad |= 1;
      p0 = 0;
    }
    if (p1 < 0 || p1 >= a.num_blocks) {
      bad |= 2;
      p1 = 0;
    }
    const int64_t hb0 = ((int64_t)p0 * a.n_kv_heads + g) * head_elems;
    const int64_t hb1 = ((int64_t)p1 * a.n_kv_heads + g) * head_elems;
    const int64_t kb = k_blk ? hb1 : hb0;
    const uint16_t *kp = a.kc + kb + (int64_t)k_row0 * D + 8 * kg;
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
      kr[2 * jt + 0] = *(const u32x4 *)(kp + jt * 4 * D);
      kr[2 * jt + 1] = *(const u32x4 *)(kp + jt * 4 * D + 32);
    }
    const uint16_t *vp = a.vc + (v_blk ? hb1 : hb0) + (int64_t)m * kBlockTokens + v_tok0;
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
      vr[nn] = *(const u32x4 *)(vp + nn * 16 * kBlockTokens);
  };

  int step = w;
  if (step < n_steps)
    load_step(step, kcur, vcur, valid_cur, bad_cur);
  for (; step < n_steps; step += NW) {
    if (step + NW < n_steps)
      load_step(step + NW, knext, vnext, valid_next, bad_next);

    // Scores of tokens 8*kg + 4*jt + r, this lane's column.
    float sc[8];
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, kcur[2 * jt + 0]), qop0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, kcur[2 * jt + 1]), qop1, acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++)
        sc[4 * jt + r] = acc[r] + swap8(acc[r]);
    }
    if (valid_cur < kStep || bad_cur) {
      // Tail of the sequence or a bad block id: those tokens get weight 0 and
      // their values (possibly never written) are replaced by zeros.
      if (bad_cur && lane == 0 && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
      const bool blk_bad = (bad_cur >> v_blk) & 1;
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (8 * kg + i >= valid_cur || blk_bad)
          sc[i] = -INFINITY;
      uint32_t keep[4];
#pragma unroll
      for (int h2 = 0; h2 < 4; h2++) {
        const int t = 8 * kg + 2 * h2;
        keep[h2] = blk_bad ? 0u
                           : ((t < valid_cur ? 0x0000ffffu : 0u) |
                              (t + 1 < valid_cur ? 0xffff0000u : 0u));
      }
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
#pragma unroll
        for (int h2 = 0; h2 < 4; h2++)
          vcur[nn][h2] &= keep[h2];
    }

    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; i++)
      mx = fmaxf(mx, sc[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // Lazy rescale: the reference max moves only when a score exceeds it by
    // more than 8 (weights stay below 2^8, harmless in fp32); the final
    // normalisation uses the same max, so the result does not change.
    if (__any(mx > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      lsum *= alpha;
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
        o[nn] *= alpha;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      p[i] = __builtin_amdgcn_exp2f(sc[i] - m_run);
      lsum += p[i];
    }
    const bf16x8 pop = pack_pieces(p, lo);
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
      o[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vcur[nn]), pop,
                                                      o[nn], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      kcur[j] = knext[j];
      vcur[j] = vnext[j];
    }
    valid_cur = valid_next;
    bad_cur = bad_next;
  }

  // Wave totals: sum over the 4 k-groups; the lo column adds its part of O.
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
#pragma unroll
  for (int nn = 0; nn < 4; nn++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      o[nn][r] += swap8(o[nn][r]);
  if (!lo) {
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        s_o[w][col][16 * nn + 4 * kg + r] = o[nn][r];
    if (kg == 0) {
      s_m[w][col] = m_run;
      s_l[w][col] = lsum;
    }
  }
  __syncthreads();

  // Merge the waves; finish single-split sequences, park the others.
  const int64_t part = ((int64_t)b * a.n_kv_heads + g) * a.max_splits + split;
  for (int idx = threadIdx.x; idx < kCols * D; idx += 64 * NW) {
    const int h = idx / D, d = idx % D;
    if (h >= a.G)
      continue;
    float M = s_m[0][h];
#pragma unroll
    for (int v = 1; v < NW; v++)
      M = fmaxf(M, s_m[v][h]);
    float Ls = 0.0f, Os = 0.0f;
#pragma unroll
    for (int v = 0; v < NW; v++) {
      const float c = __builtin_amdgcn_exp2f(s_m[v][h] - M);
      Ls = fmaf(s_l[v][h], c, Ls);
      Os = fmaf(s_o[v][h][d], c, Os);
    }
    if (n_splits == 1) {
      const float sk = a.sinks[g * a.G + h] * kLog2e;
      const float M2 = fmaxf(M, sk);
      const float f = __builtin_amdgcn_exp2f(M - M2);
      const float Lt = fmaf(Ls, f, __builtin_amdgcn_exp2f(sk - M2));
      store_out(a.out, (int64_t)b * a.out_stride + (g * a.G + h) * D + d, Os * f / Lt,
                a.out_bf16);
    } else {
      a.ws_o[part * (kCols * D) + idx] = Os;
      if (d == 0) {
        a.ws_ml[part * kMlStride + 2 * h] = M;
        a.ws_ml[part * kMlStride + 2 * h + 1] = Ls;
      }
    }
  }
}

// One workgroup per (kv head, sequence): merge the splits of the G query heads
// with the sink. M = max(sink, m_s), L = 2^(sink-M) + sum l_s 2^(m_s-M),
// out = sum o_s 2^(m_s-M) / L  (the merge of fast_attention.hpp:403-424, across
// workgroups).
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  const int g = blockIdx.x, b = blockIdx.y;
  const int n = min(seq_tokens(a, a.seq_lens[b]), capacity(a));
  const int n_splits = max(1, (n + a.split_tokens - 1) / a.split_tokens);
  if (n_splits <= 1)
    return;
  const int64_t part0 = ((int64_t)b * a.n_kv_heads + g) * a.max_splits;
  for (int idx = threadIdx.x; idx < kCols * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    if (h >= a.G)
      continue;
    const float sk = a.sinks[g * a.G + h] * kLog2e;
    float M = sk;
    for (int s = 0; s < n_splits; s++)
      M = fmaxf(M, a.ws_ml[(part0 + s) * kMlStride + 2 * h]);
    float Ls = __builtin_amdgcn_exp2f(sk - M), Os = 0.0f;
    for (int s = 0; s < n_splits; s++) {
      const float c = __builtin_amdgcn_exp2f(a.ws_ml[(part0 + s) * kMlStride + 2 * h] - M);
      Ls = fmaf(a.ws_ml[(part0 + s) * kMlStride + 2 * h + 1], c, Ls);
      Os = fmaf(a.ws_o[(part0 + s) * (kCols * D) + idx], c, Os);
    }
    store_out(a.out, (int64_t)b * a.out_stride + (g * a.G + h) * D + d, Os / Ls, a.out_bf16);
  }
}

constexpr int kDefaultSplitTokens = 512;
constexpr int kWaves = 4;

static int max_splits_of(int max_seq_len, int window, int split_tokens) {
  const int n = window > 0 ? std::min(max_seq_len, window) : max_seq_len;
  return std::max(1, (n + split_tokens - 1) / split_tokens);
}

static size_t workspace_bytes(int B, int n_kv_heads, int max_splits) {
  const size_t parts = (size_t)B * n_kv_heads * max_splits;
  return parts * (kCols * kHeadDim + kMlStride) * sizeof(float);
}

static int prepare(DecodeArgs &a, int32_t B, int32_t n_q_heads, const float *q, int64_t q_stride,
                   const float *cos_tab, const float *sin_tab, const int32_t *seq_lens,
                   int32_t max_seq_len, const gkv_cache_view &cache, int32_t window,
                   const float *sinks, int32_t split_tokens, void *workspace,
                   size_t workspace_bytes_given, void *out, int64_t out_stride,
                   int32_t out_dtype, uint32_t *dev_err, bool need_q) {
  if (B < 0 || n_q_heads <= 0 || cache.n_kv_heads <= 0 || !seq_lens || !sinks || !out ||
      max_seq_len < 0 || window < 0 || (out_dtype != GKV_F32 && out_dtype != GKV_BF16))
    return GKV_ERR_ARG;
  if (need_q && (!q || !cache.k || !cache.v || !cache.block_table || cache.table_stride <= 0 ||
                 cache.num_blocks <= 0 || (cos_tab && !sin_tab)))
    return GKV_ERR_ARG;
  if (n_q_heads % cache.n_kv_heads != 0)
    return GKV_ERR_ARG;
  const int G = n_q_heads / cache.n_kv_heads;
  if (G > kCols)
    return GKV_ERR_UNSUPPORTED;
  if (need_q && q_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  if (out_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  if (split_tokens == 0)
    split_tokens = kDefaultSplitTokens;
  if (split_tokens < 0 || split_tokens % (kStep * kWaves) != 0)
    return GKV_ERR_ARG;
  if (window > 0 && cache.ring > 0 && cache.ring != window)
    return GKV_ERR_ARG;
  if (cache.ring > 0 && window == 0)
    return GKV_ERR_ARG; // a ring holds only the last W tokens
  const int max_splits = max_splits_of(max_seq_len, window, split_tokens);
  if (max_splits > 1) {
    if (!workspace || workspace_bytes_given < workspace_bytes(B, cache.n_kv_heads, max_splits))
      return GKV_ERR_WORKSPACE;
  }
  a.q = q;
  a.q_stride = q_stride;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.seq_lens = seq_lens;
  a.kc = (const uint16_t *)cache.k;
  a.vc = (const uint16_t *)cache.v;
  a.table = cache.block_table;
  a.table_stride = cache.table_stride;
  a.num_blocks = cache.num_blocks;
  a.n_kv_heads = cache.n_kv_heads;
  a.ring = cache.ring;
  a.window = window;
  a.sinks = sinks;
  a.G = G;
  a.split_tokens = split_tokens;
  a.max_splits = max_splits;
  const size_t parts = (size_t)B * cache.n_kv_heads * max_splits;
  a.ws_o = (float *)workspace;
  a.ws_ml = workspace ? (float *)workspace + parts * kCols * kHeadDim : nullptr;
  a.out = out;
  a.out_stride = out_stride;
  a.out_bf16 = out_dtype == GKV_BF16;
  a.dev_err = dev_err;
  return GKV_OK;
}

} // namespace gkv

using namespace gkv;

extern "C" size_t gkv_decode_workspace_bytes(int32_t B, int32_t n_kv_heads, int32_t max_seq_len,
                                             int32_t window, int32_t split_tokens) {
  if (B <= 0 || n_kv_heads <= 0 || max_seq_len < 0)
    return 0;
  if (split_tokens <= 0)
    split_tokens = kDefaultSplitTokens;
  const int ms = max_splits_of(max_seq_len, window, split_tokens);
  return ms > 1 ? workspace_bytes(B, n_kv_heads, ms) : 0;
}

extern "C" int gkv_decode_split(void *stream, int32_t B, int32_t n_q_heads, const float *q,
                                int64_t q_stride, const float *cos_tab, const float *sin_tab,
                                const int32_t *seq_lens, int32_t max_seq_len,
                                gkv_cache_view cache, int32_t window, const float *sinks,
                                int32_t split_tokens, void *workspace, size_t workspace_bytes_,
                                void *out, int64_t out_stride, int32_t out_dtype,
                                uint32_t *dev_err) {
  DecodeArgs a;
  const int st = prepare(a, B, n_q_heads, q, q_stride, cos_tab, sin_tab, seq_lens, max_seq_len,
                         cache, window, sinks, split_tokens, workspace, workspace_bytes_, out,
                         out_stride, out_dtype, dev_err, true);
  if (st != GKV_OK || B == 0)
    return st;
  hipLaunchKernelGGL(decode_split_kernel<kWaves>, dim3(a.max_splits, cache.n_kv_heads, B),
                     dim3(64 * kWaves), 0, (hipStream_t)stream, a);
  return launch_status(__func__);
}

extern "C" int gkv_decode_combine(void *stream, int32_t B, int32_t n_q_heads, int32_t n_kv_heads,
                                  const int32_t *seq_lens, int32_t max_seq_len, int32_t window,
                                  const float *sinks, int32_t split_tokens,
                                  const void *workspace, size_t workspace_bytes_, void *out,
                                  int64_t out_stride, int32_t out_dtype) {
  // The combine reads only the table capacity from the cache view.
  DecodeArgs a;
  gkv_cache_view cache{};
  cache.n_kv_heads = n_kv_heads;
  cache.table_stride = (max_seq_len + kBlockTokens - 1) / kBlockTokens + 1;
  cache.ring = 0;
  const int st = prepare(a, B, n_q_heads, nullptr, 0, nullptr, nullptr, seq_lens, max_seq_len,
                         cache, window, sinks, split_tokens, const_cast<void *>(workspace),
                         workspace_bytes_, out, out_stride, out_dtype, nullptr, false);
  if (st != GKV_OK || B == 0 || a.max_splits <= 1)
    return st;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(n_kv_heads, B), dim3(256), 0,
                     (hipStream_t)stream, a);
  return launch_status(__func__);
}

extern "C" int gkv_decode_attention(void *stream, int32_t B, int32_t n_q_heads, const float *q,
                                    int64_t q_stride, const float *cos_tab, const float *sin_tab,
                                    const int32_t *seq_lens, int32_t max_seq_len,
                                    gkv_cache_view cache, int32_t window, const float *sinks,
                                    int32_t split_tokens, void *workspace,
                                    size_t workspace_bytes_, void *out, int64_t out_stride,
                                    int32_t out_dtype, uint32_t *dev_err) {
  DecodeArgs a;
  int st = prepare(a, B, n_q_heads, q, q_stride, cos_tab, sin_tab, seq_lens, max_seq_len, cache,
                   window, sinks, split_tokens, workspace, workspace_bytes_, out, out_stride,
                   out_dtype, dev_err, true);
  if (st != GKV_OK || B == 0)
    return st;
  hipLaunchKernelGGL(decode_split_kernel<kWaves>, dim3(a.max_splits, cache.n_kv_heads, B),
                     dim3(64 * kWaves), 0, (hipStream_t)stream, a);
  if (int st2 = launch_status("decode_split_kernel"))
    return st2;
  if (a.max_splits > 1) {
    hipLaunchKernelGGL(decode_combine_kernel, dim3(cache.n_kv_heads, B), dim3(256), 0,
                       (hipStream_t)stream, a);
    if (int st2 = launch_status("decode_combine_kernel"))
      return st2;
  }
  return GKV_OK;
}

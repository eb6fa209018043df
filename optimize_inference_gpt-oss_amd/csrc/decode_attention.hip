// Split-K GQA flash-decoding over the paged bf16 KV cache, with per-head sink
// logits and the sliding window, plus the cross-split combine.
//
// Semantics: run.cpp:597-642 (score = q.k / sqrt(64), the sink as one more
// logit, softmax, weighted sum of values); window layers attend to the last W
// positions (run.cpp:170-176, 617-619), which a ring of W slots holds exactly
// (the slots in use are 0 .. min(len, W) - 1, and softmax does not depend on
// their order). Replaces attention_q8v_chunk64 / attention_bf16_chunk64
// (getp-csrc/kernels/fast_attention.hpp:566-622) and its in-workgroup merge
// (:383-424) with a paged, variable-length, token-balanced design.
//
// Work split (three launches).
//   plan     one workgroup: prefix sums of the sequences' token counts, each
//            padded to a multiple of 32, into `cu`; the total T is cut into
//            equal ranges of S tokens, one per split workgroup, and the first
//            sequence of each range is recorded. Lengths vary from 1 to
//            thousands of tokens; equal ranges keep every workgroup equally
//            busy, with as many workgroups as the GPU holds at once.
//   split    workgroup w owns tokens [w*S, (w+1)*S) of the concatenated
//            sequences, which can span several sequences (segments). Wave g
//            works on kv head g, so the workgroup's waves stream the H_kv
//            contiguous 2 KB head slices of each block together; each K/V byte
//            is read once for all G query heads of its group. A segment that
//            is a whole sequence is finished in place (sink added, output
//            written); a piece of a longer sequence leaves (m, l, o) partials
//            in the workspace at index b + w (unique: ranges are contiguous).
//            Waves raise their issue priority while they have more of their
//            range left, so that co-resident workgroups advance together
//            instead of the oldest waves running first and the others alone
//            at the end.
//   combine  one workgroup per sequence split over several ranges: merges the
//            partials with the sink; writes zeros for empty sequences.
//
// Matrix cores: v_mfma_f32_16x16x32_bf16, 16x16 output, K = 32.
//   scores  S^T[token][col] = K[token][dims] * Q^T[dims][col]      (2 MFMAs per 16 tokens)
//   output  O^T[dim][col]  += V^T[dim][tokens] * P^T[tokens][col]  (4 MFMAs per 32 tokens)
//   Columns 0..7 carry the bf16 of q (and p) of query head col, columns 8..15
//   the bf16 of what that rounding left over, so q and p keep ~16 bits; the
//   two column halves are added after the MFMA (DPP lane swap).
//   A step is 2 blocks (32 tokens); score tile jt is block jt, row m token m,
//   so lane (kg = lane/16, col) holds the scores of tokens 4kg..4kg+3 of each
//   block -- exactly its P^T operand slots, whose V^T operand is the same 4
//   tokens of one dim: an 8-byte piece of each transposed V block. No
//   register transposes, no LDS.
//
// Memory: raw buffer loads, one block of one head per instruction (scalar
// base, constant per-lane offset, 2 KB range); R - 1 steps (8 KB each) of
// every wave in flight. Every load is unconditional (indices are clamped), so
// the compiler's wait counts are exact and a step never waits for the
// prefetches issued after it.
#include "gkv_device.hpp"

#include <algorithm>
#include <cstdlib>

namespace gkv {

constexpr int kStep = 32;              // tokens per wave step
constexpr int kCols = 8;               // query heads per kv head handled (G <= 8)
constexpr int kMlStride = 16;          // floats of (m, l) per partial: 8 heads x 2
constexpr int kPartFloats = kCols * kHeadDim;
constexpr int kMaxWorkgroups = 2048;   // split workgroups per launch (workspace bound)
constexpr int kPlanHeader = 4;         // ints: T, S, workgroups used, unused
constexpr int kIdRegs = 4;             // block-id registers per wave: segments of <= 4096 tokens
constexpr int kMaxRange = kIdRegs * 64 * kBlockTokens;

struct DecodeArgs {
  const float *q;
  int64_t q_stride;
  const float *cos_tab, *sin_tab;
  const int32_t *seq_lens;
  const uint16_t *kc, *vc;
  const int32_t *table;
  int table_stride, num_blocks, n_kv_heads, window;
  int max_len;        // host bound of the tokens attended per sequence
  const float *sinks;
  int G;              // query heads per kv head
  int B;
  int n_wg;           // split workgroups launched
  int fixed_S;        // 0: S = T / n_wg (balanced); > 0: this S
  int prio;           // 1: waves raise their priority while behind
  int32_t *plan;      // [kPlanHeader][cu: B + 1][first sequence per workgroup: n_wg]
  float *ws_o;        // [B + kMaxWorkgroups][Hkv][8][64]
  float *ws_ml;       // [B + kMaxWorkgroups][Hkv][8][2]
  void *out;
  int64_t out_stride;
  int out_bf16;
  uint32_t *dev_err;
};

// Tokens attended by sequence b: its length, or the window, clamped to what
// the table row and the launch were sized for.
__device__ __forceinline__ int seq_tokens(const DecodeArgs &a, int b, bool *over = nullptr) {
  int n = a.seq_lens[b];
  if (a.window > 0)
    n = min(n, a.window);
  const int cap = min(a.table_stride * kBlockTokens, a.max_len);
  if (over)
    *over = n > cap;
  return max(min(n, cap), 0);
}

__device__ __forceinline__ int pad_step(int n) { return (n + kStep - 1) & ~(kStep - 1); }

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

// Wave issue priority 0..3 (s_setprio takes an immediate).
__device__ __forceinline__ void set_priority(int p) {
  switch (p) {
  case 3:
    __builtin_amdgcn_s_setprio(3);
    break;
  case 2:
    __builtin_amdgcn_s_setprio(2);
    break;
  case 1:
    __builtin_amdgcn_s_setprio(1);
    break;
  default:
    __builtin_amdgcn_s_setprio(0);
  }
}

// ---- plan ---------------------------------------------------------------------

constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(DecodeArgs a) {
  __shared__ int s_scan[2][kPlanThreads];
  __shared__ int s_total;
  const int t = threadIdx.x, B = a.B;
  int32_t *cu = a.plan + kPlanHeader, *first = cu + B + 1;
  const int per = (B + kPlanThreads - 1) / kPlanThreads;
  const int b0 = t * per;
  int local = 0;
  bool any_over = false;
  for (int i = 0; i < per; i++) {
    const int b = b0 + i;
    if (b < B) {
      bool over;
      local += pad_step(seq_tokens(a, b, &over));
      any_over |= over;
    }
  }
  if (any_over && a.dev_err)
    atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
  // inclusive scan of the per-thread sums (Hillis-Steele, double buffered)
  int buf = 0;
  s_scan[0][t] = local;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int v = s_scan[buf][t] + (t >= off ? s_scan[buf][t - off] : 0);
    s_scan[buf ^ 1][t] = v;
    buf ^= 1;
    __syncthreads();
  }
  int run = s_scan[buf][t] - local;
  for (int i = 0; i < per; i++) {
    const int b = b0 + i;
    if (b < B) {
      cu[b] = run;
      run += pad_step(seq_tokens(a, b));
    }
  }
  if (t == kPlanThreads - 1) {
    s_total = s_scan[buf][t];
    cu[B] = s_total;
  }
  // Every range starts as "no sequence" (B); then each sequence claims the
  // ranges whose first token it holds.
  for (int w = t; w < a.n_wg; w += kPlanThreads)
    first[w] = B;
  __syncthreads();
  const int T = s_total;
  int S = a.fixed_S;
  if (S == 0)
    S = max(kStep, pad_step((T + a.n_wg - 1) / a.n_wg));
  for (int i = 0; i < per; i++) {
    const int b = b0 + i;
    if (b < B) {
      const int c0 = cu[b], c1 = cu[b + 1];
      for (int w = (c0 + S - 1) / S; w * S < c1 && w < a.n_wg; w++)
        first[w] = b;
    }
  }
  if (t == 0) {
    a.plan[0] = T;
    a.plan[1] = S;
    a.plan[2] = min(a.n_wg, (T + S - 1) / S);
  }
}

// ---- split ----------------------------------------------------------------------

// R: depth of the register ring of loaded steps (R - 1 steps in flight ahead
// of the one being computed).
template <int R>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(R == 2 ? 4 : (R == 3 ? 3 : 2))))
void decode_split_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  const int w_id = blockIdx.x;
  const int T = a.plan[0], S = a.plan[1];
  const int rs = w_id * S;
  if (rs >= T)
    return;
  const int re = min(rs + S, T);
  const int32_t *cu = a.plan + kPlanHeader;
  const int first_b = a.plan[kPlanHeader + a.B + 1 + w_id];

  const int lane = threadIdx.x & 63;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // wave-uniform: kv head
  const int col = lane & 15, kg = lane >> 4;
  const bool lo = col >= 8;
  const int head = col & 7;
  const bool head_ok = head < a.G;
  const int hq = g * a.G + head;
  const int hq_c = head_ok ? hq : g * a.G; // a valid head for the padding columns

  // Per-lane load offsets (bytes), the same for every step.
  const uint32_t k_off = (uint32_t)(col * D + 8 * kg) * 2;
  const uint32_t v_off = (uint32_t)(col * kBlockTokens + 4 * kg) * 2; // + nn * 512
  const size_t head_bytes = (size_t)kBlockTokens * D * 2;               // 2 KB

  if (a.prio)
    if (a.prio)
    set_priority(3);

  // Block ids, up to kIdRegs * 64 per segment, one per lane per register:
  // loaded for the first segment here and for each next segment while the
  // current one streams, so a segment never starts with a dependent table
  // load. Rows are read with clamped indices (always inside the table).
  auto load_ids = [&](int bb, int blk0, int (&ids)[kIdRegs]) {
    const int32_t *row = a.table + (int64_t)bb * a.table_stride;
#pragma unroll
    for (int i = 0; i < kIdRegs; i++)
      ids[i] = row[min(blk0 + 64 * i + lane, a.table_stride - 1)];
  };
  int tv[kIdRegs];
  load_ids(min(first_b, a.B - 1), max(rs - cu[min(first_b, a.B - 1)], 0) / kBlockTokens, tv);

  for (int b = first_b; b < a.B; b++) {
    const int c0 = cu[b], c1 = cu[b + 1];
    if (c0 >= re)
      break;
    // ids of the segment after this one (the next sequence from its start)
    int tvn[kIdRegs];
    load_ids(min(b + 1, a.B - 1), 0, tvn);
    if (c1 == c0) { // empty sequence: the combine writes its zeros
#pragma unroll
      for (int i = 0; i < kIdRegs; i++)
        tv[i] = tvn[i];
      continue;
    }
    const int n = seq_tokens(a, b);
    const int t_begin = max(rs, c0) - c0;         // multiple of 32
    const int t_end = min(min(re, c1) - c0, n);   // real tokens of this segment end here
    const bool complete = rs <= c0 && c1 <= re;
    const int n_tok = max(t_end - t_begin, 0);
    const int n_steps = (n_tok + kStep - 1) / kStep;
    const int n_blk = (n_tok + kBlockTokens - 1) / kBlockTokens;
    const int L = a.seq_lens[b];
    const int seg0 = c0 + t_begin - rs; // tokens of the range before this segment
    uint32_t seg_bad = 0;               // a bad block id met in this segment

    // Block id j of the segment (j < n_blk <= 64 * kIdRegs); ids outside the
    // pool read block 0 and set bit (j & 1) of `bad`.
    auto block_id = [&](int j, uint32_t &bad) -> int {
      const int w = j >> 6, l = j & 63;
      int v = __builtin_amdgcn_readlane(tv[0], l);
#pragma unroll
      for (int i = 1; i < kIdRegs; i++)
        if (w == i)
          v = __builtin_amdgcn_readlane(tv[i], l);
      if (v < 0 || v >= a.num_blocks) {
        bad |= 1u << (j & 1);
        v = 0;
      }
      return v;
    };

    u32x4 kbuf[R][4], vbuf[R][4];
    uint32_t bad_ring[R];
    auto load_step = [&](int step, u32x4 (&kr)[4], u32x4 (&vr)[4], uint32_t &bad) {
      const int j0 = 2 * step;
      bad = 0;
      const int p0 = block_id(j0, bad);
      const int p1 = j0 + 1 < n_blk ? block_id(j0 + 1, bad) : p0;
      const size_t h0 = ((size_t)p0 * a.n_kv_heads + g) * head_bytes;
      const size_t h1 = ((size_t)p1 * a.n_kv_heads + g) * head_bytes;
      const __amdgpu_buffer_rsrc_t k0 = head_rsrc((const char *)a.kc + h0);
      const __amdgpu_buffer_rsrc_t k1 = head_rsrc((const char *)a.kc + h1);
      const __amdgpu_buffer_rsrc_t v0 = head_rsrc((const char *)a.vc + h0);
      const __amdgpu_buffer_rsrc_t v1 = head_rsrc((const char *)a.vc + h1);
      kr[0] = __builtin_amdgcn_raw_buffer_load_b128(k0, k_off, 0, 0);
      kr[1] = __builtin_amdgcn_raw_buffer_load_b128(k0, k_off + 64, 0, 0);
      kr[2] = __builtin_amdgcn_raw_buffer_load_b128(k1, k_off, 0, 0);
      kr[3] = __builtin_amdgcn_raw_buffer_load_b128(k1, k_off + 64, 0, 0);
#pragma unroll
      for (int nn = 0; nn < 4; nn++) {
        const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(v0, v_off + nn * 512, 0, 0);
        const u32x2 y = __builtin_amdgcn_raw_buffer_load_b64(v1, v_off + nn * 512, 0, 0);
        vr[nn] = u32x4{x[0], x[1], y[0], y[1]};
      }
    };

    // First loads out before the query work, so their latency overlaps it.
    // Every load is unconditional (indices clamped): the compiler's wait
    // counts are then exact, and a step never waits for later prefetches.
    const int last_step = max(n_steps - 1, 0);
#pragma unroll
    for (int r = 0; r < R - 1; r++)
      load_step(min(r, last_step), kbuf[r], vbuf[r], bad_ring[r]);

    // Query: dims 8*kg + i (first MFMA) and 32 + 8*kg + i (second); the two
    // halves of a RoPE pair sit in the same lane.
    float qa[8], qb[8];
    {
      const float *qp = a.q + (int64_t)b * a.q_stride + hq_c * D + 8 * kg;
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
        const float4 cc0 = *(const float4 *)cp, cc1 = *(const float4 *)(cp + 4);
        const float4 ss0 = *(const float4 *)sp, ss1 = *(const float4 *)(sp + 4);
        const float cv[8] = {cc0.x, cc0.y, cc0.z, cc0.w, cc1.x, cc1.y, cc1.z, cc1.w};
        const float sv[8] = {ss0.x, ss0.y, ss0.z, ss0.w, ss1.x, ss1.y, ss1.z, ss1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float x1v = qa[i], x2v = qb[i];
          qa[i] = rope_first(x1v, x2v, cv[i], sv[i]);
          qb[i] = rope_second(x1v, x2v, cv[i], sv[i]);
        }
      }
      const float qscale = head_ok ? 0.125f * kLog2e : 0.0f; // 1/sqrt(64); exp -> exp2
#pragma unroll
      for (int i = 0; i < 8; i++) {
        qa[i] *= qscale;
        qb[i] *= qscale;
      }
    }
    const bf16x8 qop0 = pack_pieces(qa, lo), qop1 = pack_pieces(qb, lo);

    const float sink2 = head_ok ? a.sinks[hq_c] * kLog2e : 0.0f;
    float m_run = sink2; // running reference max (log2 units) of this column
    float lsum = 0.0f;
    f32x4 o[4];
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
      o[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute_step = [&](int step, u32x4 (&kr)[4], u32x4 (&vr)[4], uint32_t bad) {
      // Scores of token 4*kg + r of block jt (slot 4*jt + r), this lane's column.
      float sc[8];
#pragma unroll
      for (int jt = 0; jt < 2; jt++) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[2 * jt + 0]),
                                                      qop0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[2 * jt + 1]),
                                                      qop1, acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++)
          sc[4 * jt + r] = acc[r] + swap8(acc[r]);
      }
      const int valid = min(kStep, n_tok - step * kStep);
      if (valid < kStep || bad) {
        // Tail of the sequence, padding, or a bad block id: those tokens get
        // weight 0 and their values (possibly never written) become zeros.
#pragma unroll
        for (int jt = 0; jt < 2; jt++) {
          const bool blk_bad = (bad >> jt) & 1;
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (16 * jt + 4 * kg + r >= valid || blk_bad)
              sc[4 * jt + r] = -INFINITY;
#pragma unroll
          for (int h2 = 0; h2 < 2; h2++) {
            const int t = 16 * jt + 4 * kg + 2 * h2;
            const uint32_t keep = blk_bad ? 0u
                                          : ((t < valid ? 0x0000ffffu : 0u) |
                                             (t + 1 < valid ? 0xffff0000u : 0u));
#pragma unroll
            for (int nn = 0; nn < 4; nn++)
              vr[nn][2 * jt + h2] &= keep;
          }
        }
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
        o[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vr[nn]), pop,
                                                        o[nn], 0, 0, 0);
    };

    // Ring: slot r holds step base + r; the load for step + R - 1 goes out
    // before step is computed. The step count is padded to a multiple of R;
    // padded steps re-load the last step (cache hits) and are fully masked.
    for (int base = 0; base < n_steps; base += R) {
      // priority from the share of the range still ahead of this wave
      if (a.prio)
        set_priority((4 * (S - seg0 - base * kStep) - 1) / S);
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int step = base + r;
        const int slot = (r + R - 1) % R;
        load_step(min(step + R - 1, last_step), kbuf[slot], vbuf[slot], bad_ring[slot]);
        seg_bad |= bad_ring[slot];
        compute_step(step, kbuf[r], vbuf[r], bad_ring[r]);
      }
    }
    if (seg_bad && lane == 0 && a.dev_err)
      atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
#pragma unroll
    for (int i = 0; i < kIdRegs; i++)
      tv[i] = tvn[i];

    // Wave totals: sum over the 4 k-groups; the lo column adds its part of O.
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        o[nn][r] += swap8(o[nn][r]);
    if (lo || !head_ok)
      continue;
    if (complete) {
      // out = o * 2^(m - M) / (l * 2^(m - M) + 2^(sink - M)), M = max(m, sink)
      const float M2 = fmaxf(m_run, sink2);
      const float f = __builtin_amdgcn_exp2f(m_run - M2);
      const float scale = f / fmaf(lsum, f, __builtin_amdgcn_exp2f(sink2 - M2));
      const int64_t ob = (int64_t)b * a.out_stride + (int64_t)hq * D + 4 * kg;
#pragma unroll
      for (int nn = 0; nn < 4; nn++) {
        if (a.out_bf16) {
          typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
          *(bf16x4 *)((__bf16 *)a.out + ob + 16 * nn) =
              bf16x4{(__bf16)(o[nn][0] * scale), (__bf16)(o[nn][1] * scale),
                     (__bf16)(o[nn][2] * scale), (__bf16)(o[nn][3] * scale)};
        } else {
          *(f32x4 *)((float *)a.out + ob + 16 * nn) = o[nn] * scale;
        }
      }
    } else {
      const int64_t part = ((int64_t)(b + w_id)) * a.n_kv_heads + g;
      float *wo = a.ws_o + part * kPartFloats + head * D + 4 * kg;
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
        *(f32x4 *)(wo + 16 * nn) = o[nn];
      if (kg == 0) {
        a.ws_ml[part * kMlStride + 2 * head] = m_run;
        a.ws_ml[part * kMlStride + 2 * head + 1] = lsum;
      }
    }
  }
}

// ---- combine --------------------------------------------------------------------

// One workgroup per sequence, wave g for kv head g; lane (h = lane / 8) merges
// dims 8*(lane % 8) .. +7 of query head h over the sequence's partials:
// M = max(sink, m_w), L = 2^(sink-M) + sum l_w 2^(m_w-M), out = sum o_w 2^(m_w-M) / L
// (the merge of fast_attention.hpp:403-424, across workgroups).
__global__ __launch_bounds__(512) void decode_combine_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  const int b = blockIdx.x;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, h = lane >> 3, d0 = 8 * (lane & 7);
  if (h >= a.G)
    return;
  const int32_t *cu = a.plan + kPlanHeader;
  const int S = a.plan[1];
  const int c0 = cu[b], c1 = cu[b + 1];
  const int64_t ob = (int64_t)b * a.out_stride + (int64_t)(g * a.G + h) * D + d0;
  if (c1 == c0) { // no tokens: all weight on the sink
    for (int i = 0; i < 8; i++)
      store_out(a.out, ob + i, 0.0f, a.out_bf16);
    return;
  }
  const int w0 = c0 / S, w1 = (c1 - 1) / S;
  if (w0 == w1)
    return; // finished by its split workgroup
  const float sk = a.sinks[g * a.G + h] * kLog2e;
  float M = sk;
  for (int w = w0; w <= w1; w++)
    M = fmaxf(M, a.ws_ml[((int64_t)(b + w) * a.n_kv_heads + g) * kMlStride + 2 * h]);
  float Ls = __builtin_amdgcn_exp2f(sk - M);
  f32x4 o0 = {0, 0, 0, 0}, o1 = {0, 0, 0, 0};
  for (int w = w0; w <= w1; w++) {
    const int64_t part = (int64_t)(b + w) * a.n_kv_heads + g;
    const float c = __builtin_amdgcn_exp2f(a.ws_ml[part * kMlStride + 2 * h] - M);
    Ls = fmaf(a.ws_ml[part * kMlStride + 2 * h + 1], c, Ls);
    const f32x4 *po = (const f32x4 *)(a.ws_o + part * kPartFloats + h * D + d0);
    o0 += po[0] * c;
    o1 += po[1] * c;
  }
  const float inv = 1.0f / Ls;
  for (int i = 0; i < 4; i++) {
    store_out(a.out, ob + i, o0[i] * inv, a.out_bf16);
    store_out(a.out, ob + 4 + i, o1[i] * inv, a.out_bf16);
  }
}

// ---- host side --------------------------------------------------------------------

constexpr int kRing = 4;

// Ring depth of the split kernel (default kRing; the tuning variable
// GKV_DECODE_RING = 2..4 picks another, read once).
static int ring_depth() {
  static const int r = [] {
    const char *e = getenv("GKV_DECODE_RING");
    const int v = e ? atoi(e) : kRing;
    return (v >= 2 && v <= 4) ? v : kRing;
  }();
  return r;
}

// Wave priority balancing (default on; GKV_DECODE_PRIO=0 switches it off).
static int prio_enabled() {
  static const int p = [] {
    const char *e = getenv("GKV_DECODE_PRIO");
    return e ? (atoi(e) != 0) : 1;
  }();
  return p;
}

static const void *split_kernel_fn(int ring) {
  switch (ring) {
  case 3:
    return (const void *)decode_split_kernel<3>;
  case 4:
    return (const void *)decode_split_kernel<4>;
  default:
    return (const void *)decode_split_kernel<2>;
  }
}

// Workgroups the GPU holds at once for the split kernel (CUs x per-CU
// occupancy), per device, measured once.
static int resident_workgroups(int n_kv_heads) {
  static int cache[64][9] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || n_kv_heads > 8)
    return 0;
  int &slot = cache[dev][n_kv_heads];
  if (slot == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, split_kernel_fn(ring_depth()),
                                                     64 * n_kv_heads, 0) != hipSuccess)
      return 0;
    slot = std::max(1, cus * per_cu);
  }
  return slot;
}

static size_t plan_bytes(int B) {
  return ((size_t)(kPlanHeader + B + 1 + kMaxWorkgroups) * 4 + 255) & ~(size_t)255;
}

static size_t workspace_bytes(int B, int n_kv_heads) {
  const size_t parts = (size_t)(B + kMaxWorkgroups) * n_kv_heads;
  return plan_bytes(B) + parts * (kPartFloats + kMlStride) * sizeof(float);
}

static int prepare(DecodeArgs &a, int32_t B, int32_t n_q_heads, const float *q, int64_t q_stride,
                   const float *cos_tab, const float *sin_tab, const int32_t *seq_lens,
                   int32_t max_seq_len, const gkv_cache_view &cache, int32_t window,
                   const float *sinks, int32_t split_tokens, void *workspace,
                   size_t workspace_bytes_given, void *out, int64_t out_stride,
                   int32_t out_dtype, uint32_t *dev_err, bool need_cache) {
  if (B < 0 || n_q_heads <= 0 || cache.n_kv_heads <= 0 || !seq_lens || !sinks || !out ||
      max_seq_len < 0 || window < 0 || (out_dtype != GKV_F32 && out_dtype != GKV_BF16))
    return GKV_ERR_ARG;
  if (need_cache && (!q || !cache.k || !cache.v || !cache.block_table ||
                     cache.table_stride <= 0 || cache.num_blocks <= 0 || (cos_tab && !sin_tab)))
    return GKV_ERR_ARG;
  if (n_q_heads % cache.n_kv_heads != 0)
    return GKV_ERR_ARG;
  if (cache.n_kv_heads > 8)
    return GKV_ERR_UNSUPPORTED; // one wave per kv head, 512 threads
  const int G = n_q_heads / cache.n_kv_heads;
  if (G > kCols)
    return GKV_ERR_UNSUPPORTED;
  if (need_cache && q_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  if (out_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  if (split_tokens < 0 || split_tokens % kStep != 0)
    return GKV_ERR_ARG;
  if (window > 0 && cache.ring > 0 && cache.ring != window)
    return GKV_ERR_ARG;
  if (cache.ring > 0 && window == 0)
    return GKV_ERR_ARG; // a ring holds only the last W tokens
  const int64_t n_max = window > 0 ? std::min(max_seq_len, window) : max_seq_len;
  const int64_t t_max = (int64_t)B * ((n_max + kStep - 1) / kStep * kStep);
  if (t_max >= INT32_MAX)
    return GKV_ERR_ARG;
  if (!workspace || workspace_bytes_given < workspace_bytes(B, cache.n_kv_heads))
    return GKV_ERR_WORKSPACE;
  // Ranges hold at most kMaxRange tokens (the block ids a wave keeps).
  const int64_t min_wg = (t_max + kMaxRange - 1) / kMaxRange;
  int64_t n_wg;
  if (split_tokens > 0) {
    if (split_tokens > kMaxRange)
      return GKV_ERR_ARG;
    n_wg = std::max<int64_t>(1, (t_max + split_tokens - 1) / split_tokens);
  } else {
    const int resident = (need_cache && B > 0) ? resident_workgroups(cache.n_kv_heads) : 1;
    if (resident <= 0)
      return GKV_ERR_HIP;
    n_wg = std::max<int64_t>(resident, min_wg);
  }
  if (n_wg > kMaxWorkgroups)
    return GKV_ERR_ARG;
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
  a.window = window;
  a.max_len = (int)n_max;
  a.sinks = sinks;
  a.G = G;
  a.B = B;
  a.n_wg = (int)n_wg;
  a.fixed_S = split_tokens;
  a.prio = prio_enabled();
  a.plan = (int32_t *)workspace;
  a.ws_o = (float *)((char *)workspace + plan_bytes(B));
  a.ws_ml = a.ws_o + (size_t)(B + kMaxWorkgroups) * cache.n_kv_heads * kPartFloats;
  a.out = out;
  a.out_stride = out_stride;
  a.out_bf16 = out_dtype == GKV_BF16;
  a.dev_err = dev_err;
  return GKV_OK;
}

static int launch_split(const DecodeArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, a);
  if (int st = launch_status("decode_plan_kernel"))
    return st;
  const dim3 grid(a.n_wg), block(64 * a.n_kv_heads);
  switch (ring_depth()) {
  case 3:
    hipLaunchKernelGGL(decode_split_kernel<3>, grid, block, 0, s, a);
    break;
  case 2:
    hipLaunchKernelGGL(decode_split_kernel<2>, grid, block, 0, s, a);
    break;
  default:
    hipLaunchKernelGGL(decode_split_kernel<4>, grid, block, 0, s, a);
  }
  return launch_status("decode_split_kernel");
}

static int launch_combine(const DecodeArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(decode_combine_kernel, dim3(a.B), dim3(64 * a.n_kv_heads), 0, s, a);
  return launch_status("decode_combine_kernel");
}

} // namespace gkv

using namespace gkv;

extern "C" size_t gkv_decode_workspace_bytes(int32_t B, int32_t n_kv_heads, int32_t max_seq_len,
                                             int32_t window, int32_t split_tokens) {
  (void)max_seq_len;
  (void)window;
  (void)split_tokens;
  if (B < 0 || n_kv_heads <= 0)
    return 0;
  return workspace_bytes(B, n_kv_heads);
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
  return launch_split(a, (hipStream_t)stream);
}

extern "C" int gkv_decode_combine(void *stream, int32_t B, int32_t n_q_heads, int32_t n_kv_heads,
                                  const int32_t *seq_lens, int32_t max_seq_len, int32_t window,
                                  const float *sinks, int32_t split_tokens,
                                  const void *workspace, size_t workspace_bytes_, void *out,
                                  int64_t out_stride, int32_t out_dtype) {
  DecodeArgs a;
  gkv_cache_view cache{};
  cache.n_kv_heads = n_kv_heads;
  const int st = prepare(a, B, n_q_heads, nullptr, 0, nullptr, nullptr, seq_lens, max_seq_len,
                         cache, window, sinks, split_tokens, const_cast<void *>(workspace),
                         workspace_bytes_, out, out_stride, out_dtype, nullptr, false);
  if (st != GKV_OK || B == 0)
    return st;
  return launch_combine(a, (hipStream_t)stream);
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
  if ((st = launch_split(a, (hipStream_t)stream)))
    return st;
  return launch_combine(a, (hipStream_t)stream);
}

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
// Three launches.
//   prep     Lays all sequences end to end in one token stream, each padded
//            to whole steps of 32 tokens (prefix sums `cu`), and cuts the
//            stream into equal ranges of S tokens, one per split workgroup
//            (as many as the GPU holds at once). For every 16-token block of
//            the stream it records the physical block id (checked against the
//            pool) and for every step its sequence, how many of its tokens
//            exist, and whether it is the sequence's first or last step. It
//            also prepares each (sequence, kv head)'s query operands: RoPE at
//            the sequence's last position, the 1/8 scale and log2(e), split
//            into bf16 high and low pieces, in the register layout of the
//            matrix-core operand.
//   split    Workgroup w streams steps [w*S, (w+1)*S)/32 of the stream for
//            every kv head, one wave per SIMD (wave i takes heads i, i+4, ...).
//            A range spans several sequences and the loads never stop at a
//            sequence boundary: each step's block ids and step record come
//            from registers loaded once per range, and its query operands
//            travel in the load ring with its K and V; at a boundary only the
//            softmax state is flushed. Each K/V byte is read once for all G
//            query heads of its group. A sequence inside one range is
//            finished in place (sink added, output written); a piece of a
//            longer sequence leaves (m, l, o) partials in the workspace at
//            index b + w (unique: ranges are contiguous).
//   combine  one workgroup per range: the range's split launch (or the prep
//            launch) recorded the sequence the range starts inside of; the
//            first range inside a sequence merges its partials with the
//            sink. Empty sequences get zeros from the split (or prep) launch.
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
//   tokens of one dim. The pool's block layouts (k_offset / v_offset) store
//   each lane's operand pieces as 16 contiguous bytes in lane order, so every
//   load instruction reads 1 KB contiguous: whole 128-byte lines. No
//   register transposes, no LDS.
//
// Memory: raw nontemporal buffer loads, half a block of one head per
// instruction (scalar base, constant per-lane offset); R - 1 steps (8 KB of K/V
// each) in flight per wave, held in VGPRs and AGPRs (one wave per SIMD: two
// waves on a SIMD are not served equally, the older one issues first, which
// leaves the younger ones running alone at the end). Every load is
// unconditional (indices are clamped), so the compiler's wait counts are
// exact and a step never waits for the prefetches issued after it.
#include "kv_append.hpp"
#include "lds_dma.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>

namespace gkv {

// Cache policy of the K/V loads: nontemporal (the cache is read once per
// step). Measured on the MI355X, a gather of random 2 KB blocks reads 6.9 TB/s
// with it against 6.1 TB/s without, provided each load instruction covers
// whole 128-byte lines (1 KB contiguous per wave).
#ifndef GKV_KV_AUX
constexpr int kKvAux = 2;
#else
constexpr int kKvAux = GKV_KV_AUX;
#endif
constexpr int kStep = 32;              // tokens per wave step
constexpr int kCols = 8;               // query heads per kv head handled (G <= 8)
constexpr int kMlStride = 16;          // floats of (m, l) per partial: 8 heads x 2
constexpr int kPartFloats = kCols * kHeadDim;
constexpr int kMaxWorkgroups = 1024;   // split workgroups per launch (workspace bound)
constexpr int kPartsPerRange = 2;      // partial results per range: its first and its last segment
constexpr int kPlanHeader = 4;         // ints: T, S, workgroups used, unused
constexpr int kMaxRange = 16384;       // tokens per range (its ids and records sit in LDS)
constexpr int kIdSlab = kMaxRange / kBlockTokens; // block ids per range (its slab in the workspace)
constexpr int kInfoSlab = kMaxRange / kStep;      // step records per range
constexpr int kSplitWaves = 4;         // split kernel: one wave per SIMD
constexpr int kStageRecs = 8;          // finished segments a stream wave holds in LDS
constexpr int kSplitThreads = 64 * kSplitWaves;
constexpr int kMaxSplitWaves = 8;      // the fused kernel's 8-wave form: two waves per SIMD
constexpr int kShortRangeTokens = 256; // stream per workgroup up to which that form is used
constexpr int kPrepThreads = 1024;
constexpr int kMaxBatch = 8192;        // sequences per call (prefix sums kept in LDS)
constexpr int kBadBlock = -1;          // F entry: id outside the pool
constexpr int kPadBlock = -2;          // F entry: no tokens (padding)
// A decode layer's plan kept for the following layers of its kind (the same
// lengths): a key naming what it was built for (the shape, the pointers and a
// hash of the lengths' contents), then each range's bounds, first sequence and
// count of sequences; the step records and the table position of every block
// (row * table_stride + column, not the id it held: a reusing launch reads the
// ids from the table afresh, so a changed table entry is never stale) stay in
// the range slabs (flat, steps).
constexpr int kKeyInts = 16;
constexpr int kPlanMagic = 0x504c4e31;
constexpr int kKeepPlan = 2;           // fused launch mode bits (bit 0: append)
constexpr int kReusePlan = 4;

// Step record: sequence << 8 | first step of the sequence << 7 | its last
// step << 6 | tokens of the step that exist (0..32).
__host__ __device__ constexpr int step_record(int b, bool first, bool last, int valid) {
  return (b << 8) | (first ? 0x80 : 0) | (last ? 0x40 : 0) | valid;
}

struct DecodeArgs {
  const float *q;
  int64_t q_stride;
  const float *cos_tab, *sin_tab;
  const int32_t *seq_lens;
  const uint16_t *kc, *vc;
  const float *vs;    // int8 V: fp32 scales [block][head][16]; e4m3 K/V: [block][head][32]
  int kv_fp8;         // K and V as e4m3 codes + scales (GKV_KV_FP8)
  const int32_t *table;
  int table_stride, num_blocks, n_kv_heads, window;
  int max_len;        // host bound of the tokens attended per sequence
  const float *sinks;
  int G;              // query heads per kv head
  int B;
  int n_wg;           // split workgroups launched
  int fixed_S;        // 0: n_wg balanced ranges (range_start); > 0: ranges of this S
  int aligned;        // ranges of whole sequences (fused launch only; no partials)
  int32_t *plan;      // [kPlanHeader][cu: B + 1][boundary sequence: one per range]
                      // [range start: one per range, then T]
  int32_t *flat;      // block id of every 16-token block of the stream, per range:
                      // [range][kIdSlab], block k of range w at w * kIdSlab + k
  int32_t *steps;     // step record of every 32-token step: [range][kInfoSlab]
  u32x4 *qops;        // [B][Hkv][64 lanes][2]: query operands
  int32_t *kept;      // kept plan: [kKeyInts] key, then int4 {rs, re, b_first, n_seq} per range
  float *ws_o;        // [range][kPartsPerRange][Hkv][8][64]: partial outputs
  float *ws_ml;       // [range][kPartsPerRange][Hkv][8][2]: their (m, l)
  int4 *crec;         // [range]: the combine's record ({b, w0, w1, cu[b]} of the sequence the
                      // range is the first to start inside of; b = -1: none)
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

__host__ __device__ __forceinline__ int pad_step(int n) { return (n + kStep - 1) & ~(kStep - 1); }

// The ranges of the stream (T tokens, whole steps of 32). S > 0: range k is
// [k S, (k + 1) S) (a forced split size); S = 0: the n ranges split the T / 32
// steps as evenly as whole steps allow, range k starting at step
// floor(k N / n), N = T / 32, so that no workgroup holds a range one step
// longer than another's plus one (a balanced S rounded up to a step would
// leave the last range short and its workgroup idle).
__device__ __forceinline__ int range_start(int k, int T, int S, int n) {
  if (S > 0)
    return min((int64_t)k * S, (int64_t)T);
  if (k >= n)
    return T;
  return (int)((int64_t)k * (T / kStep) / n) * kStep;
}

// The range holding stream position p (0 <= p < T): the last k with
// range_start(k) <= p.
__device__ __forceinline__ int range_of(int p, int T, int S, int n) {
  if (S > 0)
    return p / S;
  const int64_t q = p / kStep;
  return (int)(((q + 1) * n - 1) / (T / kStep));
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

// Four int8 codes (one per byte) -> four bf16 (exact: |code| <= 127), in order.
// (Each conversion compiles to one v_cvt_f32_i32 with a sign-extended byte
// select.)
__device__ __forceinline__ u32x2 int8x4_to_bf16x4(uint32_t w) {
  uint32_t h[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = (int)(w << (24 - 8 * i)) >> 24; // sign-extended byte i
    h[i] = __float_as_uint((float)c) >> 16;
  }
  return u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
}

// The combine's record for range w, which starts at stream position rs and
// inside sequence b ([c0, c1) of the stream; b = -1: at a sequence's start or
// past the stream): the sequence's pieces are in ranges w0 = w - 1 .. w1,
// and range w merges them if it is the first range to start inside it.
__device__ __forceinline__ int4 combine_record(int w, int b, int c0, int c1, int T, int S,
                                               int n) {
  if (b < 0 || w == 0 || range_start(w - 1, T, S, n) > c0)
    return int4{-1, 0, 0, 0};
  return int4{b, w - 1, range_of(c1 - 1, T, S, n), c0};
}

// ---- prep -----------------------------------------------------------------------

// Query operands of sequence b, kv head g, for one wave. Lane (kg = lane/16,
// col): column col is query head g*G + (col & 7) (zero past G), the high bf16
// piece for col < 8, the low piece for col >= 8; operand 0 holds dims
// 8kg .. 8kg+7, operand 1 dims 32 + 8kg .. +7 (the two halves of each RoPE
// pair sit in the same lane).
__device__ void prep_queries(const DecodeArgs &a, int item) {
  constexpr int D = kHeadDim;
  const int b = item / a.n_kv_heads, g = item - b * a.n_kv_heads;
  const int lane = threadIdx.x & 63, col = lane & 15, kg = lane >> 4;
  const bool lo = col >= 8;
  const int head = col & 7;
  const bool head_ok = head < a.G;
  const int hq = g * a.G + (head_ok ? head : 0);
  const float *qp = a.q + (int64_t)b * a.q_stride + hq * D + 8 * kg;
  float qa[8], qb[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    qa[i] = qp[i];
    qb[i] = qp[32 + i];
  }
  if (a.cos_tab) {
    const int pos = max(a.seq_lens[b] - 1, 0);
    const float *cp = a.cos_tab + (int64_t)pos * (D / 2) + 8 * kg;
    const float *sp = a.sin_tab + (int64_t)pos * (D / 2) + 8 * kg;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x1 = qa[i], x2 = qb[i], c = cp[i], s = sp[i];
      qa[i] = rope_first(x1, x2, c, s);
      qb[i] = rope_second(x1, x2, c, s);
    }
  }
  const float qscale = head_ok ? 0.125f * kLog2e : 0.0f; // 1/sqrt(64); exp -> exp2
#pragma unroll
  for (int i = 0; i < 8; i++) {
    qa[i] *= qscale;
    qb[i] *= qscale;
  }
  u32x4 *dst = a.qops + ((int64_t)item * 64 + lane) * 2;
  dst[0] = __builtin_bit_cast(u32x4, pack_pieces(qa, lo));
  dst[1] = __builtin_bit_cast(u32x4, pack_pieces(qb, lo));
}

// Query operands: one wave per (sequence, kv head). wg / n_wgs: this
// workgroup's index among the query workgroups and their count.
__device__ __forceinline__ void prep_query_items(const DecodeArgs &a, int wg, int n_wgs) {
  const int waves = kPrepThreads / 64;
  for (int item = wg * waves + (threadIdx.x >> 6); item < a.B * a.n_kv_heads;
       item += n_wgs * waves)
    prep_queries(a, item);
}

// Every block workgroup computes the prefix sums in LDS (the lengths are 4
// bytes per sequence, cheap to read again), then takes its share of the
// stream blocks; workgroup 0 also publishes the plan. wg / n_wgs: this
// workgroup's index among the block workgroups and their count.
__device__ __forceinline__ void prep_blocks(const DecodeArgs &a, int wg, int n_wgs) {
  constexpr int kWaves = kPrepThreads / 64;
  constexpr int kPer = (kMaxBatch + kPrepThreads - 1) / kPrepThreads;
  __shared__ int s_cu[kMaxBatch + 1];
  __shared__ int s_wave[kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, B = a.B;
  const int per = (B + kPrepThreads - 1) / kPrepThreads;
  const int b0 = t * per;
  // padded lengths of this thread's sequences, kept in registers for the
  // second pass (a reload after the barriers would be one more round trip)
  int len[kPer];
  int local = 0;
  bool any_over = false;
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    len[i] = 0;
    if (i < per && b0 + i < B) {
      bool over;
      len[i] = pad_step(seq_tokens(a, b0 + i, &over));
      any_over |= over;
    }
    local += len[i];
  }
  if (any_over && wg == 0 && a.dev_err)
    atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
  // inclusive scan: within each wave by shuffles, then over the wave totals
  int incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off)
      incl += v;
  }
  if (lane == 63)
    s_wave[wave] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; w++) {
    const int v = s_wave[w];
    before += w < wave ? v : 0;
    total += v;
  }
  int run = before + incl - local;
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    if (i < per && b0 + i < B) {
      s_cu[b0 + i] = run;
      run += len[i];
    }
  }
  if (t == 0)
    s_cu[B] = total;
  __syncthreads();
  const int T = s_cu[B];
  const int S = a.fixed_S, n_r = a.n_wg;
  if (wg == 0) {
    int32_t *cu = a.plan + kPlanHeader;
    for (int b = t; b <= B; b += kPrepThreads)
      cu[b] = s_cu[b];
    if (t == 0) {
      a.plan[0] = T;
      a.plan[1] = S;
      a.plan[2] = n_r;
      a.plan[3] = 0;
      if (a.kept)
        a.kept[0] = 0; // a kept plan is valid until a launch plans afresh
    }
    // per range, the sequence it starts inside of (-1: none), for the combine
    for (int w = t; w < a.n_wg; w += kPrepThreads) {
      const int tok = range_start(w, T, S, n_r);
      int v = -1;
      if (tok < T) {
        int lo = 0, hi = B - 1; // the last b with cu[b] <= tok
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (s_cu[mid] <= tok)
            lo = mid;
          else
            hi = mid - 1;
        }
        v = tok > s_cu[lo] ? lo : -1;
      }
      a.plan[kPlanHeader + B + 1 + w] = v;
      a.crec[w] = combine_record(w, v, v >= 0 ? s_cu[v] : 0, v >= 0 ? s_cu[v + 1] : 0, T, S, n_r);
    }
    for (int w = t; w <= a.n_wg; w += kPrepThreads)
      a.plan[kPlanHeader + B + 1 + a.n_wg + w] = range_start(w, T, S, n_r);
  }
  // sequences without tokens: output 0
  {
    const int n_out = a.n_kv_heads * a.G * kHeadDim;
    for (int b = wg; b < B; b += n_wgs)
      if (s_cu[b + 1] == s_cu[b])
        for (int i = t; i < n_out; i += kPrepThreads)
          store_out(a.out, (int64_t)b * a.out_stride + i, 0.0f, a.out_bf16);
  }

  // Stream blocks (and the step records at even blocks), grid-strided.
  bool any_bad = false;
  const int n_e = T / kBlockTokens;
  for (int e = wg * kPrepThreads + t; e < n_e; e += n_wgs * kPrepThreads) {
    const int tok = e * kBlockTokens;
    int lo = 0, hi = B - 1; // the sequence holding the block: last b with cu[b] <= tok
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cu[mid] <= tok)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int b = lo;
    const int off = tok - s_cu[b];
    const int n = seq_tokens(a, b);
    int id = kPadBlock;
    if (off < n) {
      id = a.table[(int64_t)b * a.table_stride + off / kBlockTokens];
      if (id < 0 || id >= a.num_blocks) {
        id = kBadBlock;
        any_bad = true;
      }
    }
    const int w = range_of(tok, T, S, n_r); // the range, and the block's place in its slab
    const int in_r = tok - range_start(w, T, S, n_r);
    a.flat[w * kIdSlab + in_r / kBlockTokens] = id;
    if ((e & 1) == 0)
      a.steps[w * kInfoSlab + in_r / kStep] =
          step_record(b, off == 0, tok + kStep == s_cu[b + 1], min(max(n - off, 0), kStep));
  }
  if (any_bad && a.dev_err)
    atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
}

// Workgroups 0 .. n_qwg-1 prepare the query operands, the others the plan
// and the stream blocks: the two chains (query loads; lengths, prefix sums,
// table loads) run side by side.
__global__ __launch_bounds__(kPrepThreads) void decode_prep_kernel(DecodeArgs a, int n_qwg) {
  if ((int)blockIdx.x < n_qwg)
    prep_query_items(a, blockIdx.x, n_qwg);
  else
    prep_blocks(a, blockIdx.x - n_qwg, gridDim.x - n_qwg);
}

// The append of a decode layer (row b = the new token of sequence b, at
// position seq_lens[b] - 1) and the prepare work in one launch: workgroups
// 0 .. n_app-1 append 4 rows each (4 waves per row), the next n_qwg
// prepare the query operands, the others the plan and the stream blocks. The
// parts touch disjoint memory (the prepare reads the raw query of the qkv
// rows, the block tables and the lengths).
constexpr int kAppendWavesPerRow = 4; // one kv-head pair per wave at Hkv = 8
constexpr int kAppendRowsPerWg = kPrepThreads / 64 / kAppendWavesPerRow;
__global__ __launch_bounds__(kPrepThreads) void decode_layer_prep_kernel(DecodeArgs a,
                                                                         AppendArgs ap,
                                                                         int n_rows,
                                                                         int n_app,
                                                                         int n_qwg) {
  // block workgroups first: theirs is the longest chain of dependent loads
  const int n_bwg = gridDim.x - n_app - n_qwg;
  const int wg = ((int)blockIdx.x + n_app + n_qwg) % gridDim.x;
  if (wg < n_app) {
    const int wave = threadIdx.x >> 6;
    const int r = wg * kAppendRowsPerWg + wave / kAppendWavesPerRow;
    if (r < n_rows)
      append_row(ap, r, threadIdx.x & 63, wave % kAppendWavesPerRow, kAppendWavesPerRow);
  } else if (wg < n_app + n_qwg) {
    prep_query_items(a, wg - n_app, n_qwg);
  } else {
    prep_blocks(a, wg - n_app - n_qwg, n_bwg);
  }
}

// ---- split ----------------------------------------------------------------------

// R: depth of the register ring of loaded steps (R - 1 steps in flight ahead
// of the one being computed). Streams range w_id (n_steps steps of 32 tokens)
// for this wave's kv heads: s_ids holds the two block ids of every step, s_rec
// its step record (both in LDS, filled by the caller).
// RAWQ: the ring carries the raw query (fp32, the 16 dims of this lane's
// column) and the RoPE angles of the sequence's last position (s_len: the
// sequences' lengths, in LDS), rotated, scaled and split into the operand
// pieces when the segment opens; otherwise the ring carries the operand
// pieces prepared by the prepare launch (a.qops).
// VF: the cache's value format, 0 bf16 K/V, 1 int8 V (+ scales), 2 e4m3 K and
// V (+ scales).
// LO: loads only (the ceiling yardstick): every load of the stream is issued
// and waited for exactly as in the attention, and its data is folded into an
// XOR instead of the softmax and the matrix ops; nothing useful is written.
template <int R, int VF, bool RAWQ, bool LO = false, int NWV = kSplitWaves>
__device__ __forceinline__ void stream_range(const DecodeArgs &a, int w_id, const int2 *s_ids,
                                             const int *s_rec, const int *s_len, int n_steps) {
  constexpr int D = kHeadDim;
  constexpr bool VQ = VF != 0;  // V as codes with a scale per token
  constexpr bool KF8 = VF == 2; // K as e4m3 codes with a scale per token
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // wave-uniform
  const int n_waves = blockDim.x >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const bool lo = col >= 8;
  const int head = col & 7;
  const bool head_ok = head < a.G;

  // Per-lane load offsets (bytes), the same for every step.
  // K and V: one 16-byte piece per lane of each 1 KB half of a head's block
  // (the block layouts k_offset / v_offset put them in lane order).
  const uint32_t kv_off = (uint32_t)lane * 16;
  const size_t head_bytes = (size_t)kBlockTokens * D * 2;               // 2 KB
  const uint32_t vq_off = (uint32_t)(col * 4 + kg) * 16;                 // int8 V piece


  // One wave per SIMD. Wave wv takes kv heads wv and wv + n_waves (at most two
  // passes over the range: Hkv <= 8 and n_waves = min(4, Hkv)). The passes form
  // one stream of virtual steps v = pass * n_steps + step, so the load ring runs
  // on across the change of head as it does across sequences.
  const int n_passes = (a.n_kv_heads - wv + n_waves - 1) / n_waves; // 1 or 2
  const int last_v = n_passes * n_steps - 1;
  float sink_p[2];
#pragma unroll
  for (int pp = 0; pp < 2; pp++) {
    const int gp = min(wv + pp * n_waves, a.n_kv_heads - 1);
    sink_p[pp] = head_ok ? a.sinks[gp * a.G + head] * kLog2e : 0.0f;
  }

  // Ring slot: K (4 x 16 B per lane), V (4 x 16 B), the query operands
  // (2 x 16 B; loaded only for a step that opens a segment), the step record,
  // and the bad-block bits | pass << 2.
  constexpr int QN = RAWQ ? 8 : 2; // 16-byte pieces of query data per ring slot
  u32x4 kbuf[R][4], vbuf[R][4], qbuf[R][QN];
  int rec[R], badb[R];
  const int hq_lane = head_ok ? head : 0; // query head of this lane's column, within the group
  auto load_step = [&](int v, u32x4 (&kr)[4], u32x4 (&vr)[4], u32x4 (&qr)[QN], int &rc,
                       int &bb) {
    const int pass = v >= n_steps ? 1 : 0;
    const int step = v - pass * n_steps;
    const int g = wv + pass * n_waves;
    const int2 ids = s_ids[step];
    int p0 = uniform(ids.x), p1 = uniform(ids.y);
    rc = uniform(s_rec[step]);
    // a bad id masks its block like padding (bit jt per block)
    bb = (p0 == kBadBlock ? 1 : 0) | (p1 == kBadBlock ? 2 : 0) | (pass << 2);
    // a bad id, or a step's missing second block (padding), reads nothing:
    // its buffer resource covers 0 bytes, so its loads return zeros (masked
    // anyway) without a memory access
    const int n0 = p0 >= 0 ? 2048 : 0, n1 = p1 >= 0 ? 2048 : 0;
    p0 = max(p0, 0);
    p1 = max(p1, 0);
    if (KF8) {
      // e4m3 K and V: per block one 16-byte piece of K codes (dims 8kg ..
      // +7 and 32+8kg .. +7 of token col), one of V codes (as int8 V), and
      // the 4 scales of tokens 4kg .. 4kg+3 for K and for V
      const size_t c0 = ((size_t)p0 * a.n_kv_heads + g) * (head_bytes / 2);
      const size_t c1 = ((size_t)p1 * a.n_kv_heads + g) * (head_bytes / 2);
      const __amdgpu_buffer_rsrc_t k0 = head_rsrc((const char *)a.kc + c0, n0);
      const __amdgpu_buffer_rsrc_t k1 = head_rsrc((const char *)a.kc + c1, n1);
      const __amdgpu_buffer_rsrc_t v0 = head_rsrc((const char *)a.vc + c0, n0);
      const __amdgpu_buffer_rsrc_t v1 = head_rsrc((const char *)a.vc + c1, n1);
      const __amdgpu_buffer_rsrc_t s0 = head_rsrc((const char *)a.vs + c0 / 8, n0);
      const __amdgpu_buffer_rsrc_t s1 = head_rsrc((const char *)a.vs + c1 / 8, n1);
      kr[0] = __builtin_amdgcn_raw_buffer_load_b128(k0, kv_off, 0, kKvAux);
      kr[1] = __builtin_amdgcn_raw_buffer_load_b128(k1, kv_off, 0, kKvAux);
      kr[2] = __builtin_amdgcn_raw_buffer_load_b128(s0, 16 * kg, 0, kKvAux);
      kr[3] = __builtin_amdgcn_raw_buffer_load_b128(s1, 16 * kg, 0, kKvAux);
      vr[0] = __builtin_amdgcn_raw_buffer_load_b128(v0, vq_off, 0, kKvAux);
      vr[1] = __builtin_amdgcn_raw_buffer_load_b128(v1, vq_off, 0, kKvAux);
      vr[2] = __builtin_amdgcn_raw_buffer_load_b128(s0, 64 + 16 * kg, 0, kKvAux);
      vr[3] = __builtin_amdgcn_raw_buffer_load_b128(s1, 64 + 16 * kg, 0, kKvAux);
    } else {
    const size_t h0 = ((size_t)p0 * a.n_kv_heads + g) * head_bytes;
    const size_t h1 = ((size_t)p1 * a.n_kv_heads + g) * head_bytes;
    const __amdgpu_buffer_rsrc_t k0 = head_rsrc((const char *)a.kc + h0, n0);
    const __amdgpu_buffer_rsrc_t k1 = head_rsrc((const char *)a.kc + h1, n1);
    const __amdgpu_buffer_rsrc_t v0 = head_rsrc((const char *)a.vc + h0, n0);
    const __amdgpu_buffer_rsrc_t v1 = head_rsrc((const char *)a.vc + h1, n1);
    kr[0] = __builtin_amdgcn_raw_buffer_load_b128(k0, kv_off, 0, kKvAux);
    kr[1] = __builtin_amdgcn_raw_buffer_load_b128(k0, kv_off + 1024, 0, kKvAux);
    kr[2] = __builtin_amdgcn_raw_buffer_load_b128(k1, kv_off, 0, kKvAux);
    kr[3] = __builtin_amdgcn_raw_buffer_load_b128(k1, kv_off + 1024, 0, kKvAux);
    if (VQ) {
      // int8 V: one 16-byte piece per block (dims col + 16nn, tokens
      // 4kg..4kg+3), then the 4 scales of those tokens per block
      const size_t q0 = ((size_t)p0 * a.n_kv_heads + g) * (head_bytes / 2);
      const size_t q1 = ((size_t)p1 * a.n_kv_heads + g) * (head_bytes / 2);
      const __amdgpu_buffer_rsrc_t c0 = head_rsrc((const char *)a.vc + q0, n0);
      const __amdgpu_buffer_rsrc_t c1 = head_rsrc((const char *)a.vc + q1, n1);
      const __amdgpu_buffer_rsrc_t s0 = head_rsrc((const char *)a.vs + q0 / 16, n0);
      const __amdgpu_buffer_rsrc_t s1 = head_rsrc((const char *)a.vs + q1 / 16, n1);
      vr[0] = __builtin_amdgcn_raw_buffer_load_b128(c0, vq_off, 0, kKvAux);
      vr[1] = __builtin_amdgcn_raw_buffer_load_b128(c1, vq_off, 0, kKvAux);
      vr[2] = __builtin_amdgcn_raw_buffer_load_b128(s0, 16 * kg, 0, kKvAux);
      vr[3] = __builtin_amdgcn_raw_buffer_load_b128(s1, 16 * kg, 0, kKvAux);
    } else {
      // half h of each block: tokens 4kg..4kg+3 of dims col + 32h and
      // col + 32h + 16; operand nn takes its 4 tokens from each block
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(v0, kv_off + h * 1024, 0, kKvAux);
        const u32x4 y = __builtin_amdgcn_raw_buffer_load_b128(v1, kv_off + h * 1024, 0, kKvAux);
        vr[2 * h] = u32x4{x[0], x[1], y[0], y[1]};
        vr[2 * h + 1] = u32x4{x[2], x[3], y[2], y[3]};
      }
    }
    }
    if ((rc & 0x80) || step == 0) { // the step opens a segment: its query
      const int b = rc >> 8;
      if (RAWQ) {
        // dims 8kg .. 8kg+7 and 32+8kg .. +7 of the column's query head, and
        // the angles of those pairs at the sequence's last position
        const u32x4 *qp = (const u32x4 *)(a.q + (int64_t)b * a.q_stride +
                                          (g * a.G + hq_lane) * D + 8 * kg);
        qr[0] = qp[0];
        qr[1] = qp[1];
        qr[2] = qp[8];
        qr[3] = qp[9];
        if (a.cos_tab) {
          const int64_t pos = max(s_len[b] - 1, 0);
          const u32x4 *cp = (const u32x4 *)(a.cos_tab + pos * (D / 2) + 8 * kg);
          const u32x4 *sp = (const u32x4 *)(a.sin_tab + pos * (D / 2) + 8 * kg);
          qr[4] = cp[0];
          qr[5] = cp[1];
          qr[6] = sp[0];
          qr[7] = sp[1];
        }
      } else {
        const u32x4 *qs = a.qops + (((int64_t)b * a.n_kv_heads + g) * 64 + lane) * 2;
        qr[0] = qs[0];
        qr[1] = qs[1];
      }
    }
  };

  // The ring's first loads go out before anything else.
#pragma unroll
  for (int r = 0; r < R - 1; r++)
    load_step(min(r, last_v), kbuf[r], vbuf[r], qbuf[r], rec[r], badb[r]);

  int cur_key = -1;           // sequence | pass << 16 of the open segment (-1: none)
  int cur_b = 0, cur_g = 0;   // its sequence and kv head
  float cur_sink = 0.0f;      // its sink (log2 units)
  bool cur_whole = false;     // the segment began at its sequence's first step
  bool cur_first = false;     // the segment began at the range's first step
  bool cur_ends = false;      // ... and has reached its last step
  float m_run = 0.0f;         // running reference max (log2 units) of this column
  float lsum = 0.0f;
  u32x4 qcur[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
  f32x4 o[4];
#pragma unroll
  for (int nn = 0; nn < 4; nn++)
    o[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Finished segments wait in LDS and go to memory after the stream: a
  // global store among the stream's loads delays the loads behind it (about
  // 2.5 us per segment measured on config 2, 15 us per launch), an LDS write
  // does not. Record r of this wave: the 16 values of each of the 32 lanes
  // that hold outputs (lane (kg, col < 8): query head col, dims 4 kg + 16 nn
  // + 0..3), the (m, l) of each query head for a partial, and what the record
  // is (a whole sequence's output, scaled, or a partial for the combine).
  constexpr int kRecs = kStageRecs * kSplitWaves / NWV; // the same LDS for 4 or 8 waves
  __shared__ f32x4 s_st_o[NWV][kRecs][32][4];
  __shared__ float2 s_st_ml[NWV][kRecs][kCols];
  __shared__ int4 s_st_meta[NWV][kRecs];
  int n_staged = 0; // wave-uniform
  const bool out_lane = !lo && head_ok;
  const int st_lane = kg * 8 + head;

  // Writes the staged records to memory: outputs (bf16 or fp32) and partials.
  auto write_out = [&]() {
    for (int r = 0; r < n_staged; r++) {
      const int4 m = s_st_meta[wv][r]; // {whole, sequence, kv head, partial index}
      if (!out_lane)
        continue;
      f32x4 oo[4];
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
        oo[nn] = s_st_o[wv][r][st_lane][nn];
      if (m.x) {
        const int64_t ob = (int64_t)m.y * a.out_stride + (int64_t)(m.z * a.G + head) * D + 4 * kg;
#pragma unroll
        for (int nn = 0; nn < 4; nn++) {
          if (a.out_bf16) {
            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
            *(bf16x4 *)((__bf16 *)a.out + ob + 16 * nn) =
                bf16x4{(__bf16)oo[nn][0], (__bf16)oo[nn][1], (__bf16)oo[nn][2],
                       (__bf16)oo[nn][3]};
          } else {
            *(f32x4 *)((float *)a.out + ob + 16 * nn) = oo[nn];
          }
        }
      } else {
        const int64_t part = m.w;
        float *wo = a.ws_o + part * kPartFloats + head * D + 4 * kg;
#pragma unroll
        for (int nn = 0; nn < 4; nn++)
          *(f32x4 *)(wo + 16 * nn) = oo[nn];
        if (kg == 0) {
          const float2 ml = s_st_ml[wv][r][head];
          a.ws_ml[part * kMlStride + 2 * head] = ml.x;
          a.ws_ml[part * kMlStride + 2 * head + 1] = ml.y;
        }
      }
    }
    n_staged = 0;
  };

  // Finishes the open segment: the output (sink added) if it is the whole
  // sequence, else the partial for the combine; staged in LDS.
  auto flush = [&]() {
    float ls = lsum;
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);
    f32x4 oo[4];
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        oo[nn][r] = o[nn][r] + swap8(o[nn][r]);
    if (cur_key < 0)
      return;
    if (n_staged == kRecs) // full (many short sequences): to memory now
      write_out();
    const bool whole = cur_whole && cur_ends;
    if (out_lane) {
      float scale = 1.0f;
      if (whole) {
        // out = o * 2^(m - M) / (l * 2^(m - M) + 2^(sink - M)), M = max(m, sink)
        const float M2 = fmaxf(m_run, cur_sink);
        const float f = __builtin_amdgcn_exp2f(m_run - M2);
        scale = f / fmaf(ls, f, __builtin_amdgcn_exp2f(cur_sink - M2));
      } else if (kg == 0) {
        s_st_ml[wv][n_staged][head] = float2{m_run, ls};
      }
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
        s_st_o[wv][n_staged][st_lane][nn] = whole ? oo[nn] * scale : oo[nn];
    }
    if (lane == 0) {
      // only a range's first and last segments can be pieces of a longer
      // sequence: partial slot 0 for the first, 1 for the last
      const int part = (w_id * kPartsPerRange + (cur_first ? 0 : 1)) * a.n_kv_heads + cur_g;
      s_st_meta[wv][n_staged] = int4{whole ? 1 : 0, cur_b, cur_g, part};
    }
    n_staged++;
  };

  uint32_t lo_acc = 0; // LO: the XOR of everything loaded
  auto compute_step = [&](u32x4 (&kr)[4], u32x4 (&vr)[4], u32x4 (&qr)[QN], int rc, int bb,
                          int v) {
    if constexpr (LO) {
      // a multiply per step keeps the steps in order (an XOR chain alone
      // would let the compiler regroup it and wait for later steps' loads)
      uint32_t x = (uint32_t)(rc ^ bb);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          x ^= kr[i][j] ^ vr[i][j];
      lo_acc = (lo_acc ^ x) * 0x01000193u;
      // and no instruction moves across the step: the ring stays a ring
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    const bool in_range = v <= last_v;
    const int pass = bb >> 2;
    const int key = (rc >> 8) | (pass << 16);
    if (in_range && key != cur_key) {
      // The step opens another segment (new sequence or new head): flush,
      // start over.
      flush();
      cur_key = key;
      cur_b = rc >> 8;
      cur_g = wv + pass * n_waves;
      cur_sink = pass ? sink_p[1] : sink_p[0];
      cur_whole = (rc & 0x80) != 0;
      cur_first = v == pass * n_steps;
      m_run = cur_sink;
      lsum = 0.0f;
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
        o[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (RAWQ) {
        // RoPE at the last position (as the append rotates K), the scale
        // 1/sqrt(64) and log2(e) (exp -> exp2), then the bf16 pieces
        float qa[8], qb[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
          qa[i] = __uint_as_float(qr[i >> 2][i & 3]);
          qb[i] = __uint_as_float(qr[2 + (i >> 2)][i & 3]);
        }
        if (a.cos_tab) {
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const float x1 = qa[i], x2 = qb[i];
            const float c = __uint_as_float(qr[4 + (i >> 2)][i & 3]);
            const float sn = __uint_as_float(qr[6 + (i >> 2)][i & 3]);
            qa[i] = rope_first(x1, x2, c, sn);
            qb[i] = rope_second(x1, x2, c, sn);
          }
        }
        const float qscale = head_ok ? 0.125f * kLog2e : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          qa[i] *= qscale;
          qb[i] *= qscale;
        }
        qcur[0] = __builtin_bit_cast(u32x4, pack_pieces(qa, lo));
        qcur[1] = __builtin_bit_cast(u32x4, pack_pieces(qb, lo));
      } else {
        qcur[0] = qr[0];
        qcur[1] = qr[1];
      }
    }
    if (in_range)
      cur_ends = (rc & 0x40) != 0;
    const int valid = in_range ? (rc & 0x3f) : 0;
    const uint32_t bad = (uint32_t)bb & 3u;
    const bf16x8 qop0 = __builtin_bit_cast(bf16x8, qcur[0]);
    const bf16x8 qop1 = __builtin_bit_cast(bf16x8, qcur[1]);
    // Scores of token 4*kg + r of block jt (slot 4*jt + r), this lane's column.
    float sc[8];
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
      bf16x8 k0, k1;
      if (KF8) {
        // the codes in bf16 (exact); the token's scale multiplies its score
        const u32x2 c0 = fp8x4_to_bf16x4(kr[jt][0]), c1 = fp8x4_to_bf16x4(kr[jt][1]);
        const u32x2 c2 = fp8x4_to_bf16x4(kr[jt][2]), c3 = fp8x4_to_bf16x4(kr[jt][3]);
        k0 = __builtin_bit_cast(bf16x8, u32x4{c0[0], c0[1], c1[0], c1[1]});
        k1 = __builtin_bit_cast(bf16x8, u32x4{c2[0], c2[1], c3[0], c3[1]});
      } else {
        k0 = __builtin_bit_cast(bf16x8, kr[2 * jt + 0]);
        k1 = __builtin_bit_cast(bf16x8, kr[2 * jt + 1]);
      }
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qop0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qop1, acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        sc[4 * jt + r] = acc[r] + swap8(acc[r]);
        if (KF8)
          sc[4 * jt + r] *= __uint_as_float(kr[2 + jt][r]);
      }
    }
    if (valid < kStep || bad) {
      // Tail of the sequence, padding, past the range, or a bad block id:
      // those tokens get weight 0 and their values (possibly never written)
      // become zeros.
#pragma unroll
      for (int jt = 0; jt < 2; jt++) {
        const bool blk_bad = (bad >> jt) & 1;
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (16 * jt + 4 * kg + r >= valid || blk_bad) {
            sc[4 * jt + r] = -INFINITY;
            if (VQ) // its weight is 0; its scale (possibly never written) too
              vr[2 + jt][r] = 0u;
          }
        if (KF8) {
          // e4m3 codes of unwritten slots may be NaN: zero them
          uint32_t keep = 0;
#pragma unroll
          for (int r = 0; r < 4; r++)
            keep |= (16 * jt + 4 * kg + r < valid && !blk_bad) ? 0xffu << (8 * r) : 0u;
#pragma unroll
          for (int nn = 0; nn < 4; nn++)
            vr[jt][nn] &= keep;
        }
#pragma unroll
        for (int h2 = 0; h2 < 2 && !VQ; h2++) {
          const int tk = 16 * jt + 4 * kg + 2 * h2;
          const uint32_t keep = blk_bad ? 0u
                                        : ((tk < valid ? 0x0000ffffu : 0u) |
                                           (tk + 1 < valid ? 0xffff0000u : 0u));
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
    // Lazy rescale: the reference max moves only when a score exceeds it by
    // more than 8 (weights stay below 2^8, harmless in fp32); the final
    // normalisation uses the same max, so the result does not change. The
    // test needs no cross-lane max (m_run is the same in the 4 lanes of a
    // column); only the rescale does.
    if (__any(mx > m_run + 8.0f)) {
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
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
    if (VQ) {
      // int8 / e4m3 V: the token's scale goes into its weight (the codes are
      // exact in bf16); a masked token's weight and scale are both 0
#pragma unroll
      for (int i = 0; i < 8; i++)
        p[i] *= __uint_as_float(vr[2 + (i >> 2)][i & 3]);
      const bf16x8 pop = pack_pieces(p, lo);
#pragma unroll
      for (int nn = 0; nn < 4; nn++) {
        const u32x2 x = KF8 ? fp8x4_to_bf16x4(vr[0][nn]) : int8x4_to_bf16x4(vr[0][nn]);
        const u32x2 y = KF8 ? fp8x4_to_bf16x4(vr[1][nn]) : int8x4_to_bf16x4(vr[1][nn]);
        const bf16x8 vop = __builtin_bit_cast(bf16x8, u32x4{x[0], x[1], y[0], y[1]});
        o[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop, o[nn], 0, 0, 0);
      }
    } else {
      const bf16x8 pop = pack_pieces(p, lo);
#pragma unroll
      for (int nn = 0; nn < 4; nn++)
        o[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vr[nn]), pop,
                                                        o[nn], 0, 0, 0);
    }
  };

  // Ring: slot r holds virtual step base + r; the load for v + R - 1 goes out
  // before v is computed. The count is padded to a multiple of R; padded
  // steps re-load the last step (cache hits) and are masked out.
  for (int base = 0; base <= last_v; base += R) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int v = base + r;
      const int slot = (r + R - 1) % R;
      load_step(min(v + R - 1, last_v), kbuf[slot], vbuf[slot], qbuf[slot], rec[slot],
                badb[slot]);
      compute_step(kbuf[r], vbuf[r], qbuf[r], rec[r], badb[r], v);
    }
  }
  if constexpr (LO) {
    // a store the compiler cannot drop, which (practically) never happens
    if (lo_acc == 0x9e3779b9u)
      ((uint32_t *)a.out)[lane] = lo_acc;
    return;
  }
  flush();
  write_out();
}

// The split launch of the staged path: the plan, block ids and step records
// come from the prepare launch through the workspace.
template <int R, int VF>
__global__ __launch_bounds__(kSplitThreads) __attribute__((amdgpu_waves_per_eu(1)))
void decode_split_kernel(DecodeArgs a) {
  const int w_id = blockIdx.x;
  // Block ids and step records of the range, staged in LDS by the whole
  // workgroup (the waves stream the same range for different kv heads). The
  // range's slab needs no plan to be found, so these loads go out with the
  // plan's; entries past the range's steps are never read.
  __shared__ int2 s_ids[kIdSlab / 2]; // the two block ids of each step
  __shared__ int s_rec[kInfoSlab];
  {
    const int4 *src = (const int4 *)(a.flat + (int64_t)w_id * kIdSlab);
    const int4 *srec = (const int4 *)(a.steps + (int64_t)w_id * kInfoSlab);
    int4 *dst = (int4 *)s_ids, *drec = (int4 *)s_rec;
    for (int i = threadIdx.x; i < kIdSlab / 4; i += blockDim.x)
      dst[i] = src[i];
    for (int i = threadIdx.x; i < kInfoSlab / 4; i += blockDim.x)
      drec[i] = srec[i];
  }
  const int T = a.plan[0], S = a.plan[1], n_r = a.plan[2];
  __syncthreads();
  const int rs = range_start(w_id, T, S, n_r);
  const int re = range_start(w_id + 1, T, S, n_r);
  if (rs >= re)
    return;
  stream_range<R, VF, false>(a, w_id, s_ids, s_rec, nullptr, (re - rs) / kStep);
}

// ---- fused: plan, append and split in one launch --------------------------------

constexpr int kStepsPerThread = kInfoSlab / 64; // record-building steps per thread (>= 64 threads)
constexpr int kShortRun = 8; // sequences per range counted rather than searched (records)

// Tokens of a sequence of length L in the stream: its length, or the window,
// clamped to what the table row and the launch were sized for.
__device__ __forceinline__ int stream_tokens(const DecodeArgs &a, int L) {
  const int n = a.window > 0 ? min(L, a.window) : L;
  return max(min(n, min(a.table_stride * kBlockTokens, a.max_len)), 0);
}

// Murmur3's 32-bit finaliser: a bijection of the 32-bit words.
__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h;
}

// Hash of the B lengths, the same in every workgroup: two sums over b of a
// bijective mix of (b, L_b), so that one changed length always changes both
// and several collide with probability ~2^-64. Called by the whole workgroup
// (it holds two barriers); s_red holds 2 ints per wave.
__device__ uint2 lengths_hash(const DecodeArgs &a, int *s_red) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, n_waves = blockDim.x >> 6;
  uint32_t h0 = 0, h1 = 0;
  for (int b = t; b < a.B; b += blockDim.x) {
    const uint32_t L = (uint32_t)a.seq_lens[b];
    h0 += fmix32(L ^ ((uint32_t)b * 0x9e3779b9u));
    h1 += fmix32((L + 0x7f4a7c15u) ^ ((uint32_t)b * 0x632be5abu) ^ 0x5bd1e995u);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    h0 += (uint32_t)__shfl_xor((int)h0, off);
    h1 += (uint32_t)__shfl_xor((int)h1, off);
  }
  __syncthreads(); // s_red may hold an earlier call's sums
  if (lane == 0) {
    s_red[2 * wave] = (int)h0;
    s_red[2 * wave + 1] = (int)h1;
  }
  __syncthreads();
  h0 = h1 = 0;
  for (int w = 0; w < n_waves; w++) {
    h0 += (uint32_t)s_red[2 * w];
    h1 += (uint32_t)s_red[2 * w + 1];
  }
  return uint2{h0, h1};
}

// Word i of a kept plan's key: the shape, the pointers and the lengths' hash.
__device__ __forceinline__ int plan_key(const DecodeArgs &a, int i, uint2 lh) {
  const uint64_t lens = (uint64_t)(uintptr_t)a.seq_lens, tab = (uint64_t)(uintptr_t)a.table;
  switch (i) {
  case 0: return kPlanMagic;
  case 1: return a.B;
  case 2: return a.n_wg;
  case 3: return a.window;
  case 4: return a.fixed_S;
  case 5: return a.aligned;
  case 6: return a.max_len;
  case 7: return a.table_stride;
  case 8: return a.num_blocks;
  case 9: return a.n_kv_heads;
  case 10: return (int)(uint32_t)lens;
  case 11: return (int)(uint32_t)(lens >> 32);
  case 12: return (int)(uint32_t)tab;
  case 13: return (int)(uint32_t)(tab >> 32);
  case 14: return (int)lh.x;
  case 15: return (int)lh.y;
  default: return 0;
  }
}

// One launch per decode layer before the combine. Every workgroup repeats the
// plan: the prefix sums of the padded lengths, in LDS (the lengths are 4
// bytes per sequence). It then builds the step records and block ids of its
// own range only, appends the new tokens that fall in its range (one wave per
// token, all kv heads) and streams the range, the query of each segment
// coming raw through the load ring. The appends' stores are ordered before
// the stream's loads by the workgroup barrier that precedes the stream, so
// every wave of the workgroup reads the new tokens back; no other workgroup
// reads them (each step of the stream belongs to one range). Workgroup 0 publishes the plan for the
// combine.
// mode: bit 0 append; kKeepPlan: also keep the plan in the workspace (each
// range's bounds, table positions and step records, under a key); kReusePlan:
// take the kept plan instead of planning, when its key (the lengths' hash
// included) matches this launch, else plan afresh and report GKV_DEVERR_PLAN.
// A reusing launch reads the block ids from the table at the kept positions,
// so a table changed since the plan was kept is read as it is now. Layers of
// one kind in one decode step share the lengths and the table, so one keeps
// and the others reuse; the ranges, and so every output bit, are the same
// either way.
template <int R, int VF, bool LO = false, int NWV = kSplitWaves>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(NWV / kSplitWaves)))
void decode_fused_kernel(DecodeArgs a, AppendArgs ap, int mode) {
  __shared__ int s_cu[kMaxBatch + 1];
  __shared__ int s_len[kMaxBatch];
  __shared__ int2 s_ids[kIdSlab / 2];
  __shared__ int s_rec[kInfoSlab];
  __shared__ int s_wave[kMaxSplitWaves];
  __shared__ int s_max[kMaxSplitWaves];
  __shared__ int s_hash[2 * kMaxSplitWaves];
  __shared__ int s_find[2];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nt = blockDim.x, B = a.B;
  const int n_waves = nt >> 6;
  const int w_id = blockIdx.x;
  const bool append = mode & 1, keep = mode & kKeepPlan;
  int4 *kept_ranges = (int4 *)(a.kept + kKeyInts);

  bool reuse = false;
  if (mode & kReusePlan) {
    const uint2 lh = lengths_hash(a, s_hash);
    bool same = true;
#pragma unroll
    for (int i = 0; i < kKeyInts; i++)
      same &= a.kept[i] == plan_key(a, i, lh);
    reuse = uniform(same);
    if (!reuse && w_id == 0 && t == 0 && a.dev_err)
      atomicOr(a.dev_err, GKV_DEVERR_PLAN);
  }

  int rs, re, b_first = 0, n_seq = 0;
  if (reuse) {
    const int4 h = kept_ranges[w_id];
    rs = h.x;
    re = h.y;
    b_first = h.z;
    n_seq = h.w;
    {
      // sequences without tokens: output 0, written by workgroup b % n_wg
      const int n_out = a.n_kv_heads * a.G * kHeadDim;
      for (int k = wave * 64; (int64_t)k * a.n_wg + w_id < B; k += nt) {
        const int b = w_id + (k + lane) * a.n_wg;
        const bool empty = b < B && stream_tokens(a, a.seq_lens[b]) == 0;
        uint64_t m = __ballot(empty);
        while (m) {
          const int be = w_id + (k + __builtin_ctzll(m)) * a.n_wg;
          m &= m - 1;
          for (int i = lane; i < n_out; i += 64)
            store_out(a.out, (int64_t)be * a.out_stride + i, 0.0f, a.out_bf16);
        }
      }
    }
    if (rs >= re)
      return;
  } else {
    // Lengths and padded lengths into LDS (coalesced loads), then the prefix
    // sums in place: thread t scans sequences t*per .. t*per+per-1.
    bool any_over = false;
    for (int b = t; b < B; b += nt) {
      const int L = a.seq_lens[b];
      int n = a.window > 0 ? min(L, a.window) : L;
      const int cap = min(a.table_stride * kBlockTokens, a.max_len);
      any_over |= n > cap;
      n = max(min(n, cap), 0);
      s_len[b] = L;
      s_cu[b] = pad_step(n);
    }
    __syncthreads();
    const int per = (B + nt - 1) / nt;
    const int b0 = min(t * per, B), b1 = min(b0 + per, B);
    int local = 0;
    for (int b = b0; b < b1; b++)
      local += s_cu[b];
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (lane >= off)
        incl += v;
    }
    if (lane == 63)
      s_wave[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < n_waves; w++) {
      const int v = s_wave[w];
      before += w < wave ? v : 0;
      total += v;
    }
    int run = before + incl - local;
    for (int b = b0; b < b1; b++) {
      const int v = s_cu[b];
      s_cu[b] = run;
      run += v;
    }
    if (t == 0)
      s_cu[B] = total;
    __syncthreads();
    const int T = s_cu[B];
    const int S = a.fixed_S;
    if (w_id == 0) {
      int32_t *cu = a.plan + kPlanHeader;
      for (int b = t; b <= B; b += nt)
        cu[b] = s_cu[b];
      if (t == 0) {
        a.plan[0] = T;
        a.plan[1] = S;
        a.plan[2] = a.n_wg;
        a.plan[3] = a.aligned;
      }
      // each range's first stream position (and the end), for the combine
      for (int k = t; k <= a.n_wg; k += nt)
        a.plan[kPlanHeader + B + 1 + a.n_wg + k] = range_start(k, T, S, a.n_wg);
      // a kept plan is valid until a launch plans afresh on this workspace
      if (a.kept) {
        if (keep) {
          const uint2 lh = lengths_hash(a, s_hash);
          if (t < kKeyInts)
            a.kept[t] = plan_key(a, t, lh);
        } else if (t == 0) {
          a.kept[0] = 0;
        }
      }
      if (any_over && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
    }
    if (a.aligned) {
      // Ranges of whole sequences, so every segment is a whole sequence,
      // finished here, and no partial is written. Two cuts, both keeping the
      // sequences in order: by count, range k holds sequences ceil(k B / n_wg)
      // .. ceil((k + 1) B / n_wg) - 1 (even when most sequences fill the
      // window, where a cut by tokens can hand a range a third sequence); by
      // tokens, range k runs from the first sequence that starts at or after
      // k T / n_wg (even when the lengths vary below the window). The cut by
      // count is taken when its longest range is within half a window of the
      // mean; every workgroup finds the same. Sequences without tokens (output
      // 0, all weight on the sink) are written by workgroup b % n_wg.
      auto first_by_count = [&](int k) -> int {
        return (int)(((int64_t)k * B + a.n_wg - 1) / a.n_wg);
      };
      auto start_by_tokens = [&](int k) -> int {
        if (k >= a.n_wg)
          return T;
        const int target = (int)(((int64_t)k * T + a.n_wg - 1) / a.n_wg);
        int lo = 0, hi = B; // the first i with s_cu[i] >= target (s_cu[B] = T)
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (s_cu[mid] >= target)
            hi = mid;
          else
            lo = mid + 1;
        }
        return s_cu[lo];
      };
      int longest = 0;
      for (int k = t; k < a.n_wg; k += nt)
        longest = max(longest, s_cu[first_by_count(k + 1)] - s_cu[first_by_count(k)]);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1)
        longest = max(longest, __shfl_xor(longest, off));
      if (lane == 0)
        s_max[wave] = longest;
      __syncthreads();
      for (int w = 0; w < n_waves; w++)
        longest = max(longest, s_max[w]);
      const bool by_count = longest <= (T + a.n_wg - 1) / a.n_wg + a.window / 2 &&
                            longest <= kMaxRange;
      rs = by_count ? s_cu[first_by_count(w_id)] : start_by_tokens(w_id);
      re = by_count ? s_cu[first_by_count(w_id + 1)] : start_by_tokens(w_id + 1);
      const int n_out = a.n_kv_heads * a.G * kHeadDim;
      for (int b = w_id; b < B; b += a.n_wg)
        if (s_cu[b + 1] == s_cu[b])
          for (int i = t; i < n_out; i += nt)
            store_out(a.out, (int64_t)b * a.out_stride + i, 0.0f, a.out_bf16);
    } else {
      rs = range_start(w_id, T, S, a.n_wg);
      re = range_start(w_id + 1, T, S, a.n_wg);
    }
    // The sequences that overlap the range, a run of consecutive indices:
    // from the one holding position rs (the last b with cu[b] <= rs) to the
    // last one starting before re. (The first is found for a range without
    // tokens too, when rs < T: the combine needs the sequence that every
    // range, empty or not, starts inside of.)
    // One pass over the prefix sums, a thread per candidate (two LDS reads
    // each, then one barrier) instead of two binary searches of dependent
    // LDS reads: exactly one b has cu[b] <= rs < cu[b + 1] (rs < T = cu[B]),
    // and exactly one b > b_first has cu[b - 1] < re <= cu[b] (rs < re <= T).
    for (int b = t; b <= B; b += nt) {
      const int c = s_cu[b];
      if (b < B && rs < T && c <= rs && s_cu[b + 1] > rs)
        s_find[0] = b;
      if (b >= 1 && rs < re && c >= re && s_cu[b - 1] < re)
        s_find[1] = b;
    }
    __syncthreads();
    if (rs < T)
      b_first = s_find[0];
    if (rs < re)
      n_seq = s_find[1] - b_first;
    if (keep && t == 0)
      kept_ranges[w_id] = int4{rs, max(re, rs), b_first, n_seq};
    if (a.aligned && t == 0)
      a.crec[w_id] = int4{-1, 0, 0, 0}; // whole sequences: nothing to combine
    if (!a.aligned) {
      // The sequence this range starts inside of (-1: none), for the combine
      // launched per range boundary; and the sequences without tokens
      // (output 0), written by workgroup b % n_wg.
      if (t == 0) {
        const int v = rs < T && rs > s_cu[b_first] ? b_first : -1;
        a.plan[kPlanHeader + B + 1 + w_id] = v;
        a.crec[w_id] = combine_record(w_id, v, v >= 0 ? s_cu[v] : 0, v >= 0 ? s_cu[v + 1] : 0, T,
                                      S, a.n_wg);
      }
      const int n_out = a.n_kv_heads * a.G * kHeadDim;
      for (int b = w_id; b < B; b += a.n_wg)
        if (s_cu[b + 1] == s_cu[b])
          for (int i = t; i < n_out; i += nt)
            store_out(a.out, (int64_t)b * a.out_stride + i, 0.0f, a.out_bf16);
    }
    if (rs >= re)
      return;
  }
  // The range is the same for every lane; saying so keeps the stream's
  // addresses in scalar registers (a bound the compiler takes for divergent,
  // e.g. one that went through a cross-lane max, makes every load of the
  // stream a loop over lanes).
  rs = uniform(rs);
  re = uniform(re);
  b_first = uniform(b_first);
  n_seq = uniform(n_seq);
  const int n_steps = (re - rs) / kStep;

  // The new tokens in the range: each sequence that overlaps it is checked
  // for its new token's place in the stream (its last position, or its ring
  // slot). Wave w appends candidates w, w + 4, ...; the loads of its first go
  // out now, before the step records' loads, and it finishes after them.
  const int32_t *plan_cu = a.plan + kPlanHeader;
  auto cu_of = [&](int b) -> int { return reuse ? plan_cu[b] : s_cu[b]; };
  auto len_of = [&](int b) -> int { return reuse ? a.seq_lens[b] : s_len[b]; };
  auto new_token_in_range = [&](int b) -> bool {
    const int L = len_of(b);
    const int slot = a.window > 0 ? (L - 1) % a.window : L - 1;
    const int at = cu_of(b) + slot;
    return L >= 1 && slot < stream_tokens(a, L) && at >= rs && at < re;
  };
  AppendLoads first_row;
  int first_b = -1;
  if (append && wave < n_seq) {
    const int b = b_first + wave;
    if (new_token_in_range(b)) {
      first_row = append_begin(ap, b, lane, len_of(b) - 1, /*direct=*/true);
      first_b = b;
    }
  }

  // Step records and block ids of the range (the table loads, or the kept
  // slabs' loads, go out here).
  int id0[kStepsPerThread], id1[kStepsPerThread], rcd[kStepsPerThread];
  int pos0[kStepsPerThread], pos1[kStepsPerThread]; // table positions (kept plans)
  if (reuse) {
    // the kept table positions, then the ids they hold now
    const int2 *src = (const int2 *)(a.flat + (int64_t)w_id * kIdSlab);
    const int *srec = a.steps + (int64_t)w_id * kInfoSlab;
    int2 pos[kStepsPerThread];
#pragma unroll
    for (int k = 0; k < kStepsPerThread; k++) {
      const int i = t + k * nt;
      pos[k] = int2{kPadBlock, kPadBlock};
      rcd[k] = 0;
      if (i < n_steps) {
        pos[k] = src[i];
        rcd[k] = srec[i];
      }
    }
#pragma unroll
    for (int k = 0; k < kStepsPerThread; k++) {
      id0[k] = pos[k].x >= 0 ? a.table[pos[k].x] : kPadBlock;
      id1[k] = pos[k].y >= 0 ? a.table[pos[k].y] : kPadBlock;
    }
    for (int j = t; j < n_seq; j += nt)
      s_len[b_first + j] = a.seq_lens[b_first + j];
  } else {
#pragma unroll
    for (int k = 0; k < kStepsPerThread; k++) {
      const int i = t + k * nt;
      id0[k] = id1[k] = kPadBlock;
      pos0[k] = pos1[k] = kPadBlock;
      rcd[k] = 0;
      if (i < n_steps) {
        const int tok = rs + i * kStep;
        // the sequence holding the step: the last b with cu[b] <= tok, one
        // of the range's run b_first .. b_first + n_seq - 1; a short run is
        // counted with independent LDS reads, a long one searched
        int lo = b_first;
        if (n_seq <= kShortRun) {
#pragma unroll
          for (int j = 1; j < kShortRun; j++)
            lo += j < n_seq && s_cu[b_first + j] <= tok ? 1 : 0;
        } else {
          int hi = b_first + n_seq - 1;
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_cu[mid] <= tok)
              lo = mid;
            else
              hi = mid - 1;
          }
        }
        const int b = lo;
        const int off = tok - s_cu[b];
        const int n = stream_tokens(a, s_len[b]);
        const int p0 = b * a.table_stride + off / kBlockTokens;
        if (off < n) {
          id0[k] = a.table[p0];
          pos0[k] = p0;
        }
        if (off + kBlockTokens < n) {
          id1[k] = a.table[p0 + 1];
          pos1[k] = p0 + 1;
        }
        rcd[k] = step_record(b, off == 0, tok + kStep == s_cu[b + 1], min(max(n - off, 0), kStep));
      }
    }
  }

  // The appends: one wave per new token, every kv head.
  if (first_b >= 0)
    append_end(ap, first_row, first_b, lane);
  if (append) {
    for (int j = wave + n_waves; j < n_seq; j += n_waves) {
      const int b = b_first + j;
      if (new_token_in_range(b))
        append_row(ap, b, lane, 0, 1, nullptr, len_of(b) - 1, /*direct=*/true);
    }
  }

  bool any_bad = false;
#pragma unroll
  for (int k = 0; k < kStepsPerThread; k++) {
    const int i = t + k * nt;
    if (i < n_steps) {
      int x = id0[k], y = id1[k];
      if (x != kPadBlock && (x < 0 || x >= a.num_blocks)) {
        x = kBadBlock;
        any_bad = true;
      }
      if (y != kPadBlock && (y < 0 || y >= a.num_blocks)) {
        y = kBadBlock;
        any_bad = true;
      }
      s_ids[i] = int2{x, y};
      s_rec[i] = rcd[k];
      if (keep && !reuse) {
        ((int2 *)(a.flat + (int64_t)w_id * kIdSlab))[i] = int2{pos0[k], pos1[k]};
        a.steps[(int64_t)w_id * kInfoSlab + i] = rcd[k];
      }
    }
  }
  if (any_bad && a.dev_err)
    atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
  // The barrier orders the appends' stores before every wave's stream loads:
  // the waves of a workgroup share one CU, whose vector memory path keeps
  // their accesses in order, so (as for any write, __syncthreads, read within
  // a workgroup) the new tokens are read back without waiting for the stores
  // to complete.
  __syncthreads();

  // The stream reads its arguments afresh from the kernel-argument segment
  // (the prologue's values are not kept live across the loop).
#if defined(__HIP_DEVICE_COMPILE__)
  typedef const __attribute__((address_space(4))) DecodeArgs *KernargPtr;
  KernargPtr pa = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(pa));
  const DecodeArgs a2 = *pa;
  stream_range<R, VF, true, LO, NWV>(a2, w_id, s_ids, s_rec, s_len, n_steps);
#endif
}

// ---- combine --------------------------------------------------------------------

// Sequence b's output from its pieces in ranges w0 .. w1 (the stream
// positions [c0, c1) meet them), one wave per kv head g; lane (h = lane / 8)
// merges dims 8*(lane % 8) .. +7 of query head h:
// M = max(sink, m_w), L = 2^(sink-M) + sum l_w 2^(m_w-M), out = sum o_w 2^(m_w-M) / L
// (the merge of fast_attention.hpp:403-424, across workgroups). The piece in
// range w is that range's last segment (slot 1) for the first range unless
// the sequence starts exactly there, else its first segment (slot 0); ranges
// without tokens (possible when there are fewer steps than ranges) hold none.
// Up to kCombineAtOnce ranges, every load goes out at once (one round trip).
constexpr int kCombineAtOnce = 4;
__device__ __forceinline__ void combine_sequence(const DecodeArgs &a, int4 rec) {
  constexpr int D = kHeadDim;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, h = lane >> 3, d0 = 8 * (lane & 7);
  if (h >= a.G)
    return;
  const int b = rec.x, w0 = rec.y, w1 = rec.z, c0 = rec.w;
  const int32_t *rsa = a.plan + kPlanHeader + a.B + 1 + a.n_wg; // range starts (+ the end)
  auto part_of = [&](int r, int rs) -> int64_t {
    const int slot = (r == w0 && c0 != rs) ? 1 : 0;
    return ((int64_t)r * kPartsPerRange + slot) * a.n_kv_heads + g;
  };
  const int64_t ob = (int64_t)b * a.out_stride + (int64_t)(g * a.G + h) * D + d0;
  const float sk = a.sinks[g * a.G + h] * kLog2e;
  float M = sk, Ls, inv;
  f32x4 o0 = {0, 0, 0, 0}, o1 = {0, 0, 0, 0};
  if (w1 - w0 < kCombineAtOnce) {
    float m[kCombineAtOnce], l[kCombineAtOnce];
    f32x4 pa[kCombineAtOnce], pb[kCombineAtOnce];
    bool ok[kCombineAtOnce];
#pragma unroll
    for (int i = 0; i < kCombineAtOnce; i++) {
      const int r = w0 + i;
      ok[i] = false;
      if (r <= w1) {
        const int rs = rsa[r];
        ok[i] = rs != rsa[r + 1];
        const int64_t part = part_of(r, rs);
        m[i] = a.ws_ml[part * kMlStride + 2 * h];
        l[i] = a.ws_ml[part * kMlStride + 2 * h + 1];
        const f32x4 *po = (const f32x4 *)(a.ws_o + part * kPartFloats + h * D + d0);
        pa[i] = po[0];
        pb[i] = po[1];
      }
    }
#pragma unroll
    for (int i = 0; i < kCombineAtOnce; i++)
      if (ok[i])
        M = fmaxf(M, m[i]);
    Ls = __builtin_amdgcn_exp2f(sk - M);
#pragma unroll
    for (int i = 0; i < kCombineAtOnce; i++)
      if (ok[i]) {
        const float c = __builtin_amdgcn_exp2f(m[i] - M);
        Ls = fmaf(l[i], c, Ls);
        o0 += pa[i] * c;
        o1 += pb[i] * c;
      }
  } else {
    for (int r = w0; r <= w1; r++)
      if (rsa[r] != rsa[r + 1])
        M = fmaxf(M, a.ws_ml[part_of(r, rsa[r]) * kMlStride + 2 * h]);
    Ls = __builtin_amdgcn_exp2f(sk - M);
    for (int r = w0; r <= w1; r++) {
      if (rsa[r] == rsa[r + 1])
        continue;
      const int64_t part = part_of(r, rsa[r]);
      const float c = __builtin_amdgcn_exp2f(a.ws_ml[part * kMlStride + 2 * h] - M);
      Ls = fmaf(a.ws_ml[part * kMlStride + 2 * h + 1], c, Ls);
      const f32x4 *po = (const f32x4 *)(a.ws_o + part * kPartFloats + h * D + d0);
      o0 += po[0] * c;
      o1 += po[1] * c;
    }
  }
  inv = 1.0f / Ls;
  for (int i = 0; i < 4; i++) {
    store_out(a.out, ob + i, o0[i] * inv, a.out_bf16);
    store_out(a.out, ob + 4 + i, o1[i] * inv, a.out_bf16);
  }
}

// One workgroup per range, a wave per kv head: the split launch (or the
// prepare launch of the staged ones) left, per range, the record of the
// sequence the range is the first to start inside of (its pieces' ranges and
// stream start), so the merge is two round trips: the record, then every
// piece at once. n_wg workgroups instead of one per sequence, most of them
// returning at once.
__global__ __launch_bounds__(512) void decode_combine_kernel(DecodeArgs a) {
  const int4 rec = a.crec[blockIdx.x];
  if (rec.x < 0)
    return;
  combine_sequence(a, rec);
}

// ---- host side --------------------------------------------------------------------

constexpr int kRing = 3;

// Ring depth of the split kernels (default kRing; the tuning variable
// GKV_DECODE_RING = 3..5 picks another, read once).
static int ring_depth() {
  static const int r = [] {
    const char *e = getenv("GKV_DECODE_RING");
    const int v = e ? atoi(e) : kRing;
    return (v >= 3 && v <= 5) ? v : kRing;
  }();
  return r;
}

template <int R>
static void launch_split_ring(const DecodeArgs &a, dim3 grid, dim3 block, hipStream_t s) {
  if (a.kv_fp8)
    hipLaunchKernelGGL((decode_split_kernel<R, 2>), grid, block, 0, s, a);
  else if (a.vs)
    hipLaunchKernelGGL((decode_split_kernel<R, 1>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((decode_split_kernel<R, 0>), grid, block, 0, s, a);
}

// The fused kernel at the given ring depth (3..5; the default otherwise).
static const void *fused_kernel_fn(int ring) {
  switch (ring) {
  case 3:
    return (const void *)decode_fused_kernel<3, 0>;
  case 5:
    return (const void *)decode_fused_kernel<5, 0>;
  default:
    return (const void *)decode_fused_kernel<4, 0>;
  }
}

static int split_block(int n_kv_heads) { return 64 * std::min(kSplitWaves, n_kv_heads); }

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
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fused_kernel_fn(ring_depth()),
                                                     split_block(n_kv_heads), 0) != hipSuccess)
      return 0;
    slot = std::max(1, cus * per_cu);
  }
  return slot;
}

static constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace layout: plan | partials (o) | partials (m, l) | then, for the
// staged launches and the kept plan only: block ids | step records | query
// operands | kept plan. The split that plans in its prologue uses the first
// three (fused_total bytes).
struct WorkspaceLayout {
  size_t plan, crec, ws_o, ws_ml, flat, steps, qops, kept, fused_total, total;
};

static constexpr WorkspaceLayout layout_of(int B, int n_kv_heads, int max_wg) {
  WorkspaceLayout L{};
  L.plan = 0;
  L.crec = align256((size_t)(kPlanHeader + B + 1 + 2 * max_wg + 1) * 4);
  L.ws_o = align256(L.crec + (size_t)max_wg * 16);
  const size_t parts = (size_t)kPartsPerRange * max_wg * n_kv_heads;
  L.ws_ml = L.ws_o + parts * kPartFloats * sizeof(float);
  L.flat = align256(L.ws_ml + parts * kMlStride * sizeof(float));
  L.fused_total = L.flat;
  L.steps = L.flat + align256((size_t)max_wg * kIdSlab * 4);
  L.qops = L.steps + align256((size_t)max_wg * kInfoSlab * 4);
  L.kept = L.qops + align256((size_t)B * n_kv_heads * 64 * 32);
  L.total = L.kept + align256((size_t)(kKeyInts + 4 * max_wg) * 4);
  return L;
}

static int64_t stream_max(int32_t B, int32_t max_seq_len, int32_t window) {
  const int64_t n_max = window > 0 ? std::min(max_seq_len, window) : max_seq_len;
  return (int64_t)B * ((n_max + kStep - 1) / kStep * kStep);
}

// Window layers with the balanced split take ranges of whole sequences: no
// sequence is split, and the fused launch needs no combine after it. A range
// then exceeds its share of the stream by at most one sequence (W tokens), so
// it stays within kMaxRange.
static bool whole_sequence_ranges(int64_t t_max, int64_t n_wg, int32_t window,
                                  int32_t split_tokens) {
  return split_tokens == 0 && window > 0 && n_wg > 0 &&
         (t_max + n_wg - 1) / n_wg + (window + kStep - 1) / kStep * kStep <= kMaxRange;
}

static int prepare(DecodeArgs &a, int32_t B, int32_t n_q_heads, const float *q, int64_t q_stride,
                   const float *cos_tab, const float *sin_tab, const int32_t *seq_lens,
                   int32_t max_seq_len, const gkv_cache_view &cache, int32_t window,
                   const float *sinks, int32_t split_tokens, void *workspace,
                   size_t workspace_bytes_given, void *out, int64_t out_stride,
                   int32_t out_dtype, uint32_t *dev_err, bool need_cache,
                   int ws_wg = kMaxWorkgroups, bool staged_parts = true) {
  if (B < 0 || n_q_heads <= 0 || cache.n_kv_heads <= 0 || !seq_lens || !sinks || !out ||
      max_seq_len < 0 || window < 0 || (out_dtype != GKV_F32 && out_dtype != GKV_BF16))
    return GKV_ERR_ARG;
  if (need_cache && (!q || !cache.k || !cache.v || !cache.block_table ||
                     cache.table_stride <= 0 || cache.num_blocks <= 0 || (cos_tab && !sin_tab)))
    return GKV_ERR_ARG;
  if (n_q_heads % cache.n_kv_heads != 0)
    return GKV_ERR_ARG;
  if (cache.v_format != GKV_V_BF16 && cache.v_format != GKV_V_INT8 &&
      cache.v_format != GKV_KV_FP8)
    return GKV_ERR_ARG;
  if (need_cache && cache.v_format != GKV_V_BF16 && !cache.v_scale)
    return GKV_ERR_ARG;
  if (cache.n_kv_heads > 8 || B > kMaxBatch)
    return GKV_ERR_UNSUPPORTED; // combine: one wave per kv head; prep: prefix sums in LDS
  const int G = n_q_heads / cache.n_kv_heads;
  if (G > kCols)
    return GKV_ERR_UNSUPPORTED;
  if (need_cache && q_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  // 16-byte loads of the query rows and the angle tables
  if (need_cache && (q_stride % 4 != 0 ||
                     ((uintptr_t)q | (uintptr_t)cos_tab | (uintptr_t)sin_tab) % 16 != 0))
    return GKV_ERR_ARG;
  if (out_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  if (split_tokens < 0 || split_tokens % kStep != 0)
    return GKV_ERR_ARG;
  if (window > 0 && cache.ring > 0 && cache.ring != window)
    return GKV_ERR_ARG;
  if (cache.ring > 0 && window == 0)
    return GKV_ERR_ARG; // a ring holds only the last W tokens
  if (need_cache && window > 0 && cache.ring == 0)
    return GKV_ERR_UNSUPPORTED; // the window is read from a ring of W slots
  const int64_t t_max = stream_max(B, max_seq_len, window);
  if (t_max >= (1 << 30) || (int64_t)B << 8 >= INT32_MAX)
    return GKV_ERR_ARG;
  // Ranges hold at most kMaxRange tokens (the block ids a wave keeps).
  const int64_t min_wg = (t_max + kMaxRange - 1) / kMaxRange;
  int64_t n_wg = 0;
  if (split_tokens > 0) {
    if (split_tokens > kMaxRange)
      return GKV_ERR_ARG;
    n_wg = std::max<int64_t>(1, (t_max + split_tokens - 1) / split_tokens);
    if (n_wg > kMaxWorkgroups)
      return GKV_ERR_ARG;
  }
  const WorkspaceLayout L = layout_of(B, cache.n_kv_heads, ws_wg);
  if (!workspace || workspace_bytes_given < (staged_parts ? L.total : L.fused_total))
    return GKV_ERR_WORKSPACE;
  if (split_tokens == 0) {
    // (the combine takes the same count: one workgroup per range)
    const int resident = B > 0 ? resident_workgroups(cache.n_kv_heads) : 1;
    if (resident <= 0)
      return GKV_ERR_HIP;
    n_wg = std::max<int64_t>(resident, min_wg);
    if (n_wg > kMaxWorkgroups)
      return GKV_ERR_ARG;
  }
  if (n_wg > ws_wg)
    return GKV_ERR_CAPACITY; // more ranges than the workspace has partial slots for
  a.q = q;
  a.q_stride = q_stride;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.seq_lens = seq_lens;
  a.kc = (const uint16_t *)cache.k;
  a.vc = (const uint16_t *)cache.v;
  a.vs = cache.v_format != GKV_V_BF16 ? (const float *)cache.v_scale : nullptr;
  a.kv_fp8 = cache.v_format == GKV_KV_FP8;
  a.table = cache.block_table;
  a.table_stride = cache.table_stride;
  a.num_blocks = cache.num_blocks;
  a.n_kv_heads = cache.n_kv_heads;
  a.window = window;
  a.max_len = (int)(window > 0 ? std::min(max_seq_len, window) : max_seq_len);
  a.sinks = sinks;
  a.G = G;
  a.B = B;
  a.n_wg = (int)n_wg;
  a.fixed_S = split_tokens;
  a.aligned = whole_sequence_ranges(t_max, n_wg, window, split_tokens);
  char *ws = (char *)workspace;
  a.plan = (int32_t *)(ws + L.plan);
  a.flat = (int32_t *)(ws + L.flat);
  a.steps = (int32_t *)(ws + L.steps);
  a.qops = (u32x4 *)(ws + L.qops);
  a.kept = staged_parts ? (int32_t *)(ws + L.kept) : nullptr;
  a.ws_o = (float *)(ws + L.ws_o);
  a.crec = (int4 *)(ws + L.crec);
  a.ws_ml = (float *)(ws + L.ws_ml);
  a.out = out;
  a.out_stride = out_stride;
  a.out_bf16 = out_dtype == GKV_BF16;
  a.dev_err = dev_err;
  return GKV_OK;
}

// Query workgroups (one wave per item) and block workgroups (one thread per
// 16-token block of the longest possible stream), each at most 1024.
static int query_workgroups(const DecodeArgs &a) {
  const int waves = kPrepThreads / 64;
  return (int)std::max<int64_t>(
      1, std::min<int64_t>(1024, ((int64_t)a.B * a.n_kv_heads + waves - 1) / waves));
}

static int block_workgroups(int64_t t_max) {
  return (int)std::max<int64_t>(
      1, std::min<int64_t>(1024, (t_max / kBlockTokens + kPrepThreads - 1) / kPrepThreads));
}

static int launch_prep(const DecodeArgs &a, int64_t t_max, hipStream_t s) {
  const int n_qwg = query_workgroups(a);
  hipLaunchKernelGGL(decode_prep_kernel, dim3(n_qwg + block_workgroups(t_max)),
                     dim3(kPrepThreads), 0, s, a, n_qwg);
  return launch_status("decode_prep_kernel");
}

static int launch_layer_prep(const DecodeArgs &a, const AppendArgs &ap, int64_t t_max,
                             hipStream_t s) {
  const int n_app = (a.B + kAppendRowsPerWg - 1) / kAppendRowsPerWg;
  const int n_qwg = query_workgroups(a);
  hipLaunchKernelGGL(decode_layer_prep_kernel, dim3(n_app + n_qwg + block_workgroups(t_max)),
                     dim3(kPrepThreads), 0, s, a, ap, a.B, n_app, n_qwg);
  return launch_status("decode_layer_prep_kernel");
}

static int launch_split(const DecodeArgs &a, hipStream_t s) {
  const dim3 grid(a.n_wg), block(split_block(a.n_kv_heads));
  switch (ring_depth()) {
  case 3:
    launch_split_ring<3>(a, grid, block, s);
    break;
  case 5:
    launch_split_ring<5>(a, grid, block, s);
    break;
  default:
    launch_split_ring<4>(a, grid, block, s);
  }
  return launch_status("decode_split_kernel");
}

template <int R>
static void launch_fused_ring(const DecodeArgs &a, const AppendArgs &ap, int mode, dim3 grid,
                              dim3 block, hipStream_t s) {
  if (a.kv_fp8) {
    // The e4m3 stream is bound by its waves' instructions (half the bytes per
    // step, the same math plus the code conversions): two waves per SIMD, one
    // kv head each, cover each other's dependency chains; at 256 registers
    // the ring is 2 steps deep (3 would spill). Measured 125.1 against
    // 130.9 us at config 2; the bf16 and int8-V streams, bound by their
    // loads, measured level or slower this way.
    hipLaunchKernelGGL((decode_fused_kernel<2, 2, false, kMaxSplitWaves>), grid,
                       dim3(64 * std::min(kMaxSplitWaves, a.n_kv_heads)), 0, s, a, ap, mode);
    return;
  }
  // Short ranges (at most kShortRangeTokens of stream per workgroup, bounded
  // on the host from the shape: a window layer of a large batch) are bound by
  // the prologue and each step's chain, not by their loads: the 8-wave form
  // too (config 3: bf16 37.4 -> 35.5 us, int8 V 32.5 -> 30.0 us; with 512
  // tokens per range, config 5's window layers, it is slower).
  const int64_t range_bound = ((int64_t)a.B * pad_step(a.max_len) + a.n_wg - 1) / a.n_wg;
  if (a.n_kv_heads == kMaxSplitWaves && a.fixed_S == 0 && range_bound <= kShortRangeTokens) {
    const dim3 b8(64 * kMaxSplitWaves);
    if (a.vs)
      hipLaunchKernelGGL((decode_fused_kernel<2, 1, false, kMaxSplitWaves>), grid, b8, 0, s, a,
                         ap, mode);
    else
      hipLaunchKernelGGL((decode_fused_kernel<2, 0, false, kMaxSplitWaves>), grid, b8, 0, s, a,
                         ap, mode);
    return;
  }
  if (a.vs)
    hipLaunchKernelGGL((decode_fused_kernel<R, 1>), grid, block, 0, s, a, ap, mode);
  else
    hipLaunchKernelGGL((decode_fused_kernel<R, 0>), grid, block, 0, s, a, ap, mode);
}

// The fused launch; ap == nullptr: no append (attention only). plan_bits:
// kKeepPlan / kReusePlan (a workspace with the kept-plan area).
static int launch_fused(const DecodeArgs &a, const AppendArgs *ap, hipStream_t s,
                        int plan_bits = 0) {
  const dim3 grid(a.n_wg), block(split_block(a.n_kv_heads));
  AppendArgs aa{};
  if (ap) {
    aa = *ap;
    aa.seq_lens = nullptr; // the kernel passes each row's position (its length - 1)
  }
  const int mode = (ap ? 1 : 0) | plan_bits;
  switch (ring_depth()) {
  case 3:
    launch_fused_ring<3>(a, aa, mode, grid, block, s);
    break;
  case 5:
    launch_fused_ring<5>(a, aa, mode, grid, block, s);
    break;
  default:
    launch_fused_ring<4>(a, aa, mode, grid, block, s);
  }
  return launch_status("decode_fused_kernel");
}

static int launch_combine(const DecodeArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(decode_combine_kernel, dim3(a.n_wg), dim3(64 * a.n_kv_heads), 0, s, a);
  return launch_status("decode_combine_kernel");
}

} // namespace gkv

using namespace gkv;

extern "C" size_t gkv_decode_workspace_bytes(int32_t B, int32_t n_kv_heads, int32_t max_seq_len,
                                             int32_t window, int32_t split_tokens) {
  (void)split_tokens;
  if (B < 0 || n_kv_heads <= 0 || max_seq_len < 0 || window < 0)
    return 0;
  return layout_of(B, n_kv_heads, kMaxWorkgroups).total;
}

extern "C" int gkv_decode_layer_combines(int32_t B, int32_t n_kv_heads, int32_t max_seq_len,
                                         int32_t window, int32_t split_tokens) {
  if (B < 0 || n_kv_heads <= 0 || n_kv_heads > 8 || max_seq_len < 0 || window < 0 ||
      split_tokens < 0)
    return GKV_ERR_ARG;
  if (B == 0)
    return 0;
  const int64_t t_max = stream_max(B, max_seq_len, window);
  const int resident = resident_workgroups(n_kv_heads);
  if (resident <= 0)
    return GKV_ERR_HIP;
  const int64_t n_wg = std::max<int64_t>(resident, (t_max + kMaxRange - 1) / kMaxRange);
  return whole_sequence_ranges(t_max, n_wg, window, split_tokens) ? 0 : 1;
}

#define GKV_DECODE_PARAMS                                                                   \
  void *stream, int32_t B, int32_t n_q_heads, const float *q, int64_t q_stride,                \
      const float *cos_tab, const float *sin_tab, const int32_t *seq_lens, int32_t max_seq_len, \
      gkv_cache_view cache, int32_t window, const float *sinks, int32_t split_tokens,          \
      void *workspace, size_t workspace_bytes_, void *out, int64_t out_stride,                  \
      int32_t out_dtype, uint32_t *dev_err
#define GKV_LAYER_PARAMS                                                                    \
  void *stream, int32_t B, int32_t n_q_heads, const float *qkv, int64_t row_stride,            \
      const float *cos_tab, const float *sin_tab, const int32_t *seq_lens, int32_t max_seq_len, \
      gkv_cache_view cache, int32_t window, const float *sinks, int32_t split_tokens,          \
      void *workspace, size_t workspace_bytes_, void *out, int64_t out_stride,                  \
      int32_t out_dtype, uint32_t *dev_err
#define GKV_DECODE_PREPARE(a)                                                                  \
  prepare(a, B, n_q_heads, q, q_stride, cos_tab, sin_tab, seq_lens, max_seq_len, cache, window, \
          sinks, split_tokens, workspace, workspace_bytes_, out, out_stride, out_dtype, dev_err, \
          true)

extern "C" int gkv_decode_prepare(GKV_DECODE_PARAMS) {
  DecodeArgs a;
  const int st = GKV_DECODE_PREPARE(a);
  if (st != GKV_OK || B == 0)
    return st;
  return launch_prep(a, stream_max(B, max_seq_len, window), (hipStream_t)stream);
}

extern "C" int gkv_decode_split(GKV_DECODE_PARAMS) {
  DecodeArgs a;
  const int st = GKV_DECODE_PREPARE(a);
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
  // always launched: after the staged launches a window layer has partials;
  // after a fused split of whole-sequence ranges the plan says so and the
  // kernel returns at once
  return launch_combine(a, (hipStream_t)stream);
}

extern "C" int gkv_decode_attention(GKV_DECODE_PARAMS) {
  DecodeArgs a;
  int st = GKV_DECODE_PREPARE(a);
  if (st != GKV_OK || B == 0)
    return st;
  if ((st = launch_fused(a, nullptr, (hipStream_t)stream)))
    return st;
  return a.aligned ? GKV_OK : launch_combine(a, (hipStream_t)stream);
}

// ---- decode layer: append + attention -----------------------------------------

static int layer_append_args(AppendArgs &ap, int32_t B, int32_t n_q_heads, const float *qkv,
                             int64_t row_stride, const float *cos_tab, const float *sin_tab,
                             const int32_t *seq_lens, const gkv_cache_view &cache,
                             uint32_t *dev_err) {
  if (!qkv || !cos_tab || !sin_tab || !cache.k || !cache.v)
    return GKV_ERR_ARG;
  if (row_stride < (int64_t)(n_q_heads + 2 * cache.n_kv_heads) * kHeadDim)
    return GKV_ERR_ARG;
  if (row_stride % 4 != 0 || ((uintptr_t)qkv | (uintptr_t)cos_tab | (uintptr_t)sin_tab) % 16 != 0)
    return GKV_ERR_ARG; // 16-byte vector loads in the append
  if (cache.ring % kBlockTokens != 0)
    return GKV_ERR_UNSUPPORTED;
  ap.qkv = qkv;
  ap.row_stride = row_stride;
  ap.n_q_heads = n_q_heads;
  ap.n_kv_heads = cache.n_kv_heads;
  ap.cos_tab = cos_tab;
  ap.sin_tab = sin_tab;
  ap.row_pos = nullptr; // position = seq_lens[b] - 1
  ap.row_seq = nullptr;
  ap.seq_lens = seq_lens;
  ap.kc = (uint16_t *)cache.k;
  ap.vc = (uint16_t *)cache.v;
  ap.table = cache.block_table;
  ap.table_stride = cache.table_stride;
  ap.num_blocks = cache.num_blocks;
  ap.ring = cache.ring;
  ap.q_out = nullptr;
  ap.q_out_stride = 0;
  ap.k_pack = ap.v_pack = nullptr;
  ap.dev_err = dev_err;
  ap.v_int8 = cache.v_format == GKV_V_INT8;
  ap.kv_fp8 = cache.v_format == GKV_KV_FP8;
  ap.vs = (float *)cache.v_scale;
  (void)B;
  return GKV_OK;
}

#define GKV_LAYER_SETUP                                                                        \
  DecodeArgs a;                                                                                \
  AppendArgs ap;                                                                               \
  int st = prepare(a, B, n_q_heads, qkv, row_stride, cos_tab, sin_tab, seq_lens, max_seq_len,  \
                   cache, window, sinks, split_tokens, workspace, workspace_bytes_, out,       \
                   out_stride, out_dtype, dev_err, true);                                     \
  if (st == GKV_OK)                                                                            \
    st = layer_append_args(ap, B, n_q_heads, qkv, row_stride, cos_tab, sin_tab, seq_lens,     \
                           cache, dev_err);                                                    \
  if (st != GKV_OK || B == 0)                                                                  \
    return st;

extern "C" int gkv_decode_layer_prepare(GKV_LAYER_PARAMS) {
  GKV_LAYER_SETUP
  return launch_layer_prep(a, ap, stream_max(B, max_seq_len, window), (hipStream_t)stream);
}

extern "C" int gkv_decode_layer_split(GKV_LAYER_PARAMS) {
  GKV_LAYER_SETUP
  return launch_fused(a, &ap, (hipStream_t)stream);
}

extern "C" int gkv_decode_layer(GKV_LAYER_PARAMS) {
  GKV_LAYER_SETUP
  if ((st = launch_fused(a, &ap, (hipStream_t)stream)))
    return st;
  return a.aligned ? GKV_OK : launch_combine(a, (hipStream_t)stream);
}

static int plan_bits(int32_t plan) {
  return plan == GKV_PLAN_KEEP ? kKeepPlan : plan == GKV_PLAN_REUSE ? kReusePlan : 0;
}

// The loads-only form of gkv_decode_layer's split launch (bf16 K/V): the same
// plan, appends and load stream, the attention math replaced by an XOR of the
// loaded data. A ceiling yardstick, as the reference's loads-only kernels
// (getp-csrc/bench/attn_bench.cpp:161-227); the outputs are not written.
extern "C" int gkv_yardstick_decode_loads(GKV_LAYER_PARAMS) {
  if (cache.v_format != GKV_V_BF16)
    return GKV_ERR_UNSUPPORTED;
  GKV_LAYER_SETUP
  AppendArgs aa = ap;
  aa.seq_lens = nullptr;
  hipLaunchKernelGGL((decode_fused_kernel<kRing, 0, true>), dim3(a.n_wg),
                     dim3(split_block(a.n_kv_heads)), 0, (hipStream_t)stream, a, aa, 1);
  return launch_status("decode_fused_kernel (loads only)");
}

extern "C" int gkv_decode_layer_planned(GKV_LAYER_PARAMS, int32_t plan) {
  if (plan != GKV_PLAN_NONE && plan != GKV_PLAN_KEEP && plan != GKV_PLAN_REUSE)
    return GKV_ERR_ARG;
  GKV_LAYER_SETUP
  if ((st = launch_fused(a, &ap, (hipStream_t)stream, plan_bits(plan))))
    return st;
  return a.aligned ? GKV_OK : launch_combine(a, (hipStream_t)stream);
}

extern "C" int gkv_decode_layer_split_planned(GKV_LAYER_PARAMS, int32_t plan) {
  if (plan != GKV_PLAN_NONE && plan != GKV_PLAN_KEEP && plan != GKV_PLAN_REUSE)
    return GKV_ERR_ARG;
  GKV_LAYER_SETUP
  return launch_fused(a, &ap, (hipStream_t)stream, plan_bits(plan));
}


// ---- decode layer without allocation ---------------------------------------------
//
// gkv_decode_layer with its workspace in this library's own device memory: a
// file-scope array, one per GPU, held until the process ends. Its address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and only that address is handed to kernels. The fused split and the
// combine use the plan and the partial slots of the workspace: the plan is
// written by the split before the combine reads it, and every partial the
// combine reads was written by the split of the same call, so nothing has to
// start at zero. Calls that overlap on one GPU share the array and race.

namespace gkv {
constexpr int kScratchWorkgroups = 512; // ranges (split workgroups) the scratch holds
constexpr size_t kScratchBytes = layout_of(kMaxBatch, 8, kScratchWorkgroups).fused_total;
static __device__ __align__(256) char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;

// The scratch array's device address on the current device (looked up on the
// first call on that device), or nullptr with the HIP error recorded.
static void *scratch_ptr() {
  static std::mutex mu;
  static void *ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hip_status(hipGetDevice(&dev), "hipGetDevice") != GKV_OK)
    return nullptr;
  if (dev < 0 || dev >= kMaxDevices)
    return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *p = nullptr;
    if (hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress") !=
        GKV_OK)
      return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}
} // namespace gkv

extern "C" int gkv_decode_layer_noalloc(void *stream, int32_t B, int32_t n_q_heads,
                                        const float *qkv, int64_t row_stride,
                                        const float *cos_tab, const float *sin_tab,
                                        const int32_t *seq_lens, int32_t max_seq_len,
                                        gkv_cache_view cache, int32_t window, const float *sinks,
                                        void *out, int64_t out_stride, int32_t out_dtype,
                                        uint32_t *dev_err) {
  if (cache.n_kv_heads > 8 || B > kMaxBatch)
    return GKV_ERR_CAPACITY; // the scratch is sized for 8 kv heads and kMaxBatch sequences
  void *ws = scratch_ptr();
  if (!ws)
    return GKV_ERR_HIP;
  DecodeArgs a;
  AppendArgs ap;
  int st = prepare(a, B, n_q_heads, qkv, row_stride, cos_tab, sin_tab, seq_lens, max_seq_len,
                   cache, window, sinks, 0, ws, kScratchBytes, out, out_stride, out_dtype,
                   dev_err, true, kScratchWorkgroups, false);
  if (st == GKV_OK)
    st = layer_append_args(ap, B, n_q_heads, qkv, row_stride, cos_tab, sin_tab, seq_lens, cache,
                           dev_err);
  if (st != GKV_OK || B == 0)
    return st;
  if ((st = launch_fused(a, &ap, (hipStream_t)stream)))
    return st;
  return a.aligned ? GKV_OK : launch_combine(a, (hipStream_t)stream);
}

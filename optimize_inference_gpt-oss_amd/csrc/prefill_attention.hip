// Causal attention of a packed batch of prompts with per-head sinks and the
// sliding window, on bf16 and fp16 matrix cores.
//
// The reference has no prefill kernel: it feeds a prompt one token at a time
// through the decode step (getp-csrc/engine/gpu_engine.hpp:811-813), so each
// query row j of a prompt is the decode attention of run.cpp:597-642 at
// pos = j -- over that prompt's positions 0..j (window W: j-W+1..j) plus the
// sink logit. This kernel computes exactly that for all rows at once.
//
// Work: one workgroup per (prompt, kv head, block of 32 query positions), one
// wave per query head of the kv head's group (all waves share the K/V tiles
// in LDS, so each K/V byte is read from L2 once per group). Blocks are
// launched longest-first (the last query blocks of the prompts see the most
// keys).
//
// Matrix cores, v_mfma_f32_16x16x32_bf16 (the decode kernel's operand
// arrangement, with 16 query columns instead of 8 heads):
//   scores  S^T[key][query] = K[key][dims] * Q^T[dims][query]; the query is
//           carried as bf16 high + low pieces accumulated into one tile, so
//           the scores keep ~16 mantissa bits of the fp32 query
//   output  O^T[dim][query] += V^T[dim][keys] * P^T[keys][query] on
//           v_mfma_f32_16x16x32_f16: P (in [0, 1]) as one fp16 piece, V as fp16
//           of v * 2^-10 (a single bf16 P leaves errors of 2^-9 of |v| on
//           queries that see few keys; fp16 keeps 2^-12)
//   A 32-key step uses two 16-key score tiles; lane (kg, n) holds keys
//   4kg..4kg+3 of each, which are its P^T operand slots; the V^T operand is
//   the same 8 keys of one dim, read from V stored transposed in LDS.
// Online softmax in the log2 domain (scale 1/8 * log2 e folded into Q), lazy
// rescale by threshold 8 (tested on the fp16 weights), the running max seeded
// with the sink, and the sink added in the final normalisation, as in the
// decode kernel. The row sums are fp32 sums of the same fp16 weights.
//
// Chunks after a history: a prompt's rows may continue a sequence that
// already holds start_pos[b] tokens (a multiple of 16) in the paged cache.
// Row j is then position start + j and attends to positions
// max(0, start + j - W + 1) .. start + j: those before start come from the
// cache (the full layer's table, or the ring of W slots, which must still
// hold them: append a ring layer's chunk after this call), those from start
// on from the packed rows (or also from the cache, when no packed rows are
// given: a full layer whose chunk was appended first).
//
// LDS (66 KB, two workgroups per CU): a pipeline of 3 K/V tile stages of 64
// keys, fed by direct-to-LDS loads 2 tiles ahead. Each 16-key group of a tile
// is one paged block's 2 KB (from the cache), staged in its block layout (a
// lane's K operand is then one 16-byte read at lane * 16), or 16 packed rows.
// Without a history, packed K and V are staged as rows with 16-byte slots
// XOR-swizzled per key row (conflict-free operand reads without padding);
// with one, packed K goes into the block layout too (one operand form), V
// stays in rows. The V of tile t + 1 is turned into V^T [64 dims][64 keys + 8 pad]
// fp16 after tile t is computed, into the other of two V^T buffers: two
// barriers per tile, and a tile's loads have two tiles' compute to land in.
#include "gkv_device.hpp"
#include "lds_dma.hpp"

#include <algorithm>
#include <climits>
#include <cstdlib>

namespace gkv {

constexpr int kQBlock = 32;         // query positions per workgroup
constexpr int kKTile = 64;          // keys per LDS tile
constexpr int kVRow = kKTile + 8;   // fp16 per V^T row in LDS
constexpr float kVScale = 0x1p-10f; // V is staged as fp16 of v * kVScale
constexpr int kStages = 3;          // K/V tile pipeline depth (tiles held in LDS)
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct PrefillArgs {
  const int32_t *cu;
  const int32_t *start;           // per prompt: tokens already cached (nullptr: none)
  const float *q;
  int64_t q_stride;
  const float *cos_tab, *sin_tab; // nullptr: q is rotated; else rotate row j at its position
  const uint16_t *k, *v;          // packed rows (nullptr: every key from the cache)
  int64_t kv_stride; // elements per packed row: Hkv * 64
  const uint16_t *kc, *vc;        // the paged cache (K and V block layouts)
  const float *vs;                // the cache's scales: int8 V [block][kv head][16];
                                  // e4m3 [block][kv head][32] (K scales, then V scales)
  const int32_t *table;
  int table_stride, num_blocks, ring;
  const float *sinks;
  int B, G, n_kv_heads, window, n_qblocks;
  int band; // query blocks per band of the grid order
  void *out;
  int64_t out_stride;
  int out_bf16;
  uint32_t *dev_err;
};

// HIST: prompts may continue a cached history (start positions, keys from
// the cache); without it every key comes from the packed rows and the
// history paths are compiled out. VF (with HIST), the cache's storage: 0
// bf16 K and V; 1 int8 V codes with a scale per token and head; 2 e4m3 K and
// V codes, each with a scale per token and head. A cached group's stage of a
// quantized K or V holds the block's 1 KB of codes, then its scales (int8 V:
// 16 floats; e4m3: the block's 32, K scales then V scales).
template <int NW, bool HIST, int VF = 0>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW >= 8 ? 4 : 1))) void prefill_kernel(PrefillArgs a) {
  static_assert(HIST || VF == 0, "codes come from the cache");
  constexpr int D = kHeadDim;
  constexpr int NT = NW * 64;
  constexpr int kPieces = kKTile * D / 8 / NT; // V^T conversion: key pairs x 4 dims per thread
  // The tile pipeline's stages: K and V tiles as they arrive, row-major with
  // each 128-byte key row's 16-byte slots XOR-swizzled by key % 8 (slot s of
  // key r holds dims 8 (s ^ (r % 8))), one array per stage so that a read of
  // one stage waits only for that stage's loads; and V^T in fp16 for the tile
  // being computed and the next one. 66 KB: two workgroups per CU.
  static_assert(kStages == 3, "one array per stage below");
  __shared__ __attribute__((aligned(16))) uint16_t k_st0[kKTile * D], k_st1[kKTile * D],
      k_st2[kKTile * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_st0[kKTile * D], v_st1[kKTile * D],
      v_st2[kKTile * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2 * D * kVRow];

  // Grid order: kv head fastest (consecutive workgroups go to different
  // XCDs, so each XCD holds the K/V of its own heads), then bands of a.band
  // query blocks taken longest first, and in a band each prompt's blocks
  // together: the blocks of one prompt-head that run side by side on one XCD
  // share their K/V tiles in its L2 (a band's blocks see nearly the same
  // keys), while the longest blocks still start first. Ids past the first
  // query block (the last band's padding) exit at once.
  int id = blockIdx.x;
  const int g = id % a.n_kv_heads;
  id /= a.n_kv_heads;
  const int band = id / (a.B * a.band), w = id - band * (a.B * a.band);
  const int b = w / a.band;
  const int qb = a.n_qblocks - 1 - (band * a.band + w % a.band);
  if (qb < 0)
    return;
  const int row0 = a.cu[b];
  const int L = a.cu[b + 1] - row0;
  const int q0 = qb * kQBlock;
  if (q0 >= L)
    return;
  int start = HIST && a.start ? a.start[b] : 0; // position of row 0
  if (HIST && (start < 0 || (start & (kBlockTokens - 1)) != 0)) {
    if (threadIdx.x == 0 && a.dev_err)
      atomicOr(a.dev_err, GKV_DEVERR_ALIGN);
    start = 0; // (the prompt's outputs are then meaningless, but finite)
  }
  // A full layer's cache holds positions below table_stride * 16, and the
  // RoPE table rows the caller passes cover them: a prompt that runs past
  // that is flagged, and its rows take their angles at the last position
  // that fits (meaningless outputs, no read past the table).
  const int p_cap = HIST && a.ring == 0 ? a.table_stride * kBlockTokens : INT_MAX;
  if (HIST && start + L > p_cap && q0 == 0 && threadIdx.x == 0 && a.dev_err)
    atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
  // positions from here on: queries p0 .. p_last, keys k_lo .. p_last
  const int p0 = start + q0, p_last = start + min(q0 + kQBlock, L) - 1;
  const int W = a.window;
  int k_lo = W > 0 ? max(0, p0 - W + 1) : 0;
  k_lo &= ~(kKTile - 1);
  const int n_tiles = (p_last + 1 - k_lo + kKTile - 1) / kKTile;
  // keys before this position come from the cache
  const int hist_end = !HIST ? 0 : a.k ? start : INT_MAX;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int n = lane & 15, kg = lane >> 4;
  const bool active = wave < a.G;
  const int h = g * a.G + (active ? wave : 0);

  // ---- K/V tile pipeline: kStages stages, tiles t+1 .. t+kStages-1 in flight while
  // tile t is computed. Direct-to-LDS loads: lane l of a wave's load lands at
  // byte 16 l of the wave's 1 KB chunk (8 key rows), and fetches the 16-byte
  // slot that the swizzle puts there. Every tile slot issues its loads (rows
  // past the prompt clamped, tiles past the last re-read), so the number of
  // loads that follow a tile's is fixed and the wait below is exact.
  auto k_stage = [&](int st) -> uint16_t * {
    return st == 0 ? k_st0 : st == 1 ? k_st1 : k_st2;
  };
  auto v_stage = [&](int st) -> uint16_t * {
    return st == 0 ? v_st0 : st == 1 ? v_st1 : v_st2;
  };
  // Block ids of the 4 cached groups of a tile (-1: none), read through the
  // scalar cache (wave-uniform) at the end of the tile before the one whose
  // loads use them, so the next tile's barrier wait covers their latency. An
  // id outside the pool is flagged and replaced by block 0 (finite data;
  // that prompt's output is then meaningless, and the error word says so).
  typedef const __attribute__((address_space(4))) int32_t *ConstI32;
  struct Ids {
    int v[4];
  };
  auto load_ids = [&](int t) -> Ids {
    Ids r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      r.v[j] = -1;
      if (HIST) {
        const int p = min(k_lo + t * kKTile + kBlockTokens * j, p_last);
        const int grp = (W > 0 && a.ring > 0 ? p % a.ring : p) / kBlockTokens;
        if (p < hist_end && grp < a.table_stride)
          r.v[j] = ((ConstI32)a.table)[(int64_t)b * a.table_stride + grp];
      }
    }
    return r;
  };
  auto cached_block = [&](const Ids &ids, int grp) -> int64_t {
    // a select chain, not an indexed access (which would put the ids in memory)
    int id = grp == 0 ? ids.v[0] : grp == 1 ? ids.v[1] : grp == 2 ? ids.v[2] : ids.v[3];
    if (id < 0 || id >= a.num_blocks) {
      if (lane == 0 && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
      id = 0;
    }
    return ((int64_t)id * a.n_kv_heads + g) * (kBlockTokens * D);
  };
  // Tile t into stage st: 16 loads of 1 KB (4 groups x K/V x 2 halves), each
  // wave 16 / NW of them. Every slot issues its loads (packed rows past the
  // prompt clamped, tiles past the last re-read), so the number of loads that
  // follow a tile's is fixed and the wait below is exact.
  auto dma = [&](int t, int st, const Ids &ids) {
    const int kt0 = k_lo + t * kKTile;
#pragma unroll
    for (int i = 0; i < 16 / NW; i++) {
      const int ins = wave + i * NW;
      const int is_v = ins >> 3, grp = (ins >> 1) & 3, half = ins & 1;
      const int p = kt0 + kBlockTokens * grp; // first position of the group
      uint16_t *dst = (is_v ? v_stage(st) : k_stage(st)) + grp * 1024 + half * 512;
      // a wave-uniform base and this lane's element offset from it. The lane
      // index is made opaque here so that the per-lane offsets are formed at
      // each load rather than hoisted out of the tile loop and kept live
      // (the history variant has no registers to spare for them)
      int lane_ = lane;
      if (HIST)
        asm volatile("" : "+v"(lane_));
      const uint16_t *src;
      uint32_t off;
      if (VF != 0 && (is_v || VF == 2) && p < hist_end) {
        // a cached block of codes: half 0 its 1 KB of codes, half 1 its
        // scales (int8 V: 16 floats, lanes 0-3; e4m3: 32 floats, lanes 0-7;
        // the other lanes repeat them)
        const int64_t blk = cached_block(ids, grp); // bf16 elements of a block = code bytes
        if (half) {
          src = (const uint16_t *)a.vs + (VF == 2 ? blk / 16 : blk / 32);
          off = (lane_ & (VF == 2 ? 7 : 3)) * 8;
        } else {
          src = (is_v ? a.vc : a.kc) + blk / 2;
          off = lane_ * 8;
        }
      } else if (HIST && p < hist_end) {
        // a cached block: its 2 KB as they are (block layouts); tiles past
        // the last re-read the last one
        src = (is_v ? a.vc : a.kc) + cached_block(ids, grp) + half * 512;
        off = lane_ * 8;
      } else if (HIST && !is_v) {
        // packed rows (clamped to the prompt's last) into the K block layout,
        // as a cached block is staged: lane (kg, t) <- dims 32 half + 8 kg ..
        // +7 of the group's row t
        src = a.k + (int64_t)row0 * a.kv_stride + g * D;
        off = (uint32_t)(min(p - start + (lane_ & 15), L - 1) * (int)a.kv_stride + 32 * half +
                         8 * (lane_ >> 4));
      } else {
        // packed rows (clamped to the prompt's last) as rows: keys 8 half ..
        // +7 of the group, 16-byte slots swizzled by key % 8
        const int key = 8 * half + (lane_ >> 3);
        const int col = 8 * ((lane_ & 7) ^ (key & 7));
        src = (is_v ? a.v : a.k) + (int64_t)row0 * a.kv_stride + g * D;
        off = (uint32_t)(min(p - start + key, L - 1) * (int)a.kv_stride + col);
      }
      if (HIST)
        dma16_s(src, off * 2, dst); // uniform base in SGPRs, 32-bit offsets
      else
        dma16(src + off, dst);
    }
  };
  // V of a stage -> V^T as fp16 of v * 2^-10 (exact for bf16 magnitudes
  // 2^-4 .. 2^26, an absolute error of at most 2^-15 below that, inf above,
  // so the output shows it): P then enters the matrix core as one fp16 piece.
  // Piece i of a thread covers keys 2pr, 2pr + 1 and dims 4pd .. 4pd+3, where
  // virtual wave vw = (tid + i*NT) / 64 and its lane ln give
  // pr = ln % 16 + 16 (vw % 2), pd = ln / 16 + 4 (vw / 2); the pair is one
  // dword per dim of V^T, and the 64 dwords a wave writes fall in 64 banks.
  auto f32_half = [](float x) -> uint32_t {
    const _Float16 h = (_Float16)(x * kVScale);
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
  };
  auto v_half = [&](uint32_t bits16) -> uint32_t { return f32_half(bf16_to_f32((uint16_t)bits16)); };
  bool v_range = false; // a V beyond the fp16 range of the staged v * 2^-10
  auto convert_v = [&](int st, int buf, int t) {
    const uint16_t *vs = v_stage(st);
    uint16_t *vt_w = v_lds + buf * (D * kVRow);
    const int kt0 = k_lo + t * kKTile;
#pragma unroll
    for (int i = 0; i < kPieces; i++) {
      const int idx = tid + i * NT;
      const int vw = idx >> 6, ln = idx & 63;
      const int pr = (ln & 15) + 16 * (vw & 1), pd = (ln >> 4) + 4 * (vw >> 1);
      const int r0 = 2 * pr, r1 = 2 * pr + 1;
      // dims 4pd + j of keys r0 (low half) and r1 (high half), as fp16 of v * 2^-10
      uint32_t hp[4];
      if (VF != 0 && kt0 + (r0 & ~(kBlockTokens - 1)) < hist_end) {
        // int8 or e4m3 block: the codes of keys r0, r1 of dim d are adjacent
        // bytes at ((d % 16) * 4 + t / 4) * 16 + (d / 16) * 4 + t % 4; the
        // value is value(code) * scale in fp32, as the cache stands for it.
        // Slots past the block's last query position become 0.
        const uint16_t *blk = vs + (r0 >> 4) * 1024;
        const float *scl = (const float *)(blk + 512) + (VF == 2 ? kBlockTokens : 0);
        const int t0 = r0 & 15;
        const bool keep0 = kt0 + r0 <= p_last, keep1 = kt0 + r1 <= p_last;
        const float s0 = scl[t0], s1 = scl[t0 + 1];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int d = 4 * pd + j;
          const uint32_t c2 = *(const uint16_t *)((const char *)blk +
                                                  ((d & 15) * 4 + (t0 >> 2)) * 16 +
                                                  (d >> 4) * 4 + (t0 & 3));
          float v0, v1;
          if (VF == 2) {
            const f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)c2, false); // bytes 0, 1
            v0 = f[0];
            v1 = f[1];
          } else {
            v0 = (float)(int8_t)(c2 & 0xffu);
            v1 = (float)(int8_t)(c2 >> 8);
          }
          const float x0 = keep0 ? v0 * s0 : 0.0f;
          const float x1 = keep1 ? v1 * s1 : 0.0f;
          hp[j] = f32_half(x0) | (f32_half(x1) << 16);
        }
      } else {
        uint32_t pair[4]; // bf16 bits
        if (HIST && kt0 + (r0 & ~(kBlockTokens - 1)) < hist_end) {
          // block layout: keys r0, r1 of one dim are adjacent. Slots past the
          // block's last query position may never have been written: their V
          // becomes 0 (their weight is 0, and 0 * NaN would not be)
          const uint16_t *blk = vs + (r0 >> 4) * 1024;
          const int t0 = r0 & 15;
          const uint32_t keep = (kt0 + r0 <= p_last ? 0x0000ffffu : 0u) |
                                (kt0 + r1 <= p_last ? 0xffff0000u : 0u);
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int d = 4 * pd + j;
            pair[j] = keep & *(const uint32_t *)(blk + (d >> 5) * 512 +
                                                 ((t0 >> 2) * 16 + (d & 15)) * 8 +
                                                 ((d >> 4) & 1) * 4 + (t0 & 3));
          }
        } else {
          const u32x2 x = *(const u32x2 *)(vs + r0 * D + 8 * ((pd >> 1) ^ (r0 & 7)) + 4 * (pd & 1));
          const u32x2 y = *(const u32x2 *)(vs + r1 * D + 8 * ((pd >> 1) ^ (r1 & 7)) + 4 * (pd & 1));
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const uint32_t wa = x[j >> 1] >> (16 * (j & 1)), wb = y[j >> 1] >> (16 * (j & 1));
            pair[j] = (wa & 0xffffu) | (wb << 16);
          }
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
          hp[j] = v_half(pair[j] & 0xffffu) | (v_half(pair[j] >> 16) << 16);
      }
      bool inf = false;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (HIST) // the entry point with an error word
          inf |= (hp[j] & 0x7fffu) == 0x7c00u || ((hp[j] >> 16) & 0x7fffu) == 0x7c00u;
        *(uint32_t *)&vt_w[(4 * pd + j) * kVRow + 2 * pr] = hp[j];
      }
      if (HIST)
        v_range |= __any(inf); // wave-uniform
    }
  };

  // ---- query operands: column tile c holds queries q0 + 16c + n; half dh dims 32dh + 8kg + j.
  // The loads of both column tiles, of the block's RoPE angles and of the
  // first K/V tiles go out together: one memory round trip before compute.
  // The angles (cos and sin of the block's 32 positions, [2][32][32] fp32, 8
  // KB) are the same for every wave: they are staged once per workgroup, one
  // 1 KB direct-to-LDS load per wave (8 positions of cos or of sin), into the
  // second V^T buffer, which the first tile's conversion of the next one
  // overwrites only after its barrier. (Loaded by every wave into registers
  // they cost each workgroup 32 KB of cache traffic and its last waves 1.4 us
  // of start.) The rotation and the bf16 split follow the first barrier.
  // the block ids of the first tiles go out first
  const Ids ids0 = load_ids(0), ids1 = load_ids(1);
  Ids ids_next = load_ids(kStages - 1);
  const bool rot = a.cos_tab != nullptr;
  float *const ang = (float *)(v_lds + D * kVRow);
  bf16x8 qhi[2][2], qlo[2][2];
  f32x4 qr[2][4];
  {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int j = min(q0 + 16 * c + n, L - 1);
      const float *qp = a.q + (int64_t)(row0 + j) * a.q_stride + h * D + 8 * kg;
      // the two halves of RoPE pairs 8kg .. 8kg+7 sit in this lane
      qr[c][0] = *(const f32x4 *)qp;
      qr[c][1] = *(const f32x4 *)(qp + 4);
      qr[c][2] = *(const f32x4 *)(qp + 32);
      qr[c][3] = *(const f32x4 *)(qp + 36);
    }
    if (rot) {
#pragma unroll
      for (int k = wave; k < 8; k += NW) {
        const int i = 8 * (k & 3) + (lane >> 3); // the position's row in the block
        const float *tab = k < 4 ? a.cos_tab : a.sin_tab;
        dma16(tab + (int64_t)min(start + min(q0 + i, L - 1), p_cap - 1) * (D / 2) + 4 * (lane & 7),
              ang + k * 256);
      }
    }
#pragma unroll
    for (int t = 0; t < kStages - 1; t++)
      dma(t, t, t == 0 ? ids0 : ids1);
  }
  const float sink2 = a.sinks[h] * kLog2e;
  float m_run[2] = {sink2, sink2}, lsum[2] = {0.0f, 0.0f};
  f32x4 o[2][4];
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int nn = 0; nn < 4; nn++)
      o[c][nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Tile t in stage st: the first barrier completes the V^T of tile t
  // (converted at the end of tile t - 1); the stage of tile t - 1, free since
  // then, takes the loads of tile t + kStages - 1. After the compute, wait
  // until this wave's loads of tile t + 1 have landed (issued one tile ago;
  // those of tile t + 2 stay in flight), and the second barrier makes every
  // wave's loads visible and frees the V^T buffer of tile t - 1, which takes
  // the V^T of tile t + 1. A tile's loads thus have two tiles' compute to
  // land in.
  auto tile = [&](const int t, const int st) {
    lds_barrier();
    dma(t + kStages - 1, (st + kStages - 1) % kStages, ids_next);
    const uint16_t *ks = k_stage(st);
    const uint16_t *vt = v_lds + (t & 1) * (D * kVRow);
    const int kt0 = k_lo + t * kKTile;
#pragma unroll
    for (int s = 0; s < kKTile / 32; s++) {
      const int kb = kt0 + 32 * s; // first key of the step
      // uniform skips: every key after the last query, or (window) older
      // than the first query's window
      if (!active || kb > p_last || (W > 0 && kb + 31 <= p0 - W))
        continue;
      const bool need_mask = kb + 31 > p0 || (W > 0 && kb <= p_last - W);
      f32x4 acc[2][2]; // [key tile][query column tile]
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        acc[kt][0] = acc[kt][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // key 16 kt + n of the step (group 2s + kt of the tile), dims
        // 32dh + 8kg .. +7: with a history (K staged in the block layout) 16
        // bytes at lane * 16 of half dh; else slot 4dh + kg of its swizzled row
        const int kr = 32 * s + 16 * kt + n;
        // e4m3 codes of a cached group: lane (kg, n) holds key n's dims
        // 8kg .. +7 (bytes 0-7) and 32 + 8kg .. +7 (bytes 8-15) at lane * 16;
        // turned into bf16 exactly, the K scale applied to the scores
        const bool f8 = VF == 2 && kb + 16 * kt < hist_end; // wave-uniform
#pragma unroll
        for (int dh = 0; dh < 2; dh++) {
          const int ki = HIST ? (2 * s + kt) * 1024 + dh * 512 + lane * 8
                              : kr * D + 8 * ((4 * dh + kg) ^ (kr & 7));
          bf16x8 kop;
          if (f8) {
            const u32x2 w = *(const u32x2 *)((const char *)(ks + (2 * s + kt) * 1024) +
                                             lane * 16 + dh * 8);
            const u32x2 lo = fp8x4_to_bf16x4(w[0]), hi = fp8x4_to_bf16x4(w[1]);
            kop = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
          } else {
            kop = *(const bf16x8 *)&ks[ki];
          }
#pragma unroll
          for (int c = 0; c < 2; c++) {
            acc[kt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qhi[c][dh], acc[kt][c], 0, 0, 0);
            acc[kt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qlo[c][dh], acc[kt][c], 0, 0, 0);
          }
        }
        if (f8) { // keys 4kg .. 4kg+3 of the group: their K scales
          const f32x4 ksc = *(const f32x4 *)((const float *)(ks + (2 * s + kt) * 1024 + 512) + 4 * kg);
#pragma unroll
          for (int c = 0; c < 2; c++)
            acc[kt][c] *= ksc;
        }
      }
      f16x8 ph[2];
#pragma unroll
      for (int c = 0; c < 2; c++) {
        float sc[8];
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            sc[4 * kt + r] = acc[kt][c][r];
        if (need_mask) {
          // key ka is kept iff 0 <= qa - ka < W (no window: below 2^31), one
          // unsigned compare per score
          const uint32_t wlim = W > 0 ? (uint32_t)W : 0x80000000u;
          const int back0 = (p0 + 16 * c + n) - (kb + 4 * kg); // qa - ka of slot 0
#pragma unroll
          for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
              if ((uint32_t)(back0 - 16 * kt - r) >= wlim)
                sc[4 * kt + r] = -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < 8; i++)
          ph[c][i] = (_Float16)__builtin_amdgcn_exp2f(sc[i] - m_run[c]);
        // Lazy rescale: the reference max moves only when a weight exceeds 2^8
        // (a score more than 8 above it; an fp16 weight of inf included). The
        // test runs on the fp16 weights with packed max; it needs no cross-lane
        // max (m_run is the same in the 4 lanes of a column), only the rescale,
        // which then recomputes the weights.
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        f16x2 w2 = __builtin_elementwise_max(
            __builtin_elementwise_max(f16x2{ph[c][0], ph[c][1]}, f16x2{ph[c][2], ph[c][3]}),
            __builtin_elementwise_max(f16x2{ph[c][4], ph[c][5]}, f16x2{ph[c][6], ph[c][7]}));
        if (__any(__builtin_elementwise_max(w2[0], w2[1]) > (_Float16)256.0f)) {
          float mx = sc[0];
#pragma unroll
          for (int i = 1; i < 8; i++)
            mx = fmaxf(mx, sc[i]);
          mx = fmaxf(mx, __shfl_xor(mx, 16));
          mx = fmaxf(mx, __shfl_xor(mx, 32));
          const float m_new = fmaxf(m_run[c], mx);
          const float alpha = __builtin_amdgcn_exp2f(m_run[c] - m_new);
          m_run[c] = m_new;
          lsum[c] *= alpha;
#pragma unroll
          for (int nn = 0; nn < 4; nn++)
            o[c][nn] *= alpha;
#pragma unroll
          for (int i = 0; i < 8; i++)
            ph[c][i] = (_Float16)__builtin_amdgcn_exp2f(sc[i] - m_run[c]);
        }
        // the row sum of the same fp16 weights the output uses (fp32 sums)
#pragma unroll
        for (int i = 0; i < 8; i += 2)
          lsum[c] = __builtin_amdgcn_fdot2(f16x2{ph[c][i], ph[c][i + 1]},
                                           f16x2{(_Float16)1.0f, (_Float16)1.0f}, lsum[c], false);
      }
#pragma unroll
      for (int nn = 0; nn < 4; nn++) {
        const uint16_t *vrow = &vt[(16 * nn + n) * kVRow + 32 * s + 4 * kg];
        const u32x2 x = *(const u32x2 *)vrow;
        const u32x2 y = *(const u32x2 *)(vrow + 16);
        const f16x8 vop = __builtin_bit_cast(f16x8, u32x4{x[0], x[1], y[0], y[1]});
#pragma unroll
        for (int c = 0; c < 2; c++)
          o[c][nn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, ph[c], o[c][nn], 0, 0, 0);
      }
    }
    // the block ids of the tile whose loads the next tile issues
    if (HIST)
      ids_next = load_ids(t + kStages);
    if (t + 1 < n_tiles) {
      wait_vmcnt<16 / NW>();
      lds_barrier();
      convert_v((st + 1) % kStages, (t + 1) & 1, t + 1);
    }
  };
  // the query (rotated, scaled, split), then tile 0's V^T, before the loop
  // (tile 1's loads may still fly)
  wait_vmcnt<2 * (8 / NW)>();
  lds_barrier();
  {
    const float qscale = 0.125f * kLog2e; // 1/sqrt(64); exp -> exp2
#pragma unroll
    for (int c = 0; c < 2; c++) {
      f32x4 cr[2] = {}, sr[2] = {};
      if (rot) {
        const float *cp = ang + (16 * c + n) * (D / 2) + 8 * kg;
        cr[0] = *(const f32x4 *)cp;
        cr[1] = *(const f32x4 *)(cp + 4);
        sr[0] = *(const f32x4 *)(cp + 1024);
        sr[1] = *(const f32x4 *)(cp + 1028);
      }
      float qv[2][8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float x1 = qr[c][j / 4][j % 4], x2 = qr[c][2 + j / 4][j % 4];
        qv[0][j] = rot ? rope_first(x1, x2, cr[j / 4][j % 4], sr[j / 4][j % 4]) : x1;
        qv[1][j] = rot ? rope_second(x1, x2, cr[j / 4][j % 4], sr[j / 4][j % 4]) : x2;
      }
#pragma unroll
      for (int dh = 0; dh < 2; dh++) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float x = qv[dh][j] * qscale;
          const __bf16 hi = (__bf16)x;
          qhi[c][dh][j] = hi;
          qlo[c][dh][j] = (__bf16)(x - (float)hi);
        }
      }
    }
  }
  convert_v(0, 0, 0);
  for (int t = 0; t < n_tiles; t += kStages) {
    tile(t, 0);
#pragma unroll
    for (int st = 1; st < kStages; st++)
      if (t + st < n_tiles)
        tile(t + st, st);
  }
  wait_vmcnt<0>(); // no load may still write into LDS when the workgroup ends
  if (v_range && lane == 0 && a.dev_err)
    atomicOr(a.dev_err, GKV_DEVERR_RANGE);
  if (!active)
    return;

  // out = o * 2^(m - M) / (l * 2^(m - M) + 2^(sink - M)), M = max(m, sink).
  // The query index is formed afresh here (kept from the query loads, it
  // would hold a register through the tile loop).
  int n_out = n;
  asm volatile("" : "+v"(n_out));
#pragma unroll
  for (int c = 0; c < 2; c++) {
    float ls = lsum[c];
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);
    const int qa = q0 + 16 * c + n_out;
    if (qa >= L)
      continue;
    const float M2 = fmaxf(m_run[c], sink2);
    const float f = __builtin_amdgcn_exp2f(m_run[c] - M2);
    const float scale = f / fmaf(ls, f, __builtin_amdgcn_exp2f(sink2 - M2)) / kVScale;
    const int64_t ob = (int64_t)(row0 + qa) * a.out_stride + (int64_t)h * D + 4 * kg;
#pragma unroll
    for (int nn = 0; nn < 4; nn++) {
      const f32x4 r = o[c][nn] * scale;
      if (a.out_bf16) {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        *(bf16x4 *)((__bf16 *)a.out + ob + 16 * nn) =
            bf16x4{(__bf16)r[0], (__bf16)r[1], (__bf16)r[2], (__bf16)r[3]};
      } else {
        *(f32x4 *)((float *)a.out + ob + 16 * nn) = r;
      }
    }
  }
}

} // namespace gkv

template <bool HIST, int VF>
static void launch_prefill(const gkv::PrefillArgs &a, int G, dim3 g, hipStream_t s) {
  using namespace gkv;
  if (G > 4)
    hipLaunchKernelGGL((prefill_kernel<8, HIST, VF>), g, dim3(512), 0, s, a);
  else if (G > 2)
    hipLaunchKernelGGL((prefill_kernel<4, HIST, VF>), g, dim3(256), 0, s, a);
  else if (G > 1)
    hipLaunchKernelGGL((prefill_kernel<2, HIST, VF>), g, dim3(128), 0, s, a);
  else
    hipLaunchKernelGGL((prefill_kernel<1, HIST, VF>), g, dim3(64), 0, s, a);
}

// Query blocks per band of the grid order (2, or GKV_PREFILL_BAND, read
// once; 1 is the plain longest-first order).
static int query_band() {
  static const int env = [] {
    const char *e = getenv("GKV_PREFILL_BAND");
    return e ? std::max(1, atoi(e)) : 2;
  }();
  return env;
}

static int prefill_launch(void *stream, int32_t B, const int32_t *cu_seqlens,
                          const int32_t *start_pos, int32_t max_len, int32_t n_q_heads,
                          int32_t n_kv_heads, const float *q, int64_t q_stride,
                          const float *cos_tab, const float *sin_tab, const void *k,
                          const void *v, const gkv_cache_view *cache, const float *sinks,
                          int32_t window, void *out, int64_t out_stride, int32_t out_dtype,
                          uint32_t *dev_err) {
  using namespace gkv;
  if (B < 0 || max_len < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || window < 0 ||
      (out_dtype != GKV_F32 && out_dtype != GKV_BF16))
    return GKV_ERR_ARG;
  if (B > 0 && (!cu_seqlens || !q || !sinks || !out))
    return GKV_ERR_ARG;
  if (n_q_heads % n_kv_heads != 0 || (cos_tab == nullptr) != (sin_tab == nullptr) ||
      (k == nullptr) != (v == nullptr))
    return GKV_ERR_ARG;
  const bool cached = cache && cache->k; // a history in the cache
  if (!k && !cached)
    return GKV_ERR_ARG; // keys from nowhere
  if (start_pos && !cached)
    return GKV_ERR_ARG; // a history needs the cache
  if (cached) {
    if (!cache->v || !cache->block_table || cache->table_stride <= 0 || cache->num_blocks <= 0 ||
        cache->n_kv_heads != n_kv_heads || cache->ring < 0)
      return GKV_ERR_ARG;
    if (cache->v_format != GKV_V_BF16 && cache->v_format != GKV_V_INT8 &&
        cache->v_format != GKV_KV_FP8)
      return GKV_ERR_ARG;
    if ((cache->v_format != GKV_V_BF16) != (cache->v_scale != nullptr) ||
        (uintptr_t)cache->v_scale % 16 != 0)
      return GKV_ERR_ARG;
    if (cache->ring > 0 && (window != cache->ring || !k))
      return GKV_ERR_ARG; // a ring holds the history only: the chunk comes as packed rows
    if (((uintptr_t)cache->k | (uintptr_t)cache->v) % 16 != 0)
      return GKV_ERR_ARG;
  }
  const int G = n_q_heads / n_kv_heads;
  if (G > 8)
    return GKV_ERR_UNSUPPORTED;
  if (q_stride < (int64_t)n_q_heads * kHeadDim || out_stride < (int64_t)n_q_heads * kHeadDim ||
      (q_stride % 4) != 0)
    return GKV_ERR_ARG;
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)q | (uintptr_t)cos_tab | (uintptr_t)sin_tab) %
          16 != 0)
    return GKV_ERR_ARG; // 16-byte vector loads
  const int n_qblocks = (max_len + kQBlock - 1) / kQBlock;
  const int band = std::min(query_band(), std::max(n_qblocks, 1));
  const int64_t grid = (int64_t)((n_qblocks + band - 1) / band) * band * B * n_kv_heads;
  if (grid == 0)
    return GKV_OK;
  if (grid >= INT32_MAX)
    return GKV_ERR_ARG;
  PrefillArgs a;
  a.cu = cu_seqlens;
  a.start = start_pos;
  a.q = q;
  a.q_stride = q_stride;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.k = (const uint16_t *)k;
  a.v = (const uint16_t *)v;
  a.kv_stride = (int64_t)n_kv_heads * kHeadDim;
  a.kc = cached ? (const uint16_t *)cache->k : nullptr;
  a.vc = cached ? (const uint16_t *)cache->v : nullptr;
  a.vs = cached ? (const float *)cache->v_scale : nullptr;
  a.table = cached ? cache->block_table : nullptr;
  a.table_stride = cached ? cache->table_stride : 0;
  a.num_blocks = cached ? cache->num_blocks : 0;
  a.ring = cached ? cache->ring : 0;
  a.sinks = sinks;
  a.B = B;
  a.G = G;
  a.n_kv_heads = n_kv_heads;
  a.window = window;
  a.n_qblocks = n_qblocks;
  a.band = band;
  a.out = out;
  a.out_stride = out_stride;
  a.out_bf16 = out_dtype == GKV_BF16;
  a.dev_err = dev_err;
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)grid);
  if (cached && cache->v_format == GKV_KV_FP8)
    launch_prefill<true, 2>(a, G, g, s);
  else if (cached && cache->v_format == GKV_V_INT8)
    launch_prefill<true, 1>(a, G, g, s);
  else if (cached)
    launch_prefill<true, 0>(a, G, g, s);
  else
    launch_prefill<false, 0>(a, G, g, s);
  return launch_status("prefill_kernel");
}

extern "C" int gkv_prefill_attention(void *stream, int32_t B, const int32_t *cu_seqlens,
                                     int32_t max_len, int32_t n_q_heads, int32_t n_kv_heads,
                                     const float *q, int64_t q_stride, const float *cos_tab,
                                     const float *sin_tab, const void *k, const void *v,
                                     const float *sinks, int32_t window, void *out,
                                     int64_t out_stride, int32_t out_dtype) {
  if (!k || !v)
    return GKV_ERR_ARG;
  return prefill_launch(stream, B, cu_seqlens, nullptr, max_len, n_q_heads, n_kv_heads, q,
                        q_stride, cos_tab, sin_tab, k, v, nullptr, sinks, window, out, out_stride,
                        out_dtype, nullptr);
}

extern "C" int gkv_prefill_paged(void *stream, int32_t B, const int32_t *cu_seqlens,
                                 const int32_t *start_pos, int32_t max_len, int32_t n_q_heads,
                                 const float *q, int64_t q_stride, const float *cos_tab,
                                 const float *sin_tab, const void *k, const void *v,
                                 gkv_cache_view cache, const float *sinks, int32_t window,
                                 void *out, int64_t out_stride, int32_t out_dtype,
                                 uint32_t *dev_err) {
  return prefill_launch(stream, B, cu_seqlens, start_pos, max_len, n_q_heads, cache.n_kv_heads,
                        q, q_stride, cos_tab, sin_tab, k, v, &cache, sinks, window, out,
                        out_stride, out_dtype, dev_err);
}

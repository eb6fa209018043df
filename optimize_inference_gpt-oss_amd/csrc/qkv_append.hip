// QKV projection with the KV append in its epilogue.
//
// Replaces the pair gemm_bf16 (getp-csrc/kernels/fast_gemm.hpp:888-899) +
// rope_kv_bf16 (fast_misc.hpp:112-127) of layer_attention
// (getp-csrc/engine/gpu_engine.hpp:493-496): qkv = x . W^T + bias, with x
// bf16 [M][K] and W bf16 [N][K] row-major, fp32 accumulation, the bias added
// to the finished sum, as gemm_bf16 computes it; then the K part rotated and
// the K and V parts rounded into the paged cache exactly as gkv_kv_append
// stores them (same rotation, rounding and placement code), without the fp32
// K/V rows going through memory. The fp32 qkv rows (Q, K, V unrotated, what
// gemm_bf16 writes) are stored too when asked: the attention reads Q from
// them.
//
// Work: one workgroup per kQkvBM x kQkvBN output tile (as built 64 x 64, one
// head, 4 waves; three workgroups per CU), the K dimension in chunks of 64
// through a 3-stage LDS pipeline fed by direct-to-LDS loads (16-byte slots
// XOR-swizzled per row, as in the prefill kernel). Each wave owns 16 rows
// (kRT row tiles of 16) and one head of the tile: kRT x 4 tiles of
// v_mfma_f32_16x16x32_bf16, so a lane holds dims d and d + 32 of its rows --
// both halves of a RoPE pair -- in registers. With the number of column
// blocks a multiple of 8, the row blocks of one column block run on one XCD
// (their W tile is read from one L2).
//
// Placement of each row (its sequence, position, slot and block) is loaded by
// the first waves in three dependent hops of direct-to-LDS loads spread over the
// first main-loop iterations, so its round trips overlap the loop instead of
// adding to it.
#include "gkv_device.hpp"
#include "kv_append.hpp"
#include "lds_dma.hpp"

namespace gkv {

// Launch shapes: output rows per workgroup (64 or 128), output columns (64 or
// 128: one or two heads), the K chunk of a pipeline stage (32 or 64), the
// LDS stages and the waves per workgroup. Few rows (a decode step): 64 x 64
// tiles, three workgroups per CU, enough of them to fill the GPU. Many rows
// (prompts): 128 x 128 tiles with 8 waves and 2 stages (two workgroups per
// CU), four times the reuse of each loaded byte.
constexpr int kQkvBM = 64;
constexpr int kQkvWaves = 4;
constexpr int kQkvBN = 64;
constexpr int kQkvBK = 64;
constexpr int kQkvStages = 3;
constexpr int kQkvBigRows = 2048; // from this many rows on, the large tiles
constexpr int kQkvBigBM = 128, kQkvBigBN = 128, kQkvBigWaves = 8, kQkvBigStages = 2;

struct QkvArgs {
  const uint16_t *x; // bf16 [M][x_stride]
  int64_t x_stride;
  const uint16_t *w; // bf16 [N][K]
  const float *bias; // [N] or nullptr
  float *out;        // fp32 [M][out_stride] or nullptr
  int64_t out_stride;
  int M, N, K, m_blocks, xcd_map;
  AppendArgs ap; // placement, tables and cache of the append (qkv/q_out/packs unused)
};

template <int kGM, int kGN, int kGK, int kGStages, int kNW>
__global__ __launch_bounds__(64 * kNW) void qkv_append_kernel(QkvArgs a) {
  constexpr int kWN = kGN / 64;                // waves along N (one head each)
  constexpr int kWM = kNW / kWN;               // waves along M
  constexpr int kRT = kGM / 16 / kWM;          // 16-row tiles per wave
  constexpr int kSPR = kGK / 8;                // 16-byte slots per row of a stage
  constexpr int kRPC = 64 / kSPR;              // rows per 1 KB direct-to-LDS load
  constexpr int kXChunks = kGM / kRPC / kNW;   // x loads per wave per chunk
  constexpr int kWChunks = kGN / kRPC / kNW;   // W loads per wave per chunk
  static_assert(kRT >= 1 && kXChunks >= 1 && kWChunks >= 1, "launch shape");
  constexpr int kGPer = kXChunks + kWChunks;   // direct-to-LDS loads per wave per chunk
  // slot swizzle of row r: 8 rows (64-wide chunk) or 4 row groups of 4
  // (32-wide chunk) see every slot, so the 16 lanes reading one slot column of
  // 16 rows hit distinct banks
  auto swz = [](int r) { return kGK == 64 ? (r & 7) : ((r >> 2) & 3); };
  __shared__ __attribute__((aligned(16))) uint16_t x_st[kGStages][kGM * kGK];
  __shared__ __attribute__((aligned(16))) uint16_t w_st[kGStages][kGN * kGK];
  __shared__ int s_pos[kGM], s_off[kGM];
  __shared__ int64_t s_base[kGM];
  // placement loads land here (direct-to-LDS, one int per row)
  __shared__ __attribute__((aligned(16))) int s_seq[kGM], s_rpos[kGM], s_len[kGM], s_id[kGM];

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int n = lane & 15, kg = lane >> 4;
  int mb, nb;
  {
    const int id = blockIdx.x;
    if (a.xcd_map) { // the m blocks of column block nb on XCD nb % 8
      const int x = id % 8, r = id / 8;
      mb = r % a.m_blocks;
      nb = x + 8 * (r / a.m_blocks);
    } else {
      mb = id % a.m_blocks;
      nb = id / a.m_blocks;
    }
  }
  const int m0 = mb * kGM, n0 = nb * kGN;
  const int nk = a.K / kGK;
  const AppendArgs &ap = a.ap;
  const bool appends = ap.kc != nullptr;

  // ---- pipeline of K chunks; a chunk past the last re-reads the last one,
  // so every iteration issues the same loads and the waits are exact.
  auto dma = [&](int kc, int st) {
    const int k0 = min(kc, nk - 1) * kGK;
#pragma unroll
    for (int i = 0; i < kXChunks; i++) {
      const int c = wave + kNW * i;
      const int r = c * kRPC + lane / kSPR, slot = lane % kSPR;
      const int row = min(m0 + r, a.M - 1);
      dma16(a.x + (int64_t)row * a.x_stride + k0 + 8 * (slot ^ swz(r)), &x_st[st][c * 512]);
    }
#pragma unroll
    for (int i = 0; i < kWChunks; i++) {
      const int c = wave + kNW * i;
      const int r = c * kRPC + lane / kSPR, slot = lane % kSPR;
      const int col = min(n0 + r, a.N - 1);
      dma16(a.w + (int64_t)col * a.K + k0 + 8 * (slot ^ swz(r)), &w_st[st][c * 512]);
    }
  };

  // ---- row placement (waves 0 .. kGM/64 - 1; lane t of wave w: row
  // m0 + 64 w + t): hop 1 loads the row's sequence and position, hop 2
  // its sequence length, hop 3 its block id, each a direct-to-LDS load (a
  // register load would be left in flight across code the compiler schedules
  // freely); hops 2 and 3 are issued inside the main loop after waits that
  // cover the hop before.
  const int prl = 64 * wave + lane; // row within the tile
  const int pr = min(m0 + prl, a.M - 1);
  const bool place = wave < kGM / 64 && appends;
  const bool need_len = ap.seq_lens && (!ap.row_pos || ap.ring > 0);
  auto place_hop1 = [&]() {
    if (!place)
      return;
    if (ap.row_seq)
      dma4(ap.row_seq + pr, s_seq + 64 * wave);
    if (ap.row_pos)
      dma4(ap.row_pos + pr, s_rpos + 64 * wave);
  };
  auto row_seq_of = [&]() { return ap.row_seq ? s_seq[prl] : pr; };
  auto place_hop2 = [&]() {
    if (!place || !need_len)
      return;
    dma4(ap.seq_lens + row_seq_of(), s_len + 64 * wave);
  };
  int p_slot = 0, p_pos = 0;
  bool p_store = false;
  auto place_hop3 = [&]() {
    if (!place)
      return;
    const int seq = row_seq_of();
    const int len = need_len ? s_len[prl] : 0;
    const int pos = ap.row_pos ? s_rpos[prl] : len - 1;
    p_pos = pos;
    p_slot = ap.ring > 0 ? pos % ap.ring : pos;
    p_store = m0 + prl < a.M && pos >= 0;
    if (p_store && ap.ring > 0 && ap.seq_lens && pos + ap.ring < len)
      p_store = false; // a later row of this call takes the ring slot
    const int blk = p_slot / kBlockTokens;
    if (p_store && blk >= ap.table_stride) {
      if (ap.dev_err)
        atomicOr(ap.dev_err, GKV_DEVERR_LENGTH);
      p_store = false;
    }
    // rows that are not stored load entry 0 (any valid address)
    dma4(ap.table + (p_store ? (int64_t)seq * ap.table_stride + blk : 0), s_id + 64 * wave);
  };
  auto place_finish = [&]() { // after the loop's final wait: every load has landed
    if (wave >= kGM / 64)
      return;
    int64_t base = -1;
    if (place && p_store) {
      const int id = s_id[prl];
      if (id < 0 || id >= ap.num_blocks) {
        if (ap.dev_err)
          atomicOr(ap.dev_err, GKV_DEVERR_BLOCK_ID);
      } else {
        base = (int64_t)id * ap.n_kv_heads * (kBlockTokens * kHeadDim);
      }
    }
    s_pos[prl] = max(p_pos, 0);
    s_off[prl] = base >= 0 ? p_slot % kBlockTokens : -1;
    s_base[prl] = base;
  };

  // ---- main loop
  const int wm = wave % kWM, wn = wave / kWM;
  f32x4 acc[kRT][4];
#pragma unroll
  for (int i = 0; i < kRT; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  place_hop1();
#pragma unroll
  for (int p = 0; p < kGStages - 1; p++)
    dma(p, p);
  int st = 0;
  for (int kc = 0; kc < nk; kc++) {
    // chunk kc landed (only the next kGStages - 2 chunks and the placement
    // loads issued after chunk kc may still fly); the barrier also frees the
    // stage of chunk kc - 1 for chunk kc + kGStages - 1
    wait_vmcnt<(kGStages - 2) * kGPer>();
    lds_barrier();
    if (kc == 0)
      place_hop2(); // hop 1 was issued before chunk 0
    else if (kc == kGStages - 1)
      place_hop3(); // hop 2 was issued in iteration 0, before chunk kGStages - 1
    dma(kc + kGStages - 1, st == 0 ? kGStages - 1 : st - 1);
    const uint16_t *xs = x_st[st], *ws = w_st[st];
#pragma unroll
    for (int ks = 0; ks < kGK / 32; ks++) {
      bf16x8 xo[kRT], wo[4];
#pragma unroll
      for (int i = 0; i < kRT; i++) {
        const int r = 16 * kRT * wm + 16 * i + n, s = 4 * ks + kg;
        xo[i] = *(const bf16x8 *)&xs[r * kGK + 8 * (s ^ swz(r))];
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int r = 64 * wn + 16 * j + n, s = 4 * ks + kg;
        wo[j] = *(const bf16x8 *)&ws[r * kGK + 8 * (s ^ swz(r))];
      }
#pragma unroll
      for (int i = 0; i < kRT; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xo[i], wo[j], acc[i][j], 0, 0, 0);
    }
    st = st == kGStages - 1 ? 0 : st + 1;
  }
  wait_vmcnt<0>(); // every load landed, none still writes LDS
  // a short K (fewer than kGStages chunks) left hop 3 for here
  if (nk <= kGStages - 1) {
    place_hop3();
    wait_vmcnt<0>();
  }
  place_finish();
  __syncthreads();

  // ---- epilogue. acc[i][j][r] is row m0 + 16 kRT wm + 16 i + 4 kg + r,
  // column n0 + 64 wn + 16 j + n: head hd, dim d = 16 j + n.
  const int hd = (n0 >> 6) + wn;
  const int c0 = 64 * hd;
  if (c0 >= a.N)
    return;
  float bias[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    bias[j] = a.bias ? a.bias[c0 + 16 * j + n] : 0.0f;
#pragma unroll
  for (int i = 0; i < kRT; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        acc[i][j][r] += bias[j];
  if (a.out) {
#pragma unroll
    for (int i = 0; i < kRT; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + 16 * kRT * wm + 16 * i + 4 * kg + r;
        if (m < a.M) {
#pragma unroll
          for (int j = 0; j < 4; j++)
            a.out[(int64_t)m * a.out_stride + c0 + 16 * j + n] = acc[i][j][r];
        }
      }
  }
  if (!appends || hd < ap.n_q_heads)
    return;
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const bool is_k = hd < ap.n_q_heads + ap.n_kv_heads;
  const int g = is_k ? hd - ap.n_q_heads : hd - ap.n_q_heads - ap.n_kv_heads;
#pragma unroll
  for (int i = 0; i < kRT; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int lr = 16 * kRT * wm + 16 * i + 4 * kg + r; // row within the tile
      const int off = s_off[lr];
      const int64_t base = s_base[lr] + (int64_t)g * (kBlockTokens * D);
      const bool st_ok = m0 + lr < a.M && off >= 0;
      if (is_k) {
        const int pos = s_pos[lr];
        float kr[4]; // dims n, 16 + n (first of their pairs), 32 + n, 48 + n
#pragma unroll
        for (int j = 0; j < 2; j++) { // dims d = 16 j + n and d + 32
          const int d = 16 * j + n;
          const float c = ap.cos_tab[(int64_t)pos * HALF + d];
          const float s = ap.sin_tab[(int64_t)pos * HALF + d];
          const float x1 = acc[i][j][r], x2 = acc[i][j + 2][r];
          kr[j] = rope_first(x1, x2, c, s);
          kr[j + 2] = rope_second(x1, x2, c, s);
        }
        if (ap.kv_fp8) {
          // e4m3 K: the head's max |k| over its 64 dims (16 lanes), one
          // scale per token and head, each code stored by its lane
          float amax = 0.0f;
#pragma unroll
          for (int j = 0; j < 4; j++)
            amax = fmaxf(amax, fabsf(kr[j]));
#pragma unroll
          for (int sh = 1; sh < 16; sh <<= 1)
            amax = fmaxf(amax, __shfl_xor(amax, sh));
          const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
          if (st_ok) {
            uint8_t *kq = (uint8_t *)ap.kc + base;
#pragma unroll
            for (int j = 0; j < 4; j++)
              kq[k_fp8_offset(off, 16 * j + n)] = (uint8_t)fp8x4(kr[j], 0.0f, 0.0f, 0.0f, inv);
            if (n == 0)
              ap.vs[base / 32 + off] = amax / 448.0f;
          }
        } else if (st_ok) {
#pragma unroll
          for (int j = 0; j < 4; j++)
            ap.kc[base + k_offset(off, 16 * j + n)] = f32_to_bf16_rne(kr[j]);
        }
      } else if (ap.kv_fp8) {
        // e4m3 V: as the key, codes in the int8 V layout, the scale after
        // the token's K scale
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
          amax = fmaxf(amax, fabsf(acc[i][j][r]));
#pragma unroll
        for (int sh = 1; sh < 16; sh <<= 1)
          amax = fmaxf(amax, __shfl_xor(amax, sh));
        const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
        if (st_ok) {
          uint8_t *vq = (uint8_t *)ap.vc + base;
#pragma unroll
          for (int j = 0; j < 4; j++)
            vq[v_int8_offset(16 * j + n, off)] = (uint8_t)fp8x4(acc[i][j][r], 0.0f, 0.0f, 0.0f, inv);
          if (n == 0)
            ap.vs[base / 32 + kBlockTokens + off] = amax / 448.0f;
        }
      } else if (ap.v_int8) {
        // the head's max |v| over its 64 dims (4 per lane, 16 lanes), then
        // the reference's rule, getp-csrc/kernels/fast_misc.hpp:74-84
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
          amax = fmaxf(amax, fabsf(acc[i][j][r]));
#pragma unroll
        for (int sh = 1; sh < 16; sh <<= 1)
          amax = fmaxf(amax, __shfl_xor(amax, sh));
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        if (st_ok) {
          int8_t *vq = (int8_t *)ap.vc + base;
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const float cq = fminf(fmaxf(rintf(acc[i][j][r] * inv), -127.0f), 127.0f);
            vq[v_int8_offset(16 * j + n, off)] = (int8_t)cq;
          }
          if (n == 0)
            ap.vs[base / D + off] = amax / 127.0f;
        }
      } else if (st_ok) {
#pragma unroll
        for (int j = 0; j < 4; j++)
          ap.vc[base + v_offset(off, 16 * j + n)] = f32_to_bf16_rne(acc[i][j][r]);
      }
    }
}

} // namespace gkv

extern "C" int gkv_qkv_append(void *stream, int32_t n_rows, const void *x, int64_t x_stride,
                              int32_t hidden, const void *w_qkv, const float *b_qkv,
                              int32_t n_q_heads, const float *cos_tab, const float *sin_tab,
                              const int32_t *row_pos, const int32_t *row_seq,
                              const int32_t *seq_lens, gkv_cache_view cache, float *qkv_out,
                              int64_t out_stride, uint32_t *dev_err) {
  using namespace gkv;
  if (n_rows < 0 || !x || !w_qkv || n_q_heads <= 0 || cache.n_kv_heads <= 0 || hidden <= 0 ||
      cache.ring < 0)
    return GKV_ERR_ARG;
  if (n_q_heads % cache.n_kv_heads != 0)
    return GKV_ERR_ARG;
  const int64_t n_cols = (int64_t)(n_q_heads + 2 * cache.n_kv_heads) * kHeadDim;
  if (n_cols >= INT32_MAX || x_stride < hidden || (qkv_out && out_stride < n_cols))
    return GKV_ERR_ARG;
  if (hidden % kQkvBK != 0)
    return GKV_ERR_UNSUPPORTED;
  // 16-byte direct-to-LDS loads of x and W rows
  if (x_stride % 8 != 0 || ((uintptr_t)x | (uintptr_t)w_qkv) % 16 != 0)
    return GKV_ERR_ARG;
  const bool to_cache = cache.k != nullptr || cache.v != nullptr;
  if (!to_cache && !qkv_out)
    return GKV_ERR_ARG; // nothing to write
  if (to_cache && (!cache.k || !cache.v || !cache.block_table || cache.table_stride <= 0 ||
                   cache.num_blocks <= 0 || !cos_tab || !sin_tab))
    return GKV_ERR_ARG;
  if (to_cache && !row_pos && !seq_lens)
    return GKV_ERR_ARG; // no way to find the rows' positions
  if (to_cache && cache.ring > 0 && !seq_lens)
    return GKV_ERR_ARG; // rows W positions apart share a ring slot: the lengths pick the kept one
  if (cache.ring % kBlockTokens != 0)
    return GKV_ERR_UNSUPPORTED;
  if (cache.v_format != GKV_V_BF16 && cache.v_format != GKV_V_INT8 &&
      cache.v_format != GKV_KV_FP8)
    return GKV_ERR_ARG;
  if (to_cache && cache.v_format != GKV_V_BF16 && !cache.v_scale)
    return GKV_ERR_ARG;
  if (n_rows == 0)
    return GKV_OK;
  QkvArgs a;
  a.x = (const uint16_t *)x;
  a.x_stride = x_stride;
  a.w = (const uint16_t *)w_qkv;
  a.bias = b_qkv;
  a.out = qkv_out;
  a.out_stride = out_stride;
  a.M = n_rows;
  a.N = (int)n_cols;
  a.K = hidden;
  const bool big = n_rows >= kQkvBigRows;
  const int bm = big ? kQkvBigBM : kQkvBM, bn = big ? kQkvBigBN : kQkvBN;
  a.m_blocks = (n_rows + bm - 1) / bm;
  const int n_blocks = (int)((n_cols + bn - 1) / bn);
  a.xcd_map = n_blocks % 8 == 0;
  const int64_t grid = (int64_t)a.m_blocks * n_blocks;
  if (grid >= INT32_MAX)
    return GKV_ERR_ARG;
  AppendArgs &ap = a.ap;
  ap.qkv = nullptr;
  ap.row_stride = 0;
  ap.n_q_heads = n_q_heads;
  ap.n_kv_heads = cache.n_kv_heads;
  ap.cos_tab = cos_tab;
  ap.sin_tab = sin_tab;
  ap.row_pos = row_pos;
  ap.row_seq = row_seq;
  ap.seq_lens = seq_lens;
  ap.kc = to_cache ? (uint16_t *)cache.k : nullptr;
  ap.vc = to_cache ? (uint16_t *)cache.v : nullptr;
  ap.table = cache.block_table;
  ap.table_stride = cache.table_stride;
  ap.num_blocks = cache.num_blocks;
  ap.ring = cache.ring;
  ap.q_out = nullptr;
  ap.q_out_stride = 0;
  ap.k_pack = nullptr;
  ap.v_pack = nullptr;
  ap.dev_err = dev_err;
  ap.v_int8 = cache.v_format == GKV_V_INT8;
  ap.kv_fp8 = cache.v_format == GKV_KV_FP8;
  ap.vs = (float *)cache.v_scale;
  if (big)
    hipLaunchKernelGGL(
        (qkv_append_kernel<kQkvBigBM, kQkvBigBN, kQkvBK, kQkvBigStages, kQkvBigWaves>),
        dim3((unsigned)grid), dim3(64 * kQkvBigWaves), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((qkv_append_kernel<kQkvBM, kQkvBN, kQkvBK, kQkvStages, kQkvWaves>),
                       dim3((unsigned)grid), dim3(64 * kQkvWaves), 0, (hipStream_t)stream, a);
  return launch_status(__func__);
}

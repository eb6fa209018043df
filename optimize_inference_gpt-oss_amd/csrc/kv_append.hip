// KV append: RoPE on K, then bf16 K and V into the paged cache.
//
// Replaces rope_kv_bf16 (getp-csrc/kernels/fast_misc.hpp:48-127) and the exact
// path's rope_exact + kv_write_kernel (kernels/misc.hpp:55-85). Semantics are
// run.cpp's: the rotated key and the value of the new token go into the cache
// at its position (run.cpp:573-576, 588-592); a window layer keeps position p
// in ring slot p % W (gpu_engine.hpp:477). The rotation uses run.cpp's
// rounding (gkv::rope_first/second) and the angles of the host table
// (gkv_rope_table), so the stored bits equal the CPU path's bf16 of its fp32
// key.
//
// Layout written: 2 KB per block and head for K and for V, in the orders of
// k_offset / v_offset (kv_append.hpp), which put each lane's matrix-core
// operand pieces of the attention kernel in 16 contiguous bytes, in lane
// order. One wave per row, 16 rows per workgroup: a row's chain of dependent
// loads (its sequence, length and block id) is short work for one wave, and a
// prompt's tens of thousands of rows keep many chains in flight. HBM-bound
// (4 KB of K/V read and 2 KB written per token per layer, twice that with the
// packed rows).
#include "kv_append.hpp"

namespace gkv {

constexpr int kRowsPerWg = 16;
constexpr int kMaxStageHeads = 8; // bf16 V rows staged in LDS up to this many kv heads

// With a bf16 V cache the rows' V goes through LDS: four rows of the
// workgroup holding slots 4m .. 4m+3 of one block (consecutive tokens of a
// prompt) are written together, as 16-byte pieces (dims d and d+16 of the 4
// tokens, contiguous in the V block layout), which fill whole 128-byte lines;
// storing one token's values alone scatters 2-byte writes over the block and
// leaves partly written lines. Rows without such a quad store element-wise.
__global__ __launch_bounds__(64 * kRowsPerWg) void kv_append_kernel(AppendArgs a, int n_rows) {
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kRowsPerWg][kMaxStageHeads * kHeadDim];
  __shared__ int s_slot[kRowsPerWg], s_seq[kRowsPerWg];
  __shared__ int64_t s_base[kRowsPerWg];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * kRowsPerWg + w;
  const bool staged = !a.v_int8 && !a.kv_fp8 && a.vc && a.n_kv_heads <= kMaxStageHeads;
  RowPlace pl{0, -1, -1, 0};
  // Without a rotated-query output the row's loads go out at once (its K or
  // V pieces, then its place and angles) and the stores follow; else the
  // general form.
  if (r < n_rows && !a.q_out && a.n_kv_heads <= 8)
    pl = append_end(a, append_begin(a, r, lane, -1), r, lane, staged ? s_v[w] : nullptr);
  else if (r < n_rows)
    pl = append_row(a, r, lane, 0, 1, staged ? s_v[w] : nullptr);
  if (!staged)
    return;
  if (lane == 0) {
    s_slot[w] = pl.store ? pl.slot : -1;
    s_seq[w] = pl.seq;
    s_base[w] = pl.base;
  }
  __syncthreads();
  auto leads = [&](int i) {
    if (i < 0 || i + 3 >= kRowsPerWg || s_slot[i] < 0 || (s_slot[i] & 3) != 0)
      return false;
    for (int k = 1; k < 4; k++)
      if (s_slot[i + k] != s_slot[i] + k || s_seq[i + k] != s_seq[i] ||
          s_base[i + k] != s_base[i])
        return false;
    return true;
  };
  const bool in_quad = leads(w) || leads(w - 1) || leads(w - 2) || leads(w - 3);
  constexpr int D = kHeadDim;
  if (pl.store && !in_quad) {
    const int off = pl.slot % kBlockTokens;
    for (int idx = lane; idx < a.n_kv_heads * D; idx += 64) {
      const int g = idx / D, d = idx % D;
      a.vc[pl.base + (int64_t)g * (kBlockTokens * D) + v_offset(off, d)] = s_v[w][idx];
    }
  }
  if (leads(w)) {
    const int t0 = pl.slot % kBlockTokens; // 4m
    for (int p = lane; p < a.n_kv_heads * 32; p += 64) {
      const int g = p / 32, d = 32 * ((p / 16) % 2) + p % 16; // dims d and d + 16
      uint16_t h[8];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        h[k] = s_v[w + k][g * D + d];
        h[4 + k] = s_v[w + k][g * D + d + 16];
      }
      *(u32x4 *)(a.vc + pl.base + (int64_t)g * (kBlockTokens * D) + v_offset(t0, d)) = pack8(h);
    }
  }
}

} // namespace gkv

extern "C" int gkv_kv_append(void *stream, int32_t n_rows, const float *qkv, int64_t row_stride,
                             int32_t n_q_heads, const float *cos_tab, const float *sin_tab,
                             const int32_t *row_pos, const int32_t *row_seq,
                             const int32_t *seq_lens, gkv_cache_view cache, float *q_out,
                             int64_t q_out_stride, void *k_pack, void *v_pack,
                             uint32_t *dev_err) {
  using namespace gkv;
  if (n_rows < 0 || !qkv || !cos_tab || !sin_tab || !row_pos || n_q_heads <= 0 ||
      cache.n_kv_heads <= 0 || cache.ring < 0)
    return GKV_ERR_ARG;
  if (n_q_heads % cache.n_kv_heads != 0)
    return GKV_ERR_ARG;
  const int64_t qkv_width = (int64_t)(n_q_heads + 2 * cache.n_kv_heads) * kHeadDim;
  if (row_stride < qkv_width || (q_out && q_out_stride < (int64_t)n_q_heads * kHeadDim))
    return GKV_ERR_ARG;
  // 16-byte vector loads and stores
  if (row_stride % 4 != 0 ||
      ((uintptr_t)qkv | (uintptr_t)cos_tab | (uintptr_t)sin_tab | (uintptr_t)k_pack |
       (uintptr_t)v_pack) % 16 != 0)
    return GKV_ERR_ARG;
  const bool to_cache = cache.k != nullptr || cache.v != nullptr;
  if (to_cache && (!cache.k || !cache.v || !cache.block_table || cache.table_stride <= 0 ||
                   cache.num_blocks <= 0))
    return GKV_ERR_ARG;
  if (cache.ring % kBlockTokens != 0)
    return GKV_ERR_UNSUPPORTED;
  if (cache.v_format != GKV_V_BF16 && cache.v_format != GKV_V_INT8 &&
      cache.v_format != GKV_KV_FP8)
    return GKV_ERR_ARG;
  if (to_cache && cache.v_format != GKV_V_BF16 && !cache.v_scale)
    return GKV_ERR_ARG;
  // On a ring, two rows of one sequence W positions apart take the same slot;
  // only the lengths tell which of them the ring keeps.
  if (to_cache && cache.ring > 0 && !seq_lens)
    return GKV_ERR_ARG;
  if (n_rows == 0)
    return GKV_OK;
  AppendArgs a;
  a.qkv = qkv;
  a.row_stride = row_stride;
  a.n_q_heads = n_q_heads;
  a.n_kv_heads = cache.n_kv_heads;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.row_pos = row_pos;
  a.row_seq = row_seq;
  a.seq_lens = seq_lens;
  a.kc = to_cache ? (uint16_t *)cache.k : nullptr;
  a.vc = to_cache ? (uint16_t *)cache.v : nullptr;
  a.table = cache.block_table;
  a.table_stride = cache.table_stride;
  a.num_blocks = cache.num_blocks;
  a.ring = cache.ring;
  a.q_out = q_out;
  a.q_out_stride = q_out_stride;
  a.k_pack = (uint16_t *)k_pack;
  a.v_pack = (uint16_t *)v_pack;
  a.dev_err = dev_err;
  a.v_int8 = cache.v_format == GKV_V_INT8;
  a.kv_fp8 = cache.v_format == GKV_KV_FP8;
  a.vs = (float *)cache.v_scale;
  hipLaunchKernelGGL(kv_append_kernel, dim3((n_rows + kRowsPerWg - 1) / kRowsPerWg),
                     dim3(64 * kRowsPerWg), 0, (hipStream_t)stream, a, n_rows);
  return launch_status(__func__);
}

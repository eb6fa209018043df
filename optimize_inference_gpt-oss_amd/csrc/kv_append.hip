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
// order. 256 threads per row, 4 rows per workgroup (a prompt's append has
// tens of thousands of rows: fewer, larger workgroups launch faster); HBM-bound
// (2 KB written per token per layer).
#include "kv_append.hpp"

namespace gkv {

constexpr int kRowThreads = 256, kRowsPerWg = 4;

__global__ __launch_bounds__(kRowThreads *kRowsPerWg) void kv_append_kernel(AppendArgs a,
                                                                           int n_rows) {
  const int r = blockIdx.x * kRowsPerWg + threadIdx.x / kRowThreads;
  if (r < n_rows)
    append_row(a, r, threadIdx.x % kRowThreads, kRowThreads);
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
  const bool to_cache = cache.k != nullptr || cache.v != nullptr;
  if (to_cache && (!cache.k || !cache.v || !cache.block_table || cache.table_stride <= 0 ||
                   cache.num_blocks <= 0))
    return GKV_ERR_ARG;
  if (cache.ring % kBlockTokens != 0)
    return GKV_ERR_UNSUPPORTED;
  if (cache.v_format != GKV_V_BF16 && cache.v_format != GKV_V_INT8)
    return GKV_ERR_ARG;
  if (to_cache && cache.v_format == GKV_V_INT8 && !cache.v_scale)
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
  a.vs = (float *)cache.v_scale;
  hipLaunchKernelGGL(kv_append_kernel, dim3((n_rows + kRowsPerWg - 1) / kRowsPerWg),
                     dim3(kRowThreads * kRowsPerWg), 0, (hipStream_t)stream, a, n_rows);
  return launch_status(__func__);
}

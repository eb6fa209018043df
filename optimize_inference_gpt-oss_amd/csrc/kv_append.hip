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
// Layout written: K [block][head][16 tokens][64], V [block][head][64][16]
// (V transposed inside its block so that the attention kernel's PV operand is
// one 16-byte load per lane). One workgroup per row; HBM-bound and tiny
// (2 KB written per token per layer).
#include "gkv_device.hpp"

namespace gkv {

struct AppendArgs {
  const float *qkv;
  int64_t row_stride;
  int n_q_heads, n_kv_heads;
  const float *cos_tab, *sin_tab;
  const int32_t *row_pos, *row_seq, *seq_lens;
  uint16_t *kc, *vc;
  const int32_t *table;
  int table_stride, num_blocks, ring;
  float *q_out;
  int64_t q_out_stride;
  uint16_t *k_pack, *v_pack;
  uint32_t *dev_err;
};

__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const int r = blockIdx.x, tid = threadIdx.x;
  const int pos = a.row_pos[r];
  const int seq = a.row_seq ? a.row_seq[r] : r;
  const float *row = a.qkv + (int64_t)r * a.row_stride;
  const float *cs = a.cos_tab + (int64_t)pos * HALF, *sn = a.sin_tab + (int64_t)pos * HALF;
  const int kv_dim = a.n_kv_heads * D;

  // Rotated query (each thread owns whole pairs, so q_out may alias qkv).
  if (a.q_out) {
    float *qo = a.q_out + (int64_t)r * a.q_out_stride;
    for (int idx = tid; idx < a.n_q_heads * HALF; idx += blockDim.x) {
      const int h = idx / HALF, i = idx % HALF;
      const float x1 = row[h * D + i], x2 = row[h * D + HALF + i];
      const float c = cs[i], s = sn[i];
      const float o1 = rope_first(x1, x2, c, s), o2 = rope_second(x1, x2, c, s);
      qo[h * D + i] = o1;
      qo[h * D + HALF + i] = o2;
    }
  }

  // Where the token goes in the paged cache (if anywhere).
  const int slot = a.ring > 0 ? pos % a.ring : pos;
  bool store = a.kc != nullptr;
  if (store && a.ring > 0 && a.seq_lens && pos + a.ring < a.seq_lens[seq])
    store = false; // a later row of this call takes the ring slot
  int64_t kbase = 0, vbase = 0;
  const int off = slot % kBlockTokens;
  if (store) {
    const int blk = slot / kBlockTokens;
    if (blk >= a.table_stride) {
      if (tid == 0 && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
      store = false;
    } else {
      const int phys = a.table[(int64_t)seq * a.table_stride + blk];
      if (phys < 0 || phys >= a.num_blocks) {
        if (tid == 0 && a.dev_err)
          atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
        store = false;
      } else {
        kbase = (int64_t)phys * a.n_kv_heads * (kBlockTokens * D);
        vbase = kbase;
      }
    }
  }

  const float *kr = row + a.n_q_heads * D, *vr = kr + kv_dim;
  for (int idx = tid; idx < a.n_kv_heads * HALF; idx += blockDim.x) {
    const int g = idx / HALF, i = idx % HALF;
    const float x1 = kr[g * D + i], x2 = kr[g * D + HALF + i];
    const float c = cs[i], s = sn[i];
    const uint16_t k1 = f32_to_bf16_rne(rope_first(x1, x2, c, s));
    const uint16_t k2 = f32_to_bf16_rne(rope_second(x1, x2, c, s));
    if (store) {
      uint16_t *kd = a.kc + kbase + ((int64_t)g * kBlockTokens + off) * D;
      kd[i] = k1;
      kd[HALF + i] = k2;
    }
    if (a.k_pack) {
      uint16_t *kp = a.k_pack + (int64_t)r * kv_dim + g * D;
      kp[i] = k1;
      kp[HALF + i] = k2;
    }
  }
  for (int idx = tid; idx < kv_dim; idx += blockDim.x) {
    const int g = idx / D, d = idx % D;
    const uint16_t v = f32_to_bf16_rne(vr[idx]);
    if (store)
      a.vc[vbase + ((int64_t)g * D + d) * kBlockTokens + off] = v;
    if (a.v_pack)
      a.v_pack[(int64_t)r * kv_dim + idx] = v;
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
  const bool to_cache = cache.k != nullptr || cache.v != nullptr;
  if (to_cache && (!cache.k || !cache.v || !cache.block_table || cache.table_stride <= 0 ||
                   cache.num_blocks <= 0))
    return GKV_ERR_ARG;
  if (cache.ring % kBlockTokens != 0)
    return GKV_ERR_UNSUPPORTED;
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
  hipLaunchKernelGGL(kv_append_kernel, dim3(n_rows), dim3(256), 0, (hipStream_t)stream, a);
  return launch_status(__func__);
}

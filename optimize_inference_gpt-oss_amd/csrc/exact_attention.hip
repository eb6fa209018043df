// The exact path: RoPE, the K/V write and decode attention over fp32 caches,
// each bit for bit with the reference's CPU forward (run.cpp:506-526 and
// 597-641), as the reference's GPTOSS_EXACT engine build runs them
// (getp-csrc/engine/gpu_engine.hpp:478-488: rope_exact, kv_write_kernel,
// attention_exact of getp-csrc/kernels/misc.hpp:55-85 and attention.hpp:18-83).
//
// Bits, not speed, set the design: every sum the CPU takes in order is taken
// in the same order here (a score's 64 products in fp64, the softmax sum over
// the positions and the sink in fp64, each output dim's weighted values with
// FMA in time order), with the CPU's rounding of every step (products rounded
// to fp32 before the fp64 add, fp32 <-> fp64 conversions where the CPU has
// them, glibc's expf). What runs in parallel is what the CPU computes
// independently: the positions' scores, their exponentials and quotients,
// the 64 output dims, the query heads.
//
// Attention: one workgroup per (sequence, kv head, chunk of hc query heads),
// one wave per query head. The kv head's K rows go through LDS in tiles of 64
// positions (read once for the hc heads, 65-float rows so that lane t reading
// row t meets no bank conflict); lane t of wave h scores position t of the
// tile for head h. The scores stay in LDS, hc x (n + 1) floats (hc is chosen
// on the host so they fit), through the max, the exponentials, the sum (lane
// 0, in order), the quotients and the weighted sum of V (lane = output dim),
// whose rows go through the same LDS tile as K's.
#include <algorithm>

#include "exact_math.hpp"
#include "gkv_device.hpp"

namespace gkv {

constexpr int kExactTile = 64;
constexpr int kExactRow = kHeadDim + 1; // LDS row of a staged K position, in floats

struct ExactAttnArgs {
  const float *q;
  int64_t q_stride;
  const float *kc, *vc;
  int slots, n_kv_heads, G, hc, n_chunks, window;
  const float *sinks;
  int pos;                  // every row's position (positions == nullptr)
  const int32_t *positions; // device [B], or nullptr
  int n_cap;                // positions attended at most (sizes the score rows)
  float *out;
  int64_t out_stride;
  uint32_t *dev_err;
};

__global__ __launch_bounds__(1024) void attention_exact_kernel(ExactAttnArgs a) {
  extern __shared__ float lds[];
  __shared__ double s_sum[16];
  const int b = blockIdx.x;
  const int g = blockIdx.y / a.n_chunks;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = g * a.G + (blockIdx.y % a.n_chunks) * a.hc + wave;
  const int kv_dim = a.n_kv_heads * kHeadDim;
  float *kt = lds;                                      // [64][65]
  float *qs = kt + kExactTile * kExactRow;              // [hc][64]
  float *att = qs + a.hc * kHeadDim + wave * (a.n_cap + 1); // this head's scores

  const int p = a.positions ? a.positions[b] : a.pos;
  const int t0 = a.window > 0 ? max(0, p - a.window + 1) : 0;
  const int n = p - t0 + 1;
  // a position the cache cannot hold (full layer: p >= slots) or beyond the
  // host bound: output zeros and the length flag (uniform per workgroup)
  if (p < 0 || n > a.n_cap || (a.window == 0 && p >= a.slots)) {
    a.out[(int64_t)b * a.out_stride + (int64_t)h * kHeadDim + lane] = 0.0f;
    if (threadIdx.x == 0 && a.dev_err)
      atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
    return;
  }
  const int ring = a.window; // a window layer's cache is a ring of window slots
  const float *kbase = a.kc + (int64_t)b * a.slots * kv_dim + (int64_t)g * kHeadDim;
  const float *vbase = a.vc + (int64_t)b * a.slots * kv_dim + (int64_t)g * kHeadDim;
  qs[wave * kHeadDim + lane] = a.q[(int64_t)b * a.q_stride + (int64_t)h * kHeadDim + lane];

  // scores: (float)((sum_i (double)(q_i * k_i)) / 8), products rounded to fp32
  const double scale = (double)__fsqrt_rn((float)kHeadDim);
  for (int tile = 0; tile < n; tile += kExactTile) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < kExactTile * kHeadDim; idx += blockDim.x) {
      const int r = idx >> 6, c = idx & 63, j = tile + r;
      if (j < n) {
        const int t = t0 + j;
        const int slot = ring > 0 ? t % ring : t;
        kt[r * kExactRow + c] = kbase[(int64_t)slot * kv_dim + c];
      }
    }
    __syncthreads();
    const int j = tile + lane;
    if (j < n) {
      double s = 0.0;
      for (int i = 0; i < kHeadDim; i++)
        s = __dadd_rn(s, (double)__fmul_rn(qs[wave * kHeadDim + i], kt[lane * kExactRow + i]));
      att[j] = (float)__ddiv_rn(s, scale);
    }
  }
  if (lane == 0)
    att[n] = a.sinks[h];
  __syncthreads();

  // softmax over att[0..n] (run.cpp:335-353): the max (exact in any order),
  // expf((float)((double)x - max)), the fp64 sum in index order, the quotients
  float m = -INFINITY;
  for (int j = lane; j <= n; j += 64)
    m = fmaxf(m, att[j]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
    m = fmaxf(m, __shfl_xor(m, off));
  const double md = (double)m;
  for (int j = lane; j <= n; j += 64)
    att[j] = expf_cpu_exact((float)__dsub_rn((double)att[j], md));
  __syncthreads();
  if (lane == 0) {
    double s = 0.0;
    for (int j = 0; j <= n; j++)
      s = __dadd_rn(s, (double)att[j]);
    s_sum[wave] = s;
  }
  __syncthreads();
  const double sum = s_sum[wave];
  for (int j = lane; j <= n; j += 64)
    att[j] = (float)__ddiv_rn((double)att[j], sum);
  __syncthreads();

  // out[d] = fma(w_t, v_t[d], out[d]) over t in order; the V rows go through
  // the K tile's LDS, 64 positions at a time, read once for the hc heads
  float acc = 0.0f;
  for (int tile = 0; tile < n; tile += kExactTile) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < kExactTile * kHeadDim; idx += blockDim.x) {
      const int r = idx >> 6, c = idx & 63, j = tile + r;
      if (j < n) {
        const int t = t0 + j;
        const int slot = ring > 0 ? t % ring : t;
        kt[r * kExactRow + c] = vbase[(int64_t)slot * kv_dim + c];
      }
    }
    __syncthreads();
    const int m_t = min(kExactTile, n - tile);
    for (int r = 0; r < m_t; r++)
      acc = __fmaf_rn(att[tile + r], kt[r * kExactRow + lane], acc);
  }
  a.out[(int64_t)b * a.out_stride + (int64_t)h * kHeadDim + lane] = acc;
}

// run.cpp's apply_rotary_emb on heads 0..n_heads-1 of each row, in place.
__global__ __launch_bounds__(256) void rope_exact_kernel(float *qkv, int64_t row_stride,
                                                         const float *cos_tab,
                                                         const float *sin_tab,
                                                         const int32_t *positions, int n_heads) {
  const int b = blockIdx.x;
  constexpr int half = kHeadDim / 2;
  const int64_t p = positions ? positions[b] : 0;
  const float *cv = cos_tab + p * half, *sv = sin_tab + p * half;
  float *row = qkv + (int64_t)b * row_stride;
  for (int idx = threadIdx.x; idx < n_heads * half; idx += blockDim.x) {
    const int hh = idx / half, i = idx % half;
    float *x = row + hh * kHeadDim;
    const float x1 = x[i], x2 = x[half + i];
    x[i] = rope_first(x1, x2, cv[i], sv[i]);
    x[half + i] = rope_second(x1, x2, cv[i], sv[i]);
  }
}

// Each row's K and V (kv_dim floats each) into the fp32 caches at its slot.
__global__ __launch_bounds__(256) void kv_write_exact_kernel(
    const float *qkv, int64_t row_stride, int k_off, int v_off, float *kc, float *vc, int slots,
    int kv_dim, int slot, const int32_t *positions, int window, uint32_t *dev_err) {
  const int b = blockIdx.x;
  int s = slot;
  if (positions) {
    const int p = positions[b];
    s = p < 0 ? -1 : window > 0 ? p % window : p;
  }
  if (s < 0 || s >= slots) {
    if (threadIdx.x == 0 && dev_err)
      atomicOr(dev_err, GKV_DEVERR_LENGTH);
    return;
  }
  const float *row = qkv + (int64_t)b * row_stride;
  const int64_t dst = ((int64_t)b * slots + s) * kv_dim;
  for (int i = threadIdx.x; i < kv_dim; i += blockDim.x) {
    kc[dst + i] = row[k_off + i];
    vc[dst + i] = row[v_off + i];
  }
}

// LDS a workgroup may take (queried once per device).
static size_t lds_limit() {
  static thread_local int dev = -1;
  static thread_local size_t lim = 0;
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess)
    return 64 * 1024;
  if (d != dev) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, d) != hipSuccess ||
        v <= 0)
      v = 64 * 1024;
    dev = d;
    lim = (size_t)v;
  }
  return lim;
}

} // namespace gkv

using namespace gkv;

extern "C" int gkv_rope_exact(void *stream, int32_t B, float *qkv, int64_t row_stride,
                              const float *cos_tab, const float *sin_tab,
                              const int32_t *positions, int32_t n_heads) {
  if (B < 0 || !qkv || !cos_tab || !sin_tab || n_heads <= 0 ||
      row_stride < (int64_t)n_heads * kHeadDim)
    return GKV_ERR_ARG;
  if (B == 0)
    return GKV_OK;
  hipLaunchKernelGGL(rope_exact_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, qkv,
                     row_stride, cos_tab, sin_tab, positions, (int)n_heads);
  return launch_status("rope_exact_kernel");
}

extern "C" int gkv_kv_write_exact(void *stream, int32_t B, const float *qkv, int64_t row_stride,
                                  int32_t k_off, int32_t v_off, float *kc, float *vc,
                                  int32_t slots, int32_t kv_dim, int32_t slot,
                                  const int32_t *positions, int32_t window, uint32_t *dev_err) {
  if (B < 0 || !qkv || !kc || !vc || slots <= 0 || kv_dim <= 0 || k_off < 0 || v_off < 0 ||
      (int64_t)k_off + kv_dim > row_stride || (int64_t)v_off + kv_dim > row_stride ||
      window < 0 || (window > 0 && slots < window) ||
      (!positions && (slot < 0 || slot >= slots)))
    return GKV_ERR_ARG;
  if (B == 0)
    return GKV_OK;
  hipLaunchKernelGGL(kv_write_exact_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, qkv,
                     row_stride, (int)k_off, (int)v_off, kc, vc, (int)slots, (int)kv_dim,
                     (int)slot, positions, (int)window, dev_err);
  return launch_status("kv_write_exact_kernel");
}

extern "C" int gkv_attention_exact(void *stream, int32_t B, int32_t n_q_heads,
                                   int32_t n_kv_heads, const float *q, int64_t q_stride,
                                   const float *kc, const float *vc, int32_t slots,
                                   const float *sinks, int32_t pos, const int32_t *positions,
                                   int32_t max_pos, int32_t window, float *out,
                                   int64_t out_stride, uint32_t *dev_err) {
  if (B < 0 || !q || !kc || !vc || !sinks || !out || n_kv_heads <= 0 || n_q_heads <= 0 ||
      n_q_heads % n_kv_heads || slots <= 0 || window < 0 || (window > 0 && slots < window) ||
      q_stride < (int64_t)n_q_heads * kHeadDim || out_stride < (int64_t)n_q_heads * kHeadDim)
    return GKV_ERR_ARG;
  const int G = n_q_heads / n_kv_heads;
  if (G > 16)
    return GKV_ERR_UNSUPPORTED;
  const int p_bound = positions ? max_pos : pos;
  if (p_bound < 0 || (!positions && window == 0 && pos >= slots))
    return GKV_ERR_ARG;
  if (B == 0)
    return GKV_OK;
  // positions attended at most, then the most query heads per workgroup whose
  // score rows fit the LDS next to the K tile and the queries
  const int n_cap = window > 0 ? std::min(p_bound + 1, (int)window) : p_bound + 1;
  const size_t fixed = (size_t)kExactTile * kExactRow * sizeof(float) + 256; // + s_sum
  const size_t lim = lds_limit();
  int hc = 0;
  for (int c = G; c >= 1; c--) {
    if (G % c)
      continue;
    const size_t need = fixed + (size_t)c * (kHeadDim + n_cap + 1) * sizeof(float);
    if (need <= lim) {
      hc = c;
      break;
    }
  }
  if (hc == 0)
    return GKV_ERR_CAPACITY;
  const size_t lds = fixed - 256 + (size_t)hc * (kHeadDim + n_cap + 1) * sizeof(float);
  ExactAttnArgs a{};
  a.q = q;
  a.q_stride = q_stride;
  a.kc = kc;
  a.vc = vc;
  a.slots = slots;
  a.n_kv_heads = n_kv_heads;
  a.G = G;
  a.hc = hc;
  a.n_chunks = G / hc;
  a.window = window;
  a.sinks = sinks;
  a.pos = pos;
  a.positions = positions;
  a.n_cap = n_cap;
  a.out = out;
  a.out_stride = out_stride;
  a.dev_err = dev_err;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute((const void *)attention_exact_kernel,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return hip_status(hipGetLastError(), "attention_exact_kernel (LDS size)");
  hipLaunchKernelGGL(attention_exact_kernel, dim3(B, n_kv_heads * a.n_chunks), dim3(64 * hc),
                     lds, (hipStream_t)stream, a);
  return launch_status("attention_exact_kernel");
}

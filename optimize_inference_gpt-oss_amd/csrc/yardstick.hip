// Ceiling yardsticks: read-only kernels that state what the memory system
// gives the decode kernel's access patterns on this GPU, with no attention
// math. They play the part of the reference's read_stream and loads-only
// kernels (getp-csrc/bench/attn_bench.cpp:66-76, 161-227), which its decode
// kernel's "% of ceiling" is quoted against.
//
//   stream   every byte of a buffer once, each wave instruction reading 1 KB
//            contiguous (16 B per lane), grid-stride over a persistent grid.
//   gather   a list of 2 KB blocks in the order given (a random permutation
//            in the bench), the decode kernel's unit: one (block, kv head) of
//            the paged cache. One wave per SIMD; wave w takes list entries
//            w, w + W, w + 2W, ... in steps of 4 blocks (8 KB, the bytes of
//            one decode step), R - 1 steps in flight, each block read as two
//            1 KB instructions through a buffer resource on the block.
// Both fold what they read into an XOR and store it only if it equals a
// constant no real data produces, so no load can be dropped and nothing
// meaningful is written. The loads-only form of the decode kernel itself is
// gkv_yardstick_decode_loads (decode_attention.hip).
#include "gkv_device.hpp"

namespace gkv {

constexpr int kYsWaves = 4;              // one wave per SIMD
constexpr int kYsBlocksPerStep = 4;      // 8 KB per wave step
constexpr uint32_t kYsMagic = 0x9e3779b9u;

__global__ __launch_bounds__(64 * kYsWaves) void ys_stream_kernel(const u32x4 *src, int64_t n16,
                                                                 uint32_t *sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // four loads in flight per lane
  for (; i + 3 * stride < n16; i += 4 * stride) {
    u32x4 x[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
      x[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
    for (int k = 0; k < 4; k++)
      acc ^= x[k][0] ^ x[k][1] ^ x[k][2] ^ x[k][3];
  }
  for (; i < n16; i += stride) {
    const u32x4 x = __builtin_nontemporal_load(src + i);
    acc ^= x[0] ^ x[1] ^ x[2] ^ x[3];
  }
  if (acc == kYsMagic)
    sink[threadIdx.x] = acc;
}

template <int R>
__global__ __launch_bounds__(64 * kYsWaves) __attribute__((amdgpu_waves_per_eu(1)))
void ys_gather_kernel(const char *base, int n_blocks, const int32_t *ids, int n_ids,
                      uint32_t *sink) {
  const int lane = threadIdx.x & 63;
  const int W = gridDim.x * kYsWaves;
  const int w = blockIdx.x * kYsWaves + uniform(threadIdx.x >> 6);
  // this wave's entries: w + W * j, j = 0 .. n_mine - 1, in steps of 4
  const int n_mine = w < n_ids ? (n_ids - w + W - 1) / W : 0;
  const int n_steps = (n_mine + kYsBlocksPerStep - 1) / kYsBlocksPerStep;
  const uint32_t off = (uint32_t)lane * 16;
  u32x4 buf[R][2 * kYsBlocksPerStep];
  auto load = [&](int step, u32x4 (&b)[2 * kYsBlocksPerStep]) {
#pragma unroll
    for (int k = 0; k < kYsBlocksPerStep; k++) {
      // entries past the list re-read the wave's last block (cache hits)
      const int j = min(step * kYsBlocksPerStep + k, n_mine - 1);
      // ids outside the buffer are clamped into it
      const int id = min(max(uniform(ids[w + (int64_t)W * j]), 0), n_blocks - 1);
      const __amdgpu_buffer_rsrc_t r = head_rsrc(base + (size_t)id * 2048);
      b[2 * k] = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
      b[2 * k + 1] = __builtin_amdgcn_raw_buffer_load_b128(r, off + 1024, 0, 2);
    }
  };
  uint32_t acc = 0;
  if (n_steps > 0) {
#pragma unroll
    for (int r = 0; r < R - 1; r++)
      load(min(r, n_steps - 1), buf[r]);
    for (int s0 = 0; s0 < n_steps; s0 += R) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        load(min(s0 + r + R - 1, n_steps - 1), buf[(r + R - 1) % R]);
        // a multiply per step keeps the steps in order (an XOR chain alone
        // would let the compiler regroup it and wait for later steps' loads)
        uint32_t x = 0;
#pragma unroll
        for (int k = 0; k < 2 * kYsBlocksPerStep; k++)
          x ^= buf[r][k][0] ^ buf[r][k][1] ^ buf[r][k][2] ^ buf[r][k][3];
        acc = (acc ^ x) * 0x01000193u;
        // and no instruction moves across the step: the ring stays a ring
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if (acc == kYsMagic)
    sink[lane] = acc;
}

} // namespace gkv

using namespace gkv;

extern "C" int gkv_yardstick_stream(void *stream, const void *src, int64_t n_bytes,
                                    int32_t n_workgroups, uint32_t *sink) {
  if (!src || !sink || n_bytes < 16 || n_bytes % 16 || n_workgroups <= 0 ||
      ((uintptr_t)src & 15))
    return GKV_ERR_ARG;
  hipLaunchKernelGGL(ys_stream_kernel, dim3(n_workgroups), dim3(64 * kYsWaves), 0,
                     (hipStream_t)stream, (const u32x4 *)src, n_bytes / 16, sink);
  return launch_status("ys_stream_kernel");
}

extern "C" int gkv_yardstick_gather(void *stream, const void *base, int64_t n_bytes,
                                    const int32_t *block_ids, int32_t n_ids,
                                    int32_t n_workgroups, uint32_t *sink) {
  if (!base || !block_ids || !sink || n_ids <= 0 || n_workgroups <= 0 || n_bytes < 2048 ||
      n_bytes / 2048 > INT32_MAX)
    return GKV_ERR_ARG;
  hipLaunchKernelGGL(ys_gather_kernel<4>, dim3(n_workgroups), dim3(64 * kYsWaves), 0,
                     (hipStream_t)stream, (const char *)base, (int)(n_bytes / 2048), block_ids,
                     n_ids, sink);
  return launch_status("ys_gather_kernel");
}

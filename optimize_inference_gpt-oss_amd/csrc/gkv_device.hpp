// Device helpers shared by the gkv kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gkv.h"

namespace gkv {

constexpr int kHeadDim = 64;    // gpt-oss head_dim; the kernels are written for it
constexpr int kBlockTokens = 16; // tokens per paged block
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Buffer resource over the 2 KB of one head of one paged block: loads take a
// scalar base and a 32-bit per-lane offset; reads past 2 KB return zero.
// Word 3 = 0x00020000: 32-bit data format, the gfx9-family raw-buffer setting.
// bytes = 0: every load through it returns zeros without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const void *base, int bytes = 2048) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet. Written out in
// integer form so the stored cache bits follow this rule exactly
// (getp-csrc/kernels/fast_common.hpp:14-20 states the same rule).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// RoPE of the pair (x1, x2) = dims (i, i + 32): the rounding of run.cpp's
// compiled apply_rotary_emb (run.cpp:506-526): x2*s and x1*s rounded, the
// other product fused.
__device__ __forceinline__ float rope_first(float x1, float x2, float c, float s) {
  return __fmaf_rn(x1, c, -__fmul_rn(x2, s));
}
__device__ __forceinline__ float rope_second(float x1, float x2, float c, float s) {
  return __fmaf_rn(x2, c, __fmul_rn(x1, s));
}

// Value of lane (l ^ 8) within each row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ float swap8(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Four e4m3 codes (one per byte) -> four bf16 (exact: every e4m3 value is a
// bf16 value), in order.
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(uint32_t w) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  return u32x2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}

} // namespace gkv

namespace gkv {
// Host side: turns the launch status into a gkv_status, keeping the HIP error
// text for gkv_last_error() (thread-local).
int hip_status(hipError_t e, const char *where);
inline int launch_status(const char *where) { return hip_status(hipGetLastError(), where); }
} // namespace gkv

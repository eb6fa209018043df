// KV append of one qkv row (shared by the append launch and the fused
// append + decode-prepare launch). See kv_append.hip for the semantics.
#pragma once

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
  float *vs;   // int8 V: fp32 scales [block][head][16]; nullptr for bf16 V
  int v_int8;  // 1: V is stored as int8 codes + scales (gkv_v_format GKV_V_INT8)
};

// Element offset of token t, dim d inside one head's bf16 K block (16 x 64
// values, 2 KB): [d / 32][(d % 32) / 8][t][d % 8]. Lane kg * 16 + t of the
// attention kernel holds dims 32m + 8kg .. +7 of token t for its m-th matrix
// op, so each 1 KB half is one 16-byte load per lane in lane order.
__host__ __device__ __forceinline__ int k_offset(int t, int d) {
  return (d / 32) * 512 + ((d % 32) / 8 * 16 + t) * 8 + d % 8;
}

// Element offset of token t, dim d inside one head's bf16 V block (2 KB):
// [d / 32][t / 4][d % 16][(d / 16) % 2][t % 4]. Lane kg * 16 + i finds tokens
// 4kg .. 4kg+3 of dims i + 32h and i + 32h + 16 in one 16-byte piece of half h.
__host__ __device__ __forceinline__ int v_offset(int t, int d) {
  return (d / 32) * 512 + ((t / 4) * 16 + d % 16) * 8 + ((d / 16) % 2) * 4 + t % 4;
}

// Offset of dim d, token t inside one head's 1 KB int8 V block: lane (kg, i)
// of the attention kernel finds the codes of dims i, i+16, i+32, i+48 for
// tokens 4kg..4kg+3 in one 16-byte piece.
__host__ __device__ __forceinline__ int v_int8_offset(int d, int t) {
  return ((d % 16) * 4 + t / 4) * 16 + (d / 16) * 4 + t % 4;
}

// Row r of the call, by nt threads numbered tid = 0 .. nt-1.
__device__ __forceinline__ void append_row(const AppendArgs &a, int r, int tid, int nt) {
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const int seq = a.row_seq ? a.row_seq[r] : r;
  // the row's position: given, or the last position of its sequence
  const int pos = a.row_pos ? a.row_pos[r] : a.seq_lens[seq] - 1;
  const float *row = a.qkv + (int64_t)r * a.row_stride;
  const float *cs = a.cos_tab + (int64_t)pos * HALF, *sn = a.sin_tab + (int64_t)pos * HALF;
  const int kv_dim = a.n_kv_heads * D;

  // Rotated query (each thread owns whole pairs, so q_out may alias qkv).
  if (a.q_out) {
    float *qo = a.q_out + (int64_t)r * a.q_out_stride;
    for (int idx = tid; idx < a.n_q_heads * HALF; idx += nt) {
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
  for (int idx = tid; idx < a.n_kv_heads * HALF; idx += nt) {
    const int g = idx / HALF, i = idx % HALF;
    const float x1 = kr[g * D + i], x2 = kr[g * D + HALF + i];
    const float c = cs[i], s = sn[i];
    const uint16_t k1 = f32_to_bf16_rne(rope_first(x1, x2, c, s));
    const uint16_t k2 = f32_to_bf16_rne(rope_second(x1, x2, c, s));
    if (store) {
      uint16_t *kd = a.kc + kbase + (int64_t)g * (kBlockTokens * D);
      kd[k_offset(off, i)] = k1;
      kd[k_offset(off, HALF + i)] = k2;
    }
    if (a.k_pack) {
      uint16_t *kp = a.k_pack + (int64_t)r * kv_dim + g * D;
      kp[i] = k1;
      kp[HALF + i] = k2;
    }
  }
  if (a.v_int8) {
    // One wave per head (nt and kv_dim are multiples of 64): the head's
    // max |v| across the wave, then the reference's rule,
    // getp-csrc/kernels/fast_misc.hpp:74-84.
    for (int idx = tid; idx < kv_dim; idx += nt) {
      const int g = idx / D, d = idx % D;
      const float x = vr[idx];
      float amax = fabsf(x);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1)
        amax = fmaxf(amax, __shfl_xor(amax, o));
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      const float c = fminf(fmaxf(rintf(x * inv), -127.0f), 127.0f);
      if (store) {
        int8_t *vq = (int8_t *)a.vc + vbase + (int64_t)g * (kBlockTokens * D);
        vq[v_int8_offset(d, off)] = (int8_t)c;
        if (d == 0)
          a.vs[vbase / D + (int64_t)g * kBlockTokens + off] = amax / 127.0f;
      }
      if (a.v_pack)
        a.v_pack[(int64_t)r * kv_dim + idx] = f32_to_bf16_rne(x);
    }
    return;
  }
  for (int idx = tid; idx < kv_dim; idx += nt) {
    const int g = idx / D, d = idx % D;
    const uint16_t v = f32_to_bf16_rne(vr[idx]);
    if (store)
      a.vc[vbase + (int64_t)g * (kBlockTokens * D) + v_offset(off, d)] = v;
    if (a.v_pack)
      a.v_pack[(int64_t)r * kv_dim + idx] = v;
  }
}

} // namespace gkv

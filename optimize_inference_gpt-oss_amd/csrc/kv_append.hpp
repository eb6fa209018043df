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
  float *vs;   // int8 V: fp32 scales [block][head][16]; fp8 K/V: [block][head][32]
  int v_int8;  // 1: V is stored as int8 codes + scales (gkv_v_format GKV_V_INT8)
  int kv_fp8;  // 1: K and V are stored as e4m3 codes + scales (GKV_KV_FP8)
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

// Offset of token t, dim d inside one head's 1 KB e4m3 K block: lane kg * 16
// + t of the attention kernel finds dims 8kg .. 8kg+7 and 32+8kg .. +7 of
// token t (its two matrix-op pieces) in one 16-byte piece, in lane order.
__host__ __device__ __forceinline__ int k_fp8_offset(int t, int d) {
  return ((d % 32) / 8 * 16 + t) * 16 + (d / 32) * 8 + d % 8;
}

// The e4m3 codes of x * inv, clamped to the largest finite value 448
// (the conversion rounds to nearest even and does not saturate), four values
// per dword, element 0 in the low byte.
__device__ __forceinline__ uint32_t fp8x4(float x0, float x1, float x2, float x3, float inv) {
  auto c = [inv](float x) { return fminf(fmaxf(x * inv, -448.0f), 448.0f); };
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(c(x0), c(x1), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c(x2), c(x3), w, true);
  return (uint32_t)w;
}

// Eight bf16 (bits) as one 16-byte piece, element 0 first.
__device__ __forceinline__ u32x4 pack8(const uint16_t *h) {
  return u32x4{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
               h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16)};
}

// The key lanes' part of a row for kv head g, lane quarter j: rotate the
// pairs (8j + i, 32 + 8j + i) of x1 (dims 8j..8j+7) and x2 (32+8j..), store
// them into the cache (bf16 or e4m3) and the packed row.
__device__ __forceinline__ void append_keys(const AppendArgs &a, int r, int g, int j,
                                            const f32x4 (&x1)[2], const f32x4 (&x2)[2],
                                            const f32x4 (&c)[2], const f32x4 (&s)[2],
                                            bool store, int64_t kbase, int off) {
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const int kv_dim = a.n_kv_heads * D;
  float f1[8], f2[8];
  uint16_t o1[8], o2[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float a1 = x1[i / 4][i % 4], a2 = x2[i / 4][i % 4];
    const float cc = c[i / 4][i % 4], ss = s[i / 4][i % 4];
    f1[i] = rope_first(a1, a2, cc, ss);
    f2[i] = rope_second(a1, a2, cc, ss);
    o1[i] = f32_to_bf16_rne(f1[i]);
    o2[i] = f32_to_bf16_rne(f2[i]);
  }
  const u32x4 p1 = pack8(o1), p2 = pack8(o2);
  if (store && a.kv_fp8) {
    // e4m3 K: the head's max |k| over its 4 lanes, then one scale per
    // token and head; the lane's 16 codes are one 16-byte piece
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++)
      amax = fmaxf(amax, fmaxf(fabsf(f1[i]), fabsf(f2[i])));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
    const u32x4 w{fp8x4(f1[0], f1[1], f1[2], f1[3], inv), fp8x4(f1[4], f1[5], f1[6], f1[7], inv),
                  fp8x4(f2[0], f2[1], f2[2], f2[3], inv), fp8x4(f2[4], f2[5], f2[6], f2[7], inv)};
    const int64_t hb = kbase + (int64_t)g * (kBlockTokens * D); // bytes: 1 KB per head
    *(u32x4 *)((uint8_t *)a.kc + hb + k_fp8_offset(off, 8 * j)) = w;
    if (j == 0)
      a.vs[hb / 32 + off] = amax / 448.0f;
  } else if (store) {
    uint16_t *kd = a.kc + kbase + (int64_t)g * (kBlockTokens * D);
    *(u32x4 *)(kd + k_offset(off, 8 * j)) = p1;
    *(u32x4 *)(kd + k_offset(off, HALF + 8 * j)) = p2;
  }
  if (a.k_pack) {
    uint16_t *kp = a.k_pack + (int64_t)r * kv_dim + g * D;
    *(u32x4 *)(kp + 8 * j) = p1;
    *(u32x4 *)(kp + HALF + 8 * j) = p2;
  }
}

// The value lanes' part of a row for kv head g, quarter q (dims 16q ..
// 16q+15 in x): the packed row, then the cache (bf16, int8 or e4m3), or the
// bf16 values into v_stage for the caller to store.
__device__ __forceinline__ void append_values(const AppendArgs &a, int r, int g, int q,
                                              const f32x4 (&x)[4], bool store, int64_t vbase,
                                              int off, uint16_t *v_stage) {
  constexpr int D = kHeadDim;
  const int kv_dim = a.n_kv_heads * D;
  uint16_t h[16];
#pragma unroll
  for (int i = 0; i < 16; i++)
    h[i] = f32_to_bf16_rne(x[i / 4][i % 4]);
  if (a.v_pack) {
    uint16_t *vpk = a.v_pack + (int64_t)r * kv_dim + g * D + 16 * q;
    *(u32x4 *)vpk = pack8(h);
    *(u32x4 *)(vpk + 8) = pack8(h + 8);
  }
  if (v_stage && !a.v_int8 && !a.kv_fp8) {
    *(u32x4 *)(v_stage + g * D + 16 * q) = pack8(h);
    *(u32x4 *)(v_stage + g * D + 16 * q + 8) = pack8(h + 8);
    return;
  }
  if (!store)
    return;
  if (a.kv_fp8) {
    // e4m3 V: the head's max |v| over its 4 lanes, one scale per token and
    // head (after the token's K scale), codes in the int8 V layout
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++)
      amax = fmaxf(amax, fabsf(x[i / 4][i % 4]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
    const int64_t hb = vbase + (int64_t)g * (kBlockTokens * D); // bytes: 1 KB per head
    uint8_t *vq = (uint8_t *)a.vc + hb;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const uint32_t w = fp8x4(x[i / 4][0], x[i / 4][1], x[i / 4][2], x[i / 4][3], inv);
#pragma unroll
      for (int k = 0; k < 4; k++)
        vq[v_int8_offset(16 * q + i + k, off)] = (uint8_t)(w >> (8 * k));
    }
    if (q == 0)
      a.vs[hb / 32 + kBlockTokens + off] = amax / 448.0f;
  } else if (a.v_int8) {
    // The head's max |v| over its 4 lanes, then the reference's rule,
    // getp-csrc/kernels/fast_misc.hpp:74-84.
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++)
      amax = fmaxf(amax, fabsf(x[i / 4][i % 4]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int8_t *vq = (int8_t *)a.vc + vbase + (int64_t)g * (kBlockTokens * D);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float c = fminf(fmaxf(rintf(x[i / 4][i % 4] * inv), -127.0f), 127.0f);
      vq[v_int8_offset(16 * q + i, off)] = (int8_t)c;
    }
    if (q == 0)
      a.vs[vbase / D + (int64_t)g * kBlockTokens + off] = amax / 127.0f;
  } else {
    uint16_t *vd = a.vc + vbase + (int64_t)g * (kBlockTokens * D);
#pragma unroll
    for (int i = 0; i < 16; i++)
      vd[v_offset(off, 16 * q + i)] = h[i];
  }
}

// Row r of the call, by one wave (lane = 0..63). Lanes 0-31 take the keys:
// lane (g, j) of head g = lane / 4 rotates the pairs (8j + i, 32 + 8j + i),
// i = 0..7, and stores dims 8j..8j+7 and 32+8j..32+8j+7 as two 16-byte pieces
// (contiguous in the K block layout and in the packed row). The qkv rows,
// tables and packed rows are 16-byte aligned (checked by the callers). Lanes 32-63 take the values:
// dims 16q .. 16q+15 of head g, with (g, q) = ((lane - 32) / 4, lane % 4).
// More kv heads than 8 loop.
// Where a row's token went: its sequence, its slot and the element offset of
// its block in the pool (store = 0: not stored).
struct RowPlace {
  int store, seq, slot;
  int64_t base;
};

// part / n_parts: the row may be shared by n_parts waves, wave `part` taking
// every n_parts-th kv head (and query pair); a head's 4 key and 4 value lanes
// stay adjacent in one wave (the int8 scale is their max). v_stage: NULL, or
// bf16 [Hkv * 64] in LDS that receives the row's V; then the bf16 V cache
// store is left to the caller. pos_known >= 0: the row's position, already
// known to the caller (no load of row_pos / seq_lens). direct: as for
// append_begin below (row r is sequence r's new token at pos_known).
__device__ __forceinline__ RowPlace append_row(const AppendArgs &a, int r, int lane,
                                               int part = 0, int n_parts = 1,
                                               uint16_t *v_stage = nullptr,
                                               int pos_known = -1, bool direct = false) {
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const int seq = direct || !a.row_seq ? r : a.row_seq[r];
  // the row's position: given, or the last position of its sequence
  const int pos = pos_known >= 0 ? pos_known : a.row_pos ? a.row_pos[r] : a.seq_lens[seq] - 1;
  const float *row = a.qkv + (int64_t)r * a.row_stride;
  const float *cs = a.cos_tab + (int64_t)pos * HALF, *sn = a.sin_tab + (int64_t)pos * HALF;
  const int kv_dim = a.n_kv_heads * D;

  // Rotated query (each lane owns whole pairs, so q_out may alias qkv).
  if (a.q_out) {
    float *qo = a.q_out + (int64_t)r * a.q_out_stride;
    for (int idx = part * 64 + lane; idx < a.n_q_heads * HALF; idx += 64 * n_parts) {
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
  if (!direct && store && a.ring > 0 && a.seq_lens && pos + a.ring < a.seq_lens[seq])
    store = false; // a later row of this call takes the ring slot
  int64_t kbase = 0, vbase = 0;
  const int off = slot % kBlockTokens;
  if (store) {
    const int blk = slot / kBlockTokens;
    if (blk >= a.table_stride) {
      if (lane == 0 && part == 0 && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
      store = false;
    } else {
      const int phys = a.table[(int64_t)seq * a.table_stride + blk];
      if (phys < 0 || phys >= a.num_blocks) {
        if (lane == 0 && part == 0 && a.dev_err)
          atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
        store = false;
      } else {
        kbase = (int64_t)phys * a.n_kv_heads * (kBlockTokens * D);
        vbase = kbase;
      }
    }
  }

  const RowPlace place{store ? 1 : 0, seq, slot, kbase};
  const float *kr = row + a.n_q_heads * D, *vr = kr + kv_dim;
  if (lane < 32) {
    for (int g = (lane / 4) * n_parts + part; g < a.n_kv_heads; g += 8 * n_parts) {
      const int j = lane % 4;
      const f32x4 *k1p = (const f32x4 *)(kr + g * D + 8 * j);
      const f32x4 *k2p = (const f32x4 *)(kr + g * D + HALF + 8 * j);
      const f32x4 *cp = (const f32x4 *)(cs + 8 * j), *sp = (const f32x4 *)(sn + 8 * j);
      const f32x4 x1[2] = {k1p[0], k1p[1]}, x2[2] = {k2p[0], k2p[1]};
      const f32x4 c[2] = {cp[0], cp[1]}, s[2] = {sp[0], sp[1]};
      append_keys(a, r, g, j, x1, x2, c, s, store, kbase, off);
    }
    return place;
  }
  for (int g = ((lane - 32) / 4) * n_parts + part; g < a.n_kv_heads; g += 8 * n_parts) {
    const int q = lane % 4;
    const f32x4 *vp = (const f32x4 *)(vr + g * D + 16 * q);
    const f32x4 x[4] = {vp[0], vp[1], vp[2], vp[3]};
    append_values(a, r, g, q, x, store, vbase, off, v_stage);
  }
  return place;
}

// A row's append in two halves, for a caller that overlaps the row's loads
// with other work: append_begin issues the loads (the lane's K or V pieces
// first, as they depend on the row only; then the placement's table entry
// and the angles), append_end rotates, rounds and stores, as append_row does.
// One wave per row, at most 8 kv heads, no rotated-query output. pos: the
// row's position if the caller knows it, else -1 (row_pos[r], or the last
// position of its sequence). direct: row r is sequence r's new token at pos
// (>= 0) and no later row of the call takes its ring slot, so neither
// row_seq nor seq_lens is read: every load then goes out at once (a possible
// load of either, even one not taken, makes the compiler wait for all the
// loads before it, one round trip each).
struct AppendLoads {
  int seq, slot, off, table_entry; // table_entry: the block id as loaded (-1: none)
  bool store;
  f32x4 x[4];  // key lanes: dims 8j..8j+7, then 32+8j..+7; value lanes: dims 16q..16q+15
  f32x4 cs[4]; // key lanes: the cos, then the sin of those pairs
};

__device__ __forceinline__ AppendLoads append_begin(const AppendArgs &a, int r, int lane,
                                                    int pos, bool direct = false) {
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  AppendLoads L;
  // The row's index loads (its sequence and position) go out first, then its
  // K or V pieces, so the wait for the indices leaves the pieces in flight;
  // then every load that depends on the indices (the length for the ring
  // rule, the table entry, the angles) goes out at once. The table entry is
  // loaded whether or not the ring rule keeps the store.
  const int seq = direct || !a.row_seq ? r : a.row_seq[r];
  const bool pos_from_len = !direct && pos < 0 && !a.row_pos;
  if (!direct && pos < 0 && a.row_pos)
    pos = a.row_pos[r];
  // The same four loads on every lane (no divergent branch, so the loaded
  // registers are not merged through memory): a key lane's dims 8j..+7 and
  // 32+8j..+7, a value lane's 16q..16q+15; lanes past the heads re-read the
  // last head.
  const float *row = a.qkv + (int64_t)r * a.row_stride;
  const int g = min((lane & 31) / 4, a.n_kv_heads - 1), j = lane % 4;
  const bool key = lane < 32;
  const float *xp = row + a.n_q_heads * D + (key ? 0 : a.n_kv_heads * D) + g * D +
                    (key ? 8 * j : 16 * j);
  const int second = key ? HALF : 8;
  L.x[0] = *(const f32x4 *)xp;
  L.x[1] = *(const f32x4 *)(xp + 4);
  L.x[2] = *(const f32x4 *)(xp + second);
  L.x[3] = *(const f32x4 *)(xp + second + 4);
  L.seq = seq;
  if (pos_from_len)
    pos = a.seq_lens[L.seq] - 1;
  L.slot = a.ring > 0 ? pos % a.ring : pos;
  L.off = L.slot % kBlockTokens;
  const int blk = L.slot / kBlockTokens;
  L.table_entry = a.kc != nullptr && blk < a.table_stride
                      ? a.table[(int64_t)L.seq * a.table_stride + blk]
                      : -1;
  L.store = a.kc != nullptr;
  if (!direct && L.store && a.ring > 0 && a.seq_lens && pos + a.ring < a.seq_lens[L.seq])
    L.store = false; // a later row of this call takes the ring slot
  const float *cp = a.cos_tab + (int64_t)pos * HALF + 8 * j;
  const float *sp = a.sin_tab + (int64_t)pos * HALF + 8 * j;
  L.cs[0] = *(const f32x4 *)cp;
  L.cs[1] = *(const f32x4 *)(cp + 4);
  L.cs[2] = *(const f32x4 *)sp;
  L.cs[3] = *(const f32x4 *)(sp + 4);
  return L;
}

__device__ __forceinline__ RowPlace append_end(const AppendArgs &a, const AppendLoads &L,
                                               int r, int lane, uint16_t *v_stage = nullptr) {
  constexpr int D = kHeadDim;
  bool store = L.store;
  int64_t base = 0;
  if (store) {
    if (L.slot / kBlockTokens >= a.table_stride) {
      if (lane == 0 && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_LENGTH);
      store = false;
    } else if (L.table_entry < 0 || L.table_entry >= a.num_blocks) {
      if (lane == 0 && a.dev_err)
        atomicOr(a.dev_err, GKV_DEVERR_BLOCK_ID);
      store = false;
    } else {
      base = (int64_t)L.table_entry * a.n_kv_heads * (kBlockTokens * D);
    }
  }
  const RowPlace place{store ? 1 : 0, L.seq, L.slot, base};
  const int g = (lane & 31) / 4, j = lane % 4;
  if (g >= a.n_kv_heads)
    return place;
  if (lane < 32) {
    const f32x4 x1[2] = {L.x[0], L.x[1]}, x2[2] = {L.x[2], L.x[3]};
    const f32x4 c[2] = {L.cs[0], L.cs[1]}, s[2] = {L.cs[2], L.cs[3]};
    append_keys(a, r, g, j, x1, x2, c, s, store, base, L.off);
  } else {
    append_values(a, r, g, j, L.x, store, base, L.off, v_stage);
  }
  return place;
}

} // namespace gkv

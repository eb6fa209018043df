// C++ engine shim: the attention entry points that the reference engine's
// layer_attention calls (getp-csrc/engine/gpu_engine.hpp:495-498), kept
// under their names and argument order and forwarded to the gkv C ABI over
// the paged cache.
//
// What changes for the caller is the cache description: the reference passes
// one contiguous cache per layer (kc16 / vq8 / vs, slots) and one position
// for the whole batch; here a layer is a gkv_cache_view into the paged pool
// and every row carries its own position (continuous batching). Error
// behaviour is the reference's: a failed call prints and exits, like its
// HIP_CHECK (gpu_engine.hpp:41-49); callers who want the status use the C ABI
// directly.
#ifndef GKV_ENGINE_HPP
#define GKV_ENGINE_HPP

#include <cstdio>
#include <cstdlib>

#include "gkv.h"

namespace gkv_engine {

typedef uint16_t bf16_t; // raw bfloat16 bits (as getp-csrc/kernels/fast_common.hpp:7)
typedef void *stream_t;  // a hipStream_t

// Per-step state of the batch. The reference keeps a scalar pos for the
// whole batch and device pointers to row pos of the cos/sin table
// (gpu_engine.hpp:476); here each row has its own position.
struct PagedBatch {
  const int32_t *row_pos;  // device int32 [B]: position of each row's new token
  const int32_t *seq_lens; // device int32 [B]: row_pos + 1
  int32_t max_seq_len;     // host bound of seq_lens
  const float *cos_tab;    // device gkv_rope_table rows [max_pos][32]
  const float *sin_tab;
  void *workspace;         // device, gkv_decode_workspace_bytes(B, Hkv, max_seq_len, 0, 0)
  size_t workspace_bytes;
  uint32_t *dev_err;       // device uint32 (GKV_DEVERR_* bits), or nullptr
};

// One layer's cache (replaces GpuLayer::kc16 / vq8 / vs / slots / window /
// sinks, gpu_engine.hpp:59-78).
struct PagedLayer {
  gkv_cache_view view; // gkv_pool_layer_view(pool, l, &view)
  int32_t window;      // 0 (full layer) or the ring size
  const float *sinks;  // device fp32 [n_q_heads]
};

inline void check(int status, const char *what) {
  if (status != GKV_OK) {
    fprintf(stderr, "%s failed: %s%s%s\n", what, gkv_status_string(status),
            status == GKV_ERR_HIP ? ": " : "", status == GKV_ERR_HIP ? gkv_last_error() : "");
    exit(EXIT_FAILURE);
  }
}

// rope_kv_bf16 (getp-csrc/kernels/fast_misc.hpp:112-127): RoPE on the K heads
// (and, with rotate_q, the Q heads in place) of B qkv rows, and the bf16 store
// of K and V at each row's position in the layer's paged cache.
inline void rope_kv_bf16(stream_t s, int B, float *qkv, int row_stride, const PagedBatch &bt,
                         int n_q_heads, const PagedLayer &layer, bool rotate_q = true) {
  check(gkv_kv_append(s, B, qkv, row_stride, n_q_heads, bt.cos_tab, bt.sin_tab, bt.row_pos,
                      nullptr, bt.seq_lens, layer.view, rotate_q ? qkv : nullptr, row_stride,
                      nullptr, nullptr, bt.dev_err),
        "rope_kv_bf16");
}

// gemm_bf16 (getp-csrc/kernels/fast_gemm.hpp:888-899) followed by
// rope_kv_bf16(rotate_q = false), the pair at gpu_engine.hpp:493-496:
// C = A . W^T + bias into fp32 rows (the Q part left unrotated, as gemm_bf16
// writes it) and each row's rotated K and its V stored into the layer's paged
// cache at its position, in one gkv_qkv_append call. N must be
// (n_q_heads + 2 Hkv) * 64. Meant for decode steps (hundreds of rows, where
// it runs level with the pair); for prompt-sized batches (thousands of rows)
// keep the library GEMM followed by rope_kv_bf16, which is faster there.
inline void gemm_bf16_rope_kv(stream_t s, const bf16_t *A, int M, const bf16_t *W,
                              const float *bias, float *C, int N, int K, const PagedBatch &bt,
                              int n_q_heads, const PagedLayer &layer) {
  if (N != (n_q_heads + 2 * layer.view.n_kv_heads) * 64)
    check(GKV_ERR_ARG, "gemm_bf16_rope_kv");
  check(gkv_qkv_append(s, M, A, K, K, W, bias, n_q_heads, bt.cos_tab, bt.sin_tab, bt.row_pos,
                       nullptr, bt.seq_lens, layer.view, C, N, bt.dev_err),
        "gemm_bf16_rope_kv");
}

// attention_bf16_chunk64 (getp-csrc/kernels/fast_attention.hpp:566-580): one
// query row per sequence against its cache (bf16 V; an int8-V layer is
// GKV_ERR_ARG) plus the head's sink, output bf16 [B][out_stride]. With q_rotated false the query is rotated on load at
// row_pos (the reference's cosv/sinv form, used after
// rope_kv_bf16(rotate_q = false)).
inline void attention_bf16_chunk64(stream_t s, const float *qkv, int row_stride,
                                   const PagedLayer &layer, int n_q_heads, bf16_t *out,
                                   int out_stride, int B, const PagedBatch &bt,
                                   bool q_rotated = false) {
  if (layer.view.v_format != GKV_V_BF16)
    check(GKV_ERR_ARG, "attention_bf16_chunk64 (the layer holds the int8-V cache: use "
                       "attention_q8v_chunk64)");
  check(gkv_decode_attention(s, B, n_q_heads, qkv, row_stride, q_rotated ? nullptr : bt.cos_tab,
                             q_rotated ? nullptr : bt.sin_tab, bt.seq_lens, bt.max_seq_len,
                             layer.view, layer.window, layer.sinks, 0, bt.workspace,
                             bt.workspace_bytes, out, out_stride, GKV_BF16, bt.dev_err),
        "attention_bf16_chunk64");
}

// rope_kv_bf16(rotate_q = false) followed by attention_q8v_chunk64 (int8-V
// layer) or attention_bf16_chunk64 (bf16 V), the pair at gpu_engine.hpp:495-498,
// as one gkv_decode_layer call (the append runs in the attention's launch).
// Row b is the new token at row_pos[b]; the output is bf16.
// plan: the engine's loop over layers (gpu_engine.hpp:652) can pass
// GKV_PLAN_KEEP for the first layer of each kind (full, window) in a step and
// GKV_PLAN_REUSE for the others of that kind, each kind with a workspace of its
// own (workspace: nullptr = bt.workspace; the same size), so that the later
// layers skip the planning (gkv_decode_layer_planned; the same output bits).
inline void rope_kv_attention_bf16(stream_t s, int B, const float *qkv, int row_stride,
                                   const PagedLayer &layer, int n_q_heads, bf16_t *out,
                                   int out_stride, const PagedBatch &bt,
                                   gkv_plan_mode plan = GKV_PLAN_NONE,
                                   void *workspace = nullptr) {
  check(gkv_decode_layer_planned(s, B, n_q_heads, qkv, row_stride, bt.cos_tab, bt.sin_tab,
                                 bt.seq_lens, bt.max_seq_len, layer.view, layer.window,
                                 layer.sinks, 0, workspace ? workspace : bt.workspace,
                                 bt.workspace_bytes, out, out_stride, GKV_BF16, bt.dev_err,
                                 plan),
        "rope_kv_attention_bf16");
}

// attention_q8v_chunk64 (getp-csrc/kernels/fast_attention.hpp:604-622), the
// call of the engine's fast path (layer_attention, gpu_engine.hpp:497-498),
// in the reference's argument order: the cache arguments (kc, vq, vs, slots)
// become the layer's paged view, which must hold the int8-V cache
// (GKV_V_INT8; else GKV_ERR_ARG), and the scalar pos becomes the batch's
// per-row positions. kv_dim = Hkv * 64 and, as in the reference's
// attention_gqa8 kernels, 8 query heads per kv head. window is the layer's
// (0 or its ring). rotate_q stands for the reference's cosv/sinv: true = the
// query is rotated on load at each row's position (cos/sin from bt).
inline void attention_q8v_chunk64(stream_t s, const float *qkv, int row_stride,
                                  const PagedLayer &layer, int kv_dim, const float *sinks,
                                  bf16_t *out, int out_stride, int B, const PagedBatch &bt,
                                  int window, bool rotate_q = true) {
  if (layer.view.v_format != GKV_V_INT8 || kv_dim != layer.view.n_kv_heads * 64 ||
      window != layer.view.ring)
    check(GKV_ERR_ARG, "attention_q8v_chunk64");
  const int n_q_heads = 8 * (kv_dim / 64);
  check(gkv_decode_attention(s, B, n_q_heads, qkv, row_stride, rotate_q ? bt.cos_tab : nullptr,
                             rotate_q ? bt.sin_tab : nullptr, bt.seq_lens, bt.max_seq_len,
                             layer.view, window, sinks, 0, bt.workspace, bt.workspace_bytes, out,
                             out_stride, GKV_BF16, bt.dev_err),
        "attention_q8v_chunk64");
}

// The exact path of a GPTOSS_EXACT build (gpu_engine.hpp:478-488), under the
// reference's names and argument order (the launch configuration replaced by
// the stream and B): fp32 caches of layout [B][slots][kv_dim] as the
// reference keeps them (not the paged pool), one position for the batch.
// The results equal the reference CPU forward's bit for bit.

// rope_exact (getp-csrc/kernels/misc.hpp:55-72): cosv/sinv are the tables'
// row at pos; rotates heads 0..n_heads-1 of each row in place.
inline void rope_exact(stream_t s, int B, float *qkv, int row_stride, const float *cosv,
                       const float *sinv, int n_heads, int head_dim) {
  if (head_dim != 64)
    check(GKV_ERR_UNSUPPORTED, "rope_exact (head_dim 64 only)");
  check(gkv_rope_exact(s, B, qkv, row_stride, cosv, sinv, nullptr, n_heads), "rope_exact");
}

// kv_write_kernel (getp-csrc/kernels/misc.hpp:74-85): each row's K and V into
// the layer's fp32 caches at `slot` (pos, or pos % window on a window layer).
inline void kv_write_kernel(stream_t s, int B, const float *qkv, int row_stride, int k_off,
                            int v_off, float *kc, float *vc, int slots, int slot, int kv_dim) {
  check(gkv_kv_write_exact(s, B, qkv, row_stride, k_off, v_off, kc, vc, slots, kv_dim, slot,
                           nullptr, 0, nullptr),
        "kv_write_kernel");
}

// attention_exact (getp-csrc/kernels/attention.hpp:18-83): every row at
// position pos; window 0 (full layer) or the ring of a window layer.
inline void attention_exact(stream_t s, int B, const float *qkv, int row_stride, const float *kc,
                            const float *vc, int slots, int kv_dim, int kv_mul,
                            const float *sinks, float *out, int out_stride, int pos,
                            int window) {
  if (kv_dim % 64)
    check(GKV_ERR_UNSUPPORTED, "attention_exact (head_dim 64 only)");
  const int n_kv_heads = kv_dim / 64;
  check(gkv_attention_exact(s, B, n_kv_heads * kv_mul, n_kv_heads, qkv, row_stride, kc, vc,
                            slots, sinks, pos, nullptr, 0, window, out, out_stride, nullptr),
        "attention_exact");
}

} // namespace gkv_engine

#endif // GKV_ENGINE_HPP

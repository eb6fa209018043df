// Harness around the reference's own CPU code (run.cpp), compiled from the
// reference sources where they lie (oracle/build_ref.sh). TEST INFRASTRUCTURE
// ONLY: used to pin the oracle restatement and to write golden vectors.
//
// It exposes run.cpp's functions through a C ABI, and runs run.cpp's real
// forward() on a synthetic single-sequence model whose QKV weights are zero, so
// that the QKV bias *is* the layer's q|k|v row (matmul gives 0, plus bias,
// exactly: run.cpp:565-570). The history of the cache is pre-filled with
// already-rotated keys, then forward(pos) appends the new token (rotating q and
// k, run.cpp:588-592) and runs the attention (run.cpp:597-642), whose output is
// left in RunState::tb.
#include "run.cpp" // -I /root/reference

#include <vector>

extern "C" {

void ref_cos_sin(int pos, float base, int head_dim, float scaling, float ctx, float beta,
                 float alpha, float *cos_out, float *sin_out) {
  compute_cos_sin(pos, base, head_dim, scaling, ctx, beta, alpha, cos_out, sin_out);
}

void ref_yarn(float base, int head_dim, float scaling, float ctx, float beta, float alpha,
              float *concentration, float *inv_freq) {
  compute_concentration_and_inv_freq(base, head_dim, scaling, ctx, beta, alpha, concentration,
                                     inv_freq);
}

void ref_rotate(float *x, float *cosv, float *sinv, int n_heads, int head_dim) {
  apply_rotary_emb(x, cosv, sinv, n_heads, head_dim);
}

void ref_softmax(float *x, int size) { softmax(x, size); }

// run.cpp's QKV projection of one row: matmul (run.cpp:355-367), then the
// bias add of forward() (run.cpp:565-570).
void ref_matmul_bias(float *out, float *x, float *w, const float *bias, int n_in, int n_out) {
  matmul(out, x, w, n_in, n_out);
  if (bias)
    for (int i = 0; i < n_out; ++i)
      out[i] += bias[i];
}

// One decode step of one sequence through run.cpp forward().
//   window_layer: 1 -> the attention runs on layer 0 (a sliding-window layer
//   when window > 0), 0 -> on layer 1 (full attention).
//   qkv_row: [Q (Hq*d) | K (Hkv*d) | V (Hkv*d)] before RoPE
//   k_hist/v_hist: positions 0..pos-1, [t][Hkv*d], keys already rotated
//   sinks: [Hq]
// Outputs: out [Hq*d] (attention output), k_rot [Hkv*d] (the rotated key
// forward() left in the cache at pos). Returns 0 or -1.
int ref_decode_one(int n_q_heads, int n_kv_heads, int head_dim, int window, int window_layer,
                   int pos, const float *qkv_row, const float *k_hist, const float *v_hist,
                   const float *sinks, float *out, float *k_rot) {
  Config c{};
  c.vocab_size = 2;
  c.hidden_dim = 4;
  c.n_experts = 2;
  c.experts_per_token = 1;
  c.intermediate_dim = 4;
  c.n_layers = window_layer ? 1 : 2;
  c.head_dim = head_dim;
  c.n_attn_heads = n_q_heads;
  c.n_kv_heads = n_kv_heads;
  c.seq_len = pos + 2;
  c.initial_context_length = 4096;
  c.rope_theta = 150000.0f;
  c.rope_scaling_factor = 32.0f;
  c.sliding_window = window;
  c.swiglu_limit = 7.0f;

  const size_t qkv_dim = (size_t)head_dim * (n_q_heads + 2 * n_kv_heads);
  const size_t kv_dim = (size_t)head_dim * n_kv_heads;
  const size_t budget = 4u << 20; // floats, far more than this tiny model needs
  std::vector<float> weights(budget, 0.0f);
  TransformerWeights w{};
  memory_map_weights(&w, &c, weights.data());
  if (w.b_mlp2 + (size_t)c.n_layers * c.n_experts * c.hidden_dim > weights.data() + budget)
    return -1;

  const int l = window_layer ? 0 : 1;
  for (size_t i = 0; i < qkv_dim; i++)
    w.b_qkv[l * qkv_dim + i] = qkv_row[i];
  for (int h = 0; h < n_q_heads; h++)
    w.attn_sinks[l * n_q_heads + h] = sinks[h];

  Transformer t{};
  t.config = c;
  t.weights = w;
  t.fd = -1;
  t.data = nullptr;
  malloc_run_state(&t.state, &t.config);
  const size_t loff = (size_t)l * c.seq_len * kv_dim;
  for (int p = 0; p < pos; p++)
    for (size_t i = 0; i < kv_dim; i++) {
      t.state.key_cache[loff + p * kv_dim + i] = k_hist[p * kv_dim + i];
      t.state.value_cache[loff + p * kv_dim + i] = v_hist[p * kv_dim + i];
    }
  forward(&t, 0, pos);
  memcpy(out, t.state.tb, sizeof(float) * head_dim * n_q_heads);
  memcpy(k_rot, t.state.key_cache + loff + (size_t)pos * kv_dim, sizeof(float) * kv_dim);
  free_run_state(&t.state);
  return 0;
}

} // extern "C"

// A decode loop written the way the reference engine drives its attention
// (layer_attention, getp-csrc/engine/gpu_engine.hpp:467-508, one position for
// the whole batch per step), but through the C++ engine shim over the paged
// pool: per step, reserve the new position of every sequence, upload the
// tables, then per layer rope_kv_bf16(rotate_q = false) and
// attention_bf16_chunk64 with the query rotated on load.
//
//   gkv_engine_demo <in.bin> <out.bin> [fused | planned | project | q8v]
// fused: the one-call form rope_kv_attention_bf16 instead of the two calls.
// planned: rope_kv_attention_bf16 with the plan kept by the first layer of
//   each kind (full, window) in a step and reused by the others, a workspace
//   per kind.
// q8v: the engine's own fast-path pair, rope_kv_bf16 + attention_q8v_chunk64
//   (gpu_engine.hpp:495-498; the pool must hold the int8-V cache).
// project: the qkv rows come from the layer input through the QKV projection
//   with the append in its epilogue (gemm_bf16_rope_kv, the pair
//   gemm_bf16 + rope_kv_bf16 of gpu_engine.hpp:493-496), then
//   attention_bf16_chunk64.
// in.bin:  int32 P, B, Hq, Hkv, n_layers, window, v_format (gkv_v_format);
//          fp32 qkv [P][n_layers][B][(Hq+2Hkv)*64];
//          fp32 sinks [n_layers][Hq];
//          project only: int32 H; bf16 x [P][n_layers][B][H];
//          bf16 W [n_layers][(Hq+2Hkv)*64][H]; fp32 bias [n_layers][(Hq+2Hkv)*64]
//          (the qkv array is then ignored)
// out.bin: bf16 [P][n_layers][B][Hq*64] attention outputs of every step
// Layer l is a window layer iff window > 0 and l is even (the pool's rule).
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "gkv_engine.hpp"

#define HIP_OK(x)                                                                                \
  do {                                                                                           \
    hipError_t e_ = (x);                                                                         \
    if (e_ != hipSuccess) {                                                                      \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                                    \
      return 1;                                                                                  \
    }                                                                                            \
  } while (0)

int main(int argc, char **argv) {
  if (argc != 3 && argc != 4) {
    fprintf(stderr, "usage: %s in.bin out.bin [fused | project | q8v | planned | exact]\n",
            argv[0]);
    return 2;
  }
  const bool fused = argc == 4 && std::string(argv[3]) == "fused";
  const bool project = argc == 4 && std::string(argv[3]) == "project";
  const bool q8v = argc == 4 && std::string(argv[3]) == "q8v";
  const bool planned = argc == 4 && std::string(argv[3]) == "planned";
  // exact: the GPTOSS_EXACT trio over fp32 caches [B][slots][kv_dim] per layer
  // (window layers: a ring of W slots), fp32 outputs
  const bool exact = argc == 4 && std::string(argv[3]) == "exact";
  FILE *f = fopen(argv[1], "rb");
  if (!f)
    return 2;
  int32_t hdr[7];
  if (fread(hdr, 4, 7, f) != 7)
    return 2;
  const int P = hdr[0], B = hdr[1], Hq = hdr[2], Hkv = hdr[3], NL = hdr[4], W = hdr[5];
  const int QKV = (Hq + 2 * Hkv) * 64, ATT = Hq * 64;
  std::vector<float> qkv((size_t)P * NL * B * QKV), sinks((size_t)NL * Hq);
  if (fread(qkv.data(), 4, qkv.size(), f) != qkv.size() ||
      fread(sinks.data(), 4, sinks.size(), f) != sinks.size())
    return 2;
  int32_t H = 0;
  std::vector<uint16_t> xs, ws;
  std::vector<float> bs;
  if (project) {
    if (fread(&H, 4, 1, f) != 1 || H <= 0)
      return 2;
    xs.resize((size_t)P * NL * B * H);
    ws.resize((size_t)NL * QKV * H);
    bs.resize((size_t)NL * QKV);
    if (fread(xs.data(), 2, xs.size(), f) != xs.size() ||
        fread(ws.data(), 2, ws.size(), f) != ws.size() ||
        fread(bs.data(), 4, bs.size(), f) != bs.size())
      return 2;
  }
  fclose(f);

  gkv_pool_config cfg{};
  cfg.n_layers = NL;
  cfg.n_kv_heads = Hkv;
  cfg.head_dim = 64;
  cfg.window = W;
  cfg.max_seqs = B;
  cfg.max_seq_len = P;
  cfg.num_blocks = (int64_t)B * ((P + 15) / 16) + 3;
  cfg.shuffle_seed = 77;
  cfg.v_format = hdr[6];
  gkv_pool *pool = nullptr;
  gkv_engine::check(gkv_pool_create(&cfg, &pool), "gkv_pool_create");
  for (int b = 0; b < B; b++) {
    int32_t id = -1;
    gkv_engine::check(gkv_pool_seq_alloc(pool, &id), "gkv_pool_seq_alloc");
  }

  std::vector<float> cos_h((size_t)P * 32), sin_h((size_t)P * 32);
  gkv_rope_config rc{150000.0f, 64, 32.0f, 4096.0f, 32.0f, 1.0f}; // gpt-oss YaRN settings
  gkv_engine::check(gkv_rope_table(&rc, P, cos_h.data(), sin_h.data()), "gkv_rope_table");

  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  float *d_qkv, *d_sinks, *d_cos, *d_sin;
  int32_t *d_pos, *d_lens;
  uint32_t *d_err;
  uint16_t *d_out;
  const size_t ws_bytes = gkv_decode_workspace_bytes(B, Hkv, P, 0, 0);
  void *d_ws, *d_ws_window;
  HIP_OK(hipMalloc(&d_qkv, (size_t)B * QKV * 4));
  HIP_OK(hipMalloc(&d_sinks, sinks.size() * 4));
  HIP_OK(hipMalloc(&d_cos, cos_h.size() * 4));
  HIP_OK(hipMalloc(&d_sin, sin_h.size() * 4));
  HIP_OK(hipMalloc(&d_pos, B * 4));
  HIP_OK(hipMalloc(&d_lens, B * 4));
  HIP_OK(hipMalloc(&d_err, 4));
  HIP_OK(hipMalloc(&d_out, (size_t)B * ATT * 2));
  HIP_OK(hipMalloc(&d_ws, ws_bytes));
  HIP_OK(hipMalloc(&d_ws_window, ws_bytes));
  uint16_t *d_x = nullptr, *d_w = nullptr;
  float *d_b = nullptr;
  if (project) {
    HIP_OK(hipMalloc(&d_x, (size_t)B * H * 2));
    HIP_OK(hipMalloc(&d_w, ws.size() * 2));
    HIP_OK(hipMalloc(&d_b, bs.size() * 4));
    HIP_OK(hipMemcpy(d_w, ws.data(), ws.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_b, bs.data(), bs.size() * 4, hipMemcpyHostToDevice));
  }
  HIP_OK(hipMemcpy(d_sinks, sinks.data(), sinks.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_cos, cos_h.data(), cos_h.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_sin, sin_h.data(), sin_h.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(d_err, 0, 4));

  std::vector<gkv_engine::PagedLayer> layers(NL);
  for (int l = 0; l < NL; l++) {
    gkv_engine::check(gkv_pool_layer_view(pool, l, &layers[l].view), "gkv_pool_layer_view");
    layers[l].window = layers[l].view.ring;
    layers[l].sinks = d_sinks + (size_t)l * Hq;
  }
  gkv_engine::PagedBatch bt{d_pos, d_lens, P, d_cos, d_sin, d_ws, ws_bytes, d_err};

  std::vector<float *> kc32(NL, nullptr), vc32(NL, nullptr);
  std::vector<int> slots32(NL, 0);
  float *d_out32 = nullptr;
  if (exact) {
    for (int l = 0; l < NL; l++) {
      slots32[l] = layers[l].window > 0 ? layers[l].window : P;
      HIP_OK(hipMalloc(&kc32[l], (size_t)B * slots32[l] * Hkv * 64 * 4));
      HIP_OK(hipMalloc(&vc32[l], (size_t)B * slots32[l] * Hkv * 64 * 4));
    }
    HIP_OK(hipMalloc(&d_out32, (size_t)B * ATT * 4));
  }
  std::vector<float> out32(exact ? (size_t)P * NL * B * ATT : 0);
  std::vector<uint16_t> out((size_t)P * NL * B * ATT);
  std::vector<int32_t> pos(B), lens(B);
  for (int p = 0; p < P; p++) {
    for (int b = 0; b < B; b++) {
      pos[b] = p;
      lens[b] = p + 1;
      gkv_engine::check(gkv_pool_seq_reserve(pool, b, p + 1), "gkv_pool_seq_reserve");
    }
    gkv_engine::check(gkv_pool_sync(pool, s), "gkv_pool_sync");
    HIP_OK(hipMemcpyAsync(d_pos, pos.data(), B * 4, hipMemcpyHostToDevice, s));
    HIP_OK(hipMemcpyAsync(d_lens, lens.data(), B * 4, hipMemcpyHostToDevice, s));
    for (int l = 0; l < NL; l++) {
      if (project) {
        HIP_OK(hipMemcpyAsync(d_x, xs.data() + ((size_t)p * NL + l) * B * H, (size_t)B * H * 2,
                              hipMemcpyHostToDevice, s));
        gkv_engine::gemm_bf16_rope_kv(s, d_x, B, d_w + (size_t)l * QKV * H, d_b + (size_t)l * QKV,
                                      d_qkv, QKV, H, bt, Hq, layers[l]);
        gkv_engine::attention_bf16_chunk64(s, d_qkv, QKV, layers[l], Hq, d_out, ATT, B, bt);
      } else {
        HIP_OK(hipMemcpyAsync(d_qkv, qkv.data() + ((size_t)p * NL + l) * B * QKV,
                              (size_t)B * QKV * 4, hipMemcpyHostToDevice, s));
        if (exact) {
          // layer_attention's exact lines (gpu_engine.hpp:480-486)
          const int KVD = Hkv * 64, slot = layers[l].window > 0 ? p % layers[l].window : p;
          gkv_engine::rope_exact(s, B, d_qkv, QKV, d_cos + (size_t)p * 32, d_sin + (size_t)p * 32,
                                 Hq + Hkv, 64);
          gkv_engine::kv_write_kernel(s, B, d_qkv, QKV, ATT, ATT + KVD, kc32[l], vc32[l],
                                      slots32[l], slot, KVD);
          gkv_engine::attention_exact(s, B, d_qkv, QKV, kc32[l], vc32[l], slots32[l], KVD,
                                      Hq / Hkv, layers[l].sinks, d_out32, ATT, p,
                                      layers[l].window);
          HIP_OK(hipMemcpyAsync(out32.data() + ((size_t)p * NL + l) * B * ATT, d_out32,
                                (size_t)B * ATT * 4, hipMemcpyDeviceToHost, s));
          HIP_OK(hipStreamSynchronize(s));
          continue;
        } else if (fused) {
          gkv_engine::rope_kv_attention_bf16(s, B, d_qkv, QKV, layers[l], Hq, d_out, ATT, bt);
        } else if (planned) {
          const bool window_kind = layers[l].window > 0;
          const bool first_of_kind = l < 2 && (l == 0 || window_kind != (layers[0].window > 0));
          gkv_engine::rope_kv_attention_bf16(s, B, d_qkv, QKV, layers[l], Hq, d_out, ATT, bt,
                                             first_of_kind ? GKV_PLAN_KEEP : GKV_PLAN_REUSE,
                                             window_kind ? d_ws_window : d_ws);
        } else if (q8v) {
          // layer_attention's lines, the cache arguments replaced by the paged layer
          gkv_engine::rope_kv_bf16(s, B, d_qkv, QKV, bt, Hq, layers[l], /*rotate_q=*/false);
          gkv_engine::attention_q8v_chunk64(s, d_qkv, QKV, layers[l], Hkv * 64, layers[l].sinks,
                                            d_out, ATT, B, bt, layers[l].window);
        } else {
          gkv_engine::rope_kv_bf16(s, B, d_qkv, QKV, bt, Hq, layers[l], /*rotate_q=*/false);
          gkv_engine::attention_bf16_chunk64(s, d_qkv, QKV, layers[l], Hq, d_out, ATT, B, bt);
        }
      }
      HIP_OK(hipMemcpyAsync(out.data() + ((size_t)p * NL + l) * B * ATT, d_out,
                            (size_t)B * ATT * 2, hipMemcpyDeviceToHost, s));
      HIP_OK(hipStreamSynchronize(s));
    }
  }
  uint32_t err = 0;
  HIP_OK(hipMemcpy(&err, d_err, 4, hipMemcpyDeviceToHost));
  if (err) {
    fprintf(stderr, "device error word %u\n", err);
    return 1;
  }
  FILE *g = fopen(argv[2], "wb");
  if (!g)
    return 2;
  if (exact ? fwrite(out32.data(), 4, out32.size(), g) != out32.size()
            : fwrite(out.data(), 2, out.size(), g) != out.size())
    return 2;
  fclose(g);
  gkv_pool_destroy(pool);
  for (void *ptr : {(void *)d_qkv, (void *)d_sinks, (void *)d_cos, (void *)d_sin, (void *)d_pos,
                    (void *)d_lens, (void *)d_err, (void *)d_out, d_ws, d_ws_window, (void *)d_x,
                    (void *)d_w,
                    (void *)d_b})
    (void)hipFree(ptr);
  for (int l = 0; l < NL; l++) {
    (void)hipFree(kc32[l]);
    (void)hipFree(vc32[l]);
  }
  (void)hipFree(d_out32);
  (void)hipStreamDestroy(s);
  printf("engine demo: %d steps x %d layers x %d sequences ok\n", P, NL, B);
  return 0;
}

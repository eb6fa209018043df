// Host RoPE (YaRN) angle table, bit-identical to the reference's
// compute_cos_sin (run.cpp:422-504), which the reference engine evaluates on
// the host once per position (getp-csrc/engine/gpu_engine.hpp:388-396).
//
// The reference binary is built by hipcc -O3 with FMA contraction; the one
// contracted expression whose rounding shows, the inv_freq blend
// `interpolation * (1 - mask) + extrapolation * mask`, compiles to
// fma(extrapolation, mask, round(interpolation * (1 - mask))). It is written
// that way here, contraction is switched off for this file, and every other
// operation keeps run.cpp's types (the M_PI product in double, logf of the
// float-rounded quotient).
#include <cmath>
#include <vector>

#include "gkv.h"

#pragma clang fp contract(off)

namespace {

constexpr double kPi = 3.14159265358979323846;

void yarn_inv_freq(const gkv_rope_config &c, float &concentration, std::vector<float> &inv) {
  const int half = c.head_dim / 2;
  inv.assign(half, 0.0f);
  std::vector<float> freq(half);
  for (int i = 0; i < half; i++)
    freq[i] = powf(c.base, (float)(2 * i) / (float)c.head_dim);
  if (c.scaling_factor > 1.0f) {
    concentration = fmaf(0.1f, logf(c.scaling_factor), 1.0f);
    const float lb = logf((float)((double)c.initial_context_length /
                                  ((double)(c.ntk_beta * 2.0f) * kPi)));
    const float la = logf((float)((double)c.initial_context_length /
                                  ((double)(c.ntk_alpha * 2.0f) * kPi)));
    const float low = (float)half * lb / logf(c.base);
    const float high = (float)half * la / logf(c.base);
    for (int i = 0; i < half; i++) {
      const float interp = 1.0f / (c.scaling_factor * freq[i]);
      const float extrap = 1.0f / freq[i];
      float ramp = ((float)i - low) / (high - low);
      ramp = ramp < 0.0f ? 0.0f : (ramp > 1.0f ? 1.0f : ramp);
      const float mask = 1.0f - ramp;
      const float interp_part = interp * (1.0f - mask);
      inv[i] = fmaf(extrap, mask, interp_part);
    }
  } else {
    concentration = 1.0f;
    for (int i = 0; i < half; i++)
      inv[i] = 1.0f / freq[i];
  }
}

} // namespace

extern "C" int gkv_rope_table(const gkv_rope_config *cfg, int32_t n_pos, float *cos_tab,
                              float *sin_tab) {
  if (!cfg || n_pos < 0 || !cos_tab || !sin_tab || cfg->head_dim <= 0 || cfg->head_dim % 2 ||
      !(cfg->base > 0.0f))
    return GKV_ERR_ARG;
  float conc;
  std::vector<float> inv;
  yarn_inv_freq(*cfg, conc, inv);
  const int half = cfg->head_dim / 2;
  for (int p = 0; p < n_pos; p++)
    for (int j = 0; j < half; j++) {
      const float val = (float)p * inv[j];
      cos_tab[(size_t)p * half + j] = cosf(val) * conc;
      sin_tab[(size_t)p * half + j] = sinf(val) * conc;
    }
  return GKV_OK;
}

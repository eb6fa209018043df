// TEST INFRASTRUCTURE ONLY: exposes the reference's host-side int8-V rule
// (quantize_v, getp-csrc/tests/attn_test.cpp:218-226) from its own test file,
// compiled where it lies, so that the oracle's orc_quantize_v is checked
// against the reference's code rather than against a second restatement. The
// test's main() is renamed so the file links into a library; nothing else of
// it runs.
#define main gkv_reference_attn_test_main
#include "tests/attn_test.cpp"
#undef main

extern "C" void ref_quantize_v(const float *v, int8_t *codes, float *scale) {
  quantize_v(v, codes, scale);
}

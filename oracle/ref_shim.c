/* ref_shim.c -- exports the reference CPU twin's dequant / dot / transcendental functions
 * (tools/qwen35_engine.c:45-347, all `static`) so tests can check the oracle against the
 * reference's own compiled code. TEST INFRASTRUCTURE ONLY.
 * Built by oracle/Makefile (target `ref`) from the source where it lies under the reference
 * checkout; the output goes to oracle/_ref/ and is never part of the product. */
#define main qwen35_engine_main
#include "qwen35_engine.c"
#undef main

float ref_half_to_float(unsigned h) { return half_to_float((uint16_t)h); }
float ref_dot_fmt(int fmt, const uint8_t* row, int cols, const float* x) { return dot_fmt(fmt, row, cols, x); }
void ref_deq_row(int fmt, const uint8_t* row, int cols, float* out) { deq_row(fmt, row, cols, out); }
float ref_hf_exp(float x) { return hf_exp(x); }
float ref_hf_silu(float x) { return hf_silu(x); }
float ref_hf_sigmoid(float x) { return hf_sigmoid(x); }
/* rms_norm (tools/qwen35_engine.c:510-515) with its EPS set for the call */
void ref_rms_norm(float* h, const float* x, const float* w, int n, float eps) {
  EPS = eps;
  rms_norm(h, x, w, n);
}

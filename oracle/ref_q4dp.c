/* ref_q4dp.c -- exports the reference's CPU twin of its Q4_K x q8 block dot (tools/q4dp/q4dp_ref.h:18-74,
 * all `static`): ref_q8x (the q8 quantizer), ref_sb (a thread's share of a superblock, with the twin's
 * mutation controls mut 1..4) and ref_row (a row's 128-thread sum), so tests can pin the oracle's q8
 * functions against the reference's own code. TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (target
 * `ref`) from the header where it lies under the reference checkout, into oracle/_ref/. */
#include "q4dp_ref.h"

void ref_q8x_c(const float* x, signed char* qx, float* dx, u32 n) { ref_q8x(x, qx, dx, n); }
float ref_sb_c(const u8* B, const signed char* qx, const float* dx, u32 n, u32 sb, u32 g, u32 k, int mut) {
  return ref_sb(B, qx, dx, n, sb, g, k, mut);
}
float ref_row_c(const u8* row, u32 nsb, const signed char* qx, const float* dx, u32 n, int mut) {
  return ref_row(row, nsb, qx, dx, n, mut);
}

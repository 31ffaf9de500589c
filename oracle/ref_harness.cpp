// ref_harness.cpp -- exports the reference's own quant.h functions through a C ABI.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile from the reference
// sources where they lie (-I <reference>/tier, nothing copied); the output goes
// to oracle/_ref/ only.  It checks the C restatement in tq_oracle.c and
// writes the golden vectors under tests/golden/.
//
// This file is built with -O2 and no -march (as check_quant.py:25 builds its
// QTEST harness), so fp32 expressions in quant.h's quantizers are not fused.
#include "quant.h"

#include <cstddef>
#include <cstdint>

extern "C" {
// quant.h:33
size_t ref_q_row_bytes(int t, int cols) { return q_row_bytes(t, cols); }
// quant.h:34
int ref_q_cols_ok(int t, int cols) { return q_cols_ok(t, cols) ? 1 : 0; }
// quant.h:37
float ref_q_h2f(uint16_t h) { return q_h2f(h); }
// quant.h:124
uint16_t ref_q_f2h(float f) { return q_f2h(f); }
// quant.h:59 over whole rows (the 'dq' mode of check_quant.py:16-17)
void ref_dequant_rows(const uint8_t* W, int t, int cols, size_t rows, float* out) {
  const size_t rb = q_row_bytes(t, cols);
  for (size_t r = 0; r < rows; ++r)
    for (int k = 0; k < cols; ++k) out[r * (size_t)cols + k] = q_val(W + r * rb, t, k);
}
// quant.h:201 over whole rows (the 'q' mode of check_quant.py:18-19)
int ref_quantize_rows(int t, const float* x, size_t rows, int cols, uint8_t* out) {
  const size_t rb = q_row_bytes(t, cols);
  for (size_t r = 0; r < rows; ++r)
    if (!q_row(t, x + r * (size_t)cols, out + r * rb, cols)) return 0;
  return 1;
}
}

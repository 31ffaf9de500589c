// tm_host.h -- internal host-side declarations shared by the library's sources.
#pragma once

#include <cstddef>
#include <cstdint>

#include "../../include/tiermm.h"

namespace tiermm {

// ggml type ids (quant.h:21-24).
enum : int {
  QT_F32 = 0, QT_F16 = 1, QT_Q4_0 = 2, QT_Q4_1 = 3, QT_Q5_0 = 6, QT_Q5_1 = 7, QT_Q8_0 = 8,
  QT_Q2_K = 10, QT_Q3_K = 11, QT_Q4_K = 12, QT_Q5_K = 13, QT_Q6_K = 14, QT_IQ4_NL = 20, QT_IQ4_XS = 23,
  QT_BF16 = 30, QT_TQ1_0 = 34, QT_TQ2_0 = 35, QT_MXFP4 = 39, QT_NF4 = 200, QT_FP4 = 201,
  QT_IQ2_XXS = 16, QT_IQ2_XS = 17, QT_IQ3_XXS = 18, QT_IQ1_S = 19, QT_IQ3_S = 21, QT_IQ2_S = 22, QT_IQ1_M = 29
};

struct BlockInfo {
  int type;
  const char* name;
  int elems;  // elements per block
  int bytes;  // bytes per block
};
// Block geometry of every type id the reference knows (quant.h:26-30), or nullptr.
const BlockInfo* block_info(int qtype);

// Record an error for tiermm_last_error() and return `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Map a HIP error code to the ABI's negative status, recording `what`.
int hip_fail(int hip_err, const char* what);

// Workspace: caller-provided (ws != nullptr) or the per-device pool.
// Returns TIERMM_OK and sets *out, or an error status.
int get_workspace(void* ws, size_t ws_bytes, size_t need, void** out, const char* who);

int quantize_rows(int qtype, const float* x, void* out, size_t rows, int cols, int nthreads);

// Device address of tiermm_x3_rows_noalloc's static scratch on the current device,
// looked up once per device (x3.hip).
int noalloc_scratch_init();

}  // namespace tiermm

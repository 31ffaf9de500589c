// chat_ops.hip -- the small element-wise steps of chat_lin's trained-row overlay
// and LoRA (tier.cpp:2333-2350), launched by chat.cpp on the set's compute stream.
#include "tm_device.h"

namespace tiermm {
namespace {

// y[t * ld + idx[j]] = src[t * r + j] for t < M, j < r: the trained rows' outputs
// over their rows of the full output (scatter_cols_k's contract, tier.cpp:1255).
__global__ __launch_bounds__(256) void scatter_cols_kernel(const float* __restrict__ src, float* __restrict__ y,
                                                           const int* __restrict__ idx, int M, int r, int ld) {
  const size_t n = (size_t)M * r, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const size_t t = i / (size_t)r;
    y[t * (size_t)ld + idx[i - t * (size_t)r]] = src[i];
  }
}

__global__ __launch_bounds__(256) void scale_kernel(float* __restrict__ u, size_t n, float s) {
  const size_t step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) u[i] *= s;
}

unsigned grid_for(size_t n) {
  const size_t want = (n + 255) / 256;
  return (unsigned)(want < 4096 ? (want ? want : 1) : 4096);
}

}  // namespace

int chat_scatter_cols(const float* src, float* y, const int* idx, int M, int r, int ld, hipStream_t s) {
  if ((size_t)M * r == 0) return TIERMM_OK;
  scatter_cols_kernel<<<grid_for((size_t)M * r), 256, 0, s>>>(src, y, idx, M, r, ld);
  TM_LAUNCH_CHECK("tiermm_chat_lin: trained rows");
  return TIERMM_OK;
}

int chat_scale(float* u, size_t n, float f, hipStream_t s) {
  if (n == 0) return TIERMM_OK;
  scale_kernel<<<grid_for(n), 256, 0, s>>>(u, n, f);
  TM_LAUNCH_CHECK("tiermm_chat_lin: lora scale");
  return TIERMM_OK;
}

}  // namespace tiermm

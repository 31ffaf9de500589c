// qgemv.hip -- tiermm_qgemv: decode-time (M=1) dequant-GEMV, gemv_q (tier.cpp:299-306).
//
// Generic kernel (every type): the block stages x in LDS once; each wave
// owns R consecutive rows and its lanes walk the row in 8-element chunks
// (lane-strided, like gemv_q's k += warpSize loop but 8 wide), decoding each
// chunk exactly as q_val and accumulating in fp32; the R row partials are then
// reduced across the wave with xor shuffles.  x is read from LDS once per chunk
// and reused for the R rows.
#include "tm_device.h"

namespace tiermm {

int check_qweight(const char* who, const void* W, int qtype, size_t rb, int cols);

namespace {

constexpr int kMaxK = 16384;  // x staged whole in LDS: 64 KiB

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int QT, int R>
__global__ __launch_bounds__(256) void qgemv_generic(const uint8_t* __restrict__ W, size_t rb,
                                                     const float* __restrict__ x, float* __restrict__ y, int N,
                                                     int K) {
  extern __shared__ float xs[];
  for (int i = threadIdx.x * 4; i < K; i += 256 * 4) *(float4*)&xs[i] = *(const float4*)&x[i];
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= N) return;
  const uint8_t* rp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rp[r] = W + (size_t)min(row0 + r, N - 1) * rb;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int c = lane * 8; c < K; c += 512) {
    const float4 xa = *(const float4*)&xs[c], xb = *(const float4*)&xs[c + 4];
    const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v[8];
      Dec<QT>::run(rp[r], c, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[r] = fmaf(v[k], xv[k], acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < N) y[row0 + r] = s;
  }
}

template <int QT>
int launch_generic(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  constexpr int R = 2;
  const unsigned grid = (unsigned)((N + 4 * R - 1) / (4 * R));
  qgemv_generic<QT, R><<<grid, 256, (size_t)K * 4, s>>>((const uint8_t*)W, rb, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_qgemv: launch");
  return TIERMM_OK;
}

}  // namespace

int qgemv_q4k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
int qgemv_q4k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
constexpr int kQ4kMaxK = 14336;  // equals the limit in qgemv_q4k.hip

int qgemv_dispatch(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  switch (qtype) {
    case QT_Q8_0: return launch_generic<QT_Q8_0>(W, rb, x, y, N, K, s);
    case QT_Q5_0: return launch_generic<QT_Q5_0>(W, rb, x, y, N, K, s);
    case QT_Q4_K:  // MFMA kernels up to kQ4kMaxK (x digits in LDS); beyond, the generic kernel
      if (K <= 8192 && (N + 15) / 16 >= 640) return qgemv_q4k_ws(W, rb, x, y, N, K, s);
      return K <= kQ4kMaxK ? qgemv_q4k(W, rb, x, y, N, K, s) : launch_generic<QT_Q4_K>(W, rb, x, y, N, K, s);
    case QT_Q5_K: return launch_generic<QT_Q5_K>(W, rb, x, y, N, K, s);
    default: return launch_generic<QT_Q6_K>(W, rb, x, y, N, K, s);
  }
}

}  // namespace tiermm

using namespace tiermm;

extern "C" int tiermm_qgemv(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K,
                            tiermm_stream_t stream) {
  int st = check_qweight("tiermm_qgemv", W, qtype, rb, K);
  if (st) return st;
  if (N < 0) return set_error(TIERMM_EINVAL, "tiermm_qgemv: N < 0");
  if (N == 0) return TIERMM_OK;
  if (K > kMaxK) return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemv: K=%d above %d", K, kMaxK);
  if (!x || !y || ((uintptr_t)x % 16)) return set_error(TIERMM_EINVAL, "tiermm_qgemv: x must be 16-byte aligned");
  return qgemv_dispatch(W, qtype, rb, x, y, N, K, (hipStream_t)stream);
}

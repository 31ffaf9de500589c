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

// ------------------------------------------------------- dense-row GEMV
// gemv<T> (tier.cpp:2261-2268) for fp32 / fp16 (tier_fp16) / bf16 rows: y[r] =
// sum_k float(W[r][k]) * x[k], fp32 accumulation.  x is staged in LDS; a wave
// owns R rows and its lanes read 16 bytes of each row per step (VEC elements),
// so every load instruction covers 1 KiB of a row; rows whose length is not a
// whole number of 16-byte chunks take the element-wise path.
template <int T>
struct Dense;
template <>
struct Dense<TIERMM_F32> {
  static constexpr int VEC = 4, BYTES = 4;
  __device__ static void load(const uint8_t* p, float (&v)[8]) {
    const float4 a = *(const float4*)p;
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  }
  __device__ static float at(const uint8_t* row, int k) { return ((const float*)row)[k]; }
};
template <>
struct Dense<TIERMM_F16> {
  static constexpr int VEC = 8, BYTES = 2;
  __device__ static void load(const uint8_t* p, float (&v)[8]) {
    const uint4 a = *(const uint4*)p;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = h2f(w[i] & 0xffffu);
      v[2 * i + 1] = h2f(w[i] >> 16);
    }
  }
  __device__ static float at(const uint8_t* row, int k) { return h2f(((const uint16_t*)row)[k]); }
};
template <>
struct Dense<TIERMM_BF16> {
  static constexpr int VEC = 8, BYTES = 2;
  __device__ static void load(const uint8_t* p, float (&v)[8]) {
    const uint4 a = *(const uint4*)p;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ static float at(const uint8_t* row, int k) {
    return __uint_as_float((uint32_t)((const uint16_t*)row)[k] << 16);
  }
};

template <int T, int R>
__global__ __launch_bounds__(256) void gemv_dense(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                  float* __restrict__ y, int N, int K) {
  using D = Dense<T>;
  extern __shared__ float xs[];
  for (int i = threadIdx.x; i < K; i += 256) xs[i] = x[i];
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= N) return;
  const size_t rbytes = (size_t)K * D::BYTES;
  const uint8_t* rp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rp[r] = W + (size_t)min(row0 + r, N - 1) * rbytes;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  if ((rbytes & 15) == 0) {
    for (int k = lane * D::VEC; k < K; k += 64 * D::VEC) {
      float v[R][8];
#pragma unroll
      for (int r = 0; r < R; ++r) D::load(rp[r] + (size_t)k * D::BYTES, v[r]);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < D::VEC; ++e) acc[r] = fmaf(v[r][e], xs[k + e], acc[r]);
    }
  } else {
    for (int k = lane; k < K; k += 64)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = fmaf(D::at(rp[r], k), xs[k], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float t = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < N) y[row0 + r] = t;
  }
}

template <int T>
int launch_dense(const void* W, const float* x, float* y, int N, int K, hipStream_t s) {
  constexpr int R = 4;
  const unsigned grid = (unsigned)((N + 4 * R - 1) / (4 * R));
  gemv_dense<T, R><<<grid, 256, (size_t)K * 4, s>>>((const uint8_t*)W, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_gemv: launch");
  return TIERMM_OK;
}

}  // namespace

int qgemv_q4k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
int qgemv_q4k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
constexpr int kQ4kMaxK = 14336;  // equals the limit in qgemv_q4k.hip

int qgemv_dispatch(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  switch (qtype) {
    // dense rows (gemv_q over q_val's F32/F16/BF16 cases): the dense-row kernel
    case QT_F32: return launch_dense<TIERMM_F32>(W, x, y, N, K, s);
    case QT_F16: return launch_dense<TIERMM_F16>(W, x, y, N, K, s);
    case QT_BF16: return launch_dense<TIERMM_BF16>(W, x, y, N, K, s);
    case QT_Q4_K:  // MFMA kernels up to kQ4kMaxK (x digits in LDS); beyond, the generic kernel
      if (K <= 8192 && (N + 15) / 16 >= 640) return qgemv_q4k_ws(W, rb, x, y, N, K, s);
      return K <= kQ4kMaxK ? qgemv_q4k(W, rb, x, y, N, K, s) : launch_generic<QT_Q4_K>(W, rb, x, y, N, K, s);
    default:
      return with_qtype(qtype, [&](auto qt) { return launch_generic<decltype(qt)::value>(W, rb, x, y, N, K, s); });
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
  if ((qtype == QT_F32 || qtype == QT_F16 || qtype == QT_BF16) && ((uintptr_t)W % 16))
    return set_error(TIERMM_EINVAL, "tiermm_qgemv: dense rows must start 16-byte aligned");
  return qgemv_dispatch(W, qtype, rb, x, y, N, K, (hipStream_t)stream);
}

extern "C" int tiermm_gemv(const void* W, int wtype, const float* x, float* y, int N, int K, tiermm_stream_t stream) {
  if (wtype != TIERMM_F32 && wtype != TIERMM_F16 && wtype != TIERMM_BF16)
    return set_error(TIERMM_UNSUPPORTED, "tiermm_gemv: weight type %d", wtype);
  if (N < 0 || K < 0) return set_error(TIERMM_EINVAL, "tiermm_gemv: negative size");
  if (N == 0) return TIERMM_OK;
  if (K > kMaxK) return set_error(TIERMM_UNSUPPORTED, "tiermm_gemv: K=%d above %d", K, kMaxK);
  if (!W || !x || !y || ((uintptr_t)W % 16))
    return set_error(TIERMM_EINVAL, "tiermm_gemv: W must be non-null and 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (wtype == TIERMM_F32) return launch_dense<TIERMM_F32>(W, x, y, N, K, s);
  if (wtype == TIERMM_F16) return launch_dense<TIERMM_F16>(W, x, y, N, K, s);
  return launch_dense<TIERMM_BF16>(W, x, y, N, K, s);
}

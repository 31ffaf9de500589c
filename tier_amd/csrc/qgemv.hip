// qgemv.hip -- tiermm_qgemv: decode-time (M=1) dequant-GEMV, gemv_q (tier.cpp:299-306).
//
// Kernel per type: Q4_K, Q5_K, Q6_K and Q8_0 run on int8 MFMA (qgemv_q4k.hip,
// qgemv_q4k_ws.hip, qgemv_q6k.hip); Q4_0/Q4_1/Q5_0/Q5_1 (and Q8_0 rows the MFMA kernel does not
// take) on the staged kernel below; every other type, and rows either kernel
// does not take, on the generic kernel.
//
// Generic kernel (every type): the block stages x in LDS once; each wave
// owns R consecutive rows and its lanes walk the row in 8-element chunks
// (lane-strided, like gemv_q's k += warpSize loop but 8 wide), decoding each
// chunk exactly as q_val and accumulating in fp32; the R row partials are then
// reduced across the wave with xor shuffles.  x is read from LDS once per chunk
// and reused for the R rows.
#include "tm_device.h"

namespace tiermm {

int check_qweight(const char* who, const void* W, int qtype, size_t rb, int cols, int dense_unit);

namespace {

constexpr int kMaxLdsK = 16384;  // x staged whole in LDS (64 KiB) up to this K; read from global above

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// XL: x staged in LDS (K <= kMaxLdsK); else read from global memory, where the
// workgroups' repeated reads of the same K floats stay in L2.
template <int QT, int R, bool XL>
__global__ __launch_bounds__(256) void qgemv_generic(const uint8_t* __restrict__ W, size_t rb,
                                                     const float* __restrict__ x, float* __restrict__ y, int N,
                                                     int K) {
  extern __shared__ float xsh[];
  const float* xs = XL ? xsh : x;
  if (XL) {
    for (int i = threadIdx.x * 4; i < K; i += 256 * 4) *(float4*)&xsh[i] = *(const float4*)&x[i];
    __syncthreads();
  }
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
  if (K <= kMaxLdsK)
    qgemv_generic<QT, R, true><<<grid, 256, (size_t)K * 4, s>>>((const uint8_t*)W, rb, x, y, N, K);
  else
    qgemv_generic<QT, R, false><<<grid, 256, 0, s>>>((const uint8_t*)W, rb, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_qgemv: launch");
  return TIERMM_OK;
}

// ------------------------------------------------------ staged block GEMV
// The 32-element block types whose two-block unit is a whole number of dwords
// (q8_0 68 B, q4_0 36, q4_1 40, q5_0 44, q5_1 48), rows 16-byte aligned.  A
// workgroup of 4 waves owns RW = 4R consecutive rows, which are one contiguous
// byte range of W: it copies them into LDS with global_load_lds_dwordx4 (1 KiB
// per instruction, every byte read once, all loads issued up front) while it
// copies x into LDS, padded 4 floats per 64 so that the lanes' 64-float units
// start on distinct banks.  Lane l of a wave then takes the units u = l, l + 64,
// ... (elements [64u, 64u + 64)) of the wave's R rows: 16 ds_read_b128 of x, DW
// dwords of each row, decoded in registers.  Per block the integer values are
// summed against x in fp32 and scaled once: d * sum(q * x) (+ m * sum(x)), the
// same products as gemv_q's sum of q_val * x (tier.cpp:299-306) in another
// order, within fp32 rounding of it.
template <int QT>
struct U2;
template <>
struct U2<QT_Q8_0> {  // quant.h:68
  static constexpr int B = 34, QS = 2, M = -1, QH = -1;
};
template <>
struct U2<QT_Q4_0> {  // quant.h:64
  static constexpr int B = 18, QS = 2, M = -1, QH = -1, OFF = 8;
};
template <>
struct U2<QT_Q4_1> {  // quant.h:65
  static constexpr int B = 20, QS = 4, M = 2, QH = -1, OFF = 0;
};
template <>
struct U2<QT_Q5_0> {  // quant.h:66
  static constexpr int B = 22, QS = 6, M = -1, QH = 2, OFF = 16;
};
template <>
struct U2<QT_Q5_1> {  // quant.h:67
  static constexpr int B = 24, QS = 8, M = 2, QH = 4, OFF = 0;
};

// byte / halfword / word at byte offset i (a compile-time constant once unrolled)
// of the dwords w; halfwords and words sit at even offsets in these layouts
template <int NW>
__device__ __forceinline__ uint32_t ubyte(const uint32_t (&w)[NW], int i) { return (w[i >> 2] >> (8 * (i & 3))) & 255u; }
template <int NW>
__device__ __forceinline__ int sbyte(const uint32_t (&w)[NW], int i) { return (int)(w[i >> 2] << (24 - 8 * (i & 3))) >> 24; }
template <int NW>
__device__ __forceinline__ uint32_t uhalf(const uint32_t (&w)[NW], int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xffffu; }
template <int NW>
__device__ __forceinline__ uint32_t uword(const uint32_t (&w)[NW], int i) {
  return (i & 3) ? (w[i >> 2] >> 16) | (w[(i >> 2) + 1] << 16) : w[i >> 2];
}

// sum over the unit's 64 elements of q_val * x; sx[b] = sum of block b's x
template <int QT, int NW>
__device__ __forceinline__ float unit_dot(const uint32_t (&w)[NW], const float (&xv)[64], const float (&sx)[2]) {
  using T = U2<QT>;
  float acc = 0.f;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int o = T::B * b;
    float sq = 0.f;
    if constexpr (QT == QT_Q8_0) {
#pragma unroll
      for (int j = 0; j < 32; ++j) sq = fmaf((float)sbyte(w, o + T::QS + j), xv[32 * b + j], sq);
    } else {
      uint32_t qh = 0;
      if constexpr (T::QH >= 0) qh = uword(w, o + T::QH);
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        int q = (int)((ubyte(w, o + T::QS + (j & 15)) >> (j < 16 ? 0 : 4)) & 15u);
        if constexpr (T::QH >= 0) q |= (int)(((qh >> j) & 1u) << 4);
        sq = fmaf((float)(q - T::OFF), xv[32 * b + j], sq);
      }
    }
    acc = fmaf(h2f(uhalf(w, o)), sq, acc);
    if constexpr (T::M >= 0) acc = fmaf(h2f(uhalf(w, o + T::M)), sx[b], acc);
  }
  return acc;
}

template <int QT, int R>
__global__ __launch_bounds__(256) void qgemv_staged(const uint8_t* __restrict__ W, size_t rb, const float* __restrict__ x,
                                                    float* __restrict__ y, int N, int K, uint32_t wbytes) {
  constexpr int UB = 2 * U2<QT>::B, NW = UB / 4, RW = 4 * R;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * RW;
  // the workgroup's rows: bytes [row0 * rb, (row0 + rows) * rb) of W; a lane past
  // them re-reads the last 16 bytes into the slack after the image
  const uint32_t total = (uint32_t)min(RW, N - row0) * (uint32_t)rb;
  const uint8_t* g0 = W + (size_t)row0 * rb;
  const uint32_t l0 = lds_addr(smem);
  const int ni = (int)((total + 1023) / 1024);
  for (int i = wave; i < ni; i += 4) {
    const uint32_t off = (uint32_t)i * 1024 + 16 * lane;
    dma16(g0 + min(off, total - 16), l0 + (uint32_t)i * 1024);
  }
  float* xs = (float*)(smem + wbytes);
  // per wave: x held a non-finite value (in the dynamic LDS, after x: the kernel
  // opts into all 160 KiB of dynamic LDS, so it has no static LDS)
  int* nf = (int*)(xs + (size_t)K / 64 * 68);
  bool bad = false;
  for (int i = tid * 4; i < K; i += 1024) {
    const float4 v = *(const float4*)&x[i];
    bad |= !__builtin_isfinite(v.x) || !__builtin_isfinite(v.y) || !__builtin_isfinite(v.z) ||
           !__builtin_isfinite(v.w);
    *(float4*)&xs[i + (i >> 6) * 4] = v;
  }
  {
    const bool wbad = __ballot(bad) != 0;
    if (lane == 0) nf[wave] = wbad ? 1 : 0;
  }
  vm_wait<0>();
  __syncthreads();
  if (nf[0] | nf[1] | nf[2] | nf[3]) {
    // NaN or +-Inf in x: d * sum(q * x) + m * sum(x) would not give the per-element
    // products' class (q = 0 times Inf), so the rows take gemv_q's non-finite sums
    for (int r = wave; r < RW; r += 4) {
      const int row = row0 + r;
      if (row < N) {
        const float s = nonfinite_terms<QT>(W + (size_t)row * rb, x, 0, K, lane);
        if (lane == 0) y[row] = s;
      }
    }
    return;
  }

  const int U = K / 64;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int u = lane; u < U; u += 64) {
    float xv[64];
    const float* xp = xs + 68 * u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4 t = *(const float4*)(xp + 4 * i);
      xv[4 * i] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
    }
    float sx[2] = {0.f, 0.f};
    if constexpr (U2<QT>::M >= 0) {
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        sx[0] += xv[j];
        sx[1] += xv[32 + j];
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t* wp = (const uint32_t*)(smem + (size_t)(wave * R + r) * rb + (size_t)UB * u);
      uint32_t w[NW];
#pragma unroll
      for (int i = 0; i < NW; ++i) w[i] = wp[i];
      acc[r] += unit_dot<QT>(w, xv, sx);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    const int row = row0 + wave * R + r;
    if (lane == 0 && row < N) y[row] = v;
  }
}

// LDS of the staged kernel: the rows (whole KiB), padded x, four non-finite flags.
size_t staged_lds(size_t rb, int K, int R) {
  return (4 * R * rb + 1023) / 1024 * 1024 + (size_t)K / 64 * 68 * 4 + 4 * sizeof(int);
}

template <int QT>
int launch_staged(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  // two rows per wave while two workgroups fit a CU, else one
  const int R = staged_lds(rb, K, 2) <= 80 * 1024 ? 2 : 1;
  const size_t lds = staged_lds(rb, K, R);
  const uint32_t wbytes = (uint32_t)((4 * R * rb + 1023) / 1024 * 1024);
  const unsigned grid = (unsigned)((N + 4 * R - 1) / (4 * R));
  static std::atomic<uint64_t> attr1{0}, attr2{0};
  int st = lds_attr_once(attr1, (const void*)qgemv_staged<QT, 1>, 160 * 1024, "tiermm_qgemv");
  if (!st) st = lds_attr_once(attr2, (const void*)qgemv_staged<QT, 2>, 160 * 1024, "tiermm_qgemv");
  if (st) return st;
  if (R == 2)
    qgemv_staged<QT, 2><<<grid, 256, lds, s>>>((const uint8_t*)W, rb, x, y, N, K, wbytes);
  else
    qgemv_staged<QT, 1><<<grid, 256, lds, s>>>((const uint8_t*)W, rb, x, y, N, K, wbytes);
  TM_LAUNCH_CHECK("tiermm_qgemv: launch");
  return TIERMM_OK;
}

// The staged kernel takes the shape: 64-element units, rows and base 16-byte
// aligned, and one workgroup's rows plus x within the LDS.
bool staged_fits(const void* W, size_t rb, int K) {
  return K % 64 == 0 && rb % 16 == 0 && ((uintptr_t)W % 16) == 0 && staged_lds(rb, K, 1) <= 160 * 1024;
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

template <int T, int R, bool XL>
__global__ __launch_bounds__(256) void gemv_dense(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                  float* __restrict__ y, int N, int K) {
  using D = Dense<T>;
  extern __shared__ float xsh[];  // x staged in LDS when XL (K <= kMaxLdsK), else read from global
  const float* xs = XL ? xsh : x;
  if (XL) {
    for (int i = threadIdx.x; i < K; i += 256) xsh[i] = x[i];
    __syncthreads();
  }
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
  if (K <= kMaxLdsK)
    gemv_dense<T, R, true><<<grid, 256, (size_t)K * 4, s>>>((const uint8_t*)W, x, y, N, K);
  else
    gemv_dense<T, R, false><<<grid, 256, 0, s>>>((const uint8_t*)W, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_gemv: launch");
  return TIERMM_OK;
}

}  // namespace

int qgemv_q4k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
int qgemv_q4k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
int qgemv_q5k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
bool qgemv_ws_takes(int qtype, int N, int K);
bool qgemv_ws_batch_takes(int qtype, const int* N, int count, int K);
int qgemv_ws_batch(const void* const* W, int qtype, size_t rb, const float* x, float* const* y, const int* N,
                   int count, int K, hipStream_t s);
bool qgemv_mfma_fits(const void* W, int qtype, size_t rb, int K);
bool qgemv_q6k_fits(const void* W, size_t rb, int N, int K);
int qgemv_q6k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
int qgemv_mfma(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K, hipStream_t s);
constexpr int kQ4kMaxK = 28672;  // equals the limit in qgemv_q4k.hip

int qgemv_dispatch(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  switch (qtype) {
    // dense rows (gemv_q over q_val's F32/F16/BF16 cases): the dense-row kernel
    case QT_F32: return launch_dense<TIERMM_F32>(W, x, y, N, K, s);
    case QT_F16: return launch_dense<TIERMM_F16>(W, x, y, N, K, s);
    case QT_BF16: return launch_dense<TIERMM_BF16>(W, x, y, N, K, s);
    case QT_Q4_K:  // MFMA kernels up to kQ4kMaxK (x digits in LDS); beyond, the generic kernel
      if (qgemv_ws_takes(QT_Q4_K, N, K)) return qgemv_q4k_ws(W, rb, x, y, N, K, s);
      return K <= kQ4kMaxK ? qgemv_q4k(W, rb, x, y, N, K, s) : launch_generic<QT_Q4_K>(W, rb, x, y, N, K, s);
    case QT_Q8_0:  // int8 MFMA kernel; rows that do not fit it staged whole in LDS
      if (qgemv_mfma_fits(W, qtype, rb, K)) return qgemv_mfma(W, qtype, rb, x, y, N, K, s);
      if (staged_fits(W, rb, K)) return launch_staged<QT_Q8_0>(W, rb, x, y, N, K, s);
      return launch_generic<QT_Q8_0>(W, rb, x, y, N, K, s);
    case QT_Q5_K:  // the whole-tile kernel where qgemv_ws_takes, the rest on the per-wave one
      if (qgemv_mfma_fits(W, qtype, rb, K) && qgemv_ws_takes(QT_Q5_K, N, K)) return qgemv_q5k_ws(W, rb, x, y, N, K, s);
      if (qgemv_mfma_fits(W, qtype, rb, K)) return qgemv_mfma(W, qtype, rb, x, y, N, K, s);
      return launch_generic<QT_Q5_K>(W, rb, x, y, N, K, s);
    case QT_Q6_K:
      if (qgemv_q6k_fits(W, rb, N, K)) return qgemv_q6k(W, rb, x, y, N, K, s);
      return launch_generic<QT_Q6_K>(W, rb, x, y, N, K, s);
    case QT_Q4_0:
      if (staged_fits(W, rb, K)) return launch_staged<QT_Q4_0>(W, rb, x, y, N, K, s);
      return launch_generic<QT_Q4_0>(W, rb, x, y, N, K, s);
    case QT_Q4_1:
      if (staged_fits(W, rb, K)) return launch_staged<QT_Q4_1>(W, rb, x, y, N, K, s);
      return launch_generic<QT_Q4_1>(W, rb, x, y, N, K, s);
    case QT_Q5_0:
      if (staged_fits(W, rb, K)) return launch_staged<QT_Q5_0>(W, rb, x, y, N, K, s);
      return launch_generic<QT_Q5_0>(W, rb, x, y, N, K, s);
    case QT_Q5_1:
      if (staged_fits(W, rb, K)) return launch_staged<QT_Q5_1>(W, rb, x, y, N, K, s);
      return launch_generic<QT_Q5_1>(W, rb, x, y, N, K, s);
    default:
      return with_qtype(qtype, [&](auto qt) { return launch_generic<decltype(qt)::value>(W, rb, x, y, N, K, s); });
  }
}

}  // namespace tiermm

using namespace tiermm;

extern "C" int tiermm_qgemv(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K,
                            tiermm_stream_t stream) {
  int st = check_qweight("tiermm_qgemv", W, qtype, rb, K, 1);
  if (st) return st;
  if (N < 0) return set_error(TIERMM_EINVAL, "tiermm_qgemv: N < 0");
  if (N == 0) return TIERMM_OK;
  if (!x || !y || ((uintptr_t)x % 16)) return set_error(TIERMM_EINVAL, "tiermm_qgemv: x must be 16-byte aligned");
  if ((qtype == QT_F32 || qtype == QT_F16 || qtype == QT_BF16) && ((uintptr_t)W % 16))
    return set_error(TIERMM_EINVAL, "tiermm_qgemv: dense rows must start 16-byte aligned");
  return qgemv_dispatch(W, qtype, rb, x, y, N, K, (hipStream_t)stream);
}

// gemv_q of up to TIERMM_QGEMV_BATCH matrices that share x, K and the block type.  Where
// the whole-tile kernel takes their concatenated rows (q4_K / q5_K, K <= 5120, its tile
// rule on the total) they run as one launch; otherwise one tiermm_qgemv each.  Either
// way every y[i] is the same, bit for bit, as tiermm_qgemv on W[i].
extern "C" int tiermm_qgemv_batch(const void* const* W, int qtype, size_t rb, const float* x, float* const* y,
                                  const int* N, int count, int K, tiermm_stream_t stream) {
  if (!W || !y || !N || count < 1 || count > TIERMM_QGEMV_BATCH)
    return set_error(TIERMM_EINVAL, "tiermm_qgemv_batch: 1..%d matrices with weight, output and row arrays",
                     TIERMM_QGEMV_BATCH);
  const void* w[TIERMM_QGEMV_BATCH];
  float* yy[TIERMM_QGEMV_BATCH];
  int n[TIERMM_QGEMV_BATCH], live = 0;
  for (int i = 0; i < count; ++i) {
    if (N[i] < 0) return set_error(TIERMM_EINVAL, "tiermm_qgemv_batch: N[%d] < 0", i);
    if (N[i] > 0) {  // matrices without rows take no part (their pointers are not read)
      int st = check_qweight("tiermm_qgemv_batch", W[i], qtype, rb, K, 1);
      if (st) return st;
      if (!y[i]) return set_error(TIERMM_EINVAL, "tiermm_qgemv_batch: y[%d] is null", i);
      w[live] = W[i];
      yy[live] = y[i];
      n[live++] = N[i];
    }
  }
  if (!live) return TIERMM_OK;
  if (!x || ((uintptr_t)x % 16)) return set_error(TIERMM_EINVAL, "tiermm_qgemv_batch: x must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  bool fits = qgemv_ws_batch_takes(qtype, n, live, K);
  for (int i = 0; fits && i < live && qtype == QT_Q5_K; ++i) fits = qgemv_mfma_fits(w[i], qtype, rb, K);
  if (fits) return qgemv_ws_batch(w, qtype, rb, x, yy, n, live, K, s);
  for (int i = 0; i < live; ++i) {
    if ((qtype == QT_F32 || qtype == QT_F16 || qtype == QT_BF16) && ((uintptr_t)w[i] % 16))
      return set_error(TIERMM_EINVAL, "tiermm_qgemv_batch: dense rows must start 16-byte aligned");
    int st = qgemv_dispatch(w[i], qtype, rb, x, yy[i], n[i], K, s);
    if (st) return st;
  }
  return TIERMM_OK;
}

extern "C" int tiermm_gemv(const void* W, int wtype, const float* x, float* y, int N, int K, tiermm_stream_t stream) {
  if (wtype != TIERMM_F32 && wtype != TIERMM_F16 && wtype != TIERMM_BF16)
    return set_error(TIERMM_UNSUPPORTED, "tiermm_gemv: weight type %d", wtype);
  if (N < 0 || K < 0) return set_error(TIERMM_EINVAL, "tiermm_gemv: negative size");
  if (N == 0) return TIERMM_OK;
  if (!W || !x || !y || ((uintptr_t)W % 16))
    return set_error(TIERMM_EINVAL, "tiermm_gemv: W must be non-null and 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (wtype == TIERMM_F32) return launch_dense<TIERMM_F32>(W, x, y, N, K, s);
  if (wtype == TIERMM_F16) return launch_dense<TIERMM_F16>(W, x, y, N, K, s);
  return launch_dense<TIERMM_BF16>(W, x, y, N, K, s);
}

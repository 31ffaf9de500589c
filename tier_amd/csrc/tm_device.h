// tm_device.h -- device helpers shared by the gfx950 kernels: fp16/bf16
// rounding, the non-finite GEMV terms, hand-issued loads and the LDS DMA.  The
// exact per-block decoders (Dec<>) are in tm_decode.h, built for host and device.
//
// fp32 -> fp16 uses v_cvt_f16_f32 (round to nearest even, fp16 denormals kept by
// the default MODE), matching tier_fp16.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <type_traits>

#include "tm_decode.h"
#include "tm_host.h"

namespace tiermm {

// The empty asm statement pins the conversion to a plain v_cvt_f16_f32 on an fp32
// value (see h2f in tm_decode.h).
__device__ __forceinline__ uint16_t f2h(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// hip_bfloat16(float): round to nearest even on the top 16 bits; NaN stays NaN.
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 1u : 0u));
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// gemv_q's sum (tier.cpp:304) restricted to the columns k in [k0, k1) (multiples
// of 8; x 16-byte aligned) where x[k] is NaN or +-Inf, by one wave: every lane
// returns the sum.  Each such term q_val * x[k] is +-Inf or NaN (0 * Inf), so
// the sum is NaN or +-Inf whenever one exists, and it is the value gemv_q's
// fp32 sum over the whole row takes: finite terms cannot turn +-Inf back into a
// finite number, and NaN or Inf + -Inf gives NaN in any order.  The int8-digit
// GEMVs, which carry only finite x, overwrite their rows with it when x holds a
// non-finite element.
template <int QT>
__device__ float nonfinite_terms(const uint8_t* row, const float* x, int k0, int k1, int lane) {
  float s = 0.f;
  for (int c = k0 + 8 * lane; c < k1; c += 512) {
    const float4 a = *(const float4*)(x + c), b = *(const float4*)(x + c + 4);
    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bool any = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) any |= !__builtin_isfinite(xv[i]);
    if (any) {
      float v[8];
      Dec<QT>::run(row, c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (!__builtin_isfinite(xv[i])) s += v[i] * xv[i];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  return s;
}

// The exponent of a row of the two-part (x3s) split: with amax = m * 2^ex (m in
// [0.5, 1)), e = 15 - ex puts amax * 2^e in [2^14, 2^15); clamped to [-100, 100], and
// 0 for an all-zero or non-finite maximum.
__device__ __forceinline__ int x3s_exp(float amax) {
  if (!(amax > 0.f) || !isfinite(amax)) return 0;
  int ex;
  (void)frexpf(amax, &ex);
  return min(100, max(-100, 15 - ex));
}

__device__ __forceinline__ float block_max_256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

// The two-part split of row `row` of src (cols fp32, a multiple of 4, at most 1024 * XR;
// rows 16-byte aligned) by a block of 256 threads, the row held in registers: hi, lo =
// the fp16 parts of x * 2^e, exps[row] = e (x3s_exp of the row's max |x|).
template <int XR>
__device__ __forceinline__ void x3s_split_row(const float* __restrict__ src, uint16_t* __restrict__ hi,
                                              uint16_t* __restrict__ lo, int32_t* __restrict__ exps, int cols,
                                              int row) {
  __shared__ float red[4];
  const size_t base = (size_t)row * cols;
  const int c4 = cols >> 2;
  float4 v[XR];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < XR; ++j) {
    const int k = threadIdx.x + 256 * j;
    v[j] = k < c4 ? ((const float4*)(src + base))[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  }
  amax = block_max_256(amax, red);
  const int e = x3s_exp(amax);
  const float sc = ldexpf(1.f, e);
#pragma unroll
  for (int j = 0; j < XR; ++j) {
    const int k = threadIdx.x + 256 * j;
    if (k >= c4) break;
    const float f[4] = {v[j].x * sc, v[j].y * sc, v[j].z * sc, v[j].w * sc};
    uint32_t h[2], l[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint16_t h0 = f2h(f[2 * q]), h1 = f2h(f[2 * q + 1]);
      const uint16_t l0 = f2h(f[2 * q] - h2f(h0)), l1 = f2h(f[2 * q + 1] - h2f(h1));
      h[q] = h0 | ((uint32_t)h1 << 16);
      l[q] = l0 | ((uint32_t)l1 << 16);
    }
    ((uint2*)(hi + base))[k] = make_uint2(h[0], h[1]);
    ((uint2*)(lo + base))[k] = make_uint2(l[0], l[1]);
  }
  if (threadIdx.x == 0) exps[row] = e;
}

// Hand-issued vector memory for the kernels that stream through LDS: the
// compiler's wait insertion cannot follow global->LDS loads (it falls back to
// waiting for everything before LDS reads), which would serialise the stream.
// Every vector load below is one instruction per wave regardless of the lane
// mask, and loads retire in order, so "s_waitcnt vmcnt(N)" means all but the N
// most recent ones have landed.  Only loads into LDS are hand-issued: a register
// that a hand-issued load fills looks ready to the compiler at once, which may
// copy it while the load is in flight, so loads into registers are plain loads
// whose waits the compiler places (x that a wave needs while its own LDS DMA is
// in flight comes into LDS by the same DMA instead).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// K-tiled plane layout of the internal fp16 operands of the big-tile GEMM:
// element (row, col) of a plane with `rows` rows at ((col / 32) * rows + row) * 32
// + col % 32, so that the 64 bytes of one K step of 16 consecutive rows are one
// contiguous kilobyte.
__device__ __forceinline__ size_t ktile_index(size_t row, int col, size_t rows) {
  return (((size_t)(col >> 5) * rows + row) << 5) + (size_t)(col & 31);
}
// The element (row, col) that starts 8-element unit u of a K-tiled plane of `rows`
// rows: writers walk the units in order, so each wave stores contiguous kilobytes.
__device__ __forceinline__ void ktile_unit(size_t u, size_t rows, size_t& row, int& col) {
  const size_t kt = u / (rows * 4), rem = u - kt * rows * 4;
  row = rem >> 2;
  col = (int)(kt * 32 + (rem & 3) * 8);
}

// 16 bytes per lane from p into LDS at lds_addr + 16*lane (lds_addr wave-uniform, through M0).
//
// dma16 / dma16_nt set M0 (the LDS destination) inside their asm, unseen by the
// compiler, which treats M0 as reserved (an "m0" clobber is not honoured).  That is
// sound while the compiler puts nothing of its own in M0 in the kernels that call
// them: no LDS-DMA builtins, s_sendmsg, indexed register access or LDS-direct reads;
// in their gfx950 code the only M0 references are these writes.  The loads are
// invisible to the compiler's wait insertion, so every pipeline waits with explicit
// vm_wait counts.  __builtin_amdgcn_global_load_lds, which lets the compiler own M0,
// makes the loads visible to it instead, and it then waits for all of them
// (s_waitcnt vmcnt(0)) before every release store of a hand-off flag and before
// every workgroup barrier: built that way, qgemv_q4k_ws.hip carries 498 -> 618
// vmcnt waits and x3.hip 4408 -> 4746, and the stage in flight behind a
// flag drains before the flag is set.  So the asm form stays.
__device__ __forceinline__ void dma16(const void* p, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(p),
               "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}
// The same with the non-temporal hint: the bytes are streamed once and should not
// displace what the caches hold.
__device__ __forceinline__ void dma16_nt(const void* p, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(p),
               "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}
// Sum over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48), as
// (row0 + row1) + (row2 + row3) in every lane -- the sums two xor shuffles by 16 and
// 32 give -- through gfx950's row-swap moves instead of two LDS-routed permutes:
// with both operands a, permlane16_swap leaves rows (0,0,2,2) in one result and
// (1,1,3,3) in the other, permlane32_swap the halves (lo,lo) and (hi,hi).
__device__ __forceinline__ float row_sum4(float a) {
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  const float s = __uint_as_float(t[0]) + __uint_as_float(t[1]);
  const auto u = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(u[0]) + __uint_as_float(u[1]);
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Longest K one fp32 accumulator sums in the MFMA GEMMs: its rounding error grows
// like sqrt(K), and above kAccChunkFrom the x3 products run as chunks of at most
// kAccChunkMax columns whose sums are added in fp32 (x3.hip run_k_chunks; the
// fused dequant GEMM splits K at least as finely).
constexpr int kAccChunkFrom = 6144, kAccChunkMax = 4096;
inline int acc_chunks(int K) { return K > kAccChunkFrom ? (K + kAccChunkMax - 1) / kAccChunkMax : 1; }

// Opts kernel `fn` into `bytes` of dynamic LDS on the current device, once per
// device and process.  `done` is the caller's per-kernel bit mask of devices
// already set; threads that race on a first call may both set the attribute,
// which is harmless (it is idempotent), and the mask is updated atomically.
inline int lds_attr_once(std::atomic<uint64_t>& done, const void* fn, int bytes, const char* who) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, who);
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return TIERMM_OK;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // reset the runtime's last error, or a later launch check would report it
    return hip_fail(e, who);
  }
  done.fetch_or(bit, std::memory_order_acq_rel);
  return TIERMM_OK;
}

// Launch-shape guard: kernels assume their block size; a mismatch is a host bug.
#define TM_LAUNCH_CHECK(what)                                  \
  do {                                                         \
    hipError_t e_ = hipGetLastError();                         \
    if (e_ != hipSuccess) return hip_fail(e_, what);           \
  } while (0)

}  // namespace tiermm

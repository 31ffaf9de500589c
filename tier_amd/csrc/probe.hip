// probe.hip -- measurement helpers for bench.py (libtiermm_probe.so; no counterpart in
// the reference and not part of the matmul path): the time one launch takes to read
// a buffer once from HBM with nothing else to do, which bounds any decode GEMV that
// must read the same bytes; a register-only fp16 MFMA loop, which bounds the x3
// GEMMs' products; and a host loop that issues a run of tiermm_qgemv calls through
// the C ABI, as the engine's token loop calls gemv_q (tier.cpp:2357), so that the
// per-call cost of Python does not set the pace of the short decode lines.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every 16-byte word of [src, src + n16 * 16) is loaded once (non-temporal), U loads
// in flight per thread; the XOR of all words decides whether one word is written, so
// no load can be dropped.  grid = gridDim.x, as an argument: like the decode GEMVs the
// kernel then reads no implicit argument (a 28-byte argument segment, without the 256
// bytes of implicit arguments a read of gridDim brings).
template <int U>
__global__ __launch_bounds__(256) void read_once(const u32x4* __restrict__ src, size_t n16, uint32_t* __restrict__ out,
                                                 int grid) {
  const size_t stride = (size_t)grid * 256 * U;
  uint32_t acc = 0;
  for (size_t i = (size_t)blockIdx.x * 256 * U + threadIdx.x; i < n16; i += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t k = i + (size_t)u * 256;
      v[u] = k < n16 ? __builtin_nontemporal_load(src + k) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;
}

// The same bytes through the LDS DMA (global_load_lds_dwordx4, non-temporal) by
// persistent workgroups of 4 waves: wave w of workgroup b streams the contiguous
// 1 KiB pieces b*4 + w, + 4 grid, ... into a ring of WIN slots, keeping WIN loads in
// flight (the weight stream of the decode GEMV without its consumers).
template <int WIN>
__global__ __launch_bounds__(256) void read_lds(const uint8_t* __restrict__ src, size_t nkb, uint32_t* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[4 * WIN * 1024];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t base = (uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t*)(ring + wave * WIN * 1024);
  const size_t step = (size_t)gridDim.x * 4;
  size_t k = (size_t)blockIdx.x * 4 + wave;
  int issued = 0;
  for (; k < nkb; k += step, ++issued) {
    if (issued >= WIN) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WIN - 1) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src + k * 1024 + lane * 16),
                 "s"(__builtin_amdgcn_readfirstlane(base + (issued % WIN) * 1024))
                 : "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const uint32_t v = ((const uint32_t*)ring)[threadIdx.x];
  if (v == 0x9e3779b9u) out[blockIdx.x] = v;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ITER x 8 independent v_mfma_f32_32x32x16_f16 per wave on operands held in registers
// (seeded from `seed`, so random-like data is multiplied); one float per thread is
// written so the products are kept.
template <int ITER>
__global__ __launch_bounds__(256) void mfma_loop(const uint32_t* __restrict__ seed, float* __restrict__ out) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  f16x8 a, b;
  uint32_t s = seed[t & 1023];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s = s * 1664525u + 1013904223u;
    a[i] = (_Float16)((float)(int)(s >> 16 & 0x7ff) * (1.f / 1024.f) - 1.f);
    s = s * 1664525u + 1013904223u;
    b[i] = (_Float16)((float)(int)(s >> 16 & 0x7ff) * (1.f / 1024.f) - 1.f);
  }
  f32x16 c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = f32x16{};
  for (int it = 0; it < ITER; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
  }
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) r += c[j][i];
  out[t] = r;
}

}  // namespace

extern "C" {

// count calls fn(W[(first + i) % ncopies], qtype, rb, x, y, N, K, s) for i = 0..count-1,
// fn being tiermm_qgemv; returns the first non-zero status.
typedef int (*qgemv_fn)(const void*, int, size_t, const float*, float*, int, int, hipStream_t);
int tiermm_bench_qgemv(void* fn, const void* const* W, int ncopies, int first, int qtype, size_t rb, const float* x,
                       float* y, int N, int K, int count, hipStream_t s) {
  const qgemv_fn f = (qgemv_fn)fn;
  for (int i = 0; i < count; ++i) {
    const int st = f(W[(first + i) % ncopies], qtype, rb, x, y, N, K, s);
    if (st) return st;
  }
  return 0;
}

// One read of `bytes` (a multiple of 16, src 16-byte aligned) by `grid` workgroups of
// 256 threads with `unroll` (1, 2, 4 or 8) loads in flight per thread; out: grid words.
int tiermm_probe_read(const void* src, size_t bytes, int grid, int unroll, void* out, hipStream_t s) {
  const size_t n16 = bytes / 16;
  const dim3 g((unsigned)grid), b(256);
  switch (unroll) {
    case 1: read_once<1><<<g, b, 0, s>>>((const u32x4*)src, n16, (uint32_t*)out, grid); break;
    case 2: read_once<2><<<g, b, 0, s>>>((const u32x4*)src, n16, (uint32_t*)out, grid); break;
    case 4: read_once<4><<<g, b, 0, s>>>((const u32x4*)src, n16, (uint32_t*)out, grid); break;
    case 8: read_once<8><<<g, b, 0, s>>>((const u32x4*)src, n16, (uint32_t*)out, grid); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The LDS-DMA stream of `bytes` (a multiple of 1 KiB) by `grid` workgroups of 4 waves
// with `win` (8, 12 or 24) loads in flight per wave.
int tiermm_probe_read_lds(const void* src, size_t bytes, int grid, int win, void* out, hipStream_t s) {
  const size_t nkb = bytes / 1024;
  const dim3 g((unsigned)grid), b(256);
  switch (win) {
    case 8: read_lds<8><<<g, b, 0, s>>>((const uint8_t*)src, nkb, (uint32_t*)out); break;
    case 12: read_lds<12><<<g, b, 0, s>>>((const uint8_t*)src, nkb, (uint32_t*)out); break;
    case 24: read_lds<24><<<g, b, 0, s>>>((const uint8_t*)src, nkb, (uint32_t*)out); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// grid workgroups x 4 waves, each 8 x iters MFMAs of 32x32x16 (32768 flop each);
// seed: 1024 words, out: grid * 256 floats.  Flops = grid * 4 * 8 * iters * 32768.
int tiermm_probe_mfma(const void* seed, int grid, int iters, void* out, hipStream_t s) {
  if (iters != 4096) return 1;
  mfma_loop<4096><<<dim3((unsigned)grid), dim3(256), 0, s>>>((const uint32_t*)seed, (float*)out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}

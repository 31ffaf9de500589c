// qgemv_q4k_ws.hip -- Q4_K decode GEMV with a producer wave per workgroup.
//
// Same arithmetic and LDS layouts as qgemv_q4k.hip (gemv_q, tier.cpp:299-306;
// q_val Q4_K, quant.h:83-84).  The difference is who moves the weights: one
// wave of the workgroup does nothing but issue the global->LDS loads into a
// ring of NS stages shared by the workgroup, keeping D stages in flight, while
// the NC consumer waves prepare x and run the MFMA + scale work.  A consumer
// that computes therefore never holds back the weight stream, and the x
// preparation at the start overlaps D stages of loads.
//
// Stage order: q = gi * NC + c (consumer c fastest, gi = c's group index), so
// the consumers advance together; stage q lives in ring slot q % NS.
// Hand-off through two LDS flag arrays (values are stage numbers):
//   full[slot] = q  -- set by the producer once stage q has landed (its own
//                      vmcnt wait: loads retire in order);
//   done[slot] = q  -- set by the consumer when it has read stage q.
// The producer reuses a slot for stage q only after done[slot] == q - NS.
// Every wait is for a stage that is already issued (full) or already marked
// full (done), so all waves finish: the producer marks stage q - D right after
// issuing q, and waits only on stages numbered <= q - NS < q - D.
#include "q4k_mfma.h"

namespace tiermm {
namespace {

__device__ __forceinline__ int lds_acquire(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_release(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Marks the stages still in flight as they land: with `total - marked`
// outstanding, the oldest has landed once at most R younger ones are.
template <int R, int NLD, int NS>
__device__ __forceinline__ void drain(int total, int& marked, int* full) {
  if constexpr (R >= 0) {
    if (total - marked > R) {
      vm_wait<NLD * R>();
      lds_release(&full[marked % NS], marked);
      ++marked;
    }
    drain<R - 1, NLD, NS>(total, marked, full);
  }
}

// CT row tiles x CK K-splits = NC consumer waves, plus NP producer waves
// (waves NC..NC+NP-1); producer p serves consumers c with c % NP == p through
// a ring of its own.
template <int CT, int CK, int NP, int GS, int NS, int D, int XP, int XK>
__global__ __launch_bounds__(64 * (CT * CK + NP)) void qgemv_q4k_ws(const uint8_t* __restrict__ W, size_t rb,
                                                                 const float* __restrict__ x,
                                                                 float* __restrict__ y, int N, int K) {
  static_assert(D >= 1 && NS > D, "ring deeper than the loads in flight");
  static_assert(Stage<GS>::NLD * D <= 63, "vmcnt counts at most 63 loads");
  constexpr int NC = CT * CK, NL = NC / NP;  // NL consumers per producer
  static_assert(NC % NP == 0, "every producer serves the same number of consumers");
  static_assert(NC + NP <= 16, "at most 1024 threads per workgroup");
  constexpr int GRP = Stage<GS>::GRP, SBYTES = Stage<GS>::BYTES, NLD = Stage<GS>::NLD;
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // NP*NS*SBYTES + NC*64 + 2*NP*NS*4
  __shared__ __attribute__((aligned(16))) uint8_t xlds[xq_bytes(XK)];
  const int nsb_all = K >> 8;
  uint8_t* xq = xlds;
  float* meta = (float*)(xq + nsb_all * XQ_SB);
  uint8_t* zero = xq + nsb_all * (XQ_SB + META_SB);
  float* red = (float*)(ring + NP * NS * SBYTES);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // K split: consumer k of a tile takes super-blocks [sbk(k), sbk(k+1)); all
  // splits are given the same number of groups (short ones re-read and skip).
  const int ngrp = ((nsb_all + CK - 1) / CK + GS - 1) / GS;
  const int total = ngrp * NL;  // stages of one producer

  if (wave >= NC) {
    // ------------------------------------------------------------ producer
    const int p = wave - NC;
    int* full = (int*)(red + NC * 16) + 2 * NS * p;
    int* done = full + NS;
    if (lane < NS) {
      full[lane] = -1;
      done[lane] = -1;
    }
    // per-lane byte of the stage image: row and column within the group
    int roff[NLD], coff[NLD];
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int f = min(j * 1024 + lane * 16, SBYTES - 16);
      roff[j] = f / GRP;
      coff[j] = f % GRP;
    }
    const uint32_t ring_lds = lds_addr(ring + p * NS * SBYTES);
    auto issue = [&](int q) __attribute__((always_inline)) {
      const int c = (q % NL) * NP + p, gi = q / NL;
      const int t = c / CK, k = c % CK;
      const int row0 = (blockIdx.x * CT + t) * 16;
      const int rbase = min(row0, N - 1), rmax = min(15, N - 1 - rbase);
      const int sbk = k * nsb_all / CK, nsb = (k + 1) * nsb_all / CK - sbk;
      const uint8_t* base0 = W + (size_t)rbase * rb + (size_t)sbk * SB_BYTES;
      int ro[NLD];
#pragma unroll
      for (int j = 0; j < NLD; ++j) ro[j] = min(roff[j], rmax);
      load_group<GS>(base0, rb, ro, coff, lane, gi, nsb, ring_lds + (q % NS) * SBYTES);
    };
    const int pro = min(D, total);
    for (int q = 0; q < pro; ++q) issue(q);
    __syncthreads();  // flags initialised; consumers have prepared x
    int marked = 0;   // stages marked full so far
    for (int q = D; q < total; ++q) {
      if (q >= NS)
        while (lds_acquire(&done[q % NS]) != q - NS) __builtin_amdgcn_s_sleep(1);
      issue(q);
      vm_wait<NLD * D>();  // stage q - D has landed
      lds_release(&full[marked % NS], marked);
      ++marked;
    }
    // drain: the last min(D, total) stages, oldest first
    drain<D - 1, NLD, NS>(total, marked, full);
    __syncthreads();  // the consumers' partial sums are in red[]
    return;
  }

  // -------------------------------------------------------------- consumers
  const int c = wave, t = c / CK, k = c % CK;
  const int n = lane & 15, g = lane >> 4;
  const int* full = (const int*)(red + NC * 16) + 2 * NS * (c % NP);
  int* done = (int*)full + NS;
  const uint8_t* myring = ring + (c % NP) * NS * SBYTES;
  const int row0 = (blockIdx.x * CT + t) * 16;
  const int sbk = k * nsb_all / CK, nsb = (k + 1) * nsb_all / CK - sbk;
  constexpr int NT = 64 * NC;

  // x: one thread per 16 elements (threads past K/16 load a clamped copy and skip)
  u32x4 xr[XP][4];
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int hh = min(tid + j * NT, (K >> 4) - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[j][i] = *(const u32x4*)(x + hh * 16 + 4 * i);
  }
  for (int i = tid; i < ZERO_BYTES / 4; i += NT) ((uint32_t*)zero)[i] = 0u;
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int hh = tid + j * NT;
    if (hh < (K >> 4)) {
      float v[16];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) v[4 * i + w] = __uint_as_float(xr[j][i][w]);
      prep_half(hh >> 1, hh & 1, v, xq, meta);
    }
  }
  __syncthreads();

  uint32_t aoff[2], astep[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const bool live = (n >> 2) == 2 * (g >> 1) + p;
    aoff[p] = live ? (uint32_t)(sbk * XQ_SB + g * 64 + (n & 3) * 16) : (uint32_t)(zero - xlds);
    astep[p] = live ? (uint32_t)XQ_SB : 0u;
  }
  float acc = 0.f;
  for (int gi = 0; gi < ngrp; ++gi) {
    const int q = gi * NL + c / NP, slot = q % NS;
    while (lds_acquire(&full[slot]) != q) __builtin_amdgcn_s_sleep(1);
    const uint8_t* st = myring + slot * SBYTES;
#pragma unroll
    for (int i = 0; i < GS; ++i) {
      const int sb = GS * gi + i;
      if (sb < nsb)
        acc = q4k_superblock(st + n * GRP + i * SB_BYTES, g, xlds + aoff[0] + (uint32_t)sb * astep[0],
                             xlds + aoff[1] + (uint32_t)sb * astep[1], meta + (sbk + sb) * 16 + g * 4, acc);
    }
    lds_release(&done[slot], q);
  }

  acc += __shfl_xor(acc, 16, 64);
  acc += __shfl_xor(acc, 32, 64);
  if (g == 0) red[c * 16 + n] = acc;
  __syncthreads();
  if (k == 0 && g == 0) {
    float s = 0.f;
#pragma unroll
    for (int kk = 0; kk < CK; ++kk) s += red[(t * CK + kk) * 16 + n];
    if (row0 + n < N) y[row0 + n] = s;
  }
}

template <int CT, int CK, int NP, int GS, int NS, int D, int XP, int XK>
int launch_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  constexpr int NC = CT * CK;
  constexpr size_t lds = (size_t)NP * NS * Stage<GS>::BYTES + NC * 64 + 2 * NP * NS * 4;  // plus the static x digits
  static_assert(xq_bytes(XK) + lds <= 160 * 1024, "LDS budget");
  static_assert(XK / 16 <= 64 * NC * XP, "x preparation: one thread per 16 elements");
  const int tiles = (N + 15) / 16;
  const unsigned grid = (unsigned)((tiles + CT - 1) / CT);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)qgemv_q4k_ws<CT, CK, NP, GS, NS, D, XP, XK>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e, "tiermm_qgemv: q4_K LDS attribute");
    attr_set = true;
  }
  qgemv_q4k_ws<CT, CK, NP, GS, NS, D, XP, XK><<<grid, 64 * (NC + NP), lds, s>>>((const uint8_t*)W, rb, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_qgemv: q4_K launch");
  return TIERMM_OK;
}

}  // namespace

// Tall matrices (enough row tiles for every CU at four tiles per workgroup):
// 4 tiles x 2 K-halves of consumers and one producer per SIMD, each with a
// ring of four 2-super-block stages, two in flight.
int qgemv_q4k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  if (K <= 5120) return launch_ws<4, 2, 4, 2, 4, 2, 1, 5120>(W, rb, x, y, N, K, s);
  if (K <= 8192) return launch_ws<4, 2, 4, 2, 4, 2, 1, 8192>(W, rb, x, y, N, K, s);
  return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemv: q4_K K=%d above %d", K, 8192);
}

}  // namespace tiermm

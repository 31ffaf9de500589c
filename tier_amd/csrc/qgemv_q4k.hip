// qgemv_q4k.hip -- Q4_K decode GEMV on int8 MFMA (the north-star path), and
// Q5_K / Q8_0 on the same kernel (their per-super-block step in q4k_mfma.h).
//
// y[n] = sum_k q_val(W_n, k) * x[k] for Q4_K rows (gemv_q, tier.cpp:299-306),
// reorganised so the bulk of the work runs on v_mfma_i32_16x16x64_i8:
//
//   q_val = d*sc_s*q - dmin*m_s          (quant.h:83-84, s = 32-element sub-block)
//   y[n]  = sum_{super-block} [ d * sum_s sc_s * (q_s . x_s) - dmin * sum_s m_s * S_s ],
//   S_s   = sum of x over sub-block s.
//
// x is prepared once per workgroup: each 32-element sub-block gets a power of
// two 2^e_s that brings its max |x| into [2^28, 2^29); x_int = trunc(x*2^e_s)
// (exact for every element within 2^5 of the sub-block max, off by < 2^-28 of
// the max otherwise) is split into four signed int8 digits
// (x_int = l3*2^24 + l2*2^16 + l1*2^8 + l0), stored in LDS in MFMA A-operand
// order.  The integer dot (q_s . x_int_s) of each digit is exact; their fp32
// combination is scaled by 2^-e_s * sc_s * d.
//
// Weight stream.  A wave owns 16 rows and streams them front to back in groups
// of four super-blocks (576 bytes per row) with the gfx950 direct global->LDS
// load (global_load_lds_dwordx4).  A group of the 16 rows lands in LDS in
// row-major order (row n at n*576): load j brings bytes [1024j, 1024j+1024) of
// that 9 KiB image, lane l the 16 bytes at 1024j+16l, so each load reads one or
// two contiguous row segments and every byte is read once.  Each wave keeps
// STAGES groups in flight in its own LDS ring, so the memory stream runs ahead
// of the compute without holding registers.
//
// MFMA layout (16x16x64; lane group g = lane/16 supplies 16 k values):
//   B (weights): lane (n, g) reads qs chunks g and g+4 (qs bytes 16g.. and
//     64+16g..) of row n's super-block from LDS; MFMA t=0/1 take the low/high nibbles of chunk g, t=2/3 those of
//     chunk g+4.  Chunk a holds elements 64(a/2) + 16(a%2) + [0,16) in its low
//     nibbles (sub-block 2(a/2)) and the same +32 in its high nibbles; chunk
//     a+4 the same plus 128.
//   A (x digits): row r = 4*sigma + digit.  Lane (r, g) gives digit r%4 of the
//     x values lane group g covers when sigma == 2(g/2) + (t&1), zeros else.
//   C: MFMAs t=0,1 accumulate into Ca, t=2,3 into Cb; lane (n, g) ends with
//     Ca[4g + digit][n] (sub-block g) and Cb[4g + digit][n] (sub-block 4+g).
// The epilogue per super-block applies d, dmin and the 6-bit scales/mins of
// sub-blocks g and 4+g; partial sums are reduced over the four lane groups.
#include "q4k_mfma.h"

namespace tiermm {
namespace {


// RT row tiles of 16 rows per block; KS waves per row tile, each streaming a
// contiguous range of super-blocks (K split) in groups of GS super-blocks;
// STAGES groups in flight per wave; XP x half-sub-blocks per thread at most;
// XK the largest K (sizes the x-digit LDS object -- a static object of its own,
// so the compiler can tell it apart from the DMA ring).
template <int QT, int RT, int KS, int GS, int STAGES, int XP, int XK>
__global__ __launch_bounds__(64 * RT * KS) void qgemv_q4k_mfma(const uint8_t* __restrict__ W, size_t rb,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int N, int K) {
  using F = MfmaFmt<QT>;
  using St = Stage<GS, F::SBB>;
  constexpr int NT = 64 * RT * KS;
  constexpr int GRP = St::GRP, SBYTES = St::BYTES, NLD = St::NLD;
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // RT*KS*STAGES*SBYTES + RT*KS*64
  __shared__ __attribute__((aligned(16))) uint8_t xlds[xq_bytes(XK)];
  const int nsb_all = K >> 8;
  uint8_t* xq = xlds;                                      // nsb_all * XQ_SB
  float* meta = (float*)(xq + nsb_all * XQ_SB);            // nsb_all * META_SB
  uint8_t* zero = xq + nsb_all * (XQ_SB + META_SB);        // ZERO_BYTES

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rt = wave / KS, kp = wave % KS;
  const int n = lane & 15, g = lane >> 4;
  const int row0 = (blockIdx.x * RT + rt) * 16;
  // this wave's K range: super-blocks [sbk, sbk + nsb)
  const int sbk = kp * nsb_all / KS, nsb = (kp + 1) * nsb_all / KS - sbk;
  // per-lane DMA source: row (clamped to N-1) and byte within the group image
  const int rbase = min(row0, N - 1);                  // a tile past N re-reads row N-1
  const int rmax = min(15, N - 1 - rbase);
  const uint8_t* base0 = W + (size_t)rbase * rb + (size_t)sbk * F::SBB;
  int roff[NLD], coff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int f = min(j * 1024 + lane * 16, SBYTES - 16);
    roff[j] = min(f / GRP, rmax);
    coff[j] = f % GRP;
  }
  uint8_t* myring = ring + wave * STAGES * SBYTES;
  float* red = (float*)(ring + RT * KS * STAGES * SBYTES);
  const int ngrp = (nsb + GS - 1) / GS;

  // ---- x first, then the first STAGES-1 groups of weights; the x preparation
  // overlaps their latency.  x (K floats, the size of the digit area xq) comes into
  // xq by the same LDS DMA, 1 KiB per load spread over the waves; each wave waits for
  // its own x loads (they are older than its weight loads), a barrier for everyone's.
  // One thread per 16 elements of x (threads past K/16 read a clamped copy and skip
  // the preparation).
  const uint32_t ring_lds = lds_addr(myring);
  for (int j = wave; j < nsb_all; j += RT * KS) dma16(x + 256 * j + 4 * lane, lds_addr(xq) + 1024 * j);
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p)
    load_group<GS, F::SBB>(base0, rb, roff, coff, lane, p, nsb, ring_lds + p * SBYTES);
  vm_wait<NLD * (STAGES - 1)>();  // this wave's x has landed; the weight groups stay in flight
  __syncthreads();                // every wave's
  u32x4 xr[XP][4];
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int hh = min(tid + j * NT, (K >> 4) - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[j][i] = *(const u32x4*)(xq + 64 * hh + 16 * i);
  }
  __syncthreads();  // x is in registers: the digits may overwrite it

  __shared__ int nf[RT * KS];  // per wave: x held a non-finite value
  for (int i = tid; i < ZERO_BYTES / 4; i += NT) ((uint32_t*)zero)[i] = 0u;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int hh = tid + j * NT;  // K/16 is even: both threads of a pair are in range together
    if (hh < (K >> 4)) {
      float v[16];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) v[4 * i + w] = __uint_as_float(xr[j][i][w]);
      bad |= nonfinite16(v);
      prep_half(hh >> 1, hh & 1, v, xq, meta);
    }
  }
  publish_nonfinite(bad, nf, wave, lane);
  __syncthreads();
  const bool xbad = flags_any(nf, RT * KS);  // uniform over the workgroup

  // ---- per-lane constants
  // A operand: digits of virtual group g, live for MFMA parity p when n/4 == 2(g/2)+p.
  uint32_t aoff[2], astep[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const bool live = (n >> 2) == 2 * (g >> 1) + p;
    aoff[p] = live ? (uint32_t)(sbk * XQ_SB + g * 64 + (n & 3) * 16) : (uint32_t)(zero - xlds);
    astep[p] = live ? (uint32_t)XQ_SB : 0u;
  }
  float acc = 0.f;

  auto superblock = [&](const uint8_t* st, int i, int sb) __attribute__((always_inline)) {
    acc = F::step(st + n * GRP + i * F::SBB, g, xlds + aoff[0] + (uint32_t)sb * astep[0],
                         xlds + aoff[1] + (uint32_t)sb * astep[1], meta + (sbk + sb) * 16 + g * 4, acc);
  };

  for (int grp = 0; grp < ngrp; ++grp) {
    // keep STAGES-1 groups in flight: issue group grp+STAGES-1, then wait for grp.
    // Past the last group nothing is issued, and the wait leaves in flight only the
    // groups after grp (no re-reads whose latency the wave would wait out at its end).
    if (grp + STAGES - 1 < ngrp) {
      load_group<GS, F::SBB>(base0, rb, roff, coff, lane, grp + STAGES - 1, nsb,
                             ring_lds + ((grp + STAGES - 1) % STAGES) * SBYTES);
      vm_wait<NLD * (STAGES - 1)>();  // group grp has landed in its stage
    } else {
      const int left = ngrp - 1 - grp;  // groups issued after grp, at most STAGES - 2
      if (STAGES > 2 && left == 1) vm_wait<(STAGES > 2 ? NLD : 0)>();
      else if (STAGES > 3 && left == 2) vm_wait<(STAGES > 3 ? 2 * NLD : 0)>();
      else vm_wait<0>();
    }
    const uint8_t* st = myring + (grp % STAGES) * SBYTES;
    if (GS * grp + GS <= nsb) {
#pragma unroll
      for (int i = 0; i < GS; ++i) superblock(st, i, GS * grp + i);
    } else {
#pragma unroll
      for (int i = 0; i < GS; ++i)
        if (GS * grp + i < nsb) superblock(st, i, GS * grp + i);
    }
  }
  vm_wait<0>();  // every load has landed (the prologue's re-reads of short K parts too)

  if (xbad) {  // NaN or +-Inf in x: the workgroup's rows take gemv_q's non-finite sums
    for (int r = wave; r < RT * 16; r += RT * KS) {
      const int row = blockIdx.x * RT * 16 + r;
      if (row < N) {
        const float s = nonfinite_terms<QT>(W + (size_t)row * rb, x, 0, K, lane);
        if (lane == 0) y[row] = s;
      }
    }
    return;
  }

  // ---- reduce over the four lane groups of a row, then over the KS waves
  acc = row_sum4(acc);
  if (KS > 1) {
    if (g == 0) red[wave * 16 + n] = acc;
    __syncthreads();
    if (kp == 0 && g == 0) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < KS; ++k) t += red[(rt * KS + k) * 16 + n];
      if (row0 + n < N) y[row0 + n] = t;
    }
  } else if (g == 0 && row0 + n < N) {
    y[row0 + n] = acc;
  }
}

template <int QT, int RT, int KS, int GS, int STAGES, int XP, int XK>
int launch(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  constexpr size_t lds = (size_t)RT * KS * (STAGES * Stage<GS, MfmaFmt<QT>::SBB>::BYTES + 64);  // plus the static x digits
  static_assert(xq_bytes(XK) + 4 * RT * KS + lds <= 160 * 1024, "LDS budget (x digits, flags, ring)");
  static_assert(XK / 16 <= 64 * RT * KS * XP, "x preparation: one thread per 16 elements");
  const int tiles = (N + 15) / 16;
  const unsigned grid = (unsigned)((tiles + RT - 1) / RT);
  static std::atomic<uint64_t> attr{0};  // dynamic LDS above 64 KiB is opted into per device
  int st = lds_attr_once(attr, (const void*)qgemv_q4k_mfma<QT, RT, KS, GS, STAGES, XP, XK>, (int)lds,
                         "tiermm_qgemv: q4_K LDS attribute");
  if (st) return st;
  qgemv_q4k_mfma<QT, RT, KS, GS, STAGES, XP, XK><<<grid, 64 * RT * KS, lds, s>>>((const uint8_t*)W, rb, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_qgemv: q4_K launch");
  return TIERMM_OK;
}

}  // namespace

// Largest K handled (the x digits of the whole row stay in LDS: 121 KiB at this K,
// with the weight ring in the remaining 39 KiB).
constexpr int kQ4kMaxK = 28672;

// Launch shapes by measurement (MI355X; 200 launches over rotated copies).  At
// most one row tile per CU: one tile per workgroup, K in four parts (q8_0
// 4096x4096: 5.7 against 8.0 us).  Many row tiles: eight waves per workgroup
// (q5_K 13824x5120: 11.7 against 15.1 us; q8_0 14336x14336: 41.5 against 46.6 us).
int qgemv_q4k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  if (K > kQ4kMaxK) return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemv: q4_K K=%d above %d", K, kQ4kMaxK);
  const int tiles = (N + 15) / 16;
  // 257..639 row tiles (taller ones take the whole-tile kernel): two tiles x four K
  // parts per workgroup (q4_K 5120x5120: 5.6 against 6.4 us; 10000x5120: 9.0 against
  // 10.2; 4608x8192: 6.6 against 8.4)
  if (K <= 5120) {
    if (tiles <= 256) return launch<QT_Q4_K, 1, 4, 1, 3, 2, 5120>(W, rb, x, y, N, K, s);
    return launch<QT_Q4_K, 2, 4, 1, 2, 1, 5120>(W, rb, x, y, N, K, s);
  }
  if (K <= 8192) {
    if (tiles <= 256) return launch<QT_Q4_K, 2, 2, 2, 3, 2, 8192>(W, rb, x, y, N, K, s);
    return launch<QT_Q4_K, 2, 4, 2, 2, 1, 8192>(W, rb, x, y, N, K, s);
  }
  // K above 14336: eight waves (two tiles x four K parts), one super-block per stage
  if (K > 14336) return launch<QT_Q4_K, 2, 4, 1, 2, 4, 28672>(W, rb, x, y, N, K, s);
  if (tiles >= 640) return launch<QT_Q4_K, 4, 1, 4, 2, 4, 14336>(W, rb, x, y, N, K, s);  // 24.2 against 25.5 us
  // up to one tile per CU: one tile, K in eight parts (4096x14336: 9.4-9.6 against 11.7 us;
  // 1024x14336: 7.1 against 9.4 us)
  if (tiles <= 256) return launch<QT_Q4_K, 1, 8, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);
  return launch<QT_Q4_K, 2, 4, 2, 2, 2, 14336>(W, rb, x, y, N, K, s);
}

// Q5_K (176-byte super-blocks) and Q8_0 (groups of eight 34-byte blocks) on the
// same kernel: K a multiple of 256 up to kQ4kMaxK, rows and base 16-byte aligned.
bool qgemv_mfma_fits(const void* W, int qtype, size_t rb, int K) {
  return (qtype == QT_Q5_K || qtype == QT_Q8_0) && K % 256 == 0 && K <= kQ4kMaxK && rb % 16 == 0 &&
         ((uintptr_t)W % 16) == 0;
}

int qgemv_mfma(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  const int tiles = (N + 15) / 16;
  if (qtype == QT_Q5_K) {
    if (K <= 5120) {
      if (tiles <= 256) return launch<QT_Q5_K, 1, 4, 1, 3, 2, 5120>(W, rb, x, y, N, K, s);
      if (tiles < 640) return launch<QT_Q5_K, 2, 4, 1, 2, 2, 5120>(W, rb, x, y, N, K, s);
      return launch<QT_Q5_K, 4, 2, 2, 2, 2, 5120>(W, rb, x, y, N, K, s);
    }
    if (K <= 8192) {
      if (tiles < 640) return launch<QT_Q5_K, 2, 2, 2, 3, 2, 8192>(W, rb, x, y, N, K, s);
      return launch<QT_Q5_K, 4, 2, 2, 2, 2, 8192>(W, rb, x, y, N, K, s);
    }
    if (K > 14336) return launch<QT_Q5_K, 2, 3, 1, 2, 5, 28672>(W, rb, x, y, N, K, s);  // six waves fit the ring
    if (tiles >= 640) return launch<QT_Q5_K, 4, 2, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);
    if (tiles <= 256) return launch<QT_Q5_K, 1, 8, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);  // 4096x14336: 11.0 against 13.8 us
    return launch<QT_Q5_K, 2, 4, 2, 2, 2, 14336>(W, rb, x, y, N, K, s);
  }
  if (K <= 5120) {
    // 2048x4096: 4.4 against 5.1 us with K in four parts
    if (tiles <= 256) return launch<QT_Q8_0, 1, 8, 1, 2, 1, 5120>(W, rb, x, y, N, K, s);
    if (tiles < 640) return launch<QT_Q8_0, 2, 2, 1, 3, 2, 5120>(W, rb, x, y, N, K, s);
    return launch<QT_Q8_0, 4, 2, 2, 2, 2, 5120>(W, rb, x, y, N, K, s);
  }
  if (K <= 8192) {
    if (tiles < 640) return launch<QT_Q8_0, 2, 2, 1, 3, 2, 8192>(W, rb, x, y, N, K, s);
    return launch<QT_Q8_0, 4, 2, 1, 2, 2, 8192>(W, rb, x, y, N, K, s);
  }
  if (K > 14336) return launch<QT_Q8_0, 1, 4, 1, 2, 7, 28672>(W, rb, x, y, N, K, s);  // four waves fit the ring
  if (tiles >= 640) return launch<QT_Q8_0, 4, 2, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);
  // 1024x14336: 9.3 against 16.7 us; 4096x14336: 14.5 against 18.9 us
  if (tiles <= 256) return launch<QT_Q8_0, 1, 8, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);
  return launch<QT_Q8_0, 2, 2, 2, 2, 4, 14336>(W, rb, x, y, N, K, s);
}

}  // namespace tiermm

// qgemv_q6k.hip -- Q6_K decode GEMV on int8 MFMA (gemv_q, tier.cpp:299-306).
//
// q_val of Q6_K (quant.h:88-90): element e of a 210-byte super-block is
//   d * sc[e/16] * (q6 - 32),  q6 = low/high nibble of ql | two bits of qh,
// with int8 scales per 16 elements.  The x preparation and its LDS layout are
// those of the Q4_K kernels (q4k_mfma.h: per 32-element sub-block a power of two
// and four balanced int8 digits), and so is the element each lane feeds to each
// MFMA step t: lane group g supplies elements 16(g&1) + [0,16) of sub-block
// sg = 4(t>>1) + 2(g>>1) + (t&1).  Two things differ:
//   * the scales cover 16 elements, so the A rows of lane group g's digits are
//     live only in C rows 4g..4g+3: C[4g + digit][n] of step t is the digit dot
//     of row n's 16 elements of lane group g, and each step has its own C;
//   * a 210-byte super-block leaves rows and super-blocks 2-byte aligned: each
//     row segment of a stage is loaded from a dword boundary at most 14 bytes
//     below its start into a row pitch that holds the shift (chosen so that the
//     16 rows of a tile sit at four dword phases, which keeps the row-strided LDS
//     reads free of bank conflicts), and the weights are read from LDS as
//     aligned dwords joined with v_alignbit.
// B: lane (n, g) in step t takes ql bytes 64(t>>1) + 32(t&1) + 16(g&1) + [0,16)
// (low nibbles for g < 2, high for g >= 2) and qh bytes 128 + 32(t>>1) +
// 16(g&1) + [0,16) (bits 4(g>>1) + 2(t&1) and the next), i.e. q6 itself (0..63)
// as int8; its scale is sc[8(t>>1) + 4(g>>1) + 2(t&1) + (g&1)].  The - 32 is
// taken off the int32 digit dots: q6 in place of q6 - 32 adds 32 T_l to digit
// row l, T_l = the sum of digit l over the lane group's 16 elements, which the
// x preparation stores (prep_half<true>), so the dots and the result are those
// of q6 - 32 exactly.
#include "q4k_mfma.h"

namespace tiermm {
namespace {

constexpr int Q6_SBB = 210;
constexpr int xq6_bytes(int kmax) { return xq_bytes(kmax) + (kmax / 256) * 128; }  // + the digit sums

// GS super-blocks of each of 16 rows; a row's bytes start up to 14 bytes into
// its pitch.
template <int GS>
struct Q6Stage {
  static constexpr int PITCH = (GS * Q6_SBB + 14 + 15) / 16 * 16;
  static constexpr int BYTES = 16 * PITCH;
  static constexpr int NLD = (BYTES + 1023) / 1024;
  static constexpr int LAST = (BYTES - (NLD - 1) * 1024) / 16;  // lanes of the last load
};

// The 128 bits that start sh bits (< 32) into the aligned dword q: five dwords
// joined with v_alignbit, so a shift below 32 bits is free.
__device__ __forceinline__ u32x4 lds16_dw(const uint32_t* q, uint32_t sh) {
  const uint32_t v0 = q[0], v1 = q[1], v2 = q[2], v3 = q[3], v4 = q[4];
  return u32x4{__builtin_amdgcn_alignbit(v1, v0, sh), __builtin_amdgcn_alignbit(v2, v1, sh),
               __builtin_amdgcn_alignbit(v3, v2, sh), __builtin_amdgcn_alignbit(v4, v3, sh)};
}

// q6 of four weights as bytes: the nibble at bits 0..3 of each ql byte, the two
// qh bits at bits 4..5 of each qh byte (both words read with those shifts).
__device__ __forceinline__ int q6_bytes(uint32_t ql, uint32_t qh) {
  return (int)((ql & 0x0f0f0f0fu) | (qh & 0x30303030u));
}

// One super-block (at LDS byte offset off of base) of row n for lane group g:
// mb = the x meta of the super-block (2^-e at [4*(sg&3) + (sg>>2)]), ap = this
// lane's A digits of the super-block (step t at +t*XQ_T), dp = lane group g's
// digit-sum terms of the super-block (step t at 2t, 2t+1).
__device__ __forceinline__ float q6k_superblock(const uint8_t* base, uint32_t off, int g, const uint8_t* ap,
                                                const float* mb, const int* dp, float acc) {
  // ql read 4(g>>1) bits late (the high nibbles at bits 0..3 for g >= 2); qh read
  // so that bits 4(g>>1) + {0, 1} of each byte sit at bits 4..5 (step t&1 = 0),
  // two more bits down for t&1 = 1
  const uint32_t* dw = (const uint32_t*)base;
  const uint32_t lbit = 8 * (off + 16 * (g & 1)) + 4 * (g >> 1);  // ql of step 0
  const uint32_t hbit = lbit + 8 * 128 - 4;                        // qh of step 0
  const uint32_t* lq = dw + (lbit >> 5);
  const uint32_t* hq = dw + (hbit >> 5);
  i32x4 B[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // h = t >> 1: the 128-element half
    const u32x4 qh = lds16_dw(hq + 8 * h, hbit & 31u);
#pragma unroll
    for (int p = 0; p < 2; ++p) {  // p = t & 1
      const u32x4 ql = lds16_dw(lq + 16 * h + 8 * p, lbit & 31u);
#pragma unroll
      for (int w = 0; w < 4; ++w) B[2 * h + p][w] = q6_bytes(ql[w], p ? qh[w] >> 2 : qh[w]);
    }
  }
  const i32x4 z = {0, 0, 0, 0};
  i32x4 C[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) C[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const i32x4*)(ap + t * XQ_T), B[t], z, 0, 0, 0);
  // scales: bytes 4(g>>1) + (g&1) + {0, 2} (t = 0, 1) and 8 more (t = 2, 3)
  const u32x4 S = lds16_dw(dw + (off >> 2) + 48, 8 * (off & 3u));
  const uint32_t s01 = ((g >> 1) ? S[1] : S[0]) >> (8 * (g & 1));
  const uint32_t s23 = ((g >> 1) ? S[3] : S[2]) >> (8 * (g & 1));
  const int sc[4] = {(int)(s01 << 24) >> 24, (int)(s01 << 8) >> 24, (int)(s23 << 24) >> 24, (int)(s23 << 8) >> 24};
  const float d = h2f(*(const uint16_t*)(base + off + 208));
  const float2 f02 = *(const float2*)(mb + 8 * (g >> 1)), f13 = *(const float2*)(mb + 8 * (g >> 1) + 4);
  const float f[4] = {f02.x, f13.x, f02.y, f13.y};
  const i32x4 T01 = *(const i32x4*)dp, T23 = *(const i32x4*)(dp + 4);
  const int th[4] = {T01[0], T01[2], T23[0], T23[2]}, tl[4] = {T01[1], T01[3], T23[1], T23[3]};
  float u = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    // the digit dots of q6 - 32 (|C| <= 16*32*128): the int32 halves are exact,
    // their conversion rounds at most once
    const float D = fmaf((float)(C[t][3] * 256 + C[t][2] - th[t]), 65536.f, (float)(C[t][1] * 256 + C[t][0] - tl[t]));
    u = fmaf((float)sc[t] * f[t], D, u);
  }
  return fmaf(d, u, acc);
}

// RT row tiles of 16 rows per block; KS waves per row tile over contiguous
// super-block ranges; GS super-blocks per stage, STAGES stages in flight; XP x
// half-sub-blocks per thread at most; XK the largest K.
template <int RT, int KS, int GS, int STAGES, int XP, int XK>
__global__ __launch_bounds__(64 * RT * KS) void qgemv_q6k_mfma(const uint8_t* __restrict__ W, size_t rb,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int N, int K) {
  // W + N*rb is 16-byte aligned (qgemv_q6k_fits).  Row N-1 is loaded from
  // 16-byte aligned windows, so its loads end within W and the clamp below moves
  // none that brings needed bytes; the other rows' windows end at most 30 bytes
  // past their segment, inside W, and are never clamped
  using St = Q6Stage<GS>;
  constexpr int NT = 64 * RT * KS, PITCH = St::PITCH, SBYTES = St::BYTES, NLD = St::NLD;
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // RT*KS*STAGES*SBYTES + RT*KS*64
  __shared__ __attribute__((aligned(16))) uint8_t xlds[xq6_bytes(XK)];
  const int nsb_all = K >> 8;
  uint8_t* xq = xlds;
  float* meta = (float*)(xq + nsb_all * XQ_SB);
  uint8_t* zero = xq + nsb_all * (XQ_SB + META_SB);
  int* dsum = (int*)(zero + ZERO_BYTES);  // 32 ints per super-block

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rt = wave / KS, kp = wave % KS;
  const int n = lane & 15, g = lane >> 4;
  const int row0 = (blockIdx.x * RT + rt) * 16;
  const int sbk = kp * nsb_all / KS, nsb = (kp + 1) * nsb_all / KS - sbk;
  const int rbase = min(row0, N - 1);  // a tile past N re-reads row N-1
  const int rmax = min(15, N - 1 - rbase);
  const int ngrp = (nsb + GS - 1) / GS;
  // DMA: load j brings bytes [1024j, 1024j + 1024) of the stage image, lane l
  // the 16 at 1024j + 16l: image row r = f / PITCH, byte f % PITCH of the window
  // that holds the row's segment.  The window starts 4(r/4 % 4) bytes below the
  // dword that holds the segment start, so that the 16 rows a lane group reads
  // at one column sit at four dword phases and spread over the LDS banks (rows at
  // one phase meet four to a bank); row N-1 keeps the 16-byte aligned window.
  const uint8_t* lrow[NLD];
  int lcol[NLD], lph[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int f = min(j * 1024 + lane * 16, SBYTES - 16);
    const int r = f / PITCH, row = rbase + min(r, rmax);
    lrow[j] = W + (size_t)row * rb + (size_t)sbk * Q6_SBB;
    lcol[j] = f % PITCH;
    lph[j] = row == N - 1 ? -1 : 4 * ((r >> 2) & 3);
  }
  const uint8_t* wlast = W + (size_t)N * rb - 16;
  auto load = [&](int grp, uint32_t stage) __attribute__((always_inline)) {
    const int gc = max(0, min(grp, ngrp - 1));  // past the end: re-load the last group
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      if (j < NLD - 1 || St::LAST == 64 || lane < St::LAST) {
        const uint8_t* seg = lrow[j] + (size_t)gc * GS * Q6_SBB;
        const uint8_t* win = lph[j] < 0 ? (const uint8_t*)((uintptr_t)seg & ~(uintptr_t)15)
                                        : (const uint8_t*)((uintptr_t)seg & ~(uintptr_t)3) - lph[j];
        dma16(min(win + lcol[j], wlast), stage + j * 1024);
      }
    }
  };
  uint8_t* myring = ring + wave * STAGES * SBYTES;
  float* red = (float*)(ring + RT * KS * STAGES * SBYTES);
  // this lane's row segment (image row n) starts shift bytes into its window:
  // 4(n/4 % 4) + its start's offset in a dword, or for row N-1 the offset in 16 bytes
  const int nrow = rbase + min(n, rmax);
  const uint32_t shift0 = (uint32_t)((uintptr_t)(W + (size_t)nrow * rb + (size_t)sbk * Q6_SBB) & 15);
  const uint32_t smask = nrow == N - 1 ? 15u : 3u, sph = nrow == N - 1 ? 0u : 4u * ((n >> 2) & 3);

  // ---- x, the first STAGES-1 groups, then the x preparation.  x (K floats, the
  // size of the digit area xq) comes into xq by the same LDS DMA, 1 KiB per load spread
  // over the waves; each wave waits for its own x loads (older than its weight loads),
  // a barrier for everyone's.
  const uint32_t ring_lds = lds_addr(myring);
  for (int j = wave; j < nsb_all; j += RT * KS) dma16(x + 256 * j + 4 * lane, lds_addr(xq) + 1024 * j);
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p) load(p, ring_lds + p * SBYTES);
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
    const int hh = tid + j * NT;
    if (hh < (K >> 4)) {
      float v[16];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) v[4 * i + w] = __uint_as_float(xr[j][i][w]);
      bad |= nonfinite16(v);
      prep_half<true>(hh >> 1, hh & 1, v, xq, meta, dsum);
    }
  }
  publish_nonfinite(bad, nf, wave, lane);
  __syncthreads();
  const bool xbad = flags_any(nf, RT * KS);  // uniform over the workgroup

  // A operand: lane (n, g) gives digit n%4 of lane group g's elements when n/4 == g
  const bool live = (n >> 2) == g;
  const uint32_t aoff = live ? (uint32_t)(sbk * XQ_SB + g * 64 + (n & 3) * 16) : (uint32_t)(zero - xlds);
  const uint32_t astep = live ? (uint32_t)XQ_SB : 0u;
  float acc = 0.f;

  for (int grp = 0; grp < ngrp; ++grp) {
    load(grp + STAGES - 1, ring_lds + ((grp + STAGES - 1) % STAGES) * SBYTES);
    vm_wait<NLD * (STAGES - 1)>();  // group grp has landed in its stage
    const uint32_t st = (uint32_t)(wave * STAGES + grp % STAGES) * SBYTES;
    const uint32_t rowoff = st + n * PITCH + sph + ((shift0 + 2u * GS * grp) & smask);  // 210 = 2 mod 16
#pragma unroll
    for (int i = 0; i < GS; ++i) {
      const int sb = GS * grp + i;
      if (GS == 1 || sb < nsb)
        acc = q6k_superblock(ring, rowoff + i * Q6_SBB, g, xlds + aoff + (uint32_t)sb * astep,
                             meta + (sbk + sb) * 16, dsum + (sbk + sb) * 32 + 8 * g, acc);
    }
  }
  vm_wait<0>();  // drain the re-loads past the end before the wave ends

  if (xbad) {  // NaN or +-Inf in x: the workgroup's rows take gemv_q's non-finite sums
    for (int r = wave; r < RT * 16; r += RT * KS) {
      const int row = blockIdx.x * RT * 16 + r;
      if (row < N) {
        const float s = nonfinite_terms<QT_Q6_K>(W + (size_t)row * rb, x, 0, K, lane);
        if (lane == 0) y[row] = s;
      }
    }
    return;
  }

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

template <int RT, int KS, int GS, int STAGES, int XP, int XK>
int launch(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  constexpr size_t lds = (size_t)RT * KS * (STAGES * Q6Stage<GS>::BYTES + 64);  // plus the static x digits
  static_assert(xq6_bytes(XK) + 4 * RT * KS + lds <= 160 * 1024, "LDS budget (x digits, flags, ring)");
  static_assert(XK / 16 <= 64 * RT * KS * XP, "x preparation: one thread per 16 elements");
  static_assert(Q6Stage<GS>::NLD * (STAGES - 1) <= 63, "vmcnt counts at most 63 loads");
  const int tiles = (N + 15) / 16;
  const unsigned grid = (unsigned)((tiles + RT - 1) / RT);
  static std::atomic<uint64_t> attr{0};
  int st = lds_attr_once(attr, (const void*)qgemv_q6k_mfma<RT, KS, GS, STAGES, XP, XK>, (int)lds,
                         "tiermm_qgemv: q6_K LDS attribute");
  if (st) return st;
  qgemv_q6k_mfma<RT, KS, GS, STAGES, XP, XK><<<grid, 64 * RT * KS, lds, s>>>((const uint8_t*)W, rb, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_qgemv: q6_K launch");
  return TIERMM_OK;
}

}  // namespace

// K a multiple of 256 up to 14336, W and its end 16-byte aligned (rows may start
// at any even byte).
bool qgemv_q6k_fits(const void* W, size_t rb, int N, int K) {
  return K % 256 == 0 && K <= 14336 && ((uintptr_t)W % 16) == 0 && ((size_t)N * rb) % 16 == 0;
}

// Launch shapes by measurement (MI355X, fraction of 8 TB/s): eight waves per
// workgroup once there are more row tiles than CUs (13824x5120: 17.2 us against
// 21.6 us with four; 5120x14336: 23.1 against 40.4 us).
int qgemv_q6k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  const int tiles = (N + 15) / 16;
  if (K <= 5120) {
    if (tiles <= 256) return launch<1, 4, 1, 3, 2, 5120>(W, rb, x, y, N, K, s);
    if (tiles <= 512) return launch<2, 4, 1, 2, 2, 5120>(W, rb, x, y, N, K, s);
    return launch<4, 2, 1, 2, 2, 5120>(W, rb, x, y, N, K, s);
  }
  if (K <= 8192) {
    if (tiles < 640) return launch<2, 4, 1, 2, 2, 8192>(W, rb, x, y, N, K, s);
    return launch<4, 2, 1, 2, 2, 8192>(W, rb, x, y, N, K, s);
  }
  if (tiles <= 256) return launch<1, 8, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);  // 1024x14336: 13.2 against 21.8 us
  if (tiles < 640) return launch<2, 4, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);
  return launch<4, 2, 1, 2, 2, 14336>(W, rb, x, y, N, K, s);
}

}  // namespace tiermm

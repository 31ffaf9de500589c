// qgemv_q4k.hip -- Q4_K decode GEMV on int8 MFMA (the north-star path).
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
#include "tm_device.h"

namespace tiermm {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int SB_BYTES = 144;          // Q4_K super-block
constexpr int GRP_BYTES = 4 * SB_BYTES;  // one group of four super-blocks of a row (36 chunks)
constexpr int STAGE_BYTES = 16 * GRP_BYTES;  // one group of 16 rows in LDS: 9 loads x 64 lanes x 16 bytes
constexpr int XQ_SB = 1024;            // LDS bytes of x digits per super-block: 4 t x 4 a x 4 digits x 16
constexpr int XQ_T = 256;              // per MFMA step t
constexpr int META_SB = 64;            // 4 g x float4 (f_g, f_4+g, S_g, S_4+g)
constexpr int ZERO_BYTES = 4 * XQ_T;   // zero rows read by the A lanes that carry no digit

// Prepare x elements [16h, 16h+16) of sub-block s (h = half, values in v): the
// partner thread (lane ^ 1) holds the other half; both reach this together.
__device__ __forceinline__ void prep_half(int s, int h, const float (&v)[16], uint8_t* xq, float* meta) {
  float amax = 0.f, sum = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    amax = fmaxf(amax, fabsf(v[i]));
    sum += v[i];
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  sum += __shfl_xor(sum, 1, 64);
  int e = 0;
  if (amax > 0.f) {
    int ex;
    (void)frexpf(amax, &ex);
    e = min(126, max(-126, 29 - ex));
  }
  const int sb = s >> 3, sg = s & 7;              // super-block, sub-block within it
  const int t = 2 * (sg >> 2) + (sg & 1);         // MFMA step covering this sub-block
  const int a = 2 * ((sg & 3) >> 1) + h;          // virtual group of these 16 elements
  if (h == 0) {
    meta[sb * 16 + (sg & 3) * 4 + (sg >> 2)] = ldexpf(1.f, -e);
    meta[sb * 16 + (sg & 3) * 4 + 2 + (sg >> 2)] = sum;
  }
  // x_int = trunc(x * 2^e): |x * 2^e| < 2^29, integral already wherever it is
  // >= 2^23, otherwise off by < 1 unit (2^-28 of the sub-block max).
  // Balanced int8 digits of x_int: with y = x_int + 0x808080, the digits are
  // bytes 0..2 of y with the top bit flipped and byte 3 of y.
  uint32_t yv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) yv[i] = (uint32_t)(int)ldexpf(v[i], e) + 0x00808080u;
  u32x4 L[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {  // 4x4 byte transpose of four elements
    const uint32_t y0 = yv[4 * w], y1 = yv[4 * w + 1], y2 = yv[4 * w + 2], y3 = yv[4 * w + 3];
    const uint32_t p01l = __builtin_amdgcn_perm(y1, y0, 0x05010400u), p01h = __builtin_amdgcn_perm(y1, y0, 0x07030602u);
    const uint32_t p23l = __builtin_amdgcn_perm(y3, y2, 0x05010400u), p23h = __builtin_amdgcn_perm(y3, y2, 0x07030602u);
    L[0][w] = __builtin_amdgcn_perm(p23l, p01l, 0x05040100u) ^ 0x80808080u;
    L[1][w] = __builtin_amdgcn_perm(p23l, p01l, 0x07060302u) ^ 0x80808080u;
    L[2][w] = __builtin_amdgcn_perm(p23h, p01h, 0x05040100u) ^ 0x80808080u;
    L[3][w] = __builtin_amdgcn_perm(p23h, p01h, 0x07060302u);
  }
  uint8_t* dst = xq + sb * XQ_SB + t * XQ_T + a * 64;
#pragma unroll
  for (int l = 0; l < 4; ++l) *(u32x4*)(dst + 16 * l) = L[l];
}

// Vector-memory traffic of this kernel is issued and waited for by hand: the
// compiler's wait insertion cannot follow global->LDS loads (it falls back to
// waiting for everything before LDS reads), which would serialise the weight
// stream.  Every vector load below is one instruction per wave regardless of
// the lane mask, and loads retire in order, so "s_waitcnt vmcnt(N)" means all
// but the N most recent ones have landed.
__device__ __forceinline__ u32x4 gload16(const void* p) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
// 16 bytes per lane from p into LDS at lds_addr + 16*lane (lds_addr wave-uniform, through M0).
__device__ __forceinline__ void dma16(const void* p, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(p),
               "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Async loads of group `grp` of this wave's 16 rows into an LDS stage in
// row-major order.  roff[j] / coff[j]: row (0..15) and byte (0..575) of the
// 16 bytes lane `lane` brings with load j; bytes past the wave's K range re-read
// the last valid 16 bytes of the row segment, so the number of loads is fixed.
__device__ __forceinline__ void load_group(const uint8_t* base0, size_t rb, const int (&roff)[9],
                                           const int (&coff)[9], int grp, int nsb, uint32_t stage) {
  const int valid = min(4, nsb - 4 * grp);
  const int lastb = valid > 0 ? SB_BYTES * valid - 16 : 0;
  const uint8_t* b = base0 + (size_t)max(0, min(grp, (nsb - 1) >> 2)) * GRP_BYTES;
#pragma unroll
  for (int j = 0; j < 9; ++j) dma16(b + (size_t)roff[j] * rb + min(coff[j], lastb), stage + j * 1024);
}

constexpr int xq_bytes(int kmax) { return (kmax / 256) * (XQ_SB + META_SB) + ZERO_BYTES; }

// RT row tiles of 16 rows per block; KS waves per row tile, each streaming a
// contiguous range of super-blocks (K split); STAGES groups of four
// super-blocks in flight per wave; XP x half-sub-blocks per thread at most;
// XK the largest K (sizes the x-digit LDS object -- a static object of its own,
// so the compiler can tell it apart from the DMA ring).
template <int RT, int KS, int STAGES, int XP, int XK>
__global__ __launch_bounds__(64 * RT * KS) void qgemv_q4k_mfma(const uint8_t* __restrict__ W, size_t rb,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int N, int K) {
  constexpr int NT = 64 * RT * KS;
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // RT*KS*STAGES*STAGE_BYTES + RT*KS*64
  __shared__ __attribute__((aligned(16))) uint8_t xlds[xq_bytes(XK)];
  const int nsb_all = K >> 8;
  uint8_t* xq = xlds;                                      // nsb_all * XQ_SB
  float* meta = (float*)(xq + nsb_all * XQ_SB);            // nsb_all * META_SB
  uint8_t* zero = xq + nsb_all * (XQ_SB + META_SB);        // ZERO_BYTES

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rt = wave / KS, kp = wave % KS;
  const int n = lane & 15, g = lane >> 4;
  const int row0 = (blockIdx.x * RT + rt) * 16;
  // this wave's K range: super-blocks [sbk, sbk + nsb), in groups of four
  const int sbk = kp * nsb_all / KS, nsb = (kp + 1) * nsb_all / KS - sbk;
  // per-lane DMA source: row (clamped to N-1) and byte within the group image
  const int rbase = min(row0, N - 1);                  // a tile past N re-reads row N-1
  const int rmax = min(15, N - 1 - rbase);
  const uint8_t* base0 = W + (size_t)rbase * rb + (size_t)sbk * SB_BYTES;
  int roff[9], coff[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    const int f = j * 1024 + lane * 16;
    roff[j] = min(f / GRP_BYTES, rmax);
    coff[j] = f % GRP_BYTES;
  }
  uint8_t* myring = ring + wave * STAGES * STAGE_BYTES;
  float* red = (float*)(ring + RT * KS * STAGES * STAGE_BYTES);
  const int ngrp = (nsb + 3) >> 2;

  // ---- x loads first, then the first STAGES-1 groups of weights; the x
  // preparation overlaps their latency.  One thread per 16 elements of x
  // (threads past K/16 load a clamped copy and skip the preparation).
  const uint32_t ring_lds = lds_addr(myring);
  u32x4 xr[XP][4];
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int hh = min(tid + j * NT, (K >> 4) - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[j][i] = gload16(x + hh * 16 + 4 * i);
  }
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p) load_group(base0, rb, roff, coff, p, nsb, ring_lds + p * STAGE_BYTES);
  vm_wait<9 * (STAGES - 1)>();  // x has landed; the weight groups stay in flight
#pragma unroll
  for (int j = 0; j < XP; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(xr[j][i]));

  for (int i = tid; i < ZERO_BYTES / 4; i += NT) ((uint32_t*)zero)[i] = 0u;
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int hh = tid + j * NT;  // K/16 is even: both threads of a pair are in range together
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

  // ---- per-lane constants
  // A operand: digits of virtual group g, live for MFMA parity p when n/4 == 2(g/2)+p.
  uint32_t aoff[2], astep[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const bool live = (n >> 2) == 2 * (g >> 1) + p;
    aoff[p] = live ? (uint32_t)(sbk * XQ_SB + g * 64 + (n & 3) * 16) : (uint32_t)(zero - xlds);
    astep[p] = live ? (uint32_t)XQ_SB : 0u;
  }
  // B operand / header offsets inside a stage for super-block i of the group
  // (row n at n*576, super-block i at +144i: header, then qs)
  uint32_t qoff[4], hoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hoff[i] = (uint32_t)(n * GRP_BYTES + i * SB_BYTES);
    qoff[i] = hoff[i] + 16 + 16 * g;
  }
  const int sh = 8 * g;  // scale byte of sub-blocks g and 4+g (quant.h:47-48)
  float acc = 0.f;

  for (int grp = 0; grp < ngrp; ++grp) {
    // keep STAGES-1 groups in flight: issue group grp+STAGES-1 (a clamped re-read
    // past the end keeps the count of outstanding loads fixed), then wait for grp
    load_group(base0, rb, roff, coff, grp + STAGES - 1, nsb, ring_lds + ((grp + STAGES - 1) % STAGES) * STAGE_BYTES);
    vm_wait<9 * (STAGES - 1)>();  // group grp has landed in its stage
    const uint8_t* st = myring + (grp % STAGES) * STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sb = 4 * grp + i;
      if (sb < nsb) {
        const u32x4 H = *(const u32x4*)(st + hoff[i]);
        const u32x4 cA = *(const u32x4*)(st + qoff[i]);
        const u32x4 cB = *(const u32x4*)(st + qoff[i] + 64);
        const uint8_t* a0p = xlds + aoff[0] + (uint32_t)sb * astep[0];
        const uint8_t* a1p = xlds + aoff[1] + (uint32_t)sb * astep[1];
        const i32x4 A0 = *(const i32x4*)(a0p), A1 = *(const i32x4*)(a1p + XQ_T);
        const i32x4 A2 = *(const i32x4*)(a0p + 2 * XQ_T), A3 = *(const i32x4*)(a1p + 3 * XQ_T);
        i32x4 B0, B1, B2, B3;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          B0[w] = (int)(cA[w] & 0x0f0f0f0fu);
          B1[w] = (int)((cA[w] >> 4) & 0x0f0f0f0fu);
          B2[w] = (int)(cB[w] & 0x0f0f0f0fu);
          B3[w] = (int)((cB[w] >> 4) & 0x0f0f0f0fu);
        }
        const i32x4 z = {0, 0, 0, 0};
        i32x4 Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, z, 0, 0, 0);
        Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, Ca, 0, 0, 0);
        i32x4 Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, B2, z, 0, 0, 0);
        Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A3, B3, Cb, 0, 0, 0);
        // |C| <= 32*15*128: both halves below 2^24, so the two conversions are exact
        const float Da = fmaf((float)(Ca[3] * 256 + Ca[2]), 65536.f, (float)(Ca[1] * 256 + Ca[0]));
        const float Db = fmaf((float)(Cb[3] * 256 + Cb[2]), 65536.f, (float)(Cb[1] * 256 + Cb[0]));
        const float4 mt = *(const float4*)(meta + (sbk + sb) * 16 + g * 4);
        const uint32_t hy = H[1], hz = H[2], hw = H[3];
        const int sca = (hy >> sh) & 63, mna = (hz >> sh) & 63;
        const int scb = ((hw >> sh) & 15) | (((hy >> (sh + 6)) & 3) << 4);
        const int mnb = ((hw >> (sh + 4)) & 15) | (((hz >> (sh + 6)) & 3) << 4);
        const float d = h2f(H[0] & 0xffffu), dmin = h2f(H[0] >> 16);
        const float u = fmaf((float)scb * mt.y, Db, (float)sca * mt.x * Da);
        const float m = fmaf((float)mnb, mt.w, (float)mna * mt.z);
        acc = fmaf(d, u, acc);
        acc = fmaf(-dmin, m, acc);
      }
    }
  }
  vm_wait<0>();  // drain the clamped tail loads before the wave ends

  // ---- reduce over the four lane groups of a row, then over the KS waves
  acc += __shfl_xor(acc, 16, 64);
  acc += __shfl_xor(acc, 32, 64);
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

template <int RT, int KS, int STAGES, int XP, int XK>
int launch(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  static_assert(xq_bytes(XK) + RT * KS * (STAGES * STAGE_BYTES + 64) <= 160 * 1024, "LDS budget");
  static_assert(XK / 16 <= 64 * RT * KS * XP, "x preparation: one thread per 16 elements");
  const int tiles = (N + 15) / 16;
  const unsigned grid = (unsigned)((tiles + RT - 1) / RT);
  const size_t lds = (size_t)RT * KS * (STAGES * STAGE_BYTES + 64);  // plus the static x digits
  static bool attr_set = false;  // dynamic LDS above 64 KiB is opted into once per instantiation
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)qgemv_q4k_mfma<RT, KS, STAGES, XP, XK>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e, "tiermm_qgemv: q4_K LDS attribute");
    attr_set = true;
  }
  qgemv_q4k_mfma<RT, KS, STAGES, XP, XK><<<grid, 64 * RT * KS, lds, s>>>((const uint8_t*)W, rb, x, y, N, K);
  TM_LAUNCH_CHECK("tiermm_qgemv: q4_K launch");
  return TIERMM_OK;
}

}  // namespace

// Largest K handled (the x digits of the whole row stay in LDS).
constexpr int kQ4kMaxK = 14336;

int qgemv_q4k(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  if (K > kQ4kMaxK) return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemv: q4_K K=%d above %d", K, kQ4kMaxK);
  const int tiles = (N + 15) / 16;
  // Tall matrices: one K pass per wave, four row tiles per block.  Short ones
  // (fewer than 640 tiles cannot fill 256 CUs at 4 tiles per block) split K
  // over two waves per tile instead.
  if (K <= 8192) {
    if (tiles >= 640) return launch<4, 1, 2, 4, 8192>(W, rb, x, y, N, K, s);
    return launch<2, 2, 2, 4, 8192>(W, rb, x, y, N, K, s);
  }
  if (tiles >= 640) return launch<4, 1, 2, 4, 14336>(W, rb, x, y, N, K, s);
  return launch<2, 2, 2, 4, 14336>(W, rb, x, y, N, K, s);
}

}  // namespace tiermm

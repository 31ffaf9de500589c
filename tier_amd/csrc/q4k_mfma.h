// q4k_mfma.h -- pieces shared by the Q4_K int8-MFMA decode GEMV kernels:
// the x preparation into int8 digits, the LDS-DMA weight stage and the
// per-super-block MFMA + scale epilogue.  The layouts are described in
// qgemv_q4k.hip.
#pragma once

#include "tm_device.h"

namespace tiermm {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int SB_BYTES = 144;          // Q4_K super-block
constexpr int XQ_SB = 1024;            // LDS bytes of x digits per super-block: 4 t x 4 a x 4 digits x 16
constexpr int XQ_T = 256;              // per MFMA step t
constexpr int META_SB = 64;            // 4 g x float4 (f_g, f_4+g, S_g, S_4+g)
constexpr int ZERO_BYTES = 4 * XQ_T;   // zero rows read by the A lanes that carry no digit

// Whether one of the 16 values is NaN or +-Inf.  The digits below carry finite
// x only; a workgroup whose x holds such a value replaces its rows by
// nonfinite_terms (tm_device.h).
__device__ __forceinline__ bool nonfinite16(const float (&v)[16]) {
  bool any = false;
#pragma unroll
  for (int i = 0; i < 16; ++i) any |= !__builtin_isfinite(v[i]);
  return any;
}

// Publishes whether any lane of the calling wave saw a non-finite x value: every
// lane of the wave calls it, lane 0 writes flags[wave].  Read back with
// flags_any once a barrier has passed.
__device__ __forceinline__ void publish_nonfinite(bool bad, int* flags, int wave, int lane) {
  const bool wbad = __ballot(bad) != 0;
  if (lane == 0) flags[wave] = wbad ? 1 : 0;
}
__device__ __forceinline__ bool flags_any(const int* flags, int n) {
  int a = 0;
  for (int i = 0; i < n; ++i) a |= flags[i];
  return a != 0;
}

// Prepare x elements [16h, 16h+16) of sub-block s (h = half, values in v): the
// partner thread (lane ^ 1) holds the other half; both reach this together.
// With DSUM, also dsum[32 sb + 8 a + 2 t + {0, 1}] = 32 (256 T3 + T2) and
// 32 (256 T1 + T0), T_l = the sum of digit l over these 16 elements: what
// (q + 32) in place of q adds to the two int32 halves of a digit dot.
template <bool DSUM = false>
__device__ __forceinline__ void prep_half(int s, int h, const float (&v)[16], uint8_t* xq, float* meta,
                                          int* dsum = nullptr) {
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
  if constexpr (DSUM) {
    int T[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      T[l] = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) T[l] = __builtin_amdgcn_sdot4((int)L[l][w], 0x01010101, T[l], false);
    }
    *(int2*)(dsum + sb * 32 + a * 8 + t * 2) = make_int2(32 * (256 * T[3] + T[2]), 32 * (256 * T[1] + T[0]));
  }
}

// Async loads of group `grp` (GS super-blocks of the wave's 16 rows) into an
// LDS stage in row-major order (row n at n*GS*144).  roff[j] / coff[j]: row
// (0..15) and byte of the 16 bytes lane `lane` brings with load j; bytes past the
// wave's K range re-read the last valid 16 bytes of the row segment, so the
// number of loads is fixed.  When the stage is not a whole number of 1 KiB
// loads, the last load runs on the lanes that still have bytes to bring.
template <int GS, int SBB = SB_BYTES>
struct Stage {
  static constexpr int GRP = GS * SBB;                    // bytes of one row's group
  static constexpr int BYTES = 16 * GRP;                  // one stage
  static constexpr int NLD = (BYTES + 1023) / 1024;       // loads per stage
  static constexpr int LAST = (BYTES - (NLD - 1) * 1024) / 16;  // lanes of the last load
};

template <int GS, int SBB = SB_BYTES>
__device__ __forceinline__ void load_group(const uint8_t* base0, size_t rb, const int (&roff)[Stage<GS, SBB>::NLD],
                                           const int (&coff)[Stage<GS, SBB>::NLD], int lane, int grp, int nsb,
                                           uint32_t stage) {
  using St = Stage<GS, SBB>;
  constexpr int NLD = St::NLD;
  const int valid = min(GS, nsb - GS * grp);
  const int lastb = valid > 0 ? SBB * valid - 16 : 0;
  const uint8_t* b = base0 + (size_t)max(0, min(grp, (nsb - 1) / GS)) * St::GRP;
#pragma unroll
  for (int j = 0; j < NLD; ++j)
    if (j < NLD - 1 || St::LAST == 64 || lane < St::LAST)
      dma16(b + (size_t)roff[j] * rb + min(coff[j], lastb), stage + j * 1024);
}

constexpr int xq_bytes(int kmax) { return (kmax / 256) * (XQ_SB + META_SB) + ZERO_BYTES; }

// This lane's A operands of one super-block column: rows a0p / a1p for MFMA
// parities 0 / 1 (see q4k_superblock).
__device__ __forceinline__ void load_a(const uint8_t* a0p, const uint8_t* a1p, i32x4 (&A)[4]) {
  A[0] = *(const i32x4*)(a0p);
  A[1] = *(const i32x4*)(a1p + XQ_T);
  A[2] = *(const i32x4*)(a0p + 2 * XQ_T);
  A[3] = *(const i32x4*)(a1p + 3 * XQ_T);
}

// One super-block of a 16-row tile (gemv_q's per-element sum, tier.cpp:299-306,
// regrouped by sub-block): hp = the header of row n's super-block in the stage
// (qs follows at +16), A = this lane's A operands of the super-block's x digits,
// mt = (2^-e_g, 2^-e_4+g, S_g, S_4+g) of the super-block's x.  Returns
// acc + d * sum_s sc_s * f_s * D_s - dmin * sum_s m_s * S_s over sub-blocks g, 4+g.
__device__ __forceinline__ float q4k_sb(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt, float acc) {
  const u32x4 H = *(const u32x4*)hp;
  const u32x4 cA = *(const u32x4*)(hp + 16 + 16 * g);
  const u32x4 cB = *(const u32x4*)(hp + 80 + 16 * g);
  i32x4 B0, B1, B2, B3;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    B0[w] = (int)(cA[w] & 0x0f0f0f0fu);
    B1[w] = (int)((cA[w] >> 4) & 0x0f0f0f0fu);
    B2[w] = (int)(cB[w] & 0x0f0f0f0fu);
    B3[w] = (int)((cB[w] >> 4) & 0x0f0f0f0fu);
  }
  const i32x4 z = {0, 0, 0, 0};
  i32x4 Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B0, z, 0, 0, 0);
  Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B1, Ca, 0, 0, 0);
  i32x4 Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B2, z, 0, 0, 0);
  Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B3, Cb, 0, 0, 0);
  // |C| <= 32*15*128: both halves below 2^24, so the two conversions are exact
  const float Da = fmaf((float)(Ca[3] * 256 + Ca[2]), 65536.f, (float)(Ca[1] * 256 + Ca[0]));
  const float Db = fmaf((float)(Cb[3] * 256 + Cb[2]), 65536.f, (float)(Cb[1] * 256 + Cb[0]));
  const int sh = 8 * g;  // scale byte of sub-blocks g and 4+g (quant.h:47-48)
  const uint32_t hy = H[1], hz = H[2], hw = H[3];
  const int sca = (hy >> sh) & 63, mna = (hz >> sh) & 63;
  const int scb = ((hw >> sh) & 15) | (((hy >> (sh + 6)) & 3) << 4);
  const int mnb = ((hw >> (sh + 4)) & 15) | (((hz >> (sh + 6)) & 3) << 4);
  const float d = h2f(H[0] & 0xffffu), dmin = h2f(H[0] >> 16);
  const float u = fmaf((float)scb * mt.y, Db, (float)sca * mt.x * Da);
  const float m = fmaf((float)mnb, mt.w, (float)mna * mt.z);
  acc = fmaf(d, u, acc);
  return fmaf(-dmin, m, acc);
}
// The same with the high nibbles taken as 16 (q - 8) = (byte ^ 0x80) & 0xf0, one
// v_bitop3 per word instead of a shift and a mask: the MFMAs of the high-nibble
// sub-blocks (rows 4 sigma + digit, sigma odd) then give 16 q.x - 128 S(digit), so Ca and
// Cb start from ca / cb = 128 S(digit) on those rows (q4k_hi_init) and the lanes that
// read them (g odd) take 2^-e / 16 in mt (q4k_hi_scale).  Every intermediate is an exact
// power-of-two multiple of q4k_sb's, so the result is the same to the bit.
__device__ __forceinline__ float q4k_sb_hb(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt,
                                           const i32x4 ca, const i32x4 cb, float acc) {
  const u32x4 H = *(const u32x4*)hp;
  const u32x4 cA = *(const u32x4*)(hp + 16 + 16 * g);
  const u32x4 cB = *(const u32x4*)(hp + 80 + 16 * g);
  i32x4 B0, B1, B2, B3;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    B0[w] = (int)(cA[w] & 0x0f0f0f0fu);
    B1[w] = (int)((cA[w] ^ 0x80808080u) & 0xf0f0f0f0u);
    B2[w] = (int)(cB[w] & 0x0f0f0f0fu);
    B3[w] = (int)((cB[w] ^ 0x80808080u) & 0xf0f0f0f0u);
  }
  i32x4 Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B0, ca, 0, 0, 0);
  Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B1, Ca, 0, 0, 0);
  i32x4 Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B2, cb, 0, 0, 0);
  Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B3, Cb, 0, 0, 0);
  // |C| <= 16*32*15*128: 16 times q4k_sb's halves, still exact through the conversions
  const float Da = fmaf((float)(Ca[3] * 256 + Ca[2]), 65536.f, (float)(Ca[1] * 256 + Ca[0]));
  const float Db = fmaf((float)(Cb[3] * 256 + Cb[2]), 65536.f, (float)(Cb[1] * 256 + Cb[0]));
  const int sh = 8 * g;
  const uint32_t hy = H[1], hz = H[2], hw = H[3];
  const int sca = (hy >> sh) & 63, mna = (hz >> sh) & 63;
  const int scb = ((hw >> sh) & 15) | (((hy >> (sh + 6)) & 3) << 4);
  const int mnb = ((hw >> (sh + 4)) & 15) | (((hz >> (sh + 6)) & 3) << 4);
  const float d = h2f(H[0] & 0xffffu), dmin = h2f(H[0] >> 16);
  const float u = fmaf((float)scb * mt.y, Db, (float)sca * mt.x * Da);
  const float m = fmaf((float)mnb, mt.w, (float)mna * mt.z);
  acc = fmaf(d, u, acc);
  return fmaf(-dmin, m, acc);
}
// Accumulator starts of q4k_sb_hb for one super-block column: 128 times the digit sums
// of the high-nibble A operands (A[1], A[3]) on their rows, zero on the others --
// minus an MFMA against a B of -128 everywhere.
__device__ __forceinline__ void q4k_hi_init(const i32x4 (&A)[4], i32x4& ca, i32x4& cb) {
  const i32x4 neg = {(int)0x80808080u, (int)0x80808080u, (int)0x80808080u, (int)0x80808080u};
  const i32x4 z = {0, 0, 0, 0};
  ca = -__builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], neg, z, 0, 0, 0);
  cb = -__builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], neg, z, 0, 0, 0);
}
// mt of q4k_sb_hb: the lanes whose accumulator rows are high-nibble sub-blocks (g odd)
// take 2^-e / 16.
__device__ __forceinline__ float4 q4k_hi_scale(float4 mt, int g) {
  if (g & 1) {
    mt.x *= 0.0625f;
    mt.y *= 0.0625f;
  }
  return mt;
}
// The same with the A operands and metadata read from LDS: a0p / a1p = this
// lane's A-operand rows for MFMA parities 0 / 1, mtp = the metadata.
__device__ __forceinline__ float q4k_superblock(const uint8_t* hp, int g, const uint8_t* a0p, const uint8_t* a1p,
                                                const float* mtp, float acc) {
  i32x4 A[4];
  load_a(a0p, a1p, A);
  return q4k_sb(hp, g, A, *(const float4*)mtp, acc);
}

// Q5_K super-block (176 bytes: d, dmin, scales as Q4_K, qh[32], qs[128]; quant.h:49,
// 85-86): the Q4_K arithmetic with the fifth bit of each weight from qh.  Element
// 64j + l of the low (high) nibbles of qs[32j + l] takes bit 2j (2j+1) of qh[l];
// lane group g's chunks g and g+4 cover l = 16(g&1) + [0,16), so its 16 qh bytes
// serve all four MFMAs, with bits s0, s0+1, s0+4, s0+5 for s0 = 2(g>>1).
// Weights reach 31: the digit combination rounds once (relative 2^-24).
__device__ __forceinline__ float q5k_sb(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt, float acc) {
  const u32x4 H = *(const u32x4*)hp;
  const u32x4 Qh = *(const u32x4*)(hp + 16 + 16 * (g & 1));
  const u32x4 cA = *(const u32x4*)(hp + 48 + 16 * g);
  const u32x4 cB = *(const u32x4*)(hp + 112 + 16 * g);
  const int s0 = 2 * (g >> 1);
  i32x4 B0, B1, B2, B3;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t qs = Qh[w] >> s0;  // bit s0 of each byte at bit 0
    B0[w] = (int)((cA[w] & 0x0f0f0f0fu) | ((qs << 4) & 0x10101010u));
    B1[w] = (int)(((cA[w] >> 4) & 0x0f0f0f0fu) | ((qs << 3) & 0x10101010u));
    B2[w] = (int)((cB[w] & 0x0f0f0f0fu) | (qs & 0x10101010u));
    B3[w] = (int)(((cB[w] >> 4) & 0x0f0f0f0fu) | ((qs >> 1) & 0x10101010u));
  }
  const i32x4 z = {0, 0, 0, 0};
  i32x4 Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B0, z, 0, 0, 0);
  Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B1, Ca, 0, 0, 0);
  i32x4 Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B2, z, 0, 0, 0);
  Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B3, Cb, 0, 0, 0);
  // |C| <= 32*31*128: the halves stay exact in int32
  const float Da = fmaf((float)(Ca[3] * 256 + Ca[2]), 65536.f, (float)(Ca[1] * 256 + Ca[0]));
  const float Db = fmaf((float)(Cb[3] * 256 + Cb[2]), 65536.f, (float)(Cb[1] * 256 + Cb[0]));
  const int sh = 8 * g;
  const uint32_t hy = H[1], hz = H[2], hw = H[3];
  const int sca = (hy >> sh) & 63, mna = (hz >> sh) & 63;
  const int scb = ((hw >> sh) & 15) | (((hy >> (sh + 6)) & 3) << 4);
  const int mnb = ((hw >> (sh + 4)) & 15) | (((hz >> (sh + 6)) & 3) << 4);
  const float d = h2f(H[0] & 0xffffu), dmin = h2f(H[0] >> 16);
  const float u = fmaf((float)scb * mt.y, Db, (float)sca * mt.x * Da);
  const float m = fmaf((float)mnb, mt.w, (float)mna * mt.z);
  acc = fmaf(d, u, acc);
  return fmaf(-dmin, m, acc);
}
__device__ __forceinline__ float q5k_superblock(const uint8_t* hp, int g, const uint8_t* a0p, const uint8_t* a1p,
                                                const float* mtp, float acc) {
  i32x4 A[4];
  load_a(a0p, a1p, A);
  return q5k_sb(hp, g, A, *(const float4*)mtp, acc);
}

// Q8_0 in groups of eight blocks (272 bytes = 256 weights, 16-byte multiple),
// the "super-block" of the MFMA GEMV (quant.h:68).  Sub-block s is block s: its
// scale d at byte 34s, its 32 int8 weights at 34s + 2.  For MFMA t lane group g
// supplies weights 16(g&1) + [0,16) of block 4(t>>1) + 2(g>>1) + (t&1), whose
// bytes sit 2 (t even) or 0 (t odd) past a dword boundary; Ca ends with block
// g's digit dots, Cb with block 4+g's.
__device__ __forceinline__ float q8_sb(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt, float acc) {
  i32x4 B[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int blk = 4 * (t >> 1) + 2 * (g >> 1) + (t & 1);
    const uint32_t* q = (const uint32_t*)(hp + 34 * blk + 16 * (g & 1) + ((t & 1) ? 2 : 0));
    if (t & 1) {
#pragma unroll
      for (int w = 0; w < 4; ++w) B[t][w] = (int)q[w];
    } else {
      uint32_t v[5];
#pragma unroll
      for (int w = 0; w < 5; ++w) v[w] = q[w];
#pragma unroll
      for (int w = 0; w < 4; ++w) B[t][w] = (int)__builtin_amdgcn_alignbyte(v[w + 1], v[w], 2);
    }
  }
  const i32x4 z = {0, 0, 0, 0};
  i32x4 Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B[0], z, 0, 0, 0);
  Ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B[1], Ca, 0, 0, 0);
  i32x4 Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B[2], z, 0, 0, 0);
  Cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B[3], Cb, 0, 0, 0);
  // |C| <= 32*127*128 < 2^19: the int32 halves are exact, their conversion rounds once
  const float Da = fmaf((float)(Ca[3] * 256 + Ca[2]), 65536.f, (float)(Ca[1] * 256 + Ca[0]));
  const float Db = fmaf((float)(Cb[3] * 256 + Cb[2]), 65536.f, (float)(Cb[1] * 256 + Cb[0]));
  const float da = h2f(*(const uint16_t*)(hp + 34 * g)), db = h2f(*(const uint16_t*)(hp + 34 * (4 + g)));
  acc = fmaf(da * mt.x, Da, acc);
  return fmaf(db * mt.y, Db, acc);
}
__device__ __forceinline__ float q8_group(const uint8_t* hp, int g, const uint8_t* a0p, const uint8_t* a1p,
                                          const float* mtp, float acc) {
  i32x4 A[4];
  load_a(a0p, a1p, A);
  return q8_sb(hp, g, A, *(const float4*)mtp, acc);
}

// Per-format pieces of the MFMA GEMV: bytes per 256 weights and the 16-row
// super-block step (A operands from LDS, or already in registers).
template <int QT>
struct MfmaFmt;
template <>
struct MfmaFmt<QT_Q4_K> {
  static constexpr int SBB = 144;
  __device__ static float step(const uint8_t* hp, int g, const uint8_t* a0p, const uint8_t* a1p, const float* mtp,
                               float acc) {
    return q4k_superblock(hp, g, a0p, a1p, mtp, acc);
  }
  __device__ static float step_reg(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt, float acc) {
    return q4k_sb(hp, g, A, mt, acc);
  }
};
template <>
struct MfmaFmt<QT_Q5_K> {
  static constexpr int SBB = 176;
  __device__ static float step(const uint8_t* hp, int g, const uint8_t* a0p, const uint8_t* a1p, const float* mtp,
                               float acc) {
    return q5k_superblock(hp, g, a0p, a1p, mtp, acc);
  }
  __device__ static float step_reg(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt, float acc) {
    return q5k_sb(hp, g, A, mt, acc);
  }
};
template <>
struct MfmaFmt<QT_Q8_0> {
  static constexpr int SBB = 272;
  __device__ static float step(const uint8_t* hp, int g, const uint8_t* a0p, const uint8_t* a1p, const float* mtp,
                               float acc) {
    return q8_group(hp, g, a0p, a1p, mtp, acc);
  }
  __device__ static float step_reg(const uint8_t* hp, int g, const i32x4 (&A)[4], const float4 mt, float acc) {
    return q8_sb(hp, g, A, mt, acc);
  }
};

}  // namespace
}  // namespace tiermm

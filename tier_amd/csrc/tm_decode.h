// tm_decode.h -- the exact per-block decoders (q_val, quant.h:59-121), built for
// both the gfx950 kernels and host code: one decode source for tiermm_dequant,
// the GEMVs and GEMMs on the device, and tiermm_dequant_host on the host.
//
// Exactness: for every block type decoded here every product in q_val is exact
// in fp32 (at most 11+7+5 significant bits), so the only fp32 rounding is the
// final addition of a minimum (Q4_1, Q5_1, Q2_K) or its subtraction (Q4_K,
// Q5_K), and a fused multiply-add rounds that sum alike; NF4/FP4 round their one
// product as q_val does.  The decoders therefore give the reference's fp32 value
// bit for bit whatever the compiler fuses, on either side.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "iq_grids.h"
#include "tm_host.h"

#define TM_HD __host__ __device__ __forceinline__

namespace tiermm {

TM_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// fp16 bits -> fp32, exact.  On the device the empty asm statement pins the
// conversion to a plain v_cvt_f32_f16 on an fp32 value: without it the compiler
// folds the conversion into v_fma_mix* (fp16 operands read in place, the result
// rounded inside the fma), which gave results that differ from fp32-then-RNE for
// some inputs (found by the bit-exact dequant tests).
TM_HD float h2f(uint32_t h16) {
  float f = (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" : "+v"(f));
#endif
  return f;
}

TM_HD uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }
// 4 bytes at a 2-byte aligned address
TM_HD uint32_t ld_u32_a2(const uint8_t* p) {
  return (uint32_t)*(const uint16_t*)p | ((uint32_t)*(const uint16_t*)(p + 2) << 16);
}
// 8 bytes at a 2-byte aligned address
TM_HD uint2 ld_u64_a2(const uint8_t* p) { return make_uint2(ld_u32_a2(p), ld_u32_a2(p + 4)); }

TM_HD uint32_t byte_at(uint2 v, int k) {
  return ((k < 4 ? v.x : v.y) >> (8 * (k & 3))) & 255u;
}

// 6-bit (scale, min) of sub-block s of a Q4_K/Q5_K super-block (quant.h:47-48).
// q0 = scale bytes 0..3, q1 = 4..7, q2 = 8..11 (block bytes 4..15).
TM_HD void kq_scale_min(int s, uint32_t q0, uint32_t q1, uint32_t q2, int& sc, int& mn) {
  const int sh = 8 * (s & 3);
  if (s < 4) {
    sc = (q0 >> sh) & 63;
    mn = (q1 >> sh) & 63;
  } else {
    sc = ((q2 >> sh) & 15) | (((q0 >> (sh + 6)) & 3) << 4);
    mn = ((q2 >> (sh + 4)) & 15) | (((q1 >> (sh + 6)) & 3) << 4);
  }
}

// Decoders: 8 consecutive elements starting at column `c` (c % 8 == 0) of a
// quantized row, exactly as q_val evaluates each of them.
template <int QT>
struct Dec;

template <>
struct Dec<QT_Q8_0> {  // quant.h:68 -- 34-byte blocks: d fp16, 32 x int8
  static constexpr int BLK = 32, BYTES = 34;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 34;
    const float d = h2f(ld_u16(b));
    const uint2 q = ld_u64_a2(b + 2 + (c & 31));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)(int8_t)byte_at(q, k);
  }
};

template <>
struct Dec<QT_Q5_0> {  // quant.h:66 -- 22-byte blocks: d, qh u32, 16 bytes of nibbles
  static constexpr int BLK = 32, BYTES = 22;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 22;
    const int i0 = c & 31;
    const float d = h2f(ld_u16(b));
    const uint32_t qh = ld_u32_a2(b + 2);
    const uint2 q = ld_u64_a2(b + 6 + (i0 & 15));
    const int sh = i0 < 16 ? 0 : 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int nib = (int)((byte_at(q, k) >> sh) & 15u) | (int)(((qh >> (i0 + k)) & 1u) << 4);
      v[k] = d * (float)(nib - 16);
    }
  }
};

template <>
struct Dec<QT_Q4_0> {  // quant.h:64 -- 18-byte blocks: d, 16 bytes of nibbles (low half first)
  static constexpr int BLK = 32, BYTES = 18;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 18;
    const int i0 = c & 31;
    const float d = h2f(ld_u16(b));
    const uint2 q = ld_u64_a2(b + 2 + (i0 & 15));
    const int sh = i0 < 16 ? 0 : 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)((int)((byte_at(q, k) >> sh) & 15u) - 8);
  }
};

template <>
struct Dec<QT_Q4_1> {  // quant.h:65 -- 20-byte blocks: d, m, 16 bytes of nibbles
  static constexpr int BLK = 32, BYTES = 20;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 20;
    const int i0 = c & 31;
    const float d = h2f(ld_u16(b)), m = h2f(ld_u16(b + 2));
    const uint2 q = ld_u64_a2(b + 4 + (i0 & 15));
    const int sh = i0 < 16 ? 0 : 4;
    // d*v is exact (11 x 4 bits), so a fused multiply-add rounds as d*v + m does
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)((byte_at(q, k) >> sh) & 15u) + m;
  }
};

template <>
struct Dec<QT_Q5_1> {  // quant.h:67 -- 24-byte blocks: d, m, qh u32, 16 bytes of nibbles
  static constexpr int BLK = 32, BYTES = 24;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 24;
    const int i0 = c & 31;
    const float d = h2f(ld_u16(b)), m = h2f(ld_u16(b + 2));
    const uint32_t qh = ld_u32_a2(b + 4);
    const uint2 q = ld_u64_a2(b + 8 + (i0 & 15));
    const int sh = i0 < 16 ? 0 : 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t nib = ((byte_at(q, k) >> sh) & 15u) | (((qh >> (i0 + k)) & 1u) << 4);
      v[k] = d * (float)nib + m;
    }
  }
};

// Dense rows (quant.h:61-63): 8 elements at a 4-byte (fp32) or 2-byte aligned address.
template <>
struct Dec<QT_F32> {
  static constexpr int BLK = 1, BYTES = 4;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const float* p = (const float*)row + c;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[k];
  }
};

template <>
struct Dec<QT_F16> {
  static constexpr int BLK = 1, BYTES = 2;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint2 a = ld_u64_a2(row + 2 * (size_t)c), b = ld_u64_a2(row + 2 * (size_t)c + 8);
    const uint32_t w[4] = {a.x, a.y, b.x, b.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = h2f((w[k >> 1] >> (16 * (k & 1))) & 0xffffu);
  }
};

template <>
struct Dec<QT_BF16> {
  static constexpr int BLK = 1, BYTES = 2;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint2 a = ld_u64_a2(row + 2 * (size_t)c), b = ld_u64_a2(row + 2 * (size_t)c + 8);
    const uint32_t w[4] = {a.x, a.y, b.x, b.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = u2f((k & 1) ? (w[k >> 1] & 0xffff0000u) : (w[k >> 1] << 16));
  }
};

template <>
struct Dec<QT_Q4_K> {  // quant.h:83-84 -- 144-byte super-blocks
  static constexpr int BLK = 256, BYTES = 144;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 144;
    const int i0 = c & 255, j = i0 >> 6, l0 = i0 & 63;
    const uint4 h = *(const uint4*)b;
    int sc, mn;
    kq_scale_min(2 * j + (l0 >= 32), h.y, h.z, h.w, sc, mn);
    const float dsc = h2f(h.x & 0xffffu) * (float)sc, dm = h2f(h.x >> 16) * (float)mn;
    const uint2 q = *(const uint2*)(b + 16 + 32 * j + (l0 & 31));
    const int sh = l0 < 32 ? 0 : 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = dsc * (float)((byte_at(q, k) >> sh) & 15u) - dm;
  }
};

template <>
struct Dec<QT_Q5_K> {  // quant.h:85-87 -- 176-byte super-blocks
  static constexpr int BLK = 256, BYTES = 176;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 176;
    const int i0 = c & 255, j = i0 >> 6, l0 = i0 & 63;
    const uint4 h = *(const uint4*)b;
    int sc, mn;
    kq_scale_min(2 * j + (l0 >= 32), h.y, h.z, h.w, sc, mn);
    const float dsc = h2f(h.x & 0xffffu) * (float)sc, dm = h2f(h.x >> 16) * (float)mn;
    const uint2 q = *(const uint2*)(b + 48 + 32 * j + (l0 & 31));
    const uint2 qh = *(const uint2*)(b + 16 + (i0 & 31));
    const int sh = l0 < 32 ? 0 : 4, hs = i0 >> 5;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t nib = ((byte_at(q, k) >> sh) & 15u) | (((byte_at(qh, k) >> hs) & 1u) << 4);
      v[k] = dsc * (float)nib - dm;
    }
  }
};

template <>
struct Dec<QT_Q6_K> {  // quant.h:88-90 -- 210-byte super-blocks (2-byte aligned)
  static constexpr int BLK = 256, BYTES = 210;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 210;
    const int i0 = c & 255, a = i0 >> 7, r = i0 & 127;
    const uint2 ql = ld_u64_a2(b + 64 * a + (r & 63));
    const uint2 qh = ld_u64_a2(b + 128 + 32 * a + (r & 31));
    const float ds = h2f(ld_u16(b + 208)) * (float)(int8_t)b[192 + (i0 >> 4)];
    const int s4 = 4 * (r >> 6), s2 = 2 * (r >> 5);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int q = (int)(((byte_at(ql, k) >> s4) & 15u) | (((byte_at(qh, k) >> s2) & 3u) << 4)) - 32;
      v[k] = ds * (float)q;
    }
  }
};

// Levels of the non-uniform 4-bit codes (formats fixed by their definitions).
constexpr int8_t kIq4Levels[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
constexpr float kNf4Levels[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, -0.28444138169288635f,
    -0.18477343022823334f, -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f,
    0.24611230194568634f, 0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f,
    1.0f};  // bitsandbytes NF4
constexpr float kFp4Levels[16] = {0.0f, 0.0052083333f, 0.6666667f, 1.0f, 0.33333334f, 0.5f,
                                             0.16666667f, 0.25f, -0.0f, -0.0052083333f, -0.6666667f, -1.0f,
                                             -0.33333334f, -0.5f, -0.16666667f, -0.25f};  // bitsandbytes FP4

TM_HD uint32_t ld_u32(const uint8_t* p) { return *(const uint32_t*)p; }
TM_HD uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 255u; }

template <>
struct Dec<QT_IQ4_NL> {  // quant.h:69 -- 18-byte blocks: d, 16 bytes of nibbles mapped through the IQ4 levels
  static constexpr int BLK = 32, BYTES = 18;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 18;
    const int i0 = c & 31;
    const float d = h2f(ld_u16(b));
    const uint2 q = ld_u64_a2(b + 2 + (i0 & 15));
    const int sh = i0 < 16 ? 0 : 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)kIq4Levels[(byte_at(q, k) >> sh) & 15u];
  }
};

template <>
struct Dec<QT_MXFP4> {  // quant.h:70-71 -- 17-byte blocks: E8M0 exponent, 16 bytes of E2M1 nibbles
  static constexpr int BLK = 32, BYTES = 17;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 5) * 17;  // blocks are byte aligned: byte loads
    const int i0 = c & 31, e = b[0];
    const float scale = __builtin_ldexpf(1.0f, e - 128);  // 2^(e-127) over the doubled levels
    const int sh = i0 < 16 ? 0 : 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int code = (b[1 + (i0 & 15) + k] >> sh) & 15, ex = (code >> 1) & 3, m = code & 1;
      const int twice = ex == 0 ? m : (2 + m) << (ex - 1);
      v[k] = scale * (float)((code & 8) ? -twice : twice);
    }
  }
};

template <int QT>
struct DecBnb {  // quant.h:72-73 -- 36-byte blocks of 64: fp32 absmax, 32 bytes of nibbles (even element high)
  static constexpr int BLK = 64, BYTES = 36;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 6) * 36;
    const float a = u2f(ld_u32(b));
    const uint32_t w = ld_u32(b + 4 + ((c & 63) >> 1));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t y = byte_of(w, k >> 1), code = (k & 1) ? (y & 15u) : (y >> 4);
      v[k] = (QT == QT_NF4 ? kNf4Levels[code] : kFp4Levels[code]) * a;
    }
  }
};
template <>
struct Dec<QT_NF4> : DecBnb<QT_NF4> {};
template <>
struct Dec<QT_FP4> : DecBnb<QT_FP4> {};

template <>
struct Dec<QT_Q2_K> {  // quant.h:76-77 -- 84-byte super-blocks: nibble scale/min pairs, 2-bit codes, d, dmin
  static constexpr int BLK = 256, BYTES = 84;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 84;
    const int i0 = c & 255;
    const uint32_t sc = b[i0 >> 4];
    const float dsc = h2f(ld_u16(b + 80)) * (float)(sc & 15u), dm = h2f(ld_u16(b + 82)) * (float)(sc >> 4);
    const uint8_t* q = b + 16 + (i0 >> 7) * 32 + (i0 & 31);
    const uint32_t q0 = ld_u32(q), q1 = ld_u32(q + 4);
    const int sh = 2 * ((i0 & 127) >> 5);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = dsc * (float)((byte_of(k < 4 ? q0 : q1, k & 3) >> sh) & 3u) - dm;
  }
};

template <>
struct Dec<QT_Q3_K> {  // quant.h:78-80 -- 110-byte super-blocks: high-bit mask, 2-bit codes, 6-bit scales, d
  static constexpr int BLK = 256, BYTES = 110;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 110;
    const int i0 = c & 255, j = i0 >> 4;
    const uint8_t* s = b + 96;
    const int sc = ((j < 8 ? (s[j] & 15) : (s[j - 8] >> 4)) | (((s[8 + (j & 3)] >> (2 * (j >> 2))) & 3) << 4)) - 32;
    const float ds = h2f(ld_u16(b + 108)) * (float)sc;
    const uint2 ql = ld_u64_a2(b + 32 + (i0 >> 7) * 32 + (i0 & 31));
    const uint2 hm = ld_u64_a2(b + (i0 & 31));
    const int sh = 2 * ((i0 & 127) >> 5), hb = i0 >> 5;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int q = (int)((byte_at(ql, k) >> sh) & 3u) - (((byte_at(hm, k) >> hb) & 1u) ? 0 : 4);
      v[k] = ds * (float)q;
    }
  }
};

template <>
struct Dec<QT_IQ4_XS> {  // quant.h:92-94 -- 136-byte super-blocks: d, 6-bit scales, nibbles mapped through the IQ4 levels
  static constexpr int BLK = 256, BYTES = 136;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 136;
    const int i0 = c & 255, j = i0 >> 5;
    const int sc = (((b[4 + (j >> 1)] >> (4 * (j & 1))) & 15) | (((ld_u16(b + 2) >> (2 * j)) & 3) << 4)) - 32;
    const float ds = h2f(ld_u16(b)) * (float)sc;  // 11 + 6 bits: exact, and times a 7-bit level still exact
    const uint2 q = ld_u64_a2(b + 8 + j * 16 + (i0 & 15));
    const int sh = 4 * ((i0 & 31) >> 4);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = ds * (float)kIq4Levels[(byte_at(q, k) >> sh) & 15u];
  }
};

template <>
struct Dec<QT_TQ2_0> {  // quant.h:116 -- 66-byte super-blocks: 2-bit codes, d; value d * (code - 1)
  static constexpr int BLK = 256, BYTES = 66;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 66;
    const int i0 = c & 255;
    const float d = h2f(ld_u16(b + 64));
    const uint2 q = ld_u64_a2(b + (i0 >> 7) * 32 + (i0 & 31));
    const int sh = 2 * ((i0 & 127) >> 5);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)((int)((byte_at(q, k) >> sh) & 3u) - 1);
  }
};

template <>
struct Dec<QT_TQ1_0> {  // quant.h:117-119 -- 54-byte super-blocks: base-3 packed trits, d; value d * (trit - 1)
  static constexpr int BLK = 256, BYTES = 54;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 54;
    const int i0 = c & 255;
    const float d = h2f(ld_u16(b + 52));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = i0 + k;
      int byte, mul;  // the byte times 3^t keeps trit t in its top bits (mod 256)
      if (i < 160) {
        byte = b[i & 31];
        mul = i >> 5;
      } else if (i < 240) {
        byte = b[32 + ((i - 160) & 15)];
        mul = (i - 160) >> 4;
      } else {
        byte = b[48 + ((i - 240) & 3)];
        mul = (i - 240) >> 2;
      }
      const int p3 = mul == 0 ? 1 : mul == 1 ? 3 : mul == 2 ? 9 : mul == 3 ? 27 : 81;
      const uint32_t x = (uint32_t)(byte * p3) & 255u;
      v[k] = d * (float)((int)((x * 3u) >> 8) - 1);
    }
  }
};

// ---- lattice-grid types (quant.h:95-115).  A grid point holds 8 (IQ2, IQ1) or 4
// (IQ3) element magnitudes, packed as codes in iq_grids.h; signs come from a
// 7-bit index whose parity gives the eighth bit (ksigns) or from a byte.  Every
// product is exact in fp32 (fp16 scale times at most 5 + 6 bits), so the values
// do not depend on the order of the multiplications.
TM_HD float iq2_level(uint32_t c) { return c == 0 ? 8.f : c == 1 ? 25.f : 43.f; }
TM_HD float iq3xxs_level(uint32_t c) { return c == 7 ? 62.f : (float)(8 * c + 4); }
TM_HD uint32_t iq_ksign(uint32_t i) { return i | ((uint32_t)(__builtin_popcount(i) & 1) << 7); }
TM_HD float iq_sign(uint32_t s, int e) { return (s >> e) & 1u ? -1.f : 1.f; }

template <>
struct Dec<QT_IQ2_XXS> {  // quant.h:95-97 -- 66 bytes: d, 8 x (4 grid bytes, 4 sign/scale bytes)
  static constexpr int BLK = 256, BYTES = 66;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 66;
    const int i0 = c & 255, g = i0 >> 5, k = (i0 & 31) >> 3;
    const uint32_t a0 = ld_u32_a2(b + 2 + 8 * g), a1 = ld_u32_a2(b + 6 + 8 * g);
    const float db = h2f(ld_u16(b)) * (0.5f + (float)(a1 >> 28)) * 0.25f;
    const uint32_t w = tm_iq2xxs_grid[(a0 >> (8 * k)) & 255u], sg = iq_ksign((a1 >> (7 * k)) & 127u);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = db * iq2_level((w >> (2 * e)) & 3u) * iq_sign(sg, e);
  }
};

template <>
struct Dec<QT_IQ2_XS> {  // quant.h:98-100 -- 74 bytes: d, 32 x u16 (9-bit point, 7-bit sign index), 8 scale bytes
  static constexpr int BLK = 256, BYTES = 74;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 74;
    const int i0 = c & 255, k = i0 >> 3, s = i0 >> 4;
    const uint32_t q = ld_u16(b + 2 + 2 * k);
    const float db = h2f(ld_u16(b)) * (0.5f + (float)((b[66 + (s >> 1)] >> (4 * (s & 1))) & 15)) * 0.25f;
    const uint32_t w = tm_iq2xs_grid[q & 511u], sg = iq_ksign(q >> 9);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = db * iq2_level((w >> (2 * e)) & 3u) * iq_sign(sg, e);
  }
};

template <>
struct Dec<QT_IQ2_S> {  // quant.h:101-103 -- 82 bytes: d, 32 point bytes, 32 sign bytes, 8 high-bit bytes, 8 scales
  static constexpr int BLK = 256, BYTES = 82;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 82;
    const int i0 = c & 255, k = i0 >> 3, s = i0 >> 4;
    const float db = h2f(ld_u16(b)) * (0.5f + (float)((b[74 + (s >> 1)] >> (4 * (s & 1))) & 15)) * 0.25f;
    const uint32_t gi = b[2 + k] | (((uint32_t)(b[66 + (k >> 2)] >> (2 * (k & 3))) & 3u) << 8);
    const uint32_t w = tm_iq2s_grid[gi], sg = b[34 + k];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = db * iq2_level((w >> (2 * e)) & 3u) * iq_sign(sg, e);
  }
};

template <>
struct Dec<QT_IQ3_XXS> {  // quant.h:104-106 -- 98 bytes: d, 64 point bytes, 8 x u32 (4 sign indices, scale)
  static constexpr int BLK = 256, BYTES = 98;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 98;
    const int i0 = c & 255, g = i0 >> 5, k = (i0 & 31) >> 3;
    const uint32_t sw = ld_u32_a2(b + 66 + 4 * g);
    const float db = h2f(ld_u16(b)) * (0.5f + (float)(sw >> 28)) * 0.5f;
    const uint32_t sg = iq_ksign((sw >> (7 * k)) & 127u);
    const uint32_t w0 = tm_iq3xxs_grid[b[2 + (i0 >> 2)]], w1 = tm_iq3xxs_grid[b[3 + (i0 >> 2)]];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = db * iq3xxs_level(((e < 4 ? w0 : w1) >> (3 * (e & 3))) & 7u) * iq_sign(sg, e);
  }
};

template <>
struct Dec<QT_IQ3_S> {  // quant.h:107-109 -- 110 bytes: d, 64 point bytes, 8 high-bit bytes, 32 sign bytes, 4 scales
  static constexpr int BLK = 256, BYTES = 110;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 110;
    const int i0 = c & 255, g = i0 >> 5, k0 = i0 >> 2;
    const float db = h2f(ld_u16(b)) * (float)(1 + 2 * ((b[106 + (g >> 1)] >> (4 * (g & 1))) & 15));
    uint32_t w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int k = k0 + j;
      w[j] = tm_iq3s_grid[b[2 + k] | (((uint32_t)(b[66 + (k >> 3)] >> (k & 7)) & 1u) << 8)];
    }
    const uint32_t sg = b[74 + (i0 >> 3)];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = db * (float)(2 * ((w[e >> 2] >> (3 * (e & 3))) & 7u) + 1) * iq_sign(sg, e);
  }
};

template <>
struct Dec<QT_IQ1_S> {  // quant.h:110-112 -- 50 bytes: d, 32 point bytes, 8 x u16 (high bits, scale, delta sign)
  static constexpr int BLK = 256, BYTES = 50;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 50;
    const int i0 = c & 255, g = i0 >> 5, k = i0 >> 3;
    const uint32_t qh = ld_u16(b + 34 + 2 * g);
    const float dl = h2f(ld_u16(b)) * (float)(2 * ((qh >> 12) & 7) + 1);
    const float dt = (qh & 0x8000u) ? -0.125f : 0.125f;
    const uint32_t w = tm_iq1s_grid[b[2 + k] | (((qh >> (3 * (k & 3))) & 7u) << 8)];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = dl * ((float)((int)((w >> (2 * e)) & 3u) - 1) + dt);
  }
};

template <>
struct Dec<QT_IQ1_M> {  // quant.h:113-115 -- 56 bytes: 32 point bytes, 16 high-bit nibbles, 4 x u16 scales (+ fp16 d in their top nibbles)
  static constexpr int BLK = 256, BYTES = 56;
  TM_HD static void run(const uint8_t* row, int c, float v[8]) {
    const uint8_t* b = row + (size_t)(c >> 8) * 56;
    const uint8_t* sc = b + 48;
    const int i0 = c & 255, k = i0 >> 3, s = i0 >> 4;
    const uint32_t s0 = ld_u16(sc), s1 = ld_u16(sc + 2), s2 = ld_u16(sc + 4), s3 = ld_u16(sc + 6);
    const uint32_t dh = (s0 >> 12) | ((s1 & 0xf000u) >> 8) | ((s2 & 0xf000u) >> 4) | (s3 & 0xf000u);
    const float dl = h2f(dh) * (float)(2 * ((ld_u16(sc + 2 * (s >> 2)) >> (3 * (s & 3))) & 7) + 1);
    const uint32_t qh = (b[32 + (k >> 1)] >> (4 * (k & 1))) & 15u;
    const float dt = (qh & 8u) ? -0.125f : 0.125f;
    const uint32_t w = tm_iq1s_grid[b[k] | ((qh & 7u) << 8)];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = dl * ((float)((int)((w >> (2 * e)) & 3u) - 1) + dt);
  }
};

// One element of a dense row (q_val's F32 / F16 / BF16 cases, quant.h:61-63), for
// rows whose length is not a whole number of 8-element chunks.
template <int QT>
TM_HD float dense_val(const uint8_t* row, size_t k) {
  static_assert(QT == QT_F32 || QT == QT_F16 || QT == QT_BF16, "dense rows only");
  if constexpr (QT == QT_F32) return u2f(*(const uint32_t*)(row + 4 * k));
  else if constexpr (QT == QT_F16) return h2f(*(const uint16_t*)(row + 2 * k));
  else return u2f((uint32_t)*(const uint16_t*)(row + 2 * k) << 16);
}

// Calls f(std::integral_constant<int, QT>{}) for the GPU-decoded type `qtype`;
// the caller has already refused every other type.
template <class F>
inline auto with_qtype(int qtype, F&& f) {
  switch (qtype) {
    case QT_F32: return f(std::integral_constant<int, QT_F32>{});
    case QT_F16: return f(std::integral_constant<int, QT_F16>{});
    case QT_BF16: return f(std::integral_constant<int, QT_BF16>{});
    case QT_Q4_0: return f(std::integral_constant<int, QT_Q4_0>{});
    case QT_Q4_1: return f(std::integral_constant<int, QT_Q4_1>{});
    case QT_Q5_0: return f(std::integral_constant<int, QT_Q5_0>{});
    case QT_Q5_1: return f(std::integral_constant<int, QT_Q5_1>{});
    case QT_Q8_0: return f(std::integral_constant<int, QT_Q8_0>{});
    case QT_Q4_K: return f(std::integral_constant<int, QT_Q4_K>{});
    case QT_Q5_K: return f(std::integral_constant<int, QT_Q5_K>{});
    case QT_Q2_K: return f(std::integral_constant<int, QT_Q2_K>{});
    case QT_Q3_K: return f(std::integral_constant<int, QT_Q3_K>{});
    case QT_IQ4_NL: return f(std::integral_constant<int, QT_IQ4_NL>{});
    case QT_IQ4_XS: return f(std::integral_constant<int, QT_IQ4_XS>{});
    case QT_TQ1_0: return f(std::integral_constant<int, QT_TQ1_0>{});
    case QT_TQ2_0: return f(std::integral_constant<int, QT_TQ2_0>{});
    case QT_MXFP4: return f(std::integral_constant<int, QT_MXFP4>{});
    case QT_NF4: return f(std::integral_constant<int, QT_NF4>{});
    case QT_FP4: return f(std::integral_constant<int, QT_FP4>{});
    case QT_IQ2_XXS: return f(std::integral_constant<int, QT_IQ2_XXS>{});
    case QT_IQ2_XS: return f(std::integral_constant<int, QT_IQ2_XS>{});
    case QT_IQ2_S: return f(std::integral_constant<int, QT_IQ2_S>{});
    case QT_IQ3_XXS: return f(std::integral_constant<int, QT_IQ3_XXS>{});
    case QT_IQ3_S: return f(std::integral_constant<int, QT_IQ3_S>{});
    case QT_IQ1_S: return f(std::integral_constant<int, QT_IQ1_S>{});
    case QT_IQ1_M: return f(std::integral_constant<int, QT_IQ1_M>{});
    default: return f(std::integral_constant<int, QT_Q6_K>{});
  }
}

}  // namespace tiermm

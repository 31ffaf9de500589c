/*
 * tq_oracle.c -- CPU restatement of the reference's frozen-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never by the product.
 * Built with -ffp-contract=off so every fp32 expression rounds exactly where
 * the written C rounds.  See tq_oracle.h for what pins each function.
 */
#include "tq_oracle.h"
#include "../tier_amd/csrc/iq_grids.h"

#include <math.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* lattice-grid helpers: magnitude of element e of a packed IQ2 point, value of
 * element e of an IQ1 point, the sign byte of a 7-bit index (its parity in bit 7)
 * and the sign of element e */
static inline float iq2_mag(uint16_t w, int e) {
  const int c = (w >> (2 * e)) & 3;
  return c == 0 ? 8.f : c == 1 ? 25.f : 43.f;
}
static inline int iq1_val(uint16_t w, int e) { return ((w >> (2 * e)) & 3) - 1; }
static inline uint32_t parity_byte(uint32_t idx) {
  uint32_t p = 0;
  for (int b = 0; b < 7; ++b) p ^= (idx >> b) & 1u;
  return idx | (p << 7);
}
static inline float sign_of(uint32_t s, int e) { return (s >> e) & 1u ? -1.f : 1.f; }
static inline uint32_t rd32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* (type, elements per block, bytes per block): the table of quant.h:26-30. */
static const int QTAB[][3] = {
  {0, 1, 4}, {1, 1, 2}, {30, 1, 2}, {2, 32, 18}, {3, 32, 20}, {6, 32, 22}, {7, 32, 24},
  {8, 32, 34}, {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
  {14, 256, 210}, {16, 256, 66}, {17, 256, 74}, {22, 256, 82}, {18, 256, 98},
  {21, 256, 110}, {19, 256, 50}, {29, 256, 56}, {20, 32, 18}, {23, 256, 136},
  {34, 256, 54}, {35, 256, 66}, {39, 32, 17}, {200, 64, 36}, {201, 64, 36},
};

int orc_q_block(int type, int* blk_elems, int* blk_bytes) {
  for (size_t i = 0; i < sizeof(QTAB) / sizeof(QTAB[0]); ++i)
    if (QTAB[i][0] == type) {
      if (blk_elems) *blk_elems = QTAB[i][1];
      if (blk_bytes) *blk_bytes = QTAB[i][2];
      return 1;
    }
  return 0;
}

/* quant.h:33 q_row_bytes: cols/blk*bytes (integer division), 0 for unknown types. */
size_t orc_q_row_bytes(int type, int cols) {
  int be, bb;
  if (!orc_q_block(type, &be, &bb)) return 0;
  return (size_t)cols / (size_t)be * (size_t)bb;
}

/* binary16 -> binary32, exact (quant.h:37-42, gpu_compat.h:175-190).
 * Normal: (1024+m) * 2^(e-25); subnormal: m * 2^-24; inf/NaN keep the payload. */
float orc_h2f(uint16_t h) {
  const uint32_t sgn = (uint32_t)(h >> 15), e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 31u) return u2f((sgn << 31) | 0x7f800000u | (m << 13));
  float v = (e == 0u) ? ldexpf((float)m, -24) : ldexpf((float)(m | 1024u), (int)e - 25);
  return sgn ? -v : v;
}

/* binary32 -> binary16, round to nearest even (gpu_compat.h:151-174). */
uint16_t orc_f2h(float f) {
  const uint32_t u = f2u(f), sgn = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sgn | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (a >= 0x477ff000u) return (uint16_t)(sgn | 0x7c00u); /* >= 65520 rounds to inf */
  if (a >= 0x38800000u) {                                  /* fp16 normal range */
    uint32_t h = ((((a >> 23) - 112u)) << 10) | ((a >> 13) & 1023u);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* carry may bump exponent */
    return (uint16_t)(sgn | h);
  }
  if (a <= 0x33000000u) return (uint16_t)sgn; /* <= 2^-25: rounds to zero (tie to even) */
  /* fp16 subnormal: count units of 2^-24 */
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  const int sh = 126 - (int)(a >> 23); /* value = mant * 2^(E-23), E=(a>>23)-127 */
  uint32_t q = mant >> sh;
  const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return (uint16_t)(sgn | q);
}

/* hip_bfloat16(float): keep the top 16 bits, round to nearest even; NaN stays NaN. */
uint16_t orc_f2bf(float f) {
  const uint32_t u = f2u(f);
  uint32_t hi = u >> 16;
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u & 0xffffu) ? (hi | 1u) : hi);
  const uint32_t rem = u & 0xffffu;
  if (rem > 0x8000u || (rem == 0x8000u && (hi & 1u))) ++hi;
  return (uint16_t)hi;
}

void orc_f2h_n(const float* x, uint16_t* h, size_t n) {
  for (size_t i = 0; i < n; ++i) h[i] = orc_f2h(x[i]);
}
void orc_h2f_n(const uint16_t* h, float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = orc_h2f(h[i]);
}
void orc_f2bf_n(const float* x, uint16_t* b, size_t n) {
  for (size_t i = 0; i < n; ++i) b[i] = orc_f2bf(x[i]);
}

static inline float fp16_at(const uint8_t* p) { return orc_h2f(rd16(p)); }

/* 6-bit scale/min pair s (0..7) of a q4_K/q5_K super-block (quant.h:47-48). */
static void kq_scale_min(int s, const uint8_t* q, int* sc, int* mn) {
  if (s < 4) {
    *sc = q[s] & 63;
    *mn = q[s + 4] & 63;
  } else {
    *sc = (q[s + 4] & 15) | ((q[s - 4] >> 6) << 4);
    *mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
  }
}

/* The 16-level maps of the non-uniform 4-bit types.  These values define the
 * formats (the reference keeps them in quant_tables.h and quant.h:50-57) and must
 * be reproduced exactly.  Pinned: tests compare every code with oracle/_ref. */
/* IQ4_NL / IQ4_XS levels (ggml's kvalues_iq4nl), times the block scale */
static const int8_t kIQ4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
/* MXFP4: an E2M1 code (sign, 2-bit exponent, 1-bit mantissa) as an integer twice its
 * value, so that the block scale 2^(e-128) gives code * 2^(e-127); code 8 is +0. */
static int mxfp4_level(int v) {
  const int e = (v >> 1) & 3, m = v & 1;
  const int twice = e == 0 ? m : (2 + m) << (e - 1);
  return (v & 8) ? -twice : twice;
}
/* NF4: the 16 normal-quantile levels of bitsandbytes' NF4 code. */
static const float kNF4[16] = {-1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
                               -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
                               0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
                               0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
                               0.7229568362236023f, 1.0f};
/* FP4: bitsandbytes' FP4 code (E2M1 magnitudes over 6, code 1 the 1/192 subnormal, bit 3 the sign) */
static const float kFP4[16] = {0.0f, 0.0052083333f, 0.6666667f, 1.0f, 0.33333334f, 0.5f, 0.16666667f, 0.25f,
                               -0.0f, -0.0052083333f, -0.6666667f, -1.0f, -0.33333334f, -0.5f, -0.16666667f, -0.25f};

/* One element of a quantized row (quant.h:59-121). */
float orc_q_val(const uint8_t* row, int type, int col) {
  switch (type) {
    case ORC_F32: return u2f(rd32(row + (size_t)col * 4));
    case ORC_F16: return orc_h2f(rd16(row + (size_t)col * 2));
    case ORC_BF16: return u2f((uint32_t)rd16(row + (size_t)col * 2) << 16);
    case ORC_Q8_0: { /* quant.h:68: d fp16 @0, int8 q[32] @2 */
      const uint8_t* b = row + (size_t)(col / 32) * 34;
      return fp16_at(b) * (float)(int8_t)b[2 + col % 32];
    }
    case ORC_Q4_0: { /* quant.h:64: d @0, qs[16] @2; element i<16 low nibble, else high */
      const uint8_t* b = row + (size_t)(col / 32) * 18;
      const int i = col % 32, v = (b[2 + i % 16] >> (i < 16 ? 0 : 4)) & 15;
      return fp16_at(b) * (float)(v - 8);
    }
    case ORC_Q4_1: { /* quant.h:65: d @0, m @2, qs @4 */
      const uint8_t* b = row + (size_t)(col / 32) * 20;
      const int i = col % 32, v = (b[4 + i % 16] >> (i < 16 ? 0 : 4)) & 15;
      return fp16_at(b) * (float)v + fp16_at(b + 2);
    }
    case ORC_Q5_0: { /* quant.h:66: d @0, qh u32 @2, qs @6; bit 4 = qh bit i */
      const uint8_t* b = row + (size_t)(col / 32) * 22;
      const int i = col % 32;
      const int v = ((b[6 + i % 16] >> (i < 16 ? 0 : 4)) & 15) | (int)(((rd32(b + 2) >> i) & 1u) << 4);
      return fp16_at(b) * (float)(v - 16);
    }
    case ORC_Q5_1: { /* quant.h:67: d @0, m @2, qh @4, qs @8 */
      const uint8_t* b = row + (size_t)(col / 32) * 24;
      const int i = col % 32;
      const int v = ((b[8 + i % 16] >> (i < 16 ? 0 : 4)) & 15) | (int)(((rd32(b + 4) >> i) & 1u) << 4);
      return fp16_at(b) * (float)v + fp16_at(b + 2);
    }
    case ORC_IQ4_NL: { /* quant.h:69: d @0, qs[16] @2 as Q4_0, the nibble maps through kIQ4 */
      const uint8_t* b = row + (size_t)(col / 32) * 18;
      const int i = col % 32, v = (b[2 + i % 16] >> (i < 16 ? 0 : 4)) & 15;
      return fp16_at(b) * (float)kIQ4[v];
    }
    case ORC_MXFP4: { /* quant.h:70-71: E8M0 exponent byte @0, qs[16] @1 */
      const uint8_t* b = row + (size_t)(col / 32) * 17;
      const int i = col % 32, v = (b[1 + i % 16] >> (i < 16 ? 0 : 4)) & 15;
      return ldexpf(1.0f, (int)b[0] - 128) * (float)mxfp4_level(v);
    }
    case ORC_NF4:
    case ORC_FP4: { /* quant.h:72-73: fp32 absmax @0, 32 bytes of nibbles @4, even element high */
      const uint8_t* b = row + (size_t)(col / 64) * 36;
      const int i = col % 64;
      const uint8_t y = b[4 + i / 2];
      const int v = (i & 1) ? (y & 15) : (y >> 4);
      return (type == ORC_NF4 ? kNF4[v] : kFP4[v]) * u2f(rd32(b));
    }
    default: break;
  }
  const int i = col % 256; /* position inside a 256-element super-block */
  switch (type) {
    case ORC_Q4_K: { /* quant.h:83-84: d @0, dmin @2, scales[12] @4, qs[128] @16 */
      const uint8_t* b = row + (size_t)(col / 256) * 144;
      const int grp = i / 64, l = i % 64;
      int sc, mn;
      kq_scale_min(2 * grp + (l >= 32), b + 4, &sc, &mn);
      const uint8_t byte = b[16 + 32 * grp + l % 32];
      const int v = (l < 32) ? (byte & 15) : (byte >> 4);
      return (fp16_at(b) * (float)sc) * (float)v - fp16_at(b + 2) * (float)mn;
    }
    case ORC_Q5_K: { /* quant.h:85-87: as Q4_K, qh[32] @16, qs[128] @48 */
      const uint8_t* b = row + (size_t)(col / 256) * 176;
      const int grp = i / 64, l = i % 64;
      int sc, mn;
      kq_scale_min(2 * grp + (l >= 32), b + 4, &sc, &mn);
      const uint8_t byte = b[48 + 32 * grp + l % 32];
      const int hbit = (b[16 + i % 32] >> (i / 32)) & 1;
      const int v = ((l < 32) ? (byte & 15) : (byte >> 4)) | (hbit << 4);
      return (fp16_at(b) * (float)sc) * (float)v - fp16_at(b + 2) * (float)mn;
    }
    case ORC_Q6_K: { /* quant.h:88-90: ql[128] @0, qh[64] @128, int8 sc[16] @192, d @208 */
      const uint8_t* b = row + (size_t)(col / 256) * 210;
      const int half128 = i / 128, r = i % 128;
      const int lo4 = (b[64 * half128 + r % 64] >> (4 * (r / 64))) & 15;
      const int hi2 = (b[128 + 32 * half128 + r % 32] >> (2 * (r / 32))) & 3;
      const int q = (lo4 | (hi2 << 4)) - 32;
      return (fp16_at(b + 208) * (float)(int8_t)b[192 + i / 16]) * (float)q;
    }
    case ORC_Q2_K: { /* quant.h:76-77: scales[16] @0 (low nibble scale, high min), qs[64] @16, d @80, dmin @82 */
      const uint8_t* b = row + (size_t)(col / 256) * 84;
      const int q = (b[16 + 32 * (i / 128) + i % 32] >> (2 * ((i % 128) / 32))) & 3;
      const uint8_t sc = b[i / 16];
      return (fp16_at(b + 80) * (float)(sc & 15)) * (float)q - fp16_at(b + 82) * (float)(sc >> 4);
    }
    case ORC_Q3_K: { /* quant.h:78-80: hmask[32] @0, qs[64] @32, 6-bit scales in 12 bytes @96, d @108 */
      const uint8_t* b = row + (size_t)(col / 256) * 110;
      const uint8_t* s = b + 96;
      const int j = i / 16;
      const int low = j < 8 ? (s[j] & 15) : (s[j - 8] >> 4);
      const int high = (s[8 + j % 4] >> (2 * (j / 4))) & 3;
      const int sc = (low | (high << 4)) - 32;
      const int ql = (b[32 + 32 * (i / 128) + i % 32] >> (2 * ((i % 128) / 32))) & 3;
      const int hbit = (b[i % 32] >> (i / 32)) & 1; /* a clear bit subtracts 4 */
      return (fp16_at(b + 108) * (float)sc) * (float)(ql - (hbit ? 0 : 4));
    }
    case ORC_IQ4_XS: { /* quant.h:92-94: d @0, high scale bits u16 @2, low nibbles [4] @4, qs[128] @8 */
      const uint8_t* b = row + (size_t)(col / 256) * 136;
      const int j = i / 32;
      const int low = (b[4 + j / 2] >> (4 * (j % 2))) & 15, high = (rd16(b + 2) >> (2 * j)) & 3;
      const int sc = (low | (high << 4)) - 32;
      const int v = (b[8 + 16 * j + i % 16] >> (4 * ((i % 32) / 16))) & 15;
      return (fp16_at(b) * (float)sc) * (float)kIQ4[v];
    }
    case ORC_TQ2_0: { /* quant.h:116: 2-bit codes qs[64] @0, d @64; value d * (code - 1) */
      const uint8_t* b = row + (size_t)(col / 256) * 66;
      const int q = (b[32 * (i / 128) + i % 32] >> (2 * ((i % 128) / 32))) & 3;
      return fp16_at(b + 64) * (float)(q - 1);
    }
    case ORC_TQ1_0: { /* quant.h:117-119: 5 trits per byte in qs[48] @0, 4 per byte in qh[4] @48, d @52 */
      const uint8_t* b = row + (size_t)(col / 256) * 54;
      static const int pow3[5] = {1, 3, 9, 27, 81};
      uint8_t x; /* the byte times 3^k keeps trit k in its top bits (mod 256) */
      if (i < 160) x = (uint8_t)(b[i % 32] * pow3[i / 32]);
      else if (i < 240) x = (uint8_t)(b[32 + (i - 160) % 16] * pow3[(i - 160) / 16]);
      else x = (uint8_t)(b[48 + (i - 240) % 4] * pow3[(i - 240) / 4]);
      const int trit = ((int)x * 3) >> 8;
      return fp16_at(b + 52) * (float)(trit - 1);
    }
    /* The lattice-grid types (quant.h:95-115).  A grid point holds 8 (IQ2, IQ1) or 4
     * (IQ3) magnitudes; iq_grids.h packs each point into codes (its header gives the
     * value of each code).  Signs: a 7-bit index whose parity is the eighth bit, or
     * a sign byte; bit e of it negates element e of the 8-element group. */
    case ORC_IQ2_XXS: { /* 66 bytes: d @0, then per 32 elements 4 point bytes and a u32 of 4 x 7-bit sign indices + 4-bit scale */
      const uint8_t* b = row + (size_t)(col / 256) * 66;
      const int grp = i / 32, sub = (i % 32) / 8, e = i % 8;
      const uint32_t pts = rd32(b + 2 + 8 * grp), aux = rd32(b + 6 + 8 * grp);
      const float db = fp16_at(b) * (0.5f + (float)(aux >> 28)) * 0.25f;
      const float mag = iq2_mag(tm_iq2xxs_grid[(pts >> (8 * sub)) & 255], e);
      return (db * mag) * sign_of(parity_byte((aux >> (7 * sub)) & 127), e);
    }
    case ORC_IQ2_XS: { /* 74 bytes: d @0, 32 x u16 @2 (9-bit point, 7-bit sign index), 4-bit scales @66 */
      const uint8_t* b = row + (size_t)(col / 256) * 74;
      const int k = i / 8, e = i % 8, s16 = i / 16;
      const uint32_t q = rd16(b + 2 + 2 * k);
      const float db = fp16_at(b) * (0.5f + (float)((b[66 + s16 / 2] >> (4 * (s16 % 2))) & 15)) * 0.25f;
      return (db * iq2_mag(tm_iq2xs_grid[q % 512], e)) * sign_of(parity_byte(q >> 9), e);
    }
    case ORC_IQ2_S: { /* 82 bytes: d @0, point low bytes @2, sign bytes @34, point high 2-bit pairs @66, scales @74 */
      const uint8_t* b = row + (size_t)(col / 256) * 82;
      const int k = i / 8, e = i % 8, s16 = i / 16;
      const float db = fp16_at(b) * (0.5f + (float)((b[74 + s16 / 2] >> (4 * (s16 % 2))) & 15)) * 0.25f;
      const int pt = b[2 + k] + 256 * ((b[66 + k / 4] >> (2 * (k % 4))) & 3);
      return (db * iq2_mag(tm_iq2s_grid[pt], e)) * sign_of(b[34 + k], e);
    }
    case ORC_IQ3_XXS: { /* 98 bytes: d @0, point bytes @2 (4 elements each), per 32 elements a u32 @66 */
      const uint8_t* b = row + (size_t)(col / 256) * 98;
      const int grp = i / 32, sub = (i % 32) / 8, e = i % 8;
      const uint32_t aux = rd32(b + 66 + 4 * grp);
      const float db = fp16_at(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
      const int code = (tm_iq3xxs_grid[b[2 + i / 4]] >> (3 * (i % 4))) & 7;
      const float mag = code == 7 ? 62.f : (float)(8 * code + 4);
      return (db * mag) * sign_of(parity_byte((aux >> (7 * sub)) & 127), e);
    }
    case ORC_IQ3_S: { /* 110 bytes: d @0, point low bytes @2, point high bits @66, sign bytes @74, 4-bit scales @106 */
      const uint8_t* b = row + (size_t)(col / 256) * 110;
      const int grp = i / 32, k = i / 4;
      const float db = fp16_at(b) * (float)(1 + 2 * ((b[106 + grp / 2] >> (4 * (grp % 2))) & 15));
      const int pt = b[2 + k] + 256 * ((b[66 + k / 8] >> (k % 8)) & 1);
      const int code = (tm_iq3s_grid[pt] >> (3 * (i % 4))) & 7;
      return (db * (float)(2 * code + 1)) * sign_of(b[74 + i / 8], i % 8);
    }
    case ORC_IQ1_S: { /* 50 bytes: d @0, point low bytes @2, per 32 elements a u16 @34 (3 x 3 high bits ..., scale, delta sign) */
      const uint8_t* b = row + (size_t)(col / 256) * 50;
      const int grp = i / 32, k = i / 8, e = i % 8;
      const uint32_t qh = rd16(b + 34 + 2 * grp);
      const float dl = fp16_at(b) * (float)(2 * ((qh >> 12) & 7) + 1);
      const float delta = (qh & 0x8000u) ? -0.125f : 0.125f;
      const int pt = b[2 + k] + 256 * (int)((qh >> (3 * (k % 4))) & 7);
      return dl * ((float)iq1_val(tm_iq1s_grid[pt], e) + delta);
    }
    case ORC_IQ1_M: { /* 56 bytes: point low bytes @0, high nibbles @32, 4 x u16 @48: 3-bit scales + fp16 d in the top nibbles */
      const uint8_t* b = row + (size_t)(col / 256) * 56;
      const int k = i / 8, e = i % 8, s16 = i / 16;
      const uint32_t d16 = (rd16(b + 48) >> 12) | ((rd16(b + 50) >> 12) << 4) | ((rd16(b + 52) >> 12) << 8) |
                           ((rd16(b + 54) >> 12) << 12);
      const float dl = orc_h2f((uint16_t)d16) * (float)(2 * ((rd16(b + 48 + 2 * (s16 / 4)) >> (3 * (s16 % 4))) & 7) + 1);
      const int hi = (b[32 + k / 2] >> (4 * (k % 2))) & 15;
      const float delta = (hi & 8) ? -0.125f : 0.125f;
      const int pt = b[k] + 256 * (hi & 7);
      return dl * ((float)iq1_val(tm_iq1s_grid[pt], e) + delta);
    }
    default: return 0.f;
  }
}

void orc_dequant(const uint8_t* W, int type, size_t rb, int cols, size_t r0, size_t nrows,
                 void* out, int out_dtype) {
  const size_t n = nrows * (size_t)cols;
  for (size_t i = 0; i < n; ++i) {
    const float v = orc_q_val(W + (r0 + i / (size_t)cols) * rb, type, (int)(i % (size_t)cols));
    if (out_dtype == ORC_OUT_F32) ((float*)out)[i] = v;
    else if (out_dtype == ORC_OUT_F16) ((uint16_t*)out)[i] = orc_f2h(v);
    else ((uint16_t*)out)[i] = orc_f2bf(v);
  }
}

void orc_gemv_f64(const uint8_t* W, int type, size_t rb, const float* x, double* y, int N, int K) {
  for (int r = 0; r < N; ++r) {
    const uint8_t* w = W + (size_t)r * rb;
    double acc = 0.0;
    for (int k = 0; k < K; ++k) acc += (double)orc_q_val(w, type, k) * (double)x[k];
    y[r] = acc;
  }
}

void orc_gemv_lanes(const uint8_t* W, int type, size_t rb, const float* x, float* y, int N, int K,
                    int wave) {
  float acc[128];
  if (wave < 1 || wave > 128) return;
  for (int r = 0; r < N; ++r) {
    const uint8_t* w = W + (size_t)r * rb;
    for (int l = 0; l < wave; ++l) {
      float a = 0.f;
      for (int k = l; k < K; k += wave) a = fmaf(orc_q_val(w, type, k), x[k], a);
      acc[l] = a;
    }
    for (int o = wave / 2; o > 0; o /= 2)
      for (int l = 0; l < o; ++l) acc[l] = acc[l] + acc[l + o];
    y[r] = acc[0];
  }
}

void orc_split3_f16(const float* x, uint16_t* parts, size_t n, size_t stride, int order) {
  for (size_t i = 0; i < n; ++i) {
    const float v = x[i];
    const uint16_t h = orc_f2h(v);
    const float r = v - orc_h2f(h);
    const uint16_t m = orc_f2h(r);
    const uint16_t l = orc_f2h(r - orc_h2f(m));
    if (order == 0) {
      parts[i] = h; parts[i + stride] = m; parts[i + 2 * stride] = l;
    } else {
      parts[i] = l; parts[i + stride] = m; parts[i + 2 * stride] = h;
    }
  }
}

int32_t orc_x3s_row_exp(const float* v, int cols) {
  float amax = 0.f;
  for (int k = 0; k < cols; ++k) {
    const float a = fabsf(v[k]);
    if (a > amax) amax = a;
  }
  if (!(amax > 0.f) || !isfinite(amax)) return 0;
  int ex;
  frexpf(amax, &ex); /* amax = f * 2^ex, f in [0.5,1): floor(log2 amax) = ex-1 */
  int e = 15 - ex;
  if (e < -100) e = -100;
  if (e > 100) e = 100;
  return e;
}

void orc_x3s_split(const float* v, uint16_t* hi, uint16_t* lo, int32_t* exps, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    const float* row = v + (size_t)r * cols;
    const int32_t e = orc_x3s_row_exp(row, cols);
    exps[r] = e;
    for (int k = 0; k < cols; ++k) {
      const float s = ldexpf(row[k], e);
      const uint16_t h = orc_f2h(s);
      hi[(size_t)r * cols + k] = h;
      lo[(size_t)r * cols + k] = orc_f2h(s - orc_h2f(h));
    }
  }
}

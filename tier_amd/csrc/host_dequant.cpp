// host_dequant.cpp -- q_val on the host, for the tools that compare a quantized
// base with its source (the --tq-check metrics) without a GPU.
//
// Element values follow q_val (quant.h:59-121) for every type except the
// lattice-grid IQ2/IQ3/IQ1 families: F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1,
// Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NF4,
// FP4.  Compiled without floating-point contraction, so (d*sc)*v - dmin*m rounds
// exactly as the reference's expression does (every product is exact; one
// rounding).
#include <cmath>
#include <cstdint>
#include <cstring>

#include "tm_host.h"

using namespace tiermm;

namespace {

inline float u2f(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
inline uint32_t rd32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// binary16 -> binary32 by fields: subnormals normalised, inf / NaN payloads kept
// (quant.h:37-42).
float f16(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u;
  uint32_t m = h & 1023u;
  if (e == 0) {
    if (!m) return u2f(s);
    int k = 0;  // shifts until the implicit bit appears
    while (!(m & 1024u)) {
      m <<= 1;
      ++k;
    }
    return u2f(s | ((uint32_t)(113 - k) << 23) | ((m & 1023u) << 13));
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112u) << 23) | (m << 13));
}

void scale_min(int j, const uint8_t* q, int& sc, int& mn) {  // 6-bit pairs, quant.h:47-48
  if (j < 4) {
    sc = q[j] & 63;
    mn = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// Levels of the non-uniform 4-bit codes (formats fixed by their definitions).
const int8_t kIq4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};  // IQ4_NL, IQ4_XS
const float kNf4[16] = {-1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
                        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
                        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
                        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};  // bitsandbytes NF4
const float kFp4[16] = {0.0f, 0.0052083333f, 0.6666667f, 1.0f, 0.33333334f, 0.5f, 0.16666667f, 0.25f,
                        -0.0f, -0.0052083333f, -0.6666667f, -1.0f, -0.33333334f, -0.5f, -0.16666667f, -0.25f};  // bitsandbytes FP4
// MXFP4: E2M1 code as an integer twice its value (code 8 is +0)
int mxfp4_twice(int v) {
  const int e = (v >> 1) & 3, m = v & 1, t = e == 0 ? m : (2 + m) << (e - 1);
  return (v & 8) ? -t : t;
}
// 2^(e-128) for the E8M0 byte e (the MXFP4 block scale, halved for the doubled levels)
float e8m0_half(int e) { return std::ldexp(1.0f, e - 128); }

float value(const uint8_t* row, int type, int col) {
  switch (type) {
    case QT_F32: return u2f(rd32(row + (size_t)col * 4));
    case QT_F16: return f16(rd16(row + (size_t)col * 2));
    case QT_BF16: return u2f((uint32_t)rd16(row + (size_t)col * 2) << 16);
    case QT_Q4_0: {
      const uint8_t* b = row + (size_t)(col >> 5) * 18;
      const int i = col & 31, v = (b[2 + (i & 15)] >> (4 * (i >> 4))) & 15;
      return f16(rd16(b)) * (float)(v - 8);
    }
    case QT_Q4_1: {
      const uint8_t* b = row + (size_t)(col >> 5) * 20;
      const int i = col & 31, v = (b[4 + (i & 15)] >> (4 * (i >> 4))) & 15;
      return f16(rd16(b)) * (float)v + f16(rd16(b + 2));
    }
    case QT_Q5_0: {
      const uint8_t* b = row + (size_t)(col >> 5) * 22;
      const int i = col & 31;
      const int v = ((b[6 + (i & 15)] >> (4 * (i >> 4))) & 15) | (int)(((rd32(b + 2) >> i) & 1u) << 4);
      return f16(rd16(b)) * (float)(v - 16);
    }
    case QT_Q5_1: {
      const uint8_t* b = row + (size_t)(col >> 5) * 24;
      const int i = col & 31;
      const int v = ((b[8 + (i & 15)] >> (4 * (i >> 4))) & 15) | (int)(((rd32(b + 4) >> i) & 1u) << 4);
      return f16(rd16(b)) * (float)v + f16(rd16(b + 2));
    }
    case QT_Q8_0: {
      const uint8_t* b = row + (size_t)(col >> 5) * 34;
      return f16(rd16(b)) * (float)(int8_t)b[2 + (col & 31)];
    }
    case QT_IQ4_NL: {
      const uint8_t* b = row + (size_t)(col >> 5) * 18;
      const int i = col & 31, v = (b[2 + (i & 15)] >> (4 * (i >> 4))) & 15;
      return f16(rd16(b)) * (float)kIq4[v];
    }
    case QT_MXFP4: {
      const uint8_t* b = row + (size_t)(col >> 5) * 17;
      const int i = col & 31, v = (b[1 + (i & 15)] >> (4 * (i >> 4))) & 15;
      return e8m0_half(b[0]) * (float)mxfp4_twice(v);
    }
    case QT_NF4:
    case QT_FP4: {
      const uint8_t* b = row + (size_t)(col >> 6) * 36;
      const int i = col & 63;
      const uint8_t y = b[4 + (i >> 1)];
      const int v = (i & 1) ? (y & 15) : (y >> 4);
      return (type == QT_NF4 ? kNf4[v] : kFp4[v]) * u2f(rd32(b));
    }
    case QT_Q2_K: {
      const uint8_t* b = row + (size_t)(col >> 8) * 84;
      const int i = col & 255, q = (b[16 + (i >> 7) * 32 + (i & 31)] >> (2 * ((i & 127) >> 5))) & 3;
      const uint8_t sc = b[i >> 4];
      return (f16(rd16(b + 80)) * (float)(sc & 15)) * (float)q - f16(rd16(b + 82)) * (float)(sc >> 4);
    }
    case QT_Q3_K: {
      const uint8_t* b = row + (size_t)(col >> 8) * 110;
      const int i = col & 255, j = i >> 4;
      const uint8_t* s = b + 96;
      const int sc = ((j < 8 ? (s[j] & 15) : (s[j - 8] >> 4)) | (((s[8 + (j & 3)] >> (2 * (j >> 2))) & 3) << 4)) - 32;
      const int ql = (b[32 + (i >> 7) * 32 + (i & 31)] >> (2 * ((i & 127) >> 5))) & 3;
      const int sub = ((b[i & 31] >> (i >> 5)) & 1) ? 0 : 4;
      return (f16(rd16(b + 108)) * (float)sc) * (float)(ql - sub);
    }
    case QT_IQ4_XS: {
      const uint8_t* b = row + (size_t)(col >> 8) * 136;
      const int i = col & 255, j = i >> 5;
      const int sc = (((b[4 + (j >> 1)] >> (4 * (j & 1))) & 15) | (((rd16(b + 2) >> (2 * j)) & 3) << 4)) - 32;
      const int v = (b[8 + j * 16 + (i & 15)] >> (4 * ((i & 31) >> 4))) & 15;
      return (f16(rd16(b)) * (float)sc) * (float)kIq4[v];
    }
    case QT_TQ2_0: {
      const uint8_t* b = row + (size_t)(col >> 8) * 66;
      const int i = col & 255, q = (b[(i >> 7) * 32 + (i & 31)] >> (2 * ((i & 127) >> 5))) & 3;
      return f16(rd16(b + 64)) * (float)(q - 1);
    }
    case QT_TQ1_0: {
      const uint8_t* b = row + (size_t)(col >> 8) * 54;
      const int i = col & 255;
      static const int p3[5] = {1, 3, 9, 27, 81};
      uint8_t x;
      if (i < 160) x = (uint8_t)(b[i & 31] * p3[i >> 5]);
      else if (i < 240) x = (uint8_t)(b[32 + ((i - 160) & 15)] * p3[(i - 160) >> 4]);
      else x = (uint8_t)(b[48 + ((i - 240) & 3)] * p3[(i - 240) >> 2]);
      return f16(rd16(b + 52)) * (float)((((int)x * 3) >> 8) - 1);
    }
    case QT_Q4_K: {
      const uint8_t* b = row + (size_t)(col >> 8) * 144;
      const int i = col & 255, j = i >> 6, l = i & 63;
      int sc, mn;
      scale_min(2 * j + (l >= 32), b + 4, sc, mn);
      const uint8_t y = b[16 + j * 32 + (l & 31)];
      const int v = l < 32 ? (y & 15) : (y >> 4);
      return (f16(rd16(b)) * (float)sc) * (float)v - f16(rd16(b + 2)) * (float)mn;
    }
    case QT_Q5_K: {
      const uint8_t* b = row + (size_t)(col >> 8) * 176;
      const int i = col & 255, j = i >> 6, l = i & 63;
      int sc, mn;
      scale_min(2 * j + (l >= 32), b + 4, sc, mn);
      const uint8_t y = b[48 + j * 32 + (l & 31)];
      const int v = (l < 32 ? (y & 15) : (y >> 4)) | (((b[16 + (i & 31)] >> (i >> 5)) & 1) << 4);
      return (f16(rd16(b)) * (float)sc) * (float)v - f16(rd16(b + 2)) * (float)mn;
    }
    case QT_Q6_K: {
      const uint8_t* b = row + (size_t)(col >> 8) * 210;
      const int i = col & 255, a = i >> 7, c = i & 63, half = (i & 127) >> 6, s = (i & 127) >> 5, l = i & 31;
      const int ql = (b[a * 64 + c] >> (4 * half)) & 15, qh = (b[128 + a * 32 + l] >> (2 * s)) & 3;
      const int q = (int)(int8_t)(uint8_t)(ql | (qh << 4)) - 32;
      return (f16(rd16(b + 208)) * (float)(int8_t)b[192 + (i >> 4)]) * (float)q;
    }
    default: return 0.f;
  }
}

}  // namespace

extern "C" int tiermm_dequant_host(const void* W, int qtype, size_t rb, int cols, size_t nrows, float* out) {
  switch (qtype) {
    case QT_F32: case QT_F16: case QT_BF16: case QT_Q4_0: case QT_Q4_1: case QT_Q5_0: case QT_Q5_1:
    case QT_Q8_0: case QT_Q2_K: case QT_Q3_K: case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: case QT_IQ4_NL:
    case QT_IQ4_XS: case QT_TQ1_0: case QT_TQ2_0: case QT_MXFP4: case QT_NF4: case QT_FP4: break;
    default: return set_error(TIERMM_UNSUPPORTED, "tiermm_dequant_host: type %d", qtype);
  }
  const BlockInfo* b = block_info(qtype);
  if (cols <= 0 || cols % b->elems || rb != (size_t)(cols / b->elems) * b->bytes)
    return set_error(TIERMM_EINVAL, "tiermm_dequant_host: rb %zu does not match %d columns", rb, cols);
  if (nrows && (!W || !out)) return set_error(TIERMM_EINVAL, "tiermm_dequant_host: null buffer");
  for (size_t r = 0; r < nrows; ++r) {
    const uint8_t* row = (const uint8_t*)W + r * rb;
    for (int c = 0; c < cols; ++c) out[r * cols + c] = value(row, qtype, c);
  }
  return TIERMM_OK;
}

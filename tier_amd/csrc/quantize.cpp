// quantize.cpp -- host quantizers for Q8_0, Q4_K, Q5_K and Q6_K rows.
//
// Restates the reference's CPU quantizers (quant.h:123-204: q_f2h, q_nearest,
// q8_0_row, q_qkx2, qk_minmax_row, q_qx, q6_k_row, q_row), which follow
// ggml's make_qkx2_quants / make_qx_quants recipes.  Output bytes must be
// identical to the reference's, so every fp32 expression keeps the reference's
// association order, and this file is compiled with -ffp-contract=off (a fused
// multiply-add would round differently).  Used to produce quantized weights on
// the host (tests, bench inputs, tier --quantize equivalent).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "tm_host.h"

namespace tiermm {
namespace {

inline uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// binary32 -> binary16 with round-to-nearest-even (quant.h:124-131 for finite inputs).
uint16_t half_rne(float f) {
  const uint32_t u = fbits(f), sgn = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sgn | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
  if (a >= 0x477ff000u) return (uint16_t)(sgn | 0x7c00u);
  if (a >= 0x38800000u) {
    uint32_t h = (((a >> 23) - 112u) << 10) | ((a >> 13) & 1023u);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sgn | h);
  }
  if (a <= 0x33000000u) return (uint16_t)sgn;
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  const int sh = 126 - (int)(a >> 23);
  uint32_t q = mant >> sh;
  const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return (uint16_t)(sgn | q);
}

// binary16 -> binary32, exact.
float half_to_float(uint16_t h) {
  const uint32_t sgn = h >> 15, e = (h >> 10) & 31u, m = h & 1023u;
  float v = (e == 0u) ? std::ldexp((float)m, -24) : std::ldexp((float)(m | 1024u), (int)e - 25);
  return sgn ? -v : v;
}

inline void put_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

// Nearest integer by the 1.5*2^23 addition (quant.h:133).  For |f| >= 2^22 the
// result is what the bit trick yields, not rint(f): the quantizers clamp it
// afterwards, and byte parity needs the same value.
inline int nearest_int(float f) {
  const float v = f + 12582912.f;
  int32_t i;
  std::memcpy(&i, &v, 4);
  return (i & 0x007fffff) - 0x00400000;
}

// 6-bit scale/min pair s of a K-quant super-block (quant.h:47-48).
inline void scale_min_6bit(int s, const uint8_t* q, int& sc, int& mn) {
  if (s < 4) {
    sc = q[s] & 63;
    mn = q[s + 4] & 63;
  } else {
    sc = (q[s + 4] & 15) | ((q[s - 4] >> 6) << 4);
    mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
  }
}

// Q8_0 row (quant.h:134-136): d = absmax/127 stored as fp16, q = round(v/d) with
// the fp32 reciprocal of the unrounded d.
void row_q8_0(const float* x, uint8_t* o, int k) {
  for (int b = 0; b < k / 32; ++b, o += 34) {
    const float* v = x + b * 32;
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(v[j]));
    const float d = amax / 127.f, id = d != 0.f ? 1.f / d : 0.f;
    put_u16(o, half_rne(d));
    for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)std::roundf(v[j] * id);
  }
}

// Weighted asymmetric fit of one 32-element sub-block to levels 0..nmax with a
// scale and a non-positive minimum (quant.h:138-152, ggml make_qkx2_quants):
// start from the min/max grid, then try nstep+1 rescaled grids and keep the
// least-squares (scale, min) of the best one.
float fit_scale_min(int n, int nmax, const float* x, const float* w, uint8_t* L, float* the_min,
                    uint8_t* Laux, float rmin, float rdelta, int nstep) {
  float mn = x[0], mx = x[0], sw = w[0], sx = sw * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < mn) mn = x[i];
    if (x[i] > mx) mx = x[i];
    sw += w[i];
    sx += w[i] * x[i];
  }
  if (mn > 0) mn = 0;
  if (mx == mn) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *the_min = -mn;
    return 0.f;
  }
  float iscale = nmax / (mx - mn), scale = 1 / iscale, best = 0;
  for (int i = 0; i < n; ++i) {
    const int l = nearest_int(iscale * (x[i] - mn));
    L[i] = (uint8_t)std::max(0, std::min(nmax, l));
    const float df = scale * L[i] + mn - x[i];
    best += w[i] * df * df;
  }
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (mx - mn);
    float sl = 0, sl2 = 0, sxl = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * (x[i] - mn));
      l = std::max(0, std::min(nmax, l));
      Laux[i] = (uint8_t)l;
      sl += w[i] * l;
      sl2 += w[i] * l * l;
      sxl += w[i] * l * x[i];
    }
    const float D = sw * sl2 - sl * sl;
    if (D > 0) {
      float ts = (sw * sxl - sx * sl) / D, tm = (sl2 * sx - sl * sxl) / D;
      if (tm > 0) {
        tm = 0;
        ts = sxl / sl2;
      }
      float mad = 0;
      for (int i = 0; i < n; ++i) {
        const float df = ts * Laux[i] + tm - x[i];
        mad += w[i] * df * df;
      }
      if (mad < best) {
        for (int i = 0; i < n; ++i) L[i] = Laux[i];
        best = mad;
        scale = ts;
        mn = tm;
      }
    }
  }
  *the_min = -mn;
  return scale;
}

// Q4_K (nmax 15) / Q5_K (nmax 31) row (quant.h:154-173).
void row_kquant_minmax(const float* x, uint8_t* o, int k, int nmax) {
  const bool q5 = nmax == 31;
  const int BB = q5 ? 176 : 144;
  uint8_t L[256], La[32];
  float w[32], mins[8], scales[8];
  for (int b = 0; b < k / 256; ++b, o += BB) {
    const float* v = x + (size_t)b * 256;
    std::memset(o, 0, BB);
    float s2 = 0;
    for (int l = 0; l < 256; ++l) s2 += v[l] * v[l];
    const float av = std::sqrt(s2 / 256);
    float ms = 0, mm = 0;
    for (int j = 0; j < 8; ++j) {
      for (int l = 0; l < 32; ++l) w[l] = av + std::fabs(v[32 * j + l]);
      scales[j] = fit_scale_min(32, nmax, v + 32 * j, w, L + 32 * j, &mins[j], La, -0.5f * (q5 ? 1 : 2),
                                0.1f, q5 ? 15 : 20);
      ms = std::max(ms, scales[j]);
      mm = std::max(mm, mins[j]);
    }
    const float is = ms > 0 ? 63.f / ms : 0.f, im = mm > 0 ? 63.f / mm : 0.f;
    uint8_t* sc = o + 4;
    for (int j = 0; j < 8; ++j) {
      const int ls = std::min(63, nearest_int(is * scales[j])), lm = std::min(63, nearest_int(im * mins[j]));
      if (j < 4) {
        sc[j] = (uint8_t)ls;
        sc[j + 4] = (uint8_t)lm;
      } else {
        sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
        sc[j] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    const uint16_t hd = half_rne(ms / 63.f), hm = half_rne(mm / 63.f);
    put_u16(o, hd);
    put_u16(o + 2, hm);
    for (int j = 0; j < 8; ++j) {
      int s, m;
      scale_min_6bit(j, sc, s, m);
      const float d = half_to_float(hd) * s;
      if (!d) continue;
      const float dm = half_to_float(hm) * m;
      for (int ii = 0; ii < 32; ++ii) {
        const int l = nearest_int((v[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)std::max(0, std::min(nmax, l));
      }
    }
    if (!q5) {
      for (int j = 0; j < 256; j += 64)
        for (int l = 0; l < 32; ++l) o[16 + j / 2 + l] = (uint8_t)((L[j + l] & 15) | ((L[j + l + 32] & 15) << 4));
    } else {
      uint8_t* qh = o + 16;
      uint8_t* ql = o + 48;
      int m1 = 1, m2 = 2;
      for (int n = 0; n < 256; n += 64) {
        for (int j = 0; j < 32; ++j) {
          int l1 = L[n + j], l2 = L[n + j + 32];
          if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
          if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
          ql[j] = (uint8_t)(l1 | (l2 << 4));
        }
        m1 <<= 2;
        m2 <<= 2;
        ql += 32;
      }
    }
  }
}

// Symmetric weighted fit of n values to levels -nmax..nmax-1 (quant.h:175-185,
// ggml make_qx_quants with weights x^2): the scale that maximises the
// least-squares gain over 19 candidate grids.
float fit_symmetric(int n, int nmax, const float* x, int8_t* L) {
  float amax = 0, mx = 0;
  for (int i = 0; i < n; ++i) {
    const float a = std::fabs(x[i]);
    if (a > amax) { amax = a; mx = x[i]; }
  }
  if (amax < 1e-15f) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = -nmax / mx, sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = std::max(-nmax, std::min(nmax - 1, l));
    L[i] = (int8_t)(l + nmax);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 > 0 ? sumlx / suml2 : 0.f, best = scale * sumlx;
  for (int is = -9; is <= 9; ++is) {
    if (!is) continue;
    iscale = -(nmax + 0.1f * is) / mx;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * x[i]);
      l = std::max(-nmax, std::min(nmax - 1, l));
      const float w = x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; ++i) {
        const int l = nearest_int(iscale * x[i]);
        L[i] = (int8_t)(nmax + std::max(-nmax, std::min(nmax - 1, l)));
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

// Q6_K row (quant.h:186-199).
void row_q6_k(const float* x, uint8_t* o, int k) {
  int8_t L[256];
  float scales[16];
  for (int b = 0; b < k / 256; ++b, o += 210) {
    const float* v = x + (size_t)b * 256;
    std::memset(o, 0, 210);
    float ma = 0, ms = 0;
    for (int j = 0; j < 16; ++j) {
      scales[j] = fit_symmetric(16, 32, v + 16 * j, L + 16 * j);
      const float a = std::fabs(scales[j]);
      if (a > ma) { ma = a; ms = scales[j]; }
    }
    if (ma < 1e-15f) continue;
    const float is = -128.f / ms;
    const uint16_t hd = half_rne(1 / is);
    put_u16(o + 208, hd);
    int8_t* sc = (int8_t*)(o + 192);
    for (int j = 0; j < 16; ++j) sc[j] = (int8_t)std::min(127, nearest_int(is * scales[j]));
    for (int j = 0; j < 16; ++j) {
      const float d = half_to_float(hd) * sc[j];
      if (!d) continue;
      for (int ii = 0; ii < 16; ++ii) {
        const int l = nearest_int(v[16 * j + ii] / d);
        L[16 * j + ii] = (int8_t)(std::max(-32, std::min(31, l)) + 32);
      }
    }
    uint8_t* ql = o;
    uint8_t* qh = o + 128;
    for (int j = 0; j < 256; j += 128) {
      for (int l = 0; l < 32; ++l) {
        const int q1 = L[j + l] & 15, q2 = L[j + l + 32] & 15, q3 = L[j + l + 64] & 15, q4 = L[j + l + 96] & 15;
        ql[l] = (uint8_t)(q1 | (q3 << 4));
        ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
        qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                          ((L[j + l + 96] >> 4) << 6));
      }
      ql += 64;
      qh += 32;
    }
  }
}

bool quantize_row(int qtype, const float* x, uint8_t* o, int k) {
  switch (qtype) {
    case QT_Q8_0: row_q8_0(x, o, k); return true;
    case QT_Q4_K: row_kquant_minmax(x, o, k, 15); return true;
    case QT_Q5_K: row_kquant_minmax(x, o, k, 31); return true;
    case QT_Q6_K: row_q6_k(x, o, k); return true;
    default: return false;
  }
}

}  // namespace

int quantize_rows(int qtype, const float* x, void* out, size_t rows, int cols, int nthreads) {
  if (!x || !out || cols <= 0) return set_error(TIERMM_EINVAL, "tiermm_quantize: null buffer or cols <= 0");
  if (qtype != QT_Q8_0 && qtype != QT_Q4_K && qtype != QT_Q5_K && qtype != QT_Q6_K)
    return set_error(TIERMM_UNSUPPORTED, "tiermm_quantize: type %d has no quantizer", qtype);
  const BlockInfo* bi = block_info(qtype);
  if (cols % bi->elems) return set_error(TIERMM_UNSUPPORTED, "tiermm_quantize: cols %d not a multiple of %d", cols, bi->elems);
  const size_t rb = (size_t)cols / bi->elems * bi->bytes;
  if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
  if ((size_t)nthreads > rows) nthreads = (int)std::max<size_t>(1, rows);
  auto work = [&](int t) {
    const size_t r0 = rows * t / nthreads, r1 = rows * (t + 1) / nthreads;
    for (size_t r = r0; r < r1; ++r) quantize_row(qtype, x + r * cols, (uint8_t*)out + r * rb, cols);
  };
  if (nthreads == 1) {
    work(0);
  } else {
    std::vector<std::thread> th;
    for (int t = 0; t < nthreads; ++t) th.emplace_back(work, t);
    for (auto& h : th) h.join();
  }
  return TIERMM_OK;
}

}  // namespace tiermm

using namespace tiermm;

// Type of one matrix under a quantization recipe (tier.cpp:2701-2713, mirrored
// by tierlm.py:1858-1874).  The recipe names a base type; "_M" recipes raise the
// v_proj and down_proj of the "more" layers to Q6_K -- the first and last eighth
// of the stack and every third layer between -- and "_S" recipes with a Q4_K
// base raise the first four v_proj and the down_proj of the first eighth of the
// layers to Q5_K.  slot: 0..6 = q, k, v, o, gate, up, down; (index, count) =
// the v_proj's rank among the layers that have one and their number for slot 2,
// the layer and the number of layers for slot 6.
extern "C" int tiermm_recipe_type(const char* recipe, int slot, int index, int count) {
  if (!recipe) return set_error(TIERMM_EINVAL, "tiermm_recipe_type: null recipe");
  const std::string r(recipe);
  int base;
  if (r == "Q8_0") base = QT_Q8_0;
  else if (r == "Q6_K") base = QT_Q6_K;
  else if (r.compare(0, 4, "Q5_K") == 0) base = QT_Q5_K;
  else if (r.compare(0, 4, "Q4_K") == 0) base = QT_Q4_K;
  else return set_error(TIERMM_EINVAL, "tiermm_recipe_type: unknown recipe %s", recipe);
  const bool m_rec = r.size() > 2 && r.compare(r.size() - 2, 2, "_M") == 0;
  const bool s_rec = r.size() > 2 && r.compare(r.size() - 2, 2, "_S") == 0;
  if (slot != 2 && slot != 6) return base;
  const int eighth = count / 8;
  const bool raised = index < eighth || index >= 7 * count / 8 || (index >= eighth && (index - eighth) % 3 == 2);
  if (m_rec && raised) return QT_Q6_K;
  const int limit = slot == 2 ? 4 : eighth;  // first four v_proj / first eighth of the down_proj
  if (s_rec && base == QT_Q4_K && index < limit) return QT_Q5_K;
  return base;
}

// qgemm_fused.hip -- fused dequant + x3-ref GEMM for prefill (M > 1): q4_K, q5_K,
// q6_K, q8_0 and q5_0 weights.
//
// Y[M][ldy] (beta)= sum over the parts p of x (lo, mid, hi) of X_p[M][K] * W16[N][K]^T,
// W16 = fp16(q_val(W_n, k)) -- the training path's dq_k<tier_fp16> (tier.cpp:515,
// 293-298) followed by fp3gemm (tier.cpp:922-943) -- without writing W16 to
// memory: the quantized rows are decoded into an LDS B tile as the K loop needs them.
//
// Tiling: a workgroup owns BM=128 rows of X x BN rows of W (BN in 64..160, a
// multiple of 16), one K step of 32 (one sub-block / block) per stage,
// v_mfma_f32_16x16x32_f16.  Optionally K is split KS ways (split-K): workgroup
// kz of a tile covers K steps [kz*nk/KS, (kz+1)*nk/KS) and stores its partial
// sums; a second kernel adds the KS partials in a fixed order.  (BN, KS) comes
// from a cost model per shape (q_plan): rounds of workgroups over the CUs times
// a per-workgroup time.  A wide BN reads fewer x bytes per MFMA, which is the
// consumers' limit (below); split-K keeps the wide tiles numerous enough.  Its 8 waves
// split into 4 consumers and 4 producers, one of each per SIMD, which hand
// stages over through flags in LDS instead of a workgroup barrier:
//   * consumer c multiplies x rows [32c, 32c+32) against all BN columns.  It
//     loads its own A fragments (3 parts x 2 row blocks, 16 bytes per lane) from
//     the pre-split x planes straight into a ring of registers, three stages
//     ahead -- each consumer reads only its rows, so staging x in LDS would buy
//     no reuse;
//   * producer p decodes W rows [p*BN/4, (p+1)*BN/4) into a ring of four B
//     stages in LDS, one or two lanes per row (16 or 32 elements of a K step
//     each).  It loads the bytes of a unit of K steps that share them into
//     registers a few units ahead and decodes each element exactly as q_val,
//     rounded to fp16 (RNE, two elements per v_cvt_pk_f16_f32):
//       q4_K, q5_K  a sub-block pair (two K steps share their 32 qs bytes: low
//                   nibbles, then high nibbles; q5_K's high bits are bit s of
//                   the 32 qh bytes), d*sc*q - dmin*m with one rounding.  Bytes
//                   widen with one mask and convert with v_cvt_f32_ubyte<n>:
//                   2.75 VALU ops per element for q4_K;
//       q6_K        a quarter super-block (four K steps share 64 ql and 32 qh
//                   bytes), d*sc*(q - 32);
//       q8_0, q5_0  one block, d*q and d*(q - 16).
//     Blocks that are only 2-byte aligned (q6_K, q8_0, q5_0) are read as
//     4-byte aligned dwords, each holding a byte the unit needs (so no load
//     reaches past the weight), and realigned with v_alignbit.
// LDS rows hold 32 halfs as four 16-byte chunks, chunk c at slot
// c ^ ((row >> 2) & 3), so the fragment reads (16 rows x 4 chunks) hit
// distinct bank groups.  x comes in K-tiled planes (ktile_index) where the
// caller's x allows it, so a fragment load is one contiguous kilobyte.
//
// F32 (tiermm_qgemm's TIERMM_MODE_F32, the chat prefill semantics, tier.cpp:2358-2359:
// fp32 dequant and an fp32-accurate product): the same kernel with the x3-2x2
// products.  x comes as the hi and lo planes of its two-part split with a power-of-two
// exponent per row; the producers scale each fp32 q_val by its weight row's power of
// two (qrow_exps, from the block scales) and emit hi = fp16(v) and lo = fp16(v - hi)
// into two B planes of the stage (Emit<true>); the consumers run x_lo*W_hi, x_hi*W_lo
// and x_hi*W_hi into one fp32 accumulator and store it scaled back by both exponents.
//
// Measured, q4_K at M = 512 (bench.py lines; x split and split-K reduce included):
// 5120x5120 81 us, 14336x5120 195 us, 5120x14336 204 us, against 97-100,
// 224-234 and 246-254 us when the producers streamed raw bytes through an LDS
// ring by DMA and decoded a stage at a time (one lane per half row, two passes
// at BN = 160).  Cycle counters in a timing copy showed that decoder at ~1450
// cycles per K step, 70 % of the producer's time, with the consumers waiting
// on it for 26 % of theirs; with the register-fed pair decoder the consumers
// wait 9 % and the MFMA issue is the larger part of their K step.
#include <climits>
#include <cstdio>
#include <cstdlib>

#include "tm_device.h"

namespace tiermm {

int device_cus(int* cus);

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int QBM = 128, QBK = 32;
constexpr int QNBR = 4;  // decoded B stages in the LDS ring

// A launch covers up to QG groups (one plain GEMM, or the experts of a routed
// batch): group g multiplies rows [row0[g], row0[g] + rows[g]) of X and Y with
// weight W[g]; its tiles are workgroups [tile0[g], tile0[g+1]).
constexpr int QG = 64;
struct QArgs {
  const uint16_t* X;  // parts at X, X + xs, X + 2 xs (hi, mid, lo; F32: hi, lo), rows of K halfs
  size_t xs;
  size_t xt;          // > 0: the planes are K-tiled (ktile_index) over xt rows
  float* Y;
  size_t rb;
  int ldy, N, K;
  int kcs;      // accumulation chunks (KS == 1): K steps per chunk, each chunk's sum added into Y
  float beta;
  float* P;   // split K: partial sums of split kz at P + kz * ps, rows of N floats
  size_t ps;
  int ngroups;
  int tile0[QG + 1];
  int row0[QG];
  int rows[QG];
  const uint8_t* W[QG];
  // F32 (one group): the exponents of x's rows (x3s_exp) and of the weight's rows
  // (qrow_exps); Y takes acc * 2^-(xexp[m] + wexp[n])
  const int32_t* xexp;
  const int32_t* wexp;
};

// Byte of 16-byte chunk `chunk` (of 4) of B-tile row `row` (64 bytes, 32 halfs of K):
// the chunk index is XORed with (row / 2) % 4, so the 8 rows that one pass of a
// 16-byte LDS access serves (8 lanes, 32 banks) start on 8 distinct bank groups,
// at one chunk (the consumers' fragment reads) and at chunks 0 and 2 of 4 rows
// (producers that write half a row per lane).  (row / 4) % 4 left rows r and r+2
// on one bank group.
__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 64 + ((chunk ^ ((row >> 1) & 3)) * 16)); }

__device__ __forceinline__ void lds_rel(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The four flags at f (16-byte aligned, LDS), one 16-byte read.
typedef int i4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i4 flags_read(const int* f) {
  return *(const volatile __attribute__((address_space(3))) i4*)(size_t)lds_addr(f);
}
// Waits until the four flags at f are all >= v, starting from the values t read
// earlier (flags_read), so the first read can be issued well before the check.  The
// flags only grow, and the data they publish is read after this returns (the empty
// asm keeps those reads below the loop).
__device__ __forceinline__ void flags_wait(const int* f, i4 t, int v) {
  while (min(min(t[0], t[1]), min(t[2], t[3])) < v) {
    __builtin_amdgcn_s_sleep(1);
    t = flags_read(f);
  }
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void poll4(const int* f, int v) { flags_wait(f, flags_read(f), v); }

// ------------------------------------------------------------ decode units
// The producers of the types other than q4_K work a unit of U K steps at a time (the
// steps whose bytes overlap).  Regs<HPL> holds one lane's bytes of a unit -- halves
// h0 .. h0 + HPL - 1 (16 elements each) of its row -- loaded DP units ahead; NL is the
// number of load instructions per unit (every lane issues all of them, so "vmcnt(N)"
// counts units).  decode() gives 16 fp16 of one half of K step k0 + t, each exactly
// q_val (Dec<> in tm_decode.h) rounded to fp16.

__device__ __forceinline__ const uint8_t* floor4(const uint8_t* p) {
  return (const uint8_t*)((uintptr_t)p & ~(uintptr_t)3);
}
__device__ __forceinline__ uint32_t abit(uint32_t hi, uint32_t lo, uint32_t sh) {
  return __builtin_amdgcn_alignbit(hi, lo, sh);
}
// 8 * (p & 3): the bit offset of a 2-byte aligned address within its dword
__device__ __forceinline__ uint32_t sh_of(const uint8_t* p) { return ((uint32_t)(uintptr_t)p & 3u) * 8u; }
// Register loads are plain loads, so the compiler places the waits before the first use
// of each loaded register: a hand-issued load (asm) would leave its destination looking
// ready at once, and a register copy the compiler inserts (at a loop back-edge, say)
// would then read it before the data lands.  Addresses are 4-byte aligned; one
// global_load_dwordx4 / _dwordx2 / _dword each.
// (Global address space, so they are global_load rather than flat loads, which would
// also count against the LDS counter the flag polls wait on.)
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
#define TM_GLOBAL __attribute__((address_space(1)))
#define WAITVM(n) (((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const TM_GLOBAL u32x4a4*)(size_t)p; }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *(const TM_GLOBAL u32x2a4*)(size_t)p; }
__device__ __forceinline__ uint32_t ld4(const void* p) { return *(const TM_GLOBAL uint32_t*)(size_t)p; }

// Four fp32 values as two words of fp16 pairs (RNE).  The empty asm keeps the fp32
// results, so no conversion is folded into the arithmetic before it.
__device__ __forceinline__ void pack4(float f0, float f1, float f2, float f3, uint32_t& lo, uint32_t& hi) {
  asm volatile("" : "+v"(f0), "+v"(f1), "+v"(f2), "+v"(f3));
  const h2v p0 = {(_Float16)f0, (_Float16)f1}, p1 = {(_Float16)f2, (_Float16)f3};
  lo = __builtin_bit_cast(uint32_t, p0);
  hi = __builtin_bit_cast(uint32_t, p1);
}

// An upper bound of |q_val| over block `blk` of a row (the F32 weight row exponent).
// q_val is monotone in the block's code and fp32 rounding is monotone, so q_val's own
// fp32 arithmetic at the extreme codes gives the largest |q_val| those scales allow:
//   q4_K / q5_K (quant.h:83-87): d*sc*q - dmin*m, q in [0, 15] / [0, 31], per sub-block;
//   q6_K (quant.h:88-90): (d*sc)*(q - 32), q - 32 in [-32, 31], per 16 elements;
//   q8_0 (quant.h:68): d*q, q in [-128, 127];  q5_0 (quant.h:66): d*(q - 16), q in [0, 31].
// The bound is the row's max |q_val| when every block holds its extreme codes, and
// above it otherwise: the split never overflows fp16 either way.
template <int QT>
__device__ __forceinline__ float blk_bound(const uint8_t* row, int blk) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
    constexpr float QMAX = QT == QT_Q4_K ? 15.f : 31.f;
    const u32x4 h = *(const u32x4*)(row + (size_t)blk * (QT == QT_Q4_K ? 144 : 176));
    const float d = h2f(h[0] & 0xffffu), dmin = h2f(h[0] >> 16);
    float b = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int sc, mn;
      kq_scale_min(j, h[1], h[2], h[3], sc, mn);
      const float dsc = d * (float)sc, dm = dmin * (float)mn;
      b = fmaxf(b, fmaxf(fabsf(fmaf(dsc, QMAX, -dm)), fabsf(dm)));
    }
    return b;
  } else if constexpr (QT == QT_Q6_K) {
    const uint8_t* b = row + (size_t)blk * 210;
    const uint2 s0 = ld_u64_a2(b + 192), s1 = ld_u64_a2(b + 200);
    const float d = h2f(ld_u16(b + 208));
    int m = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) m = max(m, max(abs((int)(int8_t)byte_at(s0, k)), abs((int)(int8_t)byte_at(s1, k))));
    return fabsf(d * (float)m) * 32.f;
  } else if constexpr (QT == QT_Q8_0) {
    return fabsf(h2f(ld_u16(row + (size_t)blk * 34))) * 128.f;
  } else {
    static_assert(QT == QT_Q5_0, "fused types");
    return fabsf(h2f(ld_u16(row + (size_t)blk * 22))) * 16.f;
  }
}

// Where a producer lane's decoded values go.  x3-ref: fp16 of q_val (RNE) into o.
// F32 (the fp32-dequant semantics of tiermm_qgemm's TIERMM_MODE_F32): v = q_val * 2^e of
// its row, split as x3s_split splits the fp32 dequant -- hi = fp16(v) into o, lo =
// fp16(v - hi) into ol.
// The producers fold 2^e into their block scales (scale()): exact, as scaling by a
// power of two commutes with the rounding of q_val, so put() receives v itself.
template <bool F32>
struct Emit {
  uint32_t o[8], ol[8];
  float sc;  // 2^e of the row (F32)
  __device__ __forceinline__ float scale(float d) const { return F32 ? d * sc : d; }
  __device__ __forceinline__ void put(int k, float f0, float f1, float f2, float f3) {
    if constexpr (!F32) {
      pack4(f0, f1, f2, f3, o[2 * k], o[2 * k + 1]);
    } else {
      float v[4] = {f0, f1, f2, f3};
      asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
      const h2v h0 = {(_Float16)v[0], (_Float16)v[1]}, h1 = {(_Float16)v[2], (_Float16)v[3]};
      float r[4] = {v[0] - (float)h0[0], v[1] - (float)h0[1], v[2] - (float)h1[0], v[3] - (float)h1[1]};
      asm volatile("" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
      const h2v l0 = {(_Float16)r[0], (_Float16)r[1]}, l1 = {(_Float16)r[2], (_Float16)r[3]};
      o[2 * k] = __builtin_bit_cast(uint32_t, h0);
      o[2 * k + 1] = __builtin_bit_cast(uint32_t, h1);
      ol[2 * k] = __builtin_bit_cast(uint32_t, l0);
      ol[2 * k + 1] = __builtin_bit_cast(uint32_t, l1);
    }
  }
};

// 16 bytes at a 2-byte aligned address s, as five dwords from s rounded down to a
// multiple of 4.  Each dword holds a byte of [s, s + 16) (the fifth repeats the fourth
// when s is 4-aligned), so no load reaches past the bytes the weight holds.
struct Win16 {
  u32x4 w;
  uint32_t e;
  __device__ __forceinline__ void issue(const uint8_t* s) {
    const uint8_t* a = floor4(s);
    w = ld16(a);
    e = ld4(((uintptr_t)s & 3) ? a + 16 : a + 12);
  }
  // the 16 bytes as four words; sh = sh_of(s)
  __device__ __forceinline__ void get(uint32_t sh, uint32_t o[4]) const {
    o[0] = abit(w[1], w[0], sh);
    o[1] = abit(w[2], w[1], sh);
    o[2] = abit(w[3], w[2], sh);
    o[3] = abit(e, w[3], sh);
  }
};

template <int QT>
struct Unit;

// q8_0 (quant.h:68): 34-byte blocks (fp16 d, 32 int8), one K step each; element i of
// the block is d * q[i].
template <>
struct Unit<QT_Q8_0> {
  static constexpr int U = 1, DP = 8;
  template <int HPL>
  struct Regs {
    static constexpr int NLD = 3 * HPL;
    uint32_t d[HPL];
    Win16 q[HPL];
    __device__ __forceinline__ void issue(const uint8_t* row, int k0, int h0) {
      const uint8_t* b = row + (size_t)k0 * 34;
#pragma unroll
      for (int i = 0; i < HPL; ++i) {
        d[i] = ld4(floor4(b));
        q[i].issue(b + 2 + 16 * (h0 + i));
      }
    }
    template <class E>
    __device__ __forceinline__ void decode(const uint8_t* row, int k0, int t, int i, int h, E& o) const {
      const uint8_t* b = row + (size_t)k0 * 34;
      const uint32_t sb = sh_of(b);  // the q bytes at b + 2 + 16h sit at bit offset sb ^ 16
      const float dv = o.scale(h2f((d[i] >> sb) & 0xffffu));
      uint32_t w[4];
      q[i].get(sb ^ 16u, w);
      // d*q as fma(d, q + 128, -128d): q + 128 is the byte with its top bit flipped
      // (one xor for four, then v_cvt_f32_ubyte<n>); both forms are the exact d*q
      const float dm = -128.f * dv;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t wb = w[k] ^ 0x80808080u;
        asm volatile("" : "+v"(wb));
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = fmaf(dv, (float)((wb >> (8 * e)) & 0xffu), dm);
        o.put(k, f[0], f[1], f[2], f[3]);
      }
    }
  };
};

// q5_0 (quant.h:66): 22-byte blocks (fp16 d, qh u32, 16 nibble bytes), one K step
// each; element i is d * (((qs[i % 16] >> 4 (i / 16)) & 15 | ((qh >> i) & 1) << 4) - 16).
// Both halves need the whole block: six dwords from its address rounded down.
template <>
struct Unit<QT_Q5_0> {
  static constexpr int U = 1, DP = 8;
  template <int HPL>
  struct Regs {
    static constexpr int NLD = 2;
    u32x4 a;
    u32x2 b;
    __device__ __forceinline__ void issue(const uint8_t* row, int k0, int) {
      const uint8_t* f = floor4(row + (size_t)k0 * 22);
      a = ld16(f);
      b = ld8(f + 16);
    }
    template <class E>
    __device__ __forceinline__ void decode(const uint8_t* row, int k0, int, int, int h, E& o) const {
      const uint32_t sh = sh_of(row + (size_t)k0 * 22);
      // the block as if 4-aligned: S[j] = bytes 4j .. 4j + 3
      const uint32_t S0 = abit(a[1], a[0], sh), S1 = abit(a[2], a[1], sh), S2 = abit(a[3], a[2], sh),
                     S3 = abit(b[0], a[3], sh), S4 = abit(b[1], b[0], sh), S5 = abit(0u, b[1], sh);
      const float dv = o.scale(h2f(S0 & 0xffffu));
      const uint32_t qh = abit(S1, S0, 16);
      const uint32_t qs[4] = {abit(S2, S1, 16), abit(S3, S2, 16), abit(S4, S3, 16), abit(S5, S4, 16)};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t hb = (qh >> (16 * h + 4 * k)) & 15u;
        // bit e of hb to bit 4 of byte e
        const uint32_t v = ((qs[k] >> (4 * h)) & 0x0f0f0f0fu) | (((hb * 0x00204081u) & 0x01010101u) << 4);
        // d*(q - 16) as fma(d, q, -16d): -16d is exact and the fma rounds the same
        // real value once (the product is exact in either form)
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = fmaf(dv, (float)((v >> (8 * e)) & 0xffu), -16.f * dv);
        o.put(k, f[0], f[1], f[2], f[3]);
      }
    }
  };
};

// q5_K (quant.h:85-87): 176-byte super-blocks (16-byte aligned rows); a unit is a
// sub-block pair s, s + 1 (s even), which shares its 32 qs bytes (low nibbles, then
// high) and the 32 qh bytes (bits s and s + 1).  Element = d*sc*q - dmin*m.
template <>
struct Unit<QT_Q5_K> {
  static constexpr int U = 2, DP = 4;
  template <int HPL>
  struct Regs {
    static constexpr int NLD = 1 + 2 * HPL;
    u32x4 hd, qh[HPL], qs[HPL];
    __device__ __forceinline__ void issue(const uint8_t* row, int k0, int h0) {
      const uint8_t* b = row + (size_t)(k0 >> 3) * 176;
      hd = ld16(b);
#pragma unroll
      for (int i = 0; i < HPL; ++i) {
        qh[i] = ld16(b + 16 + 16 * (h0 + i));
        qs[i] = ld16(b + 48 + 32 * ((k0 & 7) >> 1) + 16 * (h0 + i));
      }
    }
    template <class E>
    __device__ __forceinline__ void decode(const uint8_t*, int k0, int t, int i, int, E& o) const {
      const int s = (k0 & 7) + t;
      int sc, mn;
      kq_scale_min(s, hd[1], hd[2], hd[3], sc, mn);
      const float dsc = o.scale(h2f(hd[0] & 0xffffu) * (float)sc), dm = o.scale(h2f(hd[0] >> 16) * (float)mn);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t v = ((qs[i][k] >> (4 * t)) & 0x0f0f0f0fu) | (((qh[i][k] >> s) & 0x01010101u) << 4);
        asm volatile("" : "+v"(v));  // keep the byte word, so each byte converts with v_cvt_f32_ubyte<n>
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = fmaf(dsc, (float)((v >> (8 * e)) & 0xffu), -dm);
        o.put(k, f[0], f[1], f[2], f[3]);
      }
    }
  };
};

// q6_K (quant.h:88-90): 210-byte super-blocks (2-byte aligned); a unit is the four
// sub-blocks 4a .. 4a + 3 (a 128-element half a of the super-block), which share
// ql[64a, 64a + 64), qh[32a, 32a + 32) and scales[8a, 8a + 8).  Sub-block 4a + t,
// element l: q = ((ql[64a + 32(t & 1) + l] >> 4(t >> 1)) & 15 | ((qh[32a + l] >> 2t) & 3)
// << 4) - 32, times d * scale[8a + 2t + l / 16].
template <>
struct Unit<QT_Q6_K> {
  static constexpr int U = 4, DP = 2;
  template <int HPL>
  struct Regs {
    static constexpr int NLD = 2 + 6 * HPL;
    Win16 l0[HPL], l1[HPL], qh[HPL];
    u32x4 sw;  // bytes 192 .. 209 (scales, d), five dwords from 192 rounded down
    uint32_t se;
    __device__ __forceinline__ void issue(const uint8_t* row, int k0, int h0) {
      const uint8_t* b = row + (size_t)(k0 >> 3) * 210;
      const int a = (k0 >> 2) & 1;
#pragma unroll
      for (int i = 0; i < HPL; ++i) {
        l0[i].issue(b + 64 * a + 16 * (h0 + i));
        l1[i].issue(b + 64 * a + 32 + 16 * (h0 + i));
        qh[i].issue(b + 128 + 32 * a + 16 * (h0 + i));
      }
      const uint8_t* f = floor4(b + 192);
      sw = ld16(f);
      se = ld4(f + 16);
    }
    template <class E>
    __device__ __forceinline__ void decode(const uint8_t* row, int k0, int t, int i, int h, E& o) const {
      const uint8_t* b = row + (size_t)(k0 >> 3) * 210;
      const uint32_t sh = sh_of(b);  // every region of the super-block shares it
      const bool a = (k0 & 4) != 0;
      // scale words 2a, 2a + 1 (bytes 8a .. 8a + 7) and d (bytes 16, 17)
      const uint32_t T0 = abit(sw[1], sw[0], sh), T1 = abit(sw[2], sw[1], sh), T2 = abit(sw[3], sw[2], sh),
                     T3 = abit(se, sw[3], sh), T4 = abit(0u, se, sh);
      const uint32_t Tw = t < 2 ? (a ? T2 : T0) : (a ? T3 : T1);
      const int sc = (int)(int8_t)(uint8_t)(Tw >> (16 * (t & 1) + 8 * h));
      const float ds = o.scale(h2f(T4 & 0xffffu) * (float)sc);
      uint32_t wl[4], wh[4];
      (t & 1 ? l1[i] : l0[i]).get(sh, wl);
      qh[i].get(sh, wh);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t v = ((wl[k] >> (4 * (t >> 1))) & 0x0f0f0f0fu) | (((wh[k] >> (2 * t)) & 0x03030303u) << 4);
        // ds*(q - 32) as fma(ds, q, -32ds): -32ds is exact and both forms round the
        // same real value once
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = fmaf(ds, (float)((v >> (8 * e)) & 0xffu), -32.f * ds);
        o.put(k, f[0], f[1], f[2], f[3]);
      }
    }
  };
};

// Flags (stage numbers, slot-major so that one poll reads all four):
//   ready[q % FL][p] = q -- producer p's B rows of stage q are stored;
//   done[q % FL][c] = q  -- consumer c has read stage q's B tile.
// Stage q's B tile is slot q % NBR.  Producer p writes stage q once every
// consumer has read stage q - NBR, the slot's previous user (the q4_K producer
// writes the pair q, q + 1 once stage q + 1 - NBR is read).  That stage is
// below q, its ready published by every producer, so each wait ends; a consumer
// waits only for its own loads and for ready.
template <int QT, int BN, int KS, bool CH, bool F32>
__global__ __launch_bounds__(512) void qgemm_fused_x3ref(const QArgs p) {
  constexpr int NB = BN / 16;
  // x fragments XR stages ahead: the depth is not what limits (2 and 4 time alike), so the
  // wide tiles, whose accumulators need the registers, and the chunked variant keep two
  constexpr int NBR = QNBR, FL = 4, XR = BN > 160 || CH ? 2 : 4, DP = 4;
  constexpr int PR = BN / 4;
  constexpr int LPR = 2 * PR <= 64 ? 2 : 1, HPL = 2 / LPR;  // decode: lanes per row, halves per lane
  constexpr int NL = 1 + HPL;                                // producer loads per sub-block pair
  constexpr int BPART = BN * 64;                     // one B plane of a stage
  constexpr int BSLOT = F32 ? 2 * BPART : BPART;      // F32: the hi plane, then the lo plane
  constexpr int NPART = F32 ? 2 : 3;                  // x planes
  constexpr int FLAGOFF = NBR * BSLOT;
  static_assert(BN % 16 == 0 && BN <= 256, "tile width");
  static_assert(LPR * PR <= 64, "one decode pass per producer");
  static_assert(NBR <= FL && NBR >= 3 && NL * DP <= 63, "ring depths");
  extern __shared__ __attribute__((aligned(16))) uint16_t lds_h[];
  uint8_t* lds = (uint8_t*)lds_h;
  int* ready = (int*)(lds + FLAGOFF);  // [FL][4]: slot-major, one 16-byte read per poll
  int* done = ready + 4 * FL;          // [FL][4]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < 8 * FL) ready[tid] = -1;

  int grp = 0;
  const int nt_all = p.tile0[p.ngroups];
  // split kz of every tile is the kz-th copy of the tile sequence, so both
  // splits of a tile go to the same XCD
  int b = (int)blockIdx.x % nt_all;
  const int kz = (int)blockIdx.x / nt_all;
  if (p.ngroups == 1 && (nt_all & 7) == 0) b = (b & 7) * (nt_all >> 3) + (b >> 3);
  while (grp + 1 < p.ngroups && b >= p.tile0[grp + 1]) ++grp;
  const int tile = b - p.tile0[grp];
  const int ntn = (p.N + BN - 1) / BN;
  const int m0 = (tile / ntn) * QBM, n0 = (tile % ntn) * BN;
  const int M = p.rows[grp];
  const uint16_t* Xg = p.X + (size_t)p.row0[grp] * p.K;
  float* Yg = p.Y + (size_t)p.row0[grp] * p.ldy;
  const uint8_t* Wg = p.W[grp];
  const int nk = p.K / QBK / KS, kq0 = kz * nk;  // this split's K steps (a multiple of 8 for q4_K)
  __syncthreads();  // flags initialised

  if constexpr (QT != QT_Q4_K) if (wave >= 4) {
    // ------------------------------------------------------------ producer
    // LPR lanes per row of the producer's PR, each decoding HPL halves of 16
    // elements of a K step; units of U K steps, DPU units in registers.
    using R = typename Unit<QT>::template Regs<HPL>;
    constexpr int U = Unit<QT>::U, DPU = Unit<QT>::DP;
    const int pw = wave - 4;
    const bool act = lane < LPR * PR;
    const int dr = min(lane / LPR, PR - 1), h0 = (lane % LPR) * HPL;
    const int r = pw * PR + dr;
    const uint8_t* rowp = Wg + (size_t)min(n0 + r, p.N - 1) * p.rb;
    Emit<F32> em;
    em.sc = F32 ? ldexpf(1.f, p.wexp[min(n0 + r, p.N - 1)]) : 1.f;
    const int nu = nk / U;  // units of this split
    R reg[DPU];
    // unit j into register slot u (j >= nu: unit nu - 1 again)
#pragma unroll
    for (int u = 0; u < DPU; ++u) reg[u].issue(rowp, kq0 + U * min(u, nu - 1), h0);
    // The loads are the compiler's (it waits before a loaded register is read); the
    // explicit wait for unit j's loads, DPU - 1 units of loads still in flight, keeps
    // its count exact across the loop.  Every pass of the unrolled body issues one
    // unit of loads, so the count holds past nu too (there the body only re-loads).
    for (int j0 = 0; j0 < nu; j0 += DPU) {
#pragma unroll
      for (int u = 0; u < DPU; ++u) {
        const int j = j0 + u;
        __builtin_amdgcn_s_waitcnt(WAITVM((DPU - 1) * R::NLD));
        if (j < nu) {
          const int k0 = kq0 + U * j;
#pragma unroll
          for (int t = 0; t < U; ++t) {
            const int q = U * j + t;
            if (q >= NBR) poll4(done + 4 * ((q - NBR) % FL), q - NBR);  // slot q % NBR read by all
            if (act) {
              uint8_t* bt = lds + (q % NBR) * BSLOT;
#pragma unroll
              for (int i = 0; i < HPL; ++i) {
                reg[u].decode(rowp, k0, t, i, h0 + i, em);
                const uint32_t* o = em.o;
                *(u32x4*)(bt + swz(r, 2 * (h0 + i))) = u32x4{o[0], o[1], o[2], o[3]};
                *(u32x4*)(bt + swz(r, 2 * (h0 + i) + 1)) = u32x4{o[4], o[5], o[6], o[7]};
                if constexpr (F32) {
                  const uint32_t* ol = em.ol;
                  *(u32x4*)(bt + BPART + swz(r, 2 * (h0 + i))) = u32x4{ol[0], ol[1], ol[2], ol[3]};
                  *(u32x4*)(bt + BPART + swz(r, 2 * (h0 + i) + 1)) = u32x4{ol[4], ol[5], ol[6], ol[7]};
                }
              }
            }
            if (lane == 0) lds_rel(&ready[4 * (q % FL) + pw], q);
          }
        }
        reg[u].issue(rowp, kq0 + U * min(j + DPU, nu - 1), h0);  // the slot of unit j is free again
      }
    }
    return;
  }
  if constexpr (QT == QT_Q4_K) if (wave >= 4) {
    // ------------------------------------------------------------ q4_K producer
    // LPR lanes per row of the producer's PR, each decoding HPL halves of 16
    // elements.  A sub-block pair (K steps q, q + 1 with q even) shares its 32 qs
    // bytes: low nibbles for q, high nibbles for q + 1.  Per pair a lane loads the
    // super-block header and its qs half (or halves) into registers, DP pairs ahead.
    const int pw = wave - 4;
    const bool act = lane < LPR * PR;
    const int dr = min(lane / LPR, PR - 1), h0 = (lane % LPR) * HPL;
    const int r = pw * PR + dr;
    const uint8_t* rowp = Wg + (size_t)min(n0 + r, p.N - 1) * p.rb;
    Emit<F32> em;
    em.sc = F32 ? ldexpf(1.f, p.wexp[min(n0 + r, p.N - 1)]) : 1.f;
    const int np = nk / 2;  // pairs of this split (a multiple of 4)
    u32x4 Hr[DP], Qr[DP][HPL];
    // pair j into register slot u (j >= np: pair np - 1 again, so every pair issues NL loads
    // and the explicit wait's count holds)
    auto issue = [&](int j, u32x4& h, u32x4 (&qv)[HPL]) __attribute__((always_inline)) {
      const int qq = kq0 + 2 * min(j, np - 1);
      const uint8_t* b = rowp + (size_t)(qq >> 3) * 144;
      h = ld16(b);
#pragma unroll
      for (int i = 0; i < HPL; ++i) qv[i] = ld16(b + 16 + 32 * ((qq & 7) >> 1) + 16 * (h0 + i));
    };
#pragma unroll
    for (int u = 0; u < DP; ++u) issue(u, Hr[u], Qr[u]);
    for (int j0 = 0; j0 < np; j0 += DP) {
#pragma unroll
      for (int u = 0; u < DP; ++u) {
        const int j = j0 + u, q = 2 * j;
        __builtin_amdgcn_s_waitcnt(WAITVM(NL * (DP - 1)));  // pair j is in registers
        // B slots of stages q, q + 1: their previous users, q + 1 - NBR and before, read by all
        if (q + 1 >= NBR) poll4(done + 4 * ((q + 1 - NBR) % FL), q + 1 - NBR);
        if (act) {
          const u32x4 H = Hr[u];
          const float d = h2f(H[0] & 0xffffu), dmin = h2f(H[0] >> 16);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            int sc, mn;
            kq_scale_min(((kq0 + q) & 7) + t, H[1], H[2], H[3], sc, mn);
            const float dsc = em.scale(d * (float)sc), dm = em.scale(dmin * (float)mn);
            uint8_t* bt = lds + ((q + t) % NBR) * BSLOT;
#pragma unroll
            for (int i = 0; i < HPL; ++i) {
#pragma unroll
              for (int w = 0; w < 4; ++w) {
                // elements 4w..4w+3 of the half, one per byte (the empty asm keeps the
                // masked word, so each byte converts with v_cvt_f32_ubyte<n>)
                uint32_t v = (Qr[u][i][w] >> (4 * t)) & 0x0f0f0f0fu;
                asm volatile("" : "+v"(v));
                // q_val (quant.h:83-84): both products exact, one rounding; then fp16 RNE
                // (the empty asm keeps the fp32 results, so fma and conversion stay two roundings)
                float f[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) f[b] = fmaf(dsc, (float)((v >> (8 * b)) & 0xffu), -dm);
                em.put(w, f[0], f[1], f[2], f[3]);
              }
              const uint32_t* o = em.o;
              *(u32x4*)(bt + swz(r, 2 * (h0 + i))) = u32x4{o[0], o[1], o[2], o[3]};
              *(u32x4*)(bt + swz(r, 2 * (h0 + i) + 1)) = u32x4{o[4], o[5], o[6], o[7]};
              if constexpr (F32) {
                const uint32_t* ol = em.ol;
                *(u32x4*)(bt + BPART + swz(r, 2 * (h0 + i))) = u32x4{ol[0], ol[1], ol[2], ol[3]};
                *(u32x4*)(bt + BPART + swz(r, 2 * (h0 + i) + 1)) = u32x4{ol[4], ol[5], ol[6], ol[7]};
              }
            }
          }
        }
        if (lane == 0) {
          lds_rel(&ready[4 * (q % FL) + pw], q);
          lds_rel(&ready[4 * ((q + 1) % FL) + pw], q + 1);
        }
        issue(j + DP, Hr[u], Qr[u]);  // the slot of pair j is free again
      }
    }
    return;
  }

  // -------------------------------------------------------------- consumer
  const int c = wave;
  if (m0 + c * 32 >= M) {
    // Every row of this consumer is past the group's (the last tile of a group that is
    // not a multiple of 128 rows): it stores nothing, so it skips the K loop, and its
    // done flags never hold a producer back.
    if (lane < FL) __hip_atomic_store(&done[4 * lane + c], INT_MAX, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return;
  }
  const int fr = lane & 15, fc = lane >> 4;
  const uint32_t fo = swz(fr, fc);
  // A fragment (part, i): row c*32 + 16i + fr of the tile, halfs 8fc.. of stage q
  // K-tiled planes: K step qq of row r at (qq * xt + r) * 32, so a fragment's 16
  // rows are one contiguous kilobyte; row-major: row r at r * K + qq * 32
  const uint16_t* xa[NPART][2];
  const size_t kstep = p.xt ? p.xt * QBK : (size_t)QBK;
#pragma unroll
  for (int part = 0; part < NPART; ++part)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const size_t r = (size_t)min(m0 + c * 32 + i * 16 + fr, M - 1);
      xa[part][i] = p.xt ? p.X + part * p.xs + ((size_t)p.row0[grp] + r) * QBK + 8 * fc
                         : Xg + part * p.xs + r * p.K + 8 * fc;
    }
  u32x4 A[XR][NPART][2];
  auto loadA = [&](int q, u32x4 (&dst)[NPART][2]) __attribute__((always_inline)) {
    const int qq = kq0 + min(q, nk - 1);  // past the end: a re-read, so every stage issues 2 NPART loads
#pragma unroll
    for (int part = 0; part < NPART; ++part)
#pragma unroll
      for (int i = 0; i < 2; ++i) dst[part][i] = ld16(xa[part][i] + (size_t)qq * kstep);
  };
  float4v acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < XR - 1; ++d) loadA(d, A[d]);
  // Stores the accumulators (register i of lane l holds row 4*(l/16) + i, column l%16
  // of a 16x16 block): into Y, Y = acc + beta Y, or split kz's partial sums.  With
  // accumulation chunks (kcs) it runs at the end of each chunk, which adds the
  // chunk's sum into Y (beta = 1 after the first) and starts the next from zero.
  // F32: acc * 2^-(xexp[row] + wexp[col]), the exponents read once per store
  auto scaled = [&](float v, int ea, int eb) __attribute__((always_inline)) {
    return F32 ? ldexpf(v, -(ea + eb)) : v;
  };
  auto store = [&](float beta) __attribute__((always_inline)) {
    int ea[2][4] = {}, eb[NB] = {};
    if constexpr (F32) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ea[i][r] = p.xexp[min(m0 + c * 32 + i * 16 + 4 * (lane >> 4) + r, M - 1)];
#pragma unroll
      for (int j = 0; j < NB; ++j) eb[j] = p.wexp[min(n0 + j * 16 + (lane & 15), p.N - 1)];
    }
    // A consumer whose 32 rows and the tile's BN columns all exist (every tile but the
    // last of a row or column of tiles) stores without per-element tests: one row
    // pointer per register row, the 16-column blocks at immediate offsets from it.
    if (m0 + c * 32 + 32 <= M && n0 + BN <= p.N) {
      const int rb0 = m0 + c * 32 + 4 * (lane >> 4), cb = n0 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t row = (size_t)(rb0 + i * 16 + r);
          float* rp = KS == 1 ? Yg + row * p.ldy + cb : p.P + (size_t)kz * p.ps + row * p.N + cb;
          if (KS == 1 && beta != 0.f) {
#pragma unroll
            for (int j = 0; j < NB; ++j) rp[16 * j] = fmaf(beta, rp[16 * j], scaled(acc[i][j][r], ea[i][r], eb[j]));
          } else {
#pragma unroll
            for (int j = 0; j < NB; ++j) rp[16 * j] = scaled(acc[i][j][r], ea[i][r], eb[j]);
          }
        }
      return;
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int col = n0 + j * 16 + (lane & 15);
      if (col >= p.N) continue;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + c * 32 + i * 16 + 4 * (lane >> 4) + r;
          if (row >= M) continue;
          if constexpr (KS == 1) {
            float* cp = Yg + (size_t)row * p.ldy + col;
            float v = scaled(acc[i][j][r], ea[i][r], eb[j]);
            if (beta != 0.f) v = fmaf(beta, *cp, v);
            *cp = v;
          } else {  // split K: one group; the reduce adds the scaled partials
            p.P[(size_t)kz * p.ps + (size_t)row * p.N + col] = scaled(acc[i][j][r], ea[i][r], eb[j]);
          }
        }
    }
  };
  float chunk_beta = p.beta;
  // B fragments one stage ahead, in two register sets (stage q in set q & 1; XR is
  // even, so the set follows u): stage q + 1's flags are read when stage q starts,
  // checked and its fragments loaded after the first part's MFMAs, so neither the
  // flag read nor the fragment reads stall the MFMA issue.  Stage q's slot is
  // released once its fragments are in registers, before its last MFMAs.
  // (At BN = 160, and with accumulation chunks, the second set does not fit in
  // registers: fragments are read when the stage starts.)  F32: only the hi plane's
  // fragments come a stage ahead; the lo plane's are read when the stage starts and
  // first used by its second part, so the first part's MFMAs cover their latency.
  constexpr bool PIPE = NB <= 8 && !CH;
  static_assert(XR % 2 == 0, "B register sets follow u");
  half8 bf[PIPE ? 2 : 1][NB];
  half8 bl[F32 ? NB : 1];  // F32: the lo plane of the stage
  auto readB = [&](int q, half8 (&dst)[NB]) __attribute__((always_inline)) {
    const uint8_t* bs = lds + (q % NBR) * BSLOT;
#pragma unroll
    for (int j = 0; j < NB; ++j) dst[j] = *(const half8*)(bs + j * 1024 + fo);
  };
  auto readBl = [&](int q) __attribute__((always_inline)) {
    const uint8_t* bs = lds + (q % NBR) * BSLOT + BPART;
#pragma unroll
    for (int j = 0; j < NB; ++j) bl[j] = *(const half8*)(bs + j * 1024 + fo);
  };
  if constexpr (PIPE) {
    poll4(ready, 0);
    readB(0, bf[0]);
  }
  for (int q0 = 0; q0 < nk; q0 += XR) {
#pragma unroll
    for (int u = 0; u < XR; ++u) {
      const int q = q0 + u;
      loadA(q + XR - 1, A[(u + XR - 1) % XR]);
      __builtin_amdgcn_s_waitcnt(WAITVM(2 * NPART * (XR - 1)));  // stage q's fragments are in registers
      if (q < nk) {
        const bool more = PIPE && q + 1 < nk;
        const int* fn = ready + 4 * ((q + 1) % FL);
        i4 t{};
        if (more) t = flags_read(fn);
        if constexpr (!PIPE) {
          poll4(ready + 4 * (q % FL), q);
          readB(q, bf[0]);
        }
        if constexpr (F32) readBl(q);
        const int cur = PIPE ? (u & 1) : 0;  // u is a constant after unrolling
        // parts lo, mid, hi (tier.cpp:940) into one fp32 accumulator; F32: x lo * W hi,
        // x hi * W lo, x hi * W hi (the x3-2x2 products, smallest first)
#pragma unroll
        for (int part = 2; part >= 0; --part) {
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
              const int ap = F32 ? (part == 2 ? 1 : 0) : part;
              const half8 b = F32 && part == 1 ? bl[j] : bf[cur][j];
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, A[u][ap][i]), b, acc[i][j],
                                                                 0, 0, 0);
            }
          if (part == 2) {
            if (lane == 0) lds_rel(&done[4 * (q % FL) + c], q);  // stage q's B tile is in registers
            if (more) {
              flags_wait(fn, t, q + 1);
              readB(q + 1, bf[PIPE ? (u + 1) & 1 : 0]);
            }
          }
        }
      }
    }
    if constexpr (CH) {
      if ((q0 + XR) % p.kcs == 0 && q0 + XR < nk) {  // end of an accumulation chunk
        store(chunk_beta);
        chunk_beta = 1.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};
      }
    }
  }

  store(chunk_beta);
}

// Y (beta)= sum of the KS partial sums, in split order, for rows [0, rows).
__global__ __launch_bounds__(256) void qgemm_splitk_reduce(const float* __restrict__ P, size_t ps, int ks,
                                                          float* __restrict__ Y, int ldy, int rows, int N, float beta) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * N) return;
  float v = P[i];
  for (int z = 1; z < ks; ++z) v += P[z * ps + i];
  float* y = Y + (i / N) * (size_t)ldy + i % N;
  if (beta != 0.f) v = fmaf(beta, *y, v);
  *y = v;
}
// The same, four columns a thread and one row per blockIdx.y (N and ldy multiples of
// 4, P and Y 16-byte aligned): 16-byte loads and stores, no index division.  Each
// element is summed in the same split order.
__global__ __launch_bounds__(256) void qgemm_splitk_reduce4(const float* __restrict__ P, size_t ps, int ks,
                                                           float* __restrict__ Y, int ldy, int N, float beta) {
  const int c4 = blockIdx.x * 256 + threadIdx.x;
  if (4 * c4 >= N) return;
  const size_t i = (size_t)blockIdx.y * N + 4 * c4;
  float4 v = *(const float4*)(P + i);
  for (int z = 1; z < ks; ++z) {
    const float4 t = *(const float4*)(P + z * ps + i);
    v.x += t.x; v.y += t.y; v.z += t.z; v.w += t.w;
  }
  float4* y = (float4*)(Y + (size_t)blockIdx.y * ldy + 4 * c4);
  if (beta != 0.f) {
    const float4 o = *y;
    v.x = fmaf(beta, o.x, v.x); v.y = fmaf(beta, o.y, v.y); v.z = fmaf(beta, o.z, v.z); v.w = fmaf(beta, o.w, v.w);
  }
  *y = v;
}

template <int QT, int BN, int KS, bool CH = false, bool F32 = false>
int launch_q(const QArgs& a, hipStream_t s, const char* who) {
  constexpr size_t lds = QNBR * (size_t)BN * 64 * (F32 ? 2 : 1) + 2 * 4 * 4 * 4;
  static_assert(lds <= 160 * 1024, "LDS budget");
  static std::atomic<uint64_t> attr{0};
  int st = lds_attr_once(attr, (const void*)qgemm_fused_x3ref<QT, BN, KS, CH, F32>, (int)lds, who);
  if (st) return st;
  qgemm_fused_x3ref<QT, BN, KS, CH, F32><<<(unsigned)a.tile0[a.ngroups] * KS, 512, lds, s>>>(a);
  TM_LAUNCH_CHECK(who);
  return TIERMM_OK;
}

// q4_K takes every tile width of kBns; the other types 256, 224, 160, 128 and 64.
template <int QT, int KS>
int launch_q_bn(int bn, const QArgs& a, hipStream_t s, const char* who) {
  if constexpr (QT == QT_Q4_K) {
    switch (bn) {
      case 256: return launch_q<QT, 256, KS>(a, s, who);
      case 224: return launch_q<QT, 224, KS>(a, s, who);
      case 192: return launch_q<QT, 192, KS>(a, s, who);
      case 160: return launch_q<QT, 160, KS>(a, s, who);
      case 128: return launch_q<QT, 128, KS>(a, s, who);
      case 112: return launch_q<QT, 112, KS>(a, s, who);
      case 96: return launch_q<QT, 96, KS>(a, s, who);
      case 80: return launch_q<QT, 80, KS>(a, s, who);
      default: return launch_q<QT, 64, KS>(a, s, who);
    }
  } else {
    switch (bn) {
      case 256: return launch_q<QT, 256, KS>(a, s, who);
      case 224: return launch_q<QT, 224, KS>(a, s, who);
      case 160: return launch_q<QT, 160, KS>(a, s, who);
      case 128: return launch_q<QT, 128, KS>(a, s, who);
      default: return launch_q<QT, 64, KS>(a, s, who);
    }
  }
}

// The F32 (fp32-dequant) kernels: BN 160, 128 or 64 (wider tiles do not keep both B
// planes' fragments in registers) and KS 1, 2 or 4; no accumulation chunks (their
// in-loop store spills at these widths), so K up to 4 x 4096.
template <int QT, int KS>
int launch_q_f32_bn(int bn, const QArgs& a, hipStream_t s, const char* who) {
  switch (bn) {
    case 160: return launch_q<QT, 160, KS, false, true>(a, s, who);
    case 128: return launch_q<QT, 128, KS, false, true>(a, s, who);
    default: return launch_q<QT, 64, KS, false, true>(a, s, who);
  }
}

template <int QT>
int launch_q_plan(int bn, int ks, const QArgs& a, hipStream_t s, const char* who) {
  if (a.xexp) {  // F32
    switch (ks) {
      case 4: return launch_q_f32_bn<QT, 4>(bn, a, s, who);
      case 2: return launch_q_f32_bn<QT, 2>(bn, a, s, who);
      default: return launch_q_f32_bn<QT, 1>(bn, a, s, who);
    }
  }
  if (a.kcs) {  // accumulation chunks: KS = 1, BN = 160 or 128 (wider ones spill with the chunk store)
    if (bn == 160) return launch_q<QT, 160, 1, true>(a, s, who);
    return launch_q<QT, 128, 1, true>(a, s, who);
  }
  switch (ks) {
    case 4: return launch_q_bn<QT, 4>(bn, a, s, who);
    case 2: return launch_q_bn<QT, 2>(bn, a, s, who);
    default: return launch_q_bn<QT, 1>(bn, a, s, who);
  }
}

// Tiles of one BN over the groups' row counts.
long q_tiles(const int* rows, int n, int N, int bn) {
  long t = 0;
  for (int g = 0; g < n; ++g) t += (long)((rows[g] + QBM - 1) / QBM) * ((N + bn - 1) / bn);
  return t;
}

constexpr int kNbn = 9;
constexpr int kBns[kNbn] = {256, 224, 192, 160, 128, 112, 96, 80, 64};
// Per-workgroup time model, us: kRound + kUnit[BN] * BN * (K steps of the split), fitted
// (log least squares, rms error 6 %) to every (BN, KS) of q4_K at M in {256, 512, 1024,
// 2048, 4096} x (N, K) in {5120, 14336, 4096, 1024} x 5120, 5120 x {14336, 4096} on
// MI355X.  Its pick is the measured best in 26 of those 29 shapes and within 2.2 % of
// it in 28.  The other types use the same model.
constexpr double kRound = 4.26;
constexpr double kUnit[kNbn] = {3.83e-3, 3.915e-3, 4.013e-3, 4.277e-3, 4.442e-3, 4.553e-3, 4.723e-3, 5.247e-3, 6.031e-3};
constexpr double kReduceBpus = 2.93e6;  // bytes per us of the split-K reduce
constexpr size_t kMaxPartials = (size_t)1 << 30;  // bytes of split-K partial sums
// KC > 1 plans run 1.12-1.27x their modelled time where the KS plans run 1.03-1.14x
// (q4_K and q5_K at M in {1024, 2048, 4096} x (N, K) in {5120 x 14336, 5120 x 8192,
// 14336 x 8192}): their kernel keeps a shallower x ring, does not pipeline B and
// flushes Y once per chunk.
constexpr double kChunkCost = 1.12;

// KS > 1: the K steps split KS ways, partial sums added by a second kernel; KC > 1:
// each workgroup sums KC consecutive K ranges in turn, adding each range's sum into its
// Y tile (for K beyond one accumulator's chunk when the partial sums would not fit).
struct QPlan {
  int bn, ks, kc;
};

// Weight types the fused kernel decodes, and the K steps of one producer unit: a split
// of K must hold whole units (q4_K: four sub-block pairs, the unroll of its loop).
int fused_unit(int qt) {
  switch (qt) {
    case QT_Q4_K: return 8;
    case QT_Q5_K: return 2;
    case QT_Q6_K: return 4;
    case QT_Q8_0:
    case QT_Q5_0: return 1;
    default: return 0;
  }
}

bool plan_ok(int qt, int bn, int ks, int kc, int K, size_t rows_total, int N, bool split, bool f32) {
  const int unit = fused_unit(qt);
  if (!unit || K % QBK || (K / QBK) % (unit * ks * kc)) return false;
  if (ks > 1 && (!split || kc > 1 || (size_t)ks * rows_total * N * 4 > kMaxPartials)) return false;
  if (ks * kc < acc_chunks(K)) return false;  // each accumulator sums at most the chunk of the x3 GEMMs
  if ((ks != 1 && ks != 2 && ks != 4) || kc < 1 || kc > 8) return false;
  if (kc > 1 && ((K / QBK / kc) % 4 || ks > 1 || (bn != 160 && bn != 128)))
    return false;  // chunks end where the consumer's unrolled steps do; the chunked widths
  if (f32) return kc == 1 && (bn == 160 || bn == 128 || bn == 64);  // the F32 kernels' plans
  if (qt == QT_Q4_K) {
    for (int b : kBns)
      if (b == bn) return true;
    return false;
  }
  return bn == 256 || bn == 224 || bn == 160 || bn == 128 || bn == 64;
}

// (BN, KS, KC) for the fused kernel.  TIERMM_QGEMM_TILE="BN,KS[,KC]" overrides the model
// when the plan is valid for the shape (tests and tuning).
QPlan q_plan(int qt, const int* rows, int n, int N, int K, int cus, bool split, bool f32 = false) {
  size_t rows_total = 0;
  for (int g = 0; g < n; ++g) rows_total += (size_t)rows[g];
  if (const char* e = getenv("TIERMM_QGEMM_TILE")) {
    int bn = 0, ks = 0, kc = 1;
    if (sscanf(e, "%d,%d,%d", &bn, &ks, &kc) >= 2 && plan_ok(qt, bn, ks, kc, K, rows_total, N, split, f32))
      return {bn, ks, kc};
  }
  const int nk = K / QBK;
  QPlan best{0, 0, 0};  // none: the shape does not take the fused kernel
  double best_t = -1;
  const int need = acc_chunks(K);
  for (int i = 0; i < kNbn; ++i)
    for (int ks = 1; ks <= 4; ks *= 2)
      for (int kc : {1, need}) {
        if (!plan_ok(qt, kBns[i], ks, kc, K, rows_total, N, split, f32)) continue;
        const long wg = q_tiles(rows, n, N, kBns[i]) * ks;
        double t = (double)((wg + cus - 1) / cus) * (kRound + kUnit[i] * kBns[i] * nk / ks);
        if (kc > 1) t *= kChunkCost;
        if (ks > 1) t += (double)rows_total * N * 4 * (ks + 1) / kReduceBpus;  // the reduce
        if (best_t < 0 || t < best_t) {
          best_t = t;
          best = {kBns[i], ks, kc};
        }
      }
  return best;
}

// CUs of the current device, or 256 (MI355X) where no device is visible (a size
// query on a host without a GPU); no error is recorded for that case.
int cus_or_default() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  return device_cus(&cus) == TIERMM_OK && cus > 0 ? cus : 256;
}

}  // namespace

// Bytes of split-K partial sums the fused GEMM of one M x N x K problem needs.
size_t qgemm_fused_partials_bytes(int qtype, int M, int N, int K, bool f32) {
  const QPlan pl = q_plan(qtype, &M, 1, N, K, cus_or_default(), true, f32);
  return pl.ks > 1 ? (size_t)pl.ks * M * N * sizeof(float) : 0;
}

// Whether the fused kernel takes n groups of these row counts of a qtype weight: the
// type is decoded in the kernel, some (BN, KS) fits, KS > 1 only when `split` (one
// group with a partial-sum workspace), and every split short enough for one fp32
// accumulator (acc_chunks).  f32: the F32 kernels (one group).
bool qgemm_fusable(int qtype, const int* rows, int n, int N, int K, bool split, bool f32) {
  if (f32 && n != 1) return false;
  return q_plan(qtype, rows, n, N, K, cus_or_default(), split && n == 1, f32).bn != 0;
}

// Fused x3-ref GEMM over n groups (rows[g] rows of x from row0[g], qtype weight W[g]);
// the x planes hold every group's rows (plane stride xs).  A single group may split K,
// with `partials` (qgemm_fused_partials_bytes) holding the partial sums.  xexp and
// wexp given: the F32 kernels (one group, two row-major x planes).
int qgemm_fused_groups(const void* const* W, int qtype, const int* row0, const int* rows, int n, size_t rb,
                       const uint16_t* xparts, size_t xs, size_t xt, float* Y, int ldy, int N, int K, float beta,
                       int cus, hipStream_t s, const char* who, float* partials, const int32_t* xexp,
                       const int32_t* wexp) {
  const bool f32 = xexp != nullptr;
  if (f32 && (n != 1 || !wexp || xt))
    return set_error(TIERMM_EINVAL, "%s: the fp32 kernels take one group of row-major planes", who);
  const QPlan pl = q_plan(qtype, rows, n, N, K, cus, n == 1 && partials != nullptr, f32);
  if (pl.bn == 0) return set_error(TIERMM_UNSUPPORTED, "%s: no fused plan for type %d N=%d K=%d", who, qtype, N, K);
  for (int g0 = 0; g0 < n; g0 += QG) {
    QArgs a{};
    a.X = xparts; a.xs = xs; a.xt = xt; a.Y = Y; a.rb = rb; a.ldy = ldy; a.N = N; a.K = K; a.beta = beta;
    a.kcs = pl.kc > 1 ? K / QBK / pl.kc : 0;
    a.P = partials; a.ps = n == 1 ? (size_t)rows[0] * N : 0;
    a.xexp = xexp; a.wexp = wexp;
    a.ngroups = 0;
    a.tile0[0] = 0;
    for (int g = g0; g < n && g < g0 + QG; ++g) {
      if (rows[g] == 0) continue;
      const int j = a.ngroups++;
      a.row0[j] = row0[g];
      a.rows[j] = rows[g];
      a.W[j] = (const uint8_t*)W[g];
      a.tile0[j + 1] = a.tile0[j] + (int)q_tiles(&rows[g], 1, N, pl.bn);
    }
    if (a.ngroups == 0) continue;
    int st;
    switch (qtype) {
      case QT_Q4_K: st = launch_q_plan<QT_Q4_K>(pl.bn, pl.ks, a, s, who); break;
      case QT_Q5_K: st = launch_q_plan<QT_Q5_K>(pl.bn, pl.ks, a, s, who); break;
      case QT_Q6_K: st = launch_q_plan<QT_Q6_K>(pl.bn, pl.ks, a, s, who); break;
      case QT_Q8_0: st = launch_q_plan<QT_Q8_0>(pl.bn, pl.ks, a, s, who); break;
      default: st = launch_q_plan<QT_Q5_0>(pl.bn, pl.ks, a, s, who); break;
    }
    if (st) return st;
    if (pl.ks > 1) {  // n == 1, kc == 1: rows row0[0].. of Y
      float* y0 = Y + (size_t)row0[0] * ldy;
      if (N % 4 == 0 && ldy % 4 == 0 && rows[0] <= 65535 && ((uintptr_t)y0 & 15) == 0 &&
          ((uintptr_t)partials & 15) == 0 && a.ps % 4 == 0) {
        const dim3 grid((unsigned)((N / 4 + 255) / 256), (unsigned)rows[0]);
        qgemm_splitk_reduce4<<<grid, 256, 0, s>>>(partials, a.ps, pl.ks, y0, ldy, N, beta);
      } else {
        const size_t cnt = (size_t)rows[0] * N;
        qgemm_splitk_reduce<<<(unsigned)((cnt + 255) / 256), 256, 0, s>>>(partials, a.ps, pl.ks, y0, ldy, rows[0], N,
                                                                         beta);
      }
      TM_LAUNCH_CHECK(who);
    }
  }
  return TIERMM_OK;
}

int qgemm_fused(const void* W, int qtype, size_t rb, const uint16_t* xparts, size_t xs, size_t xt, float* Y, int ldy,
                int M, int N, int K, float beta, int cus, hipStream_t s, const char* who, float* partials,
                const int32_t* xexp, const int32_t* wexp) {
  const int row0 = 0;
  return qgemm_fused_groups(&W, qtype, &row0, &M, 1, rb, xparts, xs, xt, Y, ldy, N, K, beta, cus, s, who, partials,
                            xexp, wexp);
}

// wexp[n] = x3s_exp(the bound of row n's |q_val|, blk_bound over its blocks): one wave a
// row, the row's blocks over its lanes.  Only the block scales are read.
template <int QT>
__global__ __launch_bounds__(256) void qrow_exp_kernel(const uint8_t* __restrict__ W, size_t rb, int N, int nblk,
                                                      int32_t* __restrict__ wexp) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const uint8_t* row = W + (size_t)n * rb;
  float b = 0.f;
  for (int i = lane; i < nblk; i += 64) b = fmaxf(b, blk_bound<QT>(row, i));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) b = fmaxf(b, __shfl_xor(b, o, 64));
  if (lane == 0) wexp[n] = x3s_exp(b);
}

// The two passes of the fp32-semantics GEMM in one launch: blocks [0, M) split x's rows
// (x3s_split_row), the rest take four weight rows each for their exponents, as
// qrow_exp_kernel does.  Small products (the chat prefill's chunks of 256 rows) save a
// launch and the gap behind it.
template <int XR, int QT>
__global__ __launch_bounds__(256) void f32_prep_kernel(const float* __restrict__ X, uint16_t* __restrict__ xhi,
                                                      uint16_t* __restrict__ xlo, int32_t* __restrict__ xexp, int M,
                                                      int K, const uint8_t* __restrict__ W, size_t rb, int N,
                                                      int nblk, int32_t* __restrict__ wexp) {
  if ((int)blockIdx.x < M) {
    x3s_split_row<XR>(X, xhi, xlo, xexp, K, blockIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int n = ((int)blockIdx.x - M) * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const uint8_t* row = W + (size_t)n * rb;
  float b = 0.f;
  for (int i = lane; i < nblk; i += 64) b = fmaxf(b, blk_bound<QT>(row, i));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) b = fmaxf(b, __shfl_xor(b, o, 64));
  if (lane == 0) wexp[n] = x3s_exp(b);
}

template <int XR>
int f32_prep_xr(const float* X, uint16_t* xhi, uint16_t* xlo, int32_t* xexp, int M, int K, const void* W, int qtype,
                size_t rb, int N, int32_t* wexp, hipStream_t s) {
  const unsigned grid = (unsigned)(M + (N + 3) / 4);
  const uint8_t* w = (const uint8_t*)W;
  switch (qtype) {
    case QT_Q4_K: f32_prep_kernel<XR, QT_Q4_K><<<grid, 256, 0, s>>>(X, xhi, xlo, xexp, M, K, w, rb, N, K / 256, wexp); break;
    case QT_Q5_K: f32_prep_kernel<XR, QT_Q5_K><<<grid, 256, 0, s>>>(X, xhi, xlo, xexp, M, K, w, rb, N, K / 256, wexp); break;
    case QT_Q6_K: f32_prep_kernel<XR, QT_Q6_K><<<grid, 256, 0, s>>>(X, xhi, xlo, xexp, M, K, w, rb, N, K / 256, wexp); break;
    case QT_Q8_0: f32_prep_kernel<XR, QT_Q8_0><<<grid, 256, 0, s>>>(X, xhi, xlo, xexp, M, K, w, rb, N, K / 32, wexp); break;
    case QT_Q5_0: f32_prep_kernel<XR, QT_Q5_0><<<grid, 256, 0, s>>>(X, xhi, xlo, xexp, M, K, w, rb, N, K / 32, wexp); break;
    default: return set_error(TIERMM_UNSUPPORTED, "f32_prep: type %d", qtype);
  }
  TM_LAUNCH_CHECK("tiermm_qgemm: split x, weight row exponents");
  return TIERMM_OK;
}

// x's two-part split and W's row exponents in one launch where x takes the register
// split (rows of a multiple of 4 up to 16384, 16-byte aligned; parts 8-byte aligned);
// TIERMM_UNSUPPORTED (nothing launched, no error recorded) otherwise.
int f32_prep(const float* X, uint16_t* xhi, uint16_t* xlo, int32_t* xexp, int M, int K, const void* W, int qtype,
             size_t rb, int N, int32_t* wexp, hipStream_t s) {
  if (K % 4 || ((uintptr_t)X & 15) || ((uintptr_t)xhi & 7) || ((uintptr_t)xlo & 7) || K > 16384)
    return TIERMM_UNSUPPORTED;
  if (K <= 4096) return f32_prep_xr<4>(X, xhi, xlo, xexp, M, K, W, qtype, rb, N, wexp, s);
  if (K <= 8192) return f32_prep_xr<8>(X, xhi, xlo, xexp, M, K, W, qtype, rb, N, wexp, s);
  return f32_prep_xr<16>(X, xhi, xlo, xexp, M, K, W, qtype, rb, N, wexp, s);
}

int qrow_exps(const void* W, int qtype, size_t rb, int N, int K, int32_t* wexp, hipStream_t s) {
  const unsigned grid = (unsigned)((N + 3) / 4);
  const uint8_t* w = (const uint8_t*)W;
  switch (qtype) {
    case QT_Q4_K: qrow_exp_kernel<QT_Q4_K><<<grid, 256, 0, s>>>(w, rb, N, K / 256, wexp); break;
    case QT_Q5_K: qrow_exp_kernel<QT_Q5_K><<<grid, 256, 0, s>>>(w, rb, N, K / 256, wexp); break;
    case QT_Q6_K: qrow_exp_kernel<QT_Q6_K><<<grid, 256, 0, s>>>(w, rb, N, K / 256, wexp); break;
    case QT_Q8_0: qrow_exp_kernel<QT_Q8_0><<<grid, 256, 0, s>>>(w, rb, N, K / 32, wexp); break;
    case QT_Q5_0: qrow_exp_kernel<QT_Q5_0><<<grid, 256, 0, s>>>(w, rb, N, K / 32, wexp); break;
    default: return set_error(TIERMM_UNSUPPORTED, "qrow_exps: type %d", qtype);
  }
  TM_LAUNCH_CHECK("tiermm_qgemm: weight row exponents");
  return TIERMM_OK;
}

}  // namespace tiermm

// The plan tiermm_qgemm's fused kernel takes for one MODE_X3REF product of this shape
// (the cost model, or TIERMM_QGEMM_TILE when valid for the shape): tile width, K
// splits and accumulation chunks.
extern "C" int tiermm_qgemm_plan(int qtype, int M, int N, int K, int* bn, int* ks, int* kc) {
  using namespace tiermm;
  if (M < 1 || N < 1 || K < 1 || !bn || !ks || !kc)
    return set_error(TIERMM_EINVAL, "tiermm_qgemm_plan: M=%d N=%d K=%d and three outputs", M, N, K);
  const QPlan pl = q_plan(qtype, &M, 1, N, K, cus_or_default(), true);
  if (!pl.bn) return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemm_plan: type %d N=%d K=%d is not decoded in the GEMM", qtype, N, K);
  *bn = pl.bn;
  *ks = pl.ks;
  *kc = pl.kc;
  return TIERMM_OK;
}

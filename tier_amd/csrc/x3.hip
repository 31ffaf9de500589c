// x3.hip -- split-precision ("x3") fp16 MFMA GEMMs and the split kernels.
//
//  * split3_f16 (split3_fp_k tier.cpp:869-870, split3s_fp16 tier.cpp:2192-2194)
//  * x3s_split: two-part split with a power-of-two exponent per row
//  * gemm_x3 core: C[M][N] = scale * sum over products (p,q) of A_p[M][K] * B_q[N][K]^T,
//    A_p/B_q fp16 row-major with K contiguous ("NT"), fp32 accumulation on
//    v_mfma_f32_32x32x16_f16.  Used with
//      - x3-ref (fp3gemm, chat_fp3): A = x split in hi/mid/lo, B = the fp16
//        weight, products (lo,W) (mid,W) (hi,W) -- the reference's part order
//        (tier.cpp:940);
//      - x3-2x2: A = X hi/lo, B = W hi/lo, products (hi,hi) (hi,lo) (lo,hi),
//        result scaled by 2^-(xexp[m]+wexp[n]).
//
// Tiling: a 256-thread workgroup (4 waves, 2x2) owns a BMxBN output tile; each
// wave a (BM/2)x(BN/2) sub-tile of 32x32 MFMA blocks.  K advances by BK=32 per
// stage through a double-buffered LDS copy of every part tile (one barrier per
// stage; the next stage's global loads are issued before the MFMAs of the
// current one).  LDS rows are 64 data bytes + 16 pad bytes so the 16-byte
// fragment reads of 8 consecutive rows hit distinct banks.
#include <algorithm>
#include <vector>

#include "tm_device.h"

namespace tiermm {

int check_qweight(const char* who, const void* W, int qtype, size_t rb, int cols, int dense_unit);
int dequant_f16_rows(const void* W, int qtype, size_t rb, int cols, size_t nrows, uint16_t* out, hipStream_t s,
                     bool tiled = false);
int dequant_f16_group(const void* const* W, uint16_t* const* out, int n, int qtype, size_t rb, int cols,
                      size_t nrows, hipStream_t s, bool tiled = false);
// Fused dequant + x3-ref GEMM (q4_K, q5_K, q6_K, q8_0, q5_0 weights).  xparts: three
// fp16 planes (stride xs), row-major (xt = 0) or K-tiled over xt rows.
// F32 (xexp and wexp given, one group): two fp16 planes, hi and lo of x's x3s split
// (row-major), and the weight decoded to fp32, scaled by 2^wexp of its row and split
// the same way inside the GEMM (the x3-2x2 products).
int qgemm_fused(const void* W, int qtype, size_t rb, const uint16_t* xparts, size_t xs, size_t xt, float* Y, int ldy,
                int M, int N, int K, float beta, int cus, hipStream_t s, const char* who, float* partials,
                const int32_t* xexp = nullptr, const int32_t* wexp = nullptr);
int qgemm_fused_groups(const void* const* W, int qtype, const int* row0, const int* rows, int n, size_t rb,
                       const uint16_t* xparts, size_t xs, size_t xt, float* Y, int ldy, int N, int K, float beta,
                       int cus, hipStream_t s, const char* who, float* partials, const int32_t* xexp = nullptr,
                       const int32_t* wexp = nullptr);
size_t qgemm_fused_partials_bytes(int qtype, int M, int N, int K, bool f32 = false);
bool qgemm_fusable(int qtype, const int* rows, int n, int N, int K, bool split, bool f32 = false);
// wexp[n] = the x3s exponent of a bound of weight row n's |q_val| (from the block
// scales), rows [0, N) of K columns, for the fused fp32 kernels.
int qrow_exps(const void* W, int qtype, size_t rb, int N, int K, int32_t* wexp, hipStream_t s);
int f32_prep(const float* X, uint16_t* xhi, uint16_t* xlo, int32_t* xexp, int M, int K, const void* W, int qtype,
             size_t rb, int N, int32_t* wexp, hipStream_t s);
int device_cus(int* cus);

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ splits
// BF = false: fp16 parts (split3_fp_k / split3s_fp16); true: bf16 parts with
// hip_bfloat16 rounding (split3_k tier.cpp:866-867, split3s 2159-2161).
template <bool BF>
__global__ __launch_bounds__(256) void split3_kernel(const float* __restrict__ x, uint16_t* __restrict__ parts,
                                                     size_t n, size_t stride, int order) {
  const size_t step = (size_t)gridDim.x * blockDim.x;
  uint16_t* p0 = parts;
  uint16_t* p1 = parts + stride;
  uint16_t* p2 = parts + 2 * stride;
  auto to16 = [](float f) __attribute__((always_inline)) { return BF ? f2bf(f) : f2h(f); };
  auto from16 = [](uint16_t u) __attribute__((always_inline)) {
    return BF ? __uint_as_float((uint32_t)u << 16) : h2f(u);
  };
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const float v = x[i];
    const uint16_t h = to16(v);
    const float r = v - from16(h);
    const uint16_t m = to16(r);
    const uint16_t l = to16(r - from16(m));
    if (order == TIERMM_HML) {
      p0[i] = h; p1[i] = m; p2[i] = l;
    } else {
      p0[i] = l; p1[i] = m; p2[i] = h;
    }
  }
}

// The same split, 8 consecutive elements per thread: two 16-byte loads, one
// 16-byte store per part (n, stride multiples of 8; x and parts 16-byte aligned).
// trows > 0: the parts in the K-tiled layout of planes of trows rows of cols
// elements (ktile_index; cols a multiple of 32), written in unit order.
template <bool BF>
__global__ __launch_bounds__(256) void split3_vec8_kernel(const float* __restrict__ x, uint16_t* __restrict__ parts,
                                                          size_t n8, size_t stride, int order, size_t trows = 0,
                                                          int cols = 0) {
  const size_t step = (size_t)gridDim.x * blockDim.x;
  auto to16 = [](float f) __attribute__((always_inline)) { return BF ? f2bf(f) : f2h(f); };
  auto from16 = [](uint16_t u) __attribute__((always_inline)) {
    return BF ? __uint_as_float((uint32_t)u << 16) : h2f(u);
  };
  uint16_t* ph = parts + (order == TIERMM_HML ? 0 : 2 * stride);
  uint16_t* pm = parts + stride;
  uint16_t* pl = parts + (order == TIERMM_HML ? 2 * stride : 0);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += step) {
    size_t src = 8 * i;  // K-tiled: unit i of the output, gathered from its row
    if (trows) {
      size_t row;
      int col;
      ktile_unit(i, trows, row, col);
      src = row * (size_t)cols + col;
    }
    const float4 a = *(const float4*)(x + src), b = *(const float4*)(x + src + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint16_t hh = to16(v[k]);
      const float r = v[k] - from16(hh);
      const uint16_t mm = to16(r);
      const uint16_t ll = to16(r - from16(mm));
      const int sh = 16 * (k & 1);
      if (sh == 0) {
        h[k >> 1] = hh; m[k >> 1] = mm; l[k >> 1] = ll;
      } else {
        h[k >> 1] |= (uint32_t)hh << 16; m[k >> 1] |= (uint32_t)mm << 16; l[k >> 1] |= (uint32_t)ll << 16;
      }
    }
    const size_t o = 8 * i;
    *(uint4*)(ph + o) = make_uint4(h[0], h[1], h[2], h[3]);
    *(uint4*)(pm + o) = make_uint4(m[0], m[1], m[2], m[3]);
    *(uint4*)(pl + o) = make_uint4(l[0], l[1], l[2], l[3]);
  }
}

// One pass over a row held in registers: 4 consecutive elements per thread and
// step (cols a multiple of 4, at most 1024 * XR; rows 16-byte aligned).
template <int XR>
__global__ __launch_bounds__(256) void x3s_split_reg_kernel(const float* __restrict__ src, uint16_t* __restrict__ hi,
                                                            uint16_t* __restrict__ lo, int32_t* __restrict__ exps,
                                                            int cols) {
  x3s_split_row<XR>(src, hi, lo, exps, cols, blockIdx.x);
}

__global__ __launch_bounds__(256) void x3s_split_kernel(const float* __restrict__ src, uint16_t* __restrict__ hi,
                                                        uint16_t* __restrict__ lo, int32_t* __restrict__ exps,
                                                        int cols) {
  __shared__ float red[4];
  const size_t base = (size_t)blockIdx.x * cols;
  float amax = 0.f;
  for (int k = threadIdx.x; k < cols; k += 256) amax = fmaxf(amax, fabsf(src[base + k]));
  amax = block_max_256(amax, red);
  const int e = x3s_exp(amax);
  const float sc = ldexpf(1.f, e);
  for (int k = threadIdx.x; k < cols; k += 256) {
    const float s = src[base + k] * sc;
    const uint16_t h = f2h(s);
    hi[base + k] = h;
    lo[base + k] = f2h(s - h2f(h));
  }
  if (threadIdx.x == 0) exps[blockIdx.x] = e;
}

// ---- two-part splits for the fp32 product (tiermm_sgemm): the x3s split of rows
// [rows][cols] with row stride ld into rows of kp (zeros past cols), and of the
// columns of a [k][ld] matrix, transposed (op(A) = A in the BLAS column-major view).

// One workgroup per row: e = x3s_exp(max |row|), hi/lo of row * 2^e, kp columns.
__global__ __launch_bounds__(256) void x3s_split_ld_kernel(const float* __restrict__ src, size_t ld, int cols,
                                                           int kp, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                           int32_t* __restrict__ exps) {
  __shared__ float red[4];
  const float* row = src + (size_t)blockIdx.x * ld;
  const size_t base = (size_t)blockIdx.x * kp;
  float amax = 0.f;
  for (int k = threadIdx.x; k < cols; k += 256) amax = fmaxf(amax, fabsf(row[k]));
  amax = block_max_256(amax, red);
  const int e = x3s_exp(amax);
  const float sc = ldexpf(1.f, e);
  for (int k = threadIdx.x; k < kp; k += 256) {
    const float v = k < cols ? row[k] * sc : 0.f;
    const uint16_t h = f2h(v);
    hi[base + k] = h;
    lo[base + k] = f2h(v - h2f(h));
  }
  if (threadIdx.x == 0) exps[blockIdx.x] = e;
}

// n words set to zero (a fill kernel rather than hipMemsetAsync: safe in graph capture).
__global__ __launch_bounds__(256) void zero32_kernel(uint32_t* __restrict__ p, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// amax[c] = max over r < rows of |src[r][c]| (c < cols), as the bits of a non-negative
// float (their integer order is the float order): 256 columns x 256 rows per workgroup.
__global__ __launch_bounds__(256) void col_absmax_kernel(const float* __restrict__ src, size_t ld, int rows, int cols,
                                                         uint32_t* __restrict__ amax) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const int r0 = blockIdx.y * 256, r1 = min(rows, r0 + 256);
  float m = 0.f;
  for (int r = r0; r < r1; ++r) m = fmaxf(m, fabsf(src[(size_t)r * ld + c]));
  atomicMax(amax + c, __float_as_uint(m));
}

// hi/lo[c][r] of src[r][c] * 2^e_c (e_c = x3s_exp(amax[c])) for c < cols, r < kp
// (zeros for r >= rows), through a 64x64 LDS tile; exps[c] = e_c.
__global__ __launch_bounds__(256) void x3s_split_t_kernel(const float* __restrict__ src, size_t ld, int rows, int cols,
                                                          int kp, const uint32_t* __restrict__ amax,
                                                          uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                          int32_t* __restrict__ exps) {
  __shared__ float t[64][65];
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    t[i][tx] = r < rows && c < cols ? src[(size_t)r * ld + c] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (c >= cols || r >= kp) continue;
    const int e = x3s_exp(__uint_as_float(amax[c]));
    const float v = t[tx][i] * ldexpf(1.f, e);
    const uint16_t h = f2h(v);
    hi[(size_t)c * kp + r] = h;
    lo[(size_t)c * kp + r] = f2h(v - h2f(h));
    if (blockIdx.y == 0 && tx == 0) exps[c] = e;
  }
}

// fp16 transpose: dst[c][r] = src[r][c] for r < rows, c < cols (src row stride ld,
// dst row stride dld >= rows), through a 64x64 LDS tile (odd column stride: no bank
// conflicts).
__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ src, int ld,
                                                          uint16_t* __restrict__ dst, int rows, int cols, int dld) {
  __shared__ uint16_t t[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    if (r < rows && c < cols) t[i][tx] = src[(size_t)r * ld + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (r < rows && c < cols) dst[(size_t)c * dld + r] = t[tx][i];
  }
}

// ---- K padding.  The GEMMs step K by 32; when K is not a multiple of 32 the
// operands are copied into the workspace as rows of Kp = roundup(K, 32) with
// zeros in columns [K, Kp), which add nothing to any product.  These copies are
// element-wise: only such shapes use them.

// dst[r][k] = k < K ? src[r * ld + k] : 0 for 16-bit elements, rows x Kp.
__global__ __launch_bounds__(256) void pad16_kernel(const uint16_t* __restrict__ src, size_t ld,
                                                    uint16_t* __restrict__ dst, size_t rows, int K, int Kp) {
  const size_t n = rows * (size_t)Kp, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const size_t r = i / (size_t)Kp;
    const int k = (int)(i - r * (size_t)Kp);
    dst[i] = k < K ? src[r * ld + k] : (uint16_t)0;
  }
}

// The same for fp32 rows.
__global__ __launch_bounds__(256) void pad32_kernel(const float* __restrict__ src, size_t ld, float* __restrict__ dst,
                                                    size_t rows, int K, int Kp) {
  const size_t n = rows * (size_t)Kp, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const size_t r = i / (size_t)Kp;
    const int k = (int)(i - r * (size_t)Kp);
    dst[i] = k < K ? src[r * ld + k] : 0.f;
  }
}

// Columns [K, Kp) of rows x Kp 16-bit rows set to zero (after a transpose into them).
__global__ __launch_bounds__(256) void zero_tail16_kernel(uint16_t* __restrict__ dst, size_t rows, int K, int Kp) {
  const int w = Kp - K;
  const size_t n = rows * (size_t)w, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const size_t r = i / (size_t)w;
    dst[r * Kp + K + (i - r * (size_t)w)] = 0;
  }
}

// The three-part split (split3_fp_k / split3_k) of x[rows][K] (row stride ldx)
// into HML planes of rows x Kp at parts + {0, n, 2n}, n = rows * Kp, zeros past K.
template <bool BF>
__global__ __launch_bounds__(256) void pad_split3_kernel(const float* __restrict__ x, size_t ldx,
                                                         uint16_t* __restrict__ parts, size_t rows, int K, int Kp) {
  auto to16 = [](float f) __attribute__((always_inline)) { return BF ? f2bf(f) : f2h(f); };
  auto from16 = [](uint16_t u) __attribute__((always_inline)) {
    return BF ? __uint_as_float((uint32_t)u << 16) : h2f(u);
  };
  const size_t n = rows * (size_t)Kp, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const size_t r = i / (size_t)Kp;
    const int k = (int)(i - r * (size_t)Kp);
    const float v = k < K ? x[r * ldx + k] : 0.f;
    const uint16_t h = to16(v);
    const float d = v - from16(h);
    const uint16_t m = to16(d);
    parts[i] = h;
    parts[n + i] = m;
    parts[2 * n + i] = to16(d - from16(m));
  }
}

// Dense q_val rows (F32 / F16 / BF16, row bytes rb) to fp16 (F16OUT: RNE, as
// dq_k<tier_fp16>) or fp32 rows of Kp elements, zeros past K.
template <int QT, bool F16OUT>
__global__ __launch_bounds__(256) void dense_pad_kernel(const uint8_t* __restrict__ W, size_t rb,
                                                        void* __restrict__ out, size_t rows, int K, int Kp) {
  const size_t n = rows * (size_t)Kp, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const size_t r = i / (size_t)Kp;
    const int k = (int)(i - r * (size_t)Kp);
    const float v = k < K ? dense_val<QT>(W + r * rb, (size_t)k) : 0.f;
    if (F16OUT) ((uint16_t*)out)[i] = f2h(v);
    else ((float*)out)[i] = v;
  }
}

// Weighted combine of routed expert outputs: out[t][n] = sum_j w[p_j] * Y[p_j][n],
// p_j = token_pairs[t*topk + j], summed in j order (deterministic).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ Y, const int* __restrict__ tp,
                                                          const float* __restrict__ pw, float* __restrict__ out,
                                                          int topk, int N) {
  const int t = blockIdx.x;
  for (int n = threadIdx.x; n < N; n += 256) {
    float acc = 0.f;
    for (int j = 0; j < topk; ++j) {
      const int p = tp[(size_t)t * topk + j];
      acc = fmaf(pw[p], Y[(size_t)p * N + n], acc);
    }
    out[(size_t)t * N + n] = acc;
  }
}
// The same, four columns a thread (N a multiple of 4, Y and out 16-byte aligned, topk
// at most 16): the token's pairs and weights are read once, then 16-byte loads of
// each pair's row; each column is summed in the same j order.
__global__ __launch_bounds__(256) void moe_combine4_kernel(const float* __restrict__ Y, const int* __restrict__ tp,
                                                           const float* __restrict__ pw, float* __restrict__ out,
                                                           int topk, int N) {
  const int t = blockIdx.x;
  int pj[16];
  float wj[16];
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (j < topk) {
      pj[j] = tp[(size_t)t * topk + j];
      wj[j] = pw[pj[j]];
    }
  for (int n = 4 * threadIdx.x; n < N; n += 1024) {
    float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < topk) {
        const float4 y = *(const float4*)(Y + (size_t)pj[j] * N + n);
        acc.x = fmaf(wj[j], y.x, acc.x);
        acc.y = fmaf(wj[j], y.y, acc.y);
        acc.z = fmaf(wj[j], y.z, acc.z);
        acc.w = fmaf(wj[j], y.w, acc.w);
      }
    *(float4*)(out + (size_t)t * N + n) = acc;
  }
}

// ------------------------------------------------------------- GEMM core
constexpr int BK = 32;            // K per LDS stage (two 32x32x16 MFMA steps)
constexpr int LDS_ROW = 40;       // halfs per LDS row: 32 data + 8 pad

// Operand parts per GEMM flavour (the products are spelled out in the kernel).
enum { X3_REF = 0, X3_2X2 = 1, X3_REF_BF16 = 2 };
template <int MODE>
struct X3Mode;
template <>
struct X3Mode<X3_REF> {  // A = x hi/mid/lo, B = the fp16 weight
  static constexpr int NA = 3, NB = 1;
};
template <>
struct X3Mode<X3_REF_BF16> {  // bf3gemm: A = x hi/mid/lo in bf16, B = the bf16 weight
  static constexpr int NA = 3, NB = 1;
};
template <>
struct X3Mode<X3_2X2> {  // A = X hi/lo, B = W hi/lo
  static constexpr int NA = 2, NB = 2;
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
// One 32x32x16 MFMA step on 16-bit operands: bf16 for X3_REF_BF16, fp16 otherwise.
template <int MODE>
__device__ __forceinline__ float16v mfma16(const half8& a, const half8& b, const float16v& c) {
  if constexpr (MODE == X3_REF_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

struct X3Args {
  const uint16_t* A[3];  // [M][lda]
  const uint16_t* B[2];  // [N][ldb]
  int lda, ldb;
  // Big-tile kernel only: K-tiled planes (ktile_index) when atile / btile is the
  // plane's row count, row-major with lda / ldb when 0.
  int atile, btile;
  float* C;
  int ldc;
  int M, N, K;
  const int32_t* aexp;  // per-row exponent of A (x3-2x2) or null
  const int32_t* bexp;  // per-row exponent of B or null
  float beta;
  // Big-tile kernel, x3-ref modes only: B[0] is given transposed, [K][ldb] with the N
  // index contiguous (the dX layout of W), and read in place (x3_big_tile<.., true>).
  int btr;
};

// Stores a wave's WM x WN blocks of 32x32 accumulators at rows r0 + 32i.., columns
// c0 + 32j.. (register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32 of
// its block): C = acc * 2^-(aexp[row] + bexp[col]) (+ beta * C).  The exponents and
// beta are read once, before any store.  A wave whose rows and columns all exist
// stores without per-element tests: one row pointer per register row, the column
// blocks at immediate offsets from it.
template <int WM, int WN>
__device__ __forceinline__ void x3_store(const X3Args& p, const float16v (&acc)[WM][WN], int r0, int c0, int lane) {
  const int M = p.M, N = p.N, ldc = p.ldc;
  const float beta = p.beta;
  const int32_t* aexp = p.aexp;
  const int32_t* bexp = p.bexp;
  float* C = p.C;
  const int lr = 4 * (lane >> 5), lc = lane & 31;
  const bool sc = aexp || bexp;
  int eb[WN], ea[WM][16];
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = c0 + 32 * j + lc;
    eb[j] = bexp && col < N ? bexp[col] : 0;
  }
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = r0 + 32 * i + 8 * (r >> 2) + lr + (r & 3);
      ea[i][r] = aexp && row < M ? aexp[row] : 0;
    }
  if (r0 + 32 * WM <= M && c0 + 32 * WN <= N) {
    if (!sc && beta == 0.f) {
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float* rp = C + (size_t)(r0 + 32 * i + 8 * (r >> 2) + lr + (r & 3)) * ldc + c0 + lc;
#pragma unroll
          for (int j = 0; j < WN; ++j) rp[32 * j] = acc[i][j][r];
        }
    } else {
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float* rp = C + (size_t)(r0 + 32 * i + 8 * (r >> 2) + lr + (r & 3)) * ldc + c0 + lc;
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            float v = acc[i][j][r];
            if (sc) v = ldexpf(v, -(ea[i][r] + eb[j]));
            if (beta != 0.f) v = fmaf(beta, rp[32 * j], v);
            rp[32 * j] = v;
          }
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = r0 + 32 * i + 8 * (r >> 2) + lr + (r & 3);
      if (row >= M) continue;
      float* rp = C + (size_t)row * ldc + c0 + lc;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        if (c0 + 32 * j + lc >= N) continue;
        float v = acc[i][j][r];
        if (sc) v = ldexpf(v, -(ea[i][r] + eb[j]));
        if (beta != 0.f) v = fmaf(beta, rp[32 * j], v);
        rp[32 * j] = v;
      }
    }
}

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256) void gemm_x3_kernel(const X3Args p) {
  using Md = X3Mode<MODE>;
  constexpr int NA = Md::NA, NB = Md::NB;
  constexpr int WM = BM / 64, WN = BN / 64;           // 32x32 blocks per wave (2x2 waves)
  constexpr int A_CH = BM * (BK / 8) / 256;          // 16-byte chunks per thread per A part
  constexpr int B_CH = BN * (BK / 8) / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  constexpr int A_PART = BM * LDS_ROW, B_PART = BN * LDS_ROW;
  constexpr int STAGE = NA * A_PART + NB * B_PART;

  // XCD-aware tile order: launches round-robin blocks over the 8 XCDs; give
  // each XCD a contiguous run of tiles so neighbours share L2.
  const int ntm = (p.M + BM - 1) / BM, ntn = (p.N + BN - 1) / BN, nt = ntm * ntn;
  int bid = blockIdx.x;
  if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
  const int tm = bid / ntn, tn = bid % ntn;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // global -> register staging (macros, not lambdas: the staging arrays must
  // stay in registers)
  u32x4 ra[NA][A_CH], rb[NB][B_CH];
#define X3_GLOAD(k0)                                                              \
  do {                                                                            \
    _Pragma("unroll") for (int q = 0; q < NA; ++q)                                \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) {                            \
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;                    \
      const int gr = min(m0 + row, p.M - 1);                                      \
      ra[q][i] = *(const u32x4*)(p.A[q] + (size_t)gr * p.lda + (k0) + 8 * c);     \
    }                                                                             \
    _Pragma("unroll") for (int q = 0; q < NB; ++q)                                \
    _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                            \
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;                    \
      const int gr = min(n0 + row, p.N - 1);                                      \
      rb[q][i] = *(const u32x4*)(p.B[q] + (size_t)gr * p.ldb + (k0) + 8 * c);     \
    }                                                                             \
  } while (0)
#define X3_SSTORE(buf)                                                                          \
  do {                                                                                          \
    uint16_t* s_ = lds + (buf) * STAGE;                                                         \
    _Pragma("unroll") for (int q = 0; q < NA; ++q)                                              \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) {                                          \
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;                                  \
      *(u32x4*)(s_ + q * A_PART + row * LDS_ROW + 8 * c) = ra[q][i];                            \
    }                                                                                           \
    _Pragma("unroll") for (int q = 0; q < NB; ++q)                                              \
    _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                                          \
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;                                  \
      *(u32x4*)(s_ + NA * A_PART + q * B_PART + row * LDS_ROW + 8 * c) = rb[q][i];              \
    }                                                                                           \
  } while (0)

  float16v acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = p.K / BK;
  X3_GLOAD(0);
  X3_SSTORE(0);
  __syncthreads();
  const int frow = lane & 31, fk = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) X3_GLOAD((kt + 1) * BK);
    const uint16_t* s = lds + buf * STAGE;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 af[NA][WM], bf[NB][WN];
#pragma unroll
      for (int q = 0; q < NA; ++q)
#pragma unroll
        for (int i = 0; i < WM; ++i)
          af[q][i] = *(const half8*)(s + q * A_PART + (wm * WM * 32 + i * 32 + frow) * LDS_ROW + kk + fk);
#pragma unroll
      for (int q = 0; q < NB; ++q)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          bf[q][j] = *(const half8*)(s + NA * A_PART + q * B_PART + (wn * WN * 32 + j * 32 + frow) * LDS_ROW + kk + fk);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          if constexpr (MODE != X3_2X2) {  // lo, mid, hi times the weight (tier.cpp:940, 918)
            acc[i][j] = mfma16<MODE>(af[2][i], bf[0][j], acc[i][j]);
            acc[i][j] = mfma16<MODE>(af[1][i], bf[0][j], acc[i][j]);
            acc[i][j] = mfma16<MODE>(af[0][i], bf[0][j], acc[i][j]);
          } else {  // hi*hi + hi*lo + lo*hi
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[0][i], bf[0][j], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[0][i], bf[1][j], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[1][i], bf[0][j], acc[i][j], 0, 0, 0);
          }
        }
    }
    if (kt + 1 < nk) X3_SSTORE(buf ^ 1);
    __syncthreads();
  }

  x3_store<WM, WN>(p, acc, m0 + wm * WM * 32, n0 + wn * WN * 32, lane);
#undef X3_GLOAD
#undef X3_SSTORE
}

// ------------------------------------------------------ big-tile GEMM core
// Same products as gemm_x3_kernel on a 256-row workgroup tile of 8 waves, K step
// 32, in two shapes: 256 x 320 (4 waves along M x 2 along N, each 64 x 160 =
// 2 x 5 blocks of 32x32) and 256 x 352 (8 waves along M, each 32 x 352 = 1 x 11
// blocks), the second for the N that 352 covers with less padding (1408 =
// 4 x 352, 2048 in 6 x 352 against 7 x 320).  Consecutive waves go along N
// first, so the waves whose rows all lie past M (a routed expert's last tile)
// sit on different SIMDs and skip their MFMAs.  The operand tiles reach LDS by
// global_load_lds_dwordx4 (no register staging), double-buffered: after the
// barrier that publishes stage k, the loads of stage k+1 go out into the other
// buffer, then stage k is multiplied.  A row of 32 halfs is four 16-byte
// chunks, chunk c stored at slot c ^ ((row >> 2) & 3): a fragment read (16
// consecutive rows, one chunk) then touches 16 distinct 16-byte bank groups.
// Per k-substep a wave reads NA*WM + NB*WN fragments for 3*WM*WN MFMAs (11 for
// 30 in the 320 shape, 14 for 33 in the 352 shape, x3-ref), which keeps LDS
// below half its bandwidth at full MFMA rate.
//
// TR (x3-ref modes): the weight comes as [K][ldb] with the N index contiguous (W
// itself in the dX product, read in place instead of transposed first).  A stage
// of it lands as 32 K-rows of TN halfs, each row padded by 16 bytes (TrB); a B
// fragment is then two ds_read_b64_tr_b16.  That instruction treats each group
// of 16 lanes as a 16 x 4 block -- lane s supplies the 4 halfs at its own address
// -- and gives lane i the halfs (4e + i/4, i%4), e = 0..3, of that block.  So
// lane s of group g addresses K-row kb + s/4, columns nb + 4(s%4).., with kb the
// fragment's k base plus 8(g/2) and nb its column base plus 16(g%2), and receives
// K-rows kb..kb+3 of column nb + s: the MFMA B operand's four k values, twice
// (kb, kb + 4) for the eight.  K-rows are padded to 16 (mod 64) dwords, so the 32
// bytes that each of a pair of groups reads from each of its four K-rows fall on
// eight distinct 8-dword bank groups.
constexpr int XB_M = 256;
template <int TN>
struct TrB {
  static constexpr int DW = TN / 2 + (16 - (TN / 2) % 64 + 64) % 64;  // dwords per K-row in LDS
  static constexpr int ROWB = DW * 4;
  static constexpr int PART = (BK * ROWB + 1023) / 1024 * 1024;      // one stage, whole 1 KiB loads
  static_assert(DW % 64 == 16 && DW * 2 >= TN, "K-row padding");
};
template <int TN>
struct XbShape;
template <>
struct XbShape<320> {
  static constexpr int WAVES_N = 2, WM = 2, WN = 5;
};
template <>
struct XbShape<352> {
  static constexpr int WAVES_N = 1, WM = 1, WN = 11;
};

// One 256 x TN output tile t of the problem p (t < ceil(M/256) * ceil(N/TN)).
template <int MODE, int TN, bool TR = false>
__device__ __forceinline__ void x3_big_tile(const X3Args& p, int t) {
  using Md = X3Mode<MODE>;
  using Sh = XbShape<TN>;
  constexpr int NA = Md::NA, NB = Md::NB, WM = Sh::WM, WN = Sh::WN, WAVES_N = Sh::WAVES_N;
  static_assert(!TR || NB == 1, "TR: the x3-ref modes");
  constexpr int A_PART = XB_M * 64, B_PART = TR ? TrB<TN>::PART : TN * 64;  // bytes of one part per stage
  constexpr int STAGE = NA * A_PART + NB * B_PART;
  constexpr int A_INST = A_PART / 1024, B_INST = B_PART / 1024;  // 1 KiB loads per part
  constexpr int NINST = NA * A_INST + NB * B_INST;
  constexpr int PER_WAVE = (NINST + 7) / 8;
  static_assert(WM * 32 * (8 / WAVES_N) == XB_M && WN * 32 * WAVES_N == TN, "wave grid covers the tile");
  extern __shared__ __attribute__((aligned(16))) uint16_t lds_h[];
  uint8_t* lds = (uint8_t*)lds_h;

  // The tile sequence walks groups of 4 tile rows column by column.
  const int ntm = (p.M + XB_M - 1) / XB_M, ntn = (p.N + TN - 1) / TN;
  constexpr int GM = 4;
  const int grp = t / (GM * ntn), first = grp * GM, gm = min(GM, ntm - first);
  const int tin = t - grp * GM * ntn;
  const int tm = first + tin % gm, tn = tin / gm;
  const int m0 = tm * XB_M, n0 = tn * TN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const bool live = m0 + wm * WM * 32 < p.M;  // some of the wave's rows exist
  const uint32_t lds0 = lds_addr(lds);

  // DMA of stage kt into buffer buf: instruction t = wave + 8u covers 16 rows
  // of one part.  Sources and LDS offsets are fixed per lane, so they are set
  // up once (no loads of kernel arguments inside the K loop, whose waits would
  // also wait for the DMA).
  const uint16_t* gsrc[PER_WAVE];
  uint32_t loff[PER_WAVE];
  size_t gstep[PER_WAVE];  // halfs between the K steps of a load's rows
  {
    const int drow = lane >> 2, dslot = lane & 3;
#pragma unroll
    for (int u = 0; u < PER_WAVE; ++u) {
      const int t = min(wave + 8 * u, NINST - 1);
      const uint16_t* src;
      int ld, lim, r0, base, ch;
      if (t < NA * A_INST) {
        const int q = t / A_INST;
        ch = t % A_INST;
        src = q == 0 ? p.A[0] : q == 1 ? p.A[1] : p.A[2];
        ld = p.atile ? 32 : p.lda; lim = p.M; r0 = m0; base = q * A_PART;
        gstep[u] = p.atile ? (size_t)p.atile * 32 : BK;
      } else if constexpr (TR) {
        // byte o of the padded [BK][ROWB] image: K-row o / ROWB, column (o % ROWB) / 2;
        // padding and the tail past BK rows load row 0's first chunk again (unread)
        ch = t - NA * A_INST;
        const int o = ch * 1024 + lane * 16, kr = o / TrB<TN>::ROWB, cb = o % TrB<TN>::ROWB;
        const bool pad = kr >= BK || cb >= TN * 2;
        gsrc[u] = p.B[0] + (size_t)(pad ? 0 : kr) * p.ldb + min(n0 + (pad ? 0 : cb / 2), p.N - 8);
        loff[u] = (uint32_t)(NA * A_PART + ch * 1024);
        gstep[u] = (size_t)BK * p.ldb;
        continue;
      } else {
        const int q = (t - NA * A_INST) / B_INST;
        ch = (t - NA * A_INST) % B_INST;
        src = q == 0 ? p.B[0] : p.B[1];
        ld = p.btile ? 32 : p.ldb; lim = p.N; r0 = n0; base = NA * A_PART + q * B_PART;
        gstep[u] = p.btile ? (size_t)p.btile * 32 : BK;
      }
      const int row = ch * 16 + drow;
      const int kc = dslot ^ ((row >> 2) & 3);
      gsrc[u] = src + (size_t)min(r0 + row, lim - 1) * ld + kc * 8;
      loff[u] = (uint32_t)(base + ch * 1024);
    }
  }
  auto issue = [&](int kt, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < PER_WAVE; ++u)
      if (wave + 8 * u < NINST) dma16(gsrc[u] + (size_t)kt * gstep[u], lds0 + buf * STAGE + loff[u]);
  };

  float16v acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int fr = lane & 31, fh = lane >> 5;
  const int sw = (fr >> 2) & 3;
  // byte offsets of this lane's fragment rows: chunk (2*kk + fh) of row fr
  const uint32_t cofs0 = (uint32_t)(fr * 64 + ((fh ^ sw) * 16));
  const uint32_t cofs1 = (uint32_t)(fr * 64 + (((2 + fh) ^ sw) * 16));
  // TR: this lane's transposed-read address within a 32-column block (kk = 0)
  const uint32_t trofs = (uint32_t)((8 * (lane >> 5) + ((lane & 15) >> 2)) * TrB<TN>::ROWB +
                                    (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2);
  const int nk = p.K / BK;
  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    vm_wait<0>();
    __syncthreads();  // stage kt is in LDS for every wave; buffer kt+1 is free
    if (kt + 1 < nk) issue(kt + 1, (kt + 1) & 1);
    if (!live) continue;
    const uint8_t* s = lds + (kt & 1) * STAGE;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint32_t co = kk ? cofs1 : cofs0;
      // all fragments of the substep first, then the MFMAs product-major, so
      // consecutive MFMAs on one accumulator are WM*WN apart
      half8 af[NA][WM], bf[NB][WN];
#pragma unroll
      for (int q = 0; q < NA; ++q)
#pragma unroll
        for (int i = 0; i < WM; ++i)
          af[q][i] = *(const half8*)(s + q * A_PART + (wm * WM * 32 + i * 32) * 64 + co);
      if constexpr (TR) {
        typedef short short4v __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) short4v lds_s4;
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const uint32_t a = lds_addr(s) + NA * A_PART + kk * 16 * TrB<TN>::ROWB + (wn * WN * 32 + j * 32) * 2 + trofs;
          const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(size_t)a);
          const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(size_t)(a + 4 * TrB<TN>::ROWB));
          const short4v v8[2] = {lo, hi};
          bf[0][j] = __builtin_bit_cast(half8, v8);
        }
      } else {
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            bf[q][j] = *(const half8*)(s + NA * A_PART + q * B_PART + (wn * WN * 32 + j * 32) * 64 + co);
      }
      if constexpr (MODE != X3_2X2) {  // lo, mid, hi times the weight (tier.cpp:940, 918)
#pragma unroll
        for (int pa = 2; pa >= 0; --pa)
#pragma unroll
          for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int i = 0; i < WM; ++i)
              acc[i][j] = mfma16<MODE>(af[pa][i], bf[0][j], acc[i][j]);
      } else {  // hi*hi + hi*lo + lo*hi
        constexpr int PA[3] = {0, 0, 1}, PB[3] = {0, 1, 0};
#pragma unroll
        for (int pr = 0; pr < 3; ++pr)
#pragma unroll
          for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int i = 0; i < WM; ++i)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[PA[pr]][i], bf[PB[pr]][j], acc[i][j], 0, 0, 0);
      }
    }
  }
  if (!live) return;
  x3_store<WM, WN>(p, acc, m0 + wm * WM * 32, n0 + wn * WN * 32, lane);
}

template <int MODE, int TN, bool TR = false>
__global__ __launch_bounds__(512) void gemm_x3_big(const X3Args p) {
  // Workgroups go round-robin over the 8 XCDs, so XCD x gets the x-th eighth of
  // the tile sequence: a compact block of tiles (4 x 8 at 4096 x 5120) whose
  // operand panels its L2 holds.
  const int nt = ((p.M + XB_M - 1) / XB_M) * ((p.N + TN - 1) / TN);
  int t = blockIdx.x;
  if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
  x3_big_tile<MODE, TN, TR>(p, t);
}

// Grouped problems (routed experts): group g multiplies rows [row0[g], row0[g] +
// rows[g]) of the A planes with its own B[g] (N x K, ldb = K) into the same rows
// of C; its tiles are [tile0[g], tile0[g+1]) of the tile sequence.
constexpr int X3G = 64;
struct X3Groups {
  int n;
  int tile0[X3G + 1];
  int row0[X3G];
  int rows[X3G];
  const uint16_t* B[X3G];
};

template <int MODE, int TN>
__global__ __launch_bounds__(512) void gemm_x3_big_grouped(const X3Args p, const X3Groups g) {
  // XCD x (workgroups b = x mod 8) takes the x-th contiguous share of the tile
  // sequence, so an expert's tiles share one L2
  const int nt = g.tile0[g.n], q8 = nt >> 3, r8 = nt & 7, x = (int)blockIdx.x & 7;
  const int b = x * q8 + min(x, r8) + ((int)blockIdx.x >> 3);
  int grp = 0;
  while (grp + 1 < g.n && b >= g.tile0[grp + 1]) ++grp;
  X3Args q = p;
  for (int k = 0; k < 3; ++k)
    if (q.A[k]) q.A[k] += (size_t)g.row0[grp] * (p.atile ? 32 : p.lda);
  q.B[0] = g.B[grp];
  q.M = g.rows[grp];
  q.C = p.C + (size_t)g.row0[grp] * p.ldc;
  x3_big_tile<MODE, TN>(q, b - g.tile0[grp]);
}

// Tile width for N: 352 where it pads N less than 320 does.
int big_tn(int N) {
  const long p352 = (long)((N + 351) / 352) * 352, p320 = (long)((N + 319) / 320) * 320;
  return p352 < p320 ? 352 : 320;
}

template <int MODE, int TN, bool TR = false>
constexpr size_t big_lds() {
  return 2 * ((size_t)X3Mode<MODE>::NA * XB_M * 64 + (TR ? TrB<TN>::PART : (size_t)X3Mode<MODE>::NB * TN * 64));
}

// ---- K chunks.  The fp32 accumulator's rounding error grows like sqrt(K): one
// accumulator over K = 14336 measured 1.4e-6 relative Frobenius error against
// fp64 (x3-ref, config-4 down_proj), above the 2^-20 bar, against ~8e-7 at
// K = 5120.  Above kAccChunkFrom a product therefore runs as balanced chunks of
// at most kAccChunkMax columns, each summed from zero and added to C in fp32
// (beta = 1 after the first chunk): chunks of 3584 bring K = 14336 to ~7e-7 (a
// CPU model of the accumulation scaled to the measured error).  Each extra
// chunk reads and writes C once more.
int k_chunks(int K) { return acc_chunks(K); }

// Element offset of column k0 (a multiple of 32) in a plane: k0 in a row-major
// plane, k0 / 32 tiles of `tile` rows x 32 in a K-tiled one (ktile_index).
size_t k_offset(int k0, int tile) { return tile ? (size_t)(k0 / 32) * tile * 32 : (size_t)k0; }

// Runs launch(q) over the K chunks of a (one call when K <= kChunkFrom); shift(q, k0)
// moves operands a launch reads beyond q.A / q.B (the grouped weights) to column k0.
template <class L, class S>
int run_k_chunks(const X3Args& a, L&& launch, S&& shift) {
  const int P = k_chunks(a.K);
  if (P == 1) return launch(a);
  const int steps = a.K / BK;
  for (int c = 0; c < P; ++c) {
    const int s0 = (int)((long)c * steps / P), s1 = (int)((long)(c + 1) * steps / P);
    X3Args q = a;
    for (int i = 0; i < 3; ++i)
      if (q.A[i]) q.A[i] += k_offset(s0 * BK, q.atile);
    for (int i = 0; i < 2; ++i)
      if (q.B[i]) q.B[i] += q.btr ? (size_t)s0 * BK * q.ldb : k_offset(s0 * BK, q.btile);
    shift(s0 * BK);
    q.K = (s1 - s0) * BK;
    if (c > 0) q.beta = 1.f;
    const int st = launch(q);
    if (st) return st;
  }
  return TIERMM_OK;
}
template <class L>
int run_k_chunks(const X3Args& a, L&& launch) {
  return run_k_chunks(a, launch, [](int) {});
}

template <int MODE, int TN, bool TR = false>
int launch_x3_big_tn(const X3Args& a, hipStream_t s, const char* who) {
  constexpr size_t lds = big_lds<MODE, TN, TR>();
  static_assert(lds <= 160 * 1024, "LDS budget");
  static std::atomic<uint64_t> attr{0};
  int st = lds_attr_once(attr, (const void*)gemm_x3_big<MODE, TN, TR>, (int)lds, who);
  if (st) return st;
  const int nt = ((a.M + XB_M - 1) / XB_M) * ((a.N + TN - 1) / TN);
  gemm_x3_big<MODE, TN, TR><<<nt, 512, lds, s>>>(a);
  TM_LAUNCH_CHECK(who);
  return TIERMM_OK;
}

template <int MODE>
int launch_x3_big(const X3Args& a, hipStream_t s, const char* who) {
  return run_k_chunks(a, [&](const X3Args& q) {
    if constexpr (MODE == X3_REF || MODE == X3_REF_BF16) {
      if (q.btr)
        return big_tn(q.N) == 352 ? launch_x3_big_tn<MODE, 352, true>(q, s, who)
                                  : launch_x3_big_tn<MODE, 320, true>(q, s, who);
    }
    return big_tn(q.N) == 352 ? launch_x3_big_tn<MODE, 352>(q, s, who) : launch_x3_big_tn<MODE, 320>(q, s, who);
  });
}

// g.tile0 counts tiles of width TN.
template <int MODE, int TN>
int launch_x3_big_grouped(const X3Args& a, const X3Groups& g, hipStream_t s, const char* who) {
  constexpr size_t lds = big_lds<MODE, TN>();
  static std::atomic<uint64_t> attr{0};
  int st = lds_attr_once(attr, (const void*)gemm_x3_big_grouped<MODE, TN>, (int)lds, who);
  if (st) return st;
  if (g.tile0[g.n] == 0) return TIERMM_OK;
  X3Groups gk = g;  // the groups' weights (ldb = K, or K-tiled) move with the K chunks
  return run_k_chunks(
      a,
      [&](const X3Args& q) {
        gemm_x3_big_grouped<MODE, TN><<<gk.tile0[gk.n], 512, lds, s>>>(q, gk);
        TM_LAUNCH_CHECK(who);
        return (int)TIERMM_OK;
      },
      [&](int k0) {
        for (int i = 0; i < g.n; ++i) gk.B[i] = g.B[i] + k_offset(k0, a.btile);
      });
}

template <int BM, int BN, int MODE>
int launch_x3_one(const X3Args& a, hipStream_t s, const char* who) {
  using Md = X3Mode<MODE>;
  const int nt = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  constexpr size_t lds = 2 * (size_t)(Md::NA * BM + Md::NB * BN) * LDS_ROW * sizeof(uint16_t);
  static std::atomic<uint64_t> attr{0};  // dynamic LDS above 64 KiB is opted into per device
  int st = lds_attr_once(attr, (const void*)gemm_x3_kernel<BM, BN, MODE>, (int)lds, who);
  if (st) return st;
  gemm_x3_kernel<BM, BN, MODE><<<nt, 256, lds, s>>>(a);
  TM_LAUNCH_CHECK(who);
  return TIERMM_OK;
}

template <int BM, int BN, int MODE>
int launch_x3(const X3Args& a, hipStream_t s, const char* who) {
  return run_k_chunks(a, [&](const X3Args& q) { return launch_x3_one<BM, BN, MODE>(q, s, who); });
}

// Tiles of the 256x320 kernel: it pays off once they occupy most of the CUs.
long big_tiles(int M, int N) {
  const int tn = big_tn(N);
  return (long)((M + XB_M - 1) / XB_M) * ((N + tn - 1) / tn);
}

int check_sizes(const char* who, int M, int N, int K) {
  if (M < 0 || N < 0 || K < 0) return set_error(TIERMM_EINVAL, "%s: negative size", who);
  return TIERMM_OK;
}

// Entry points whose operands come pre-split (no copy to pad them) need K in whole steps.
int check_nt(const char* who, int M, int N, int K) {
  const int st = check_sizes(who, M, N, K);
  if (st) return st;
  if (K % BK) return set_error(TIERMM_UNSUPPORTED, "%s: K=%d is not a multiple of %d", who, K, BK);
  return TIERMM_OK;
}

int pad32(int K) { return (K + BK - 1) / BK * BK; }

// Grid of the element-wise kernels (grid-stride loops).
unsigned elem_grid(size_t n) {
  const size_t want = (n + 255) / 256;
  return (unsigned)(want < 16384 ? (want ? want : 1) : 16384);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

// Whether the routed experts of type qt take the fused kernel in one launch (one group
// per expert, no split-K); experts of the types it does not take are staged in fp16.
bool grouped_fused(int qt, const int* qts, const int* offs, int n_experts, int N, int K) {
  std::vector<int> rows;
  for (int e = 0; e < n_experts; ++e)
    if (offs[e + 1] > offs[e] && qts[e] == qt) rows.push_back(offs[e + 1] - offs[e]);
  return !rows.empty() && qgemm_fusable(qt, rows.data(), (int)rows.size(), N, K, false);
}

// The distinct weight types of the routed experts, each with whether grouped_fused takes it.
std::vector<std::pair<int, bool>> routed_types(const int* qts, const int* offs, int n_experts, int N, int K) {
  std::vector<std::pair<int, bool>> t;
  for (int e = 0; e < n_experts; ++e) {
    if (offs[e + 1] == offs[e]) continue;
    bool seen = false;
    for (auto& x : t) seen = seen || x.first == qts[e];
    if (!seen) t.push_back({qts[e], grouped_fused(qts[e], qts, offs, n_experts, N, K)});
  }
  return t;
}

bool type_fused(const std::vector<std::pair<int, bool>>& t, int qt) {
  for (auto& x : t)
    if (x.first == qt) return x.second;
  return false;
}

// Routed experts through the grouped 256x320 launch: the number of experts whose
// fp16 weights are decoded at once (at most 64 and 1 GiB), or 0 when the experts'
// 256-row tiles do not fill the chip or are mostly empty rows.
int big_group_chunk(const int* offs, int n_experts, int N, int K) {
  long tiles = 0, rows = 0, cap = 0;
  for (int e = 0; e < n_experts; ++e) {
    const int Me = offs[e + 1] - offs[e];
    if (Me <= 0) continue;
    tiles += big_tiles(Me, N);
    rows += Me;
    cap += (long)((Me + XB_M - 1) / XB_M) * XB_M;
  }
  if (tiles < 192 || 2 * rows < cap) return 0;
  const size_t per = al256((size_t)N * K * sizeof(uint16_t));
  return (int)std::max<size_t>(1, std::min<size_t>(X3G, (size_t(1) << 30) / per));
}

}  // namespace

// x3-ref product on pre-split activations: C[M][ldc] (beta)= sum_parts Xpart[M][K] * W[N][K]^T,
// parts at xparts + {0, stride, 2*stride} in HML order, W fp16 with row stride ldw.
int x3ref_nt(const uint16_t* xparts, size_t stride, const uint16_t* W, int ldw, float* C, int ldc, int M, int N,
             int K, float beta, hipStream_t s, const char* who, bool bf16 = false) {
  X3Args a{};
  a.A[0] = xparts;
  a.A[1] = xparts + stride;
  a.A[2] = xparts + 2 * stride;
  a.B[0] = W;
  a.lda = K;
  a.ldb = ldw;
  a.C = C;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  a.aexp = nullptr;
  a.bexp = nullptr;
  a.beta = beta;
  if (bf16) {
    if (big_tiles(M, N) >= 192) return launch_x3_big<X3_REF_BF16>(a, s, who);
    return launch_x3<128, 128, X3_REF_BF16>(a, s, who);
  }
  if (big_tiles(M, N) >= 192) return launch_x3_big<X3_REF>(a, s, who);
  return launch_x3<128, 128, X3_REF>(a, s, who);
}

// Rows held in registers where they fit (one read of the source), else two passes.
void x3s_split_launch(const float* src, uint16_t* hi, uint16_t* lo, int32_t* exps, int rows, int cols, hipStream_t s) {
  const bool vec = cols % 4 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)hi & 7) == 0 && ((uintptr_t)lo & 7) == 0;
  if (vec && cols <= 4096)
    x3s_split_reg_kernel<4><<<rows, 256, 0, s>>>(src, hi, lo, exps, cols);
  else if (vec && cols <= 8192)
    x3s_split_reg_kernel<8><<<rows, 256, 0, s>>>(src, hi, lo, exps, cols);
  else if (vec && cols <= 16384)
    x3s_split_reg_kernel<16><<<rows, 256, 0, s>>>(src, hi, lo, exps, cols);
  else
    x3s_split_kernel<<<rows, 256, 0, s>>>(src, hi, lo, exps, cols);
}

// trows > 0: fp16 parts in the K-tiled layout of planes of trows rows of cols
// elements (needs the vectorised kernel's alignment and cols % 32 == 0).
int split3_launch(const float* x, uint16_t* parts, size_t n, size_t stride, int order, hipStream_t s, bool bf16 = false,
                  size_t trows = 0, int cols = 0) {
  if (n == 0) return TIERMM_OK;
  if (trows) {
    if (n % 8 || stride % 8 || ((uintptr_t)x & 15) || ((uintptr_t)parts & 15) || cols % 32 || bf16)
      return set_error(TIERMM_EINVAL, "split3: K-tiled parts need 16-byte aligned rows of a multiple of 32");
    const size_t n8 = n / 8, want = (n8 + 255) / 256;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    split3_vec8_kernel<false><<<grid, 256, 0, s>>>(x, parts, n8, stride, order, trows, cols);
    TM_LAUNCH_CHECK("split3: launch");
    return TIERMM_OK;
  }
  if (n % 8 == 0 && stride % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)parts & 15) == 0) {
    const size_t n8 = n / 8, want = (n8 + 255) / 256;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    if (bf16)
      split3_vec8_kernel<true><<<grid, 256, 0, s>>>(x, parts, n8, stride, order);
    else
      split3_vec8_kernel<false><<<grid, 256, 0, s>>>(x, parts, n8, stride, order);
    TM_LAUNCH_CHECK("split3: launch");
    return TIERMM_OK;
  }
  const size_t want = (n + 255) / 256;
  const unsigned grid = (unsigned)(want < 16384 ? want : 16384);
  if (bf16)
    split3_kernel<true><<<grid, 256, 0, s>>>(x, parts, n, stride, order);
  else
    split3_kernel<false><<<grid, 256, 0, s>>>(x, parts, n, stride, order);
  TM_LAUNCH_CHECK("split3: launch");
  return TIERMM_OK;
}

}  // namespace tiermm

using namespace tiermm;

extern "C" {

int tiermm_split3_f16(const float* x, uint16_t* parts, size_t n, size_t part_stride, int order,
                      tiermm_stream_t stream) {
  if (order != TIERMM_HML && order != TIERMM_LMH)
    return set_error(TIERMM_EINVAL, "tiermm_split3_f16: order %d", order);
  if (part_stride < n) return set_error(TIERMM_EINVAL, "tiermm_split3_f16: part_stride < n");
  if (n && (!x || !parts)) return set_error(TIERMM_EINVAL, "tiermm_split3_f16: null buffer");
  return split3_launch(x, parts, n, part_stride, order, (hipStream_t)stream);
}

int tiermm_split3_f16_ktiled(const float* x, uint16_t* parts, int M, int K, size_t part_stride,
                             tiermm_stream_t stream) {
  const char* who = "tiermm_split3_f16_ktiled";
  if (M < 0 || K < 0) return set_error(TIERMM_EINVAL, "%s: negative size", who);
  if (K % BK) return set_error(TIERMM_UNSUPPORTED, "%s: K=%d is not a multiple of %d", who, K, BK);
  const size_t mk = (size_t)M * K;
  if (mk == 0) return TIERMM_OK;
  if (!x || !parts || part_stride < mk) return set_error(TIERMM_EINVAL, "%s: null buffer or part_stride < M*K", who);
  return split3_launch(x, parts, mk, part_stride, TIERMM_HML, (hipStream_t)stream, false, (size_t)M, K);
}

int tiermm_split3_bf16(const float* x, uint16_t* parts, size_t n, size_t part_stride, int order,
                       tiermm_stream_t stream) {
  if (order != TIERMM_HML && order != TIERMM_LMH)
    return set_error(TIERMM_EINVAL, "tiermm_split3_bf16: order %d", order);
  if (part_stride < n) return set_error(TIERMM_EINVAL, "tiermm_split3_bf16: part_stride < n");
  if (n && (!x || !parts)) return set_error(TIERMM_EINVAL, "tiermm_split3_bf16: null buffer");
  return split3_launch(x, parts, n, part_stride, order, (hipStream_t)stream, true);
}

int tiermm_x3s_split(const float* src, uint16_t* hi, uint16_t* lo, int32_t* exps, int rows, int cols,
                     tiermm_stream_t stream) {
  if (rows < 0 || cols < 0) return set_error(TIERMM_EINVAL, "tiermm_x3s_split: negative size");
  if (rows == 0) return TIERMM_OK;
  if (!src || !hi || !lo || !exps) return set_error(TIERMM_EINVAL, "tiermm_x3s_split: null buffer");
  x3s_split_launch(src, hi, lo, exps, rows, cols, (hipStream_t)stream);
  TM_LAUNCH_CHECK("tiermm_x3s_split: launch");
  return TIERMM_OK;
}

int tiermm_x3s_gemm(const uint16_t* Xhi, const uint16_t* Xlo, const int32_t* xexp, const uint16_t* Whi,
                    const uint16_t* Wlo, const int32_t* wexp, float* Y, int M, int N, int K, int ldy,
                    tiermm_stream_t stream) {
  int st = check_nt("tiermm_x3s_gemm", M, N, K);
  if (st) return st;
  if (ldy < N) return set_error(TIERMM_EINVAL, "tiermm_x3s_gemm: ldy < N");
  if (M == 0 || N == 0) return TIERMM_OK;
  if (!aligned16(Xhi) || !aligned16(Xlo) || !aligned16(Whi) || !aligned16(Wlo) || !Y || !xexp || !wexp)
    return set_error(TIERMM_EINVAL, "tiermm_x3s_gemm: operands must be non-null and 16-byte aligned");
  X3Args a{};
  a.A[0] = Xhi;
  a.A[1] = Xlo;
  a.B[0] = Whi;
  a.B[1] = Wlo;
  a.lda = K;
  a.ldb = K;
  a.C = Y;
  a.ldc = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.aexp = xexp;
  a.bexp = wexp;
  a.beta = 0.f;
  // the 256x320 tile needs enough tiles to occupy the CUs; smaller problems use 128x128
  if (big_tiles(M, N) >= 192) return launch_x3_big<X3_2X2>(a, (hipStream_t)stream, "tiermm_x3s_gemm: launch");
  return launch_x3<128, 128, X3_2X2>(a, (hipStream_t)stream, "tiermm_x3s_gemm: launch");
}

size_t tiermm_x3_gemm_ws_bytes(int m, int n, int k) {
  // three fp16 planes of B, and the weight rows for TIERMM_OP_N (transposed) or an
  // odd k (padded), both with rows of k rounded up to 32
  const size_t kp = (size_t)pad32(k);
  return (size_t)3 * (size_t)n * kp * sizeof(uint16_t) + (size_t)m * kp * sizeof(uint16_t);
}

static int x3_gemm_impl(int opA, int m, int n, int k, const uint16_t* A, int lda, const float* B, float beta, float* C,
                        int ldc, void* ws, size_t ws_bytes, tiermm_stream_t stream, bool bf16, const char* who) {
  if (opA != TIERMM_OP_T && opA != TIERMM_OP_N) return set_error(TIERMM_EINVAL, "%s: opA %d", who, opA);
  int st = check_sizes(who, n, m, k);
  if (st) return st;
  if ((opA == TIERMM_OP_T && lda < k) || (opA == TIERMM_OP_N && lda < m) || ldc < m)
    return set_error(TIERMM_EINVAL, "%s: lda or ldc too small", who);
  if (m == 0 || n == 0) return TIERMM_OK;
  const int kp = pad32(k);
  if (!A || !B || !C || (opA == TIERMM_OP_T && kp == k && (!aligned16(A) || (lda % 8))))
    return set_error(TIERMM_EINVAL, "%s: A must be 16-byte aligned with lda a multiple of 8", who);
  void* w = nullptr;
  const size_t nk = (size_t)n * kp;
  st = get_workspace(ws, ws_bytes, tiermm_x3_gemm_ws_bytes(m, n, k), &w, who);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  uint16_t* parts = (uint16_t*)w;
  uint16_t* t = parts + 3 * nk;  // transposed or padded weight rows
  if (kp == k) {
    st = split3_launch(B, parts, nk, nk, TIERMM_HML, s, bf16);
  } else {  // rows of kp with zeros past k (k not a multiple of the 32-wide K step)
    if (bf16)
      pad_split3_kernel<true><<<elem_grid(nk), 256, 0, s>>>(B, (size_t)k, parts, (size_t)n, k, kp);
    else
      pad_split3_kernel<false><<<elem_grid(nk), 256, 0, s>>>(B, (size_t)k, parts, (size_t)n, k, kp);
    TM_LAUNCH_CHECK("tiermm_x3_gemm: padded split");
  }
  if (st) return st;
  const uint16_t* At = A;
  int ldt = lda;
  if (opA == TIERMM_OP_N && kp == k && m % 8 == 0 && lda % 8 == 0 && aligned16(A) && big_tiles(n, m) >= 192) {
    // the big-tile kernel reads A ([k][lda], m contiguous) in place: no transpose
    X3Args a{};
    a.A[0] = parts; a.A[1] = parts + nk; a.A[2] = parts + 2 * nk;
    a.B[0] = A; a.btr = 1;
    a.lda = kp; a.ldb = lda; a.C = C; a.ldc = ldc; a.M = n; a.N = m; a.K = kp; a.beta = beta;
    return bf16 ? launch_x3_big<X3_REF_BF16>(a, s, who) : launch_x3_big<X3_REF>(a, s, who);
  }
  if (opA == TIERMM_OP_N) {
    // A is m x k column-major ([k][lda] in memory, the dX layout of tier.cpp:1226):
    // transpose it to [m][kp] so the product runs in the NT form below
    dim3 grid((unsigned)((m + 63) / 64), (unsigned)((k + 63) / 64));
    transpose16_kernel<<<grid, 256, 0, s>>>(A, lda, t, k, m, kp);
    TM_LAUNCH_CHECK("tiermm_x3_gemm: transpose");
    if (kp != k) {
      zero_tail16_kernel<<<elem_grid((size_t)m * (kp - k)), 256, 0, s>>>(t, (size_t)m, k, kp);
      TM_LAUNCH_CHECK("tiermm_x3_gemm: padding");
    }
    At = t;
    ldt = kp;
  } else if (kp != k) {
    pad16_kernel<<<elem_grid((size_t)m * kp), 256, 0, s>>>(A, (size_t)lda, t, (size_t)m, k, kp);
    TM_LAUNCH_CHECK("tiermm_x3_gemm: padding");
    At = t;
    ldt = kp;
  }
  // column-major C(m x n) with ldc == row-major out[n][ldc] = x[n][k] * W[m][k]^T
  return x3ref_nt(parts, nk, At, ldt, C, ldc, n, m, kp, beta, s, who, bf16);
}

int tiermm_x3_gemm(int opA, int m, int n, int k, const uint16_t* A, int lda, const float* B, float beta, float* C,
                   int ldc, void* ws, size_t ws_bytes, tiermm_stream_t stream) {
  return x3_gemm_impl(opA, m, n, k, A, lda, B, beta, C, ldc, ws, ws_bytes, stream, false, "tiermm_x3_gemm");
}

int tiermm_x3_gemm_bf16(int opA, int m, int n, int k, const uint16_t* A, int lda, const float* B, float beta,
                        float* C, int ldc, void* ws, size_t ws_bytes, tiermm_stream_t stream) {
  return x3_gemm_impl(opA, m, n, k, A, lda, B, beta, C, ldc, ws, ws_bytes, stream, true, "tiermm_x3_gemm_bf16");
}

size_t tiermm_x3_rows_ws_bytes(int M, int K, int N) {
  // three fp16 planes of x; for an odd K (not a multiple of 32) rows padded to a
  // multiple of 32, and the weight copied to such rows
  const size_t kp = (size_t)pad32(K);
  return (size_t)3 * (size_t)M * kp * sizeof(uint16_t) + (kp != (size_t)K ? (size_t)N * kp * sizeof(uint16_t) : 0);
}

static int x3_rows_impl(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo, void* ws,
                        size_t ws_bytes, tiermm_stream_t stream, bool bf16, const char* who) {
  int st = check_sizes(who, M, N, K);
  if (st) return st;
  if (ldo < N) return set_error(TIERMM_EINVAL, "%s: ldo < N", who);
  if (M == 0 || N == 0) return TIERMM_OK;
  if (!aligned16(W) || !x || !y) return set_error(TIERMM_EINVAL, "%s: W must be 16-byte aligned", who);
  void* w = nullptr;
  st = get_workspace(ws, ws_bytes, tiermm_x3_rows_ws_bytes(M, K, N), &w, who);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  const int kp = pad32(K);
  const size_t mk = (size_t)M * kp;
  if (kp == K) {
    st = split3_launch(x, (uint16_t*)w, mk, mk, TIERMM_HML, s, bf16);
    if (st) return st;
    return x3ref_nt((const uint16_t*)w, mk, W, K, y, ldo, M, N, K, 0.f, s, who, bf16);
  }
  uint16_t* parts = (uint16_t*)w;
  uint16_t* wp = parts + 3 * mk;
  if (bf16)
    pad_split3_kernel<true><<<elem_grid(mk), 256, 0, s>>>(x, (size_t)K, parts, (size_t)M, K, kp);
  else
    pad_split3_kernel<false><<<elem_grid(mk), 256, 0, s>>>(x, (size_t)K, parts, (size_t)M, K, kp);
  TM_LAUNCH_CHECK("x3_rows: padded split");
  pad16_kernel<<<elem_grid((size_t)N * kp), 256, 0, s>>>(W, (size_t)K, wp, (size_t)N, K, kp);
  TM_LAUNCH_CHECK("x3_rows: padding");
  return x3ref_nt(parts, mk, wp, kp, y, ldo, M, N, kp, 0.f, s, who, bf16);
}

int tiermm_x3_rows(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo, void* ws,
                   size_t ws_bytes, tiermm_stream_t stream) {
  return x3_rows_impl(W, x, y, M, K, N, ldo, ws, ws_bytes, stream, false, "tiermm_x3_rows");
}

int tiermm_x3_rows_bf16(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo, void* ws,
                        size_t ws_bytes, tiermm_stream_t stream) {
  return x3_rows_impl(W, x, y, M, K, N, ldo, ws, ws_bytes, stream, true, "tiermm_x3_rows_bf16");
}


// Weight rows the unfused fp32 path expands at a time: fp32 rows and their two-part
// split take 8 bytes a weight, kept within kF32ExpandBytes in whole 320-row big tiles;
// where N allows, at least the rows that give an M-row product 192 big tiles (the
// big-tile kernel's threshold: 3840 rows at M = 4096, where smaller chunks ran on the
// 128x128 kernel at half the speed).
constexpr size_t kF32ExpandBytes = (size_t)256 << 20;
static int f32_rows(int N, int kp, int M) {
  const size_t r = kF32ExpandBytes / ((size_t)kp * 8);
  if (r >= (size_t)N) return N;
  const int ntm = (M + 255) / 256, big = (192 + ntm - 1) / ntm * 320;
  const int bounded = std::max(320, (int)(r / 320 * 320));
  return std::min(N, big <= N ? std::max(big, bounded) : bounded);
}

// tiermm_qgemm for dense rows (F32 / F16 / BF16) whose length K is not a multiple of
// the 32-wide K step (every block type is): W and x are copied into the workspace
// as rows of Kp = roundup(K, 32) with zeros past K, then multiplied as usual.
static int qgemm_padded(const void* W, int qtype, size_t rb, const float* X, float* Y, int M, int N, int K, int ldy,
                        int mode, float beta, void* w, hipStream_t s, const char* who) {
  if (qtype != TIERMM_F32 && qtype != TIERMM_F16 && qtype != TIERMM_BF16)
    return set_error(TIERMM_EINVAL, "%s: K=%d is not whole blocks of type %d", who, K, qtype);
  const int kp = pad32(K);
  const size_t nkp = (size_t)N * kp, mkp = (size_t)M * kp;
  const uint8_t* wq = (const uint8_t*)W;
  // rows [n0, n0 + nr) of W into out, as rows of kp
  auto dense_pad = [&](void* out, bool f16, int n0, int nr) {
    const unsigned g = elem_grid((size_t)nr * kp);
    const uint8_t* src = wq + (size_t)n0 * rb;
    if (qtype == TIERMM_F32) {
      if (f16) dense_pad_kernel<QT_F32, true><<<g, 256, 0, s>>>(src, rb, out, (size_t)nr, K, kp);
      else dense_pad_kernel<QT_F32, false><<<g, 256, 0, s>>>(src, rb, out, (size_t)nr, K, kp);
    } else if (qtype == TIERMM_F16) {
      if (f16) dense_pad_kernel<QT_F16, true><<<g, 256, 0, s>>>(src, rb, out, (size_t)nr, K, kp);
      else dense_pad_kernel<QT_F16, false><<<g, 256, 0, s>>>(src, rb, out, (size_t)nr, K, kp);
    } else {
      if (f16) dense_pad_kernel<QT_BF16, true><<<g, 256, 0, s>>>(src, rb, out, (size_t)nr, K, kp);
      else dense_pad_kernel<QT_BF16, false><<<g, 256, 0, s>>>(src, rb, out, (size_t)nr, K, kp);
    }
  };
  if (mode == TIERMM_MODE_F32) {  // chunks of f32_rows weight rows, as in tiermm_qgemm
    const int nc = f32_rows(N, kp, M);
    uint8_t* b = (uint8_t*)w;
    float* wf = (float*)b;       b += al256((size_t)nc * kp * 4);
    uint16_t* whi = (uint16_t*)b; b += al256((size_t)nc * kp * 2);
    uint16_t* wlo = (uint16_t*)b; b += al256((size_t)nc * kp * 2);
    int32_t* wexp = (int32_t*)b;  b += al256((size_t)nc * 4);
    float* xf = (float*)b;        b += al256(mkp * 4);
    uint16_t* xhi = (uint16_t*)b; b += al256(mkp * 2);
    uint16_t* xlo = (uint16_t*)b; b += al256(mkp * 2);
    int32_t* xexp = (int32_t*)b;
    pad32_kernel<<<elem_grid(mkp), 256, 0, s>>>(X, (size_t)K, xf, (size_t)M, K, kp);
    TM_LAUNCH_CHECK("tiermm_qgemm: padded x");
    x3s_split_launch(xf, xhi, xlo, xexp, M, kp, s);
    TM_LAUNCH_CHECK("tiermm_qgemm: split x");
    for (int n0 = 0; n0 < N; n0 += nc) {
      const int nr = std::min(nc, N - n0);
      dense_pad(wf, false, n0, nr);
      TM_LAUNCH_CHECK("tiermm_qgemm: padded W");
      x3s_split_launch(wf, whi, wlo, wexp, nr, kp, s);
      TM_LAUNCH_CHECK("tiermm_qgemm: split W");
      X3Args a{};
      a.A[0] = xhi; a.A[1] = xlo; a.B[0] = whi; a.B[1] = wlo;
      a.lda = kp; a.ldb = kp; a.C = Y + n0; a.ldc = ldy; a.M = M; a.N = nr; a.K = kp;
      a.aexp = xexp; a.bexp = wexp; a.beta = beta;
      int st = big_tiles(M, nr) >= 192 ? launch_x3_big<X3_2X2>(a, s, who) : launch_x3<128, 128, X3_2X2>(a, s, who);
      if (st) return st;
    }
    return TIERMM_OK;
  }
  uint16_t* w16 = (uint16_t*)w;
  uint16_t* parts = (uint16_t*)((uint8_t*)w + al256(nkp * 2));
  dense_pad(w16, true, 0, N);
  TM_LAUNCH_CHECK("tiermm_qgemm: padded W");
  pad_split3_kernel<false><<<elem_grid(mkp), 256, 0, s>>>(X, (size_t)K, parts, (size_t)M, K, kp);
  TM_LAUNCH_CHECK("tiermm_qgemm: padded split");
  return x3ref_nt(parts, mkp, w16, kp, Y, ldy, M, N, kp, beta, s, who);
}

size_t tiermm_sgemm_ws_bytes(int opA, int m, int n, int k) {
  // hi/lo planes and exponents of op(A) (m rows) and of B (n rows), rows of kp; for
  // TIERMM_OP_N the column maxima of A
  const size_t kp = (size_t)pad32(k);
  return 2 * al256((size_t)m * kp * 2) + al256((size_t)m * 4) + 2 * al256((size_t)n * kp * 2) + al256((size_t)n * 4) +
         (opA == TIERMM_OP_N ? al256((size_t)m * 4) : 0);
}

int tiermm_sgemm(int opA, int m, int n, int k, const float* A, int lda, const float* B, int ldb, float beta, float* C,
                 int ldc, void* ws, size_t ws_bytes, tiermm_stream_t stream) {
  const char* who = "tiermm_sgemm";
  if (opA != TIERMM_OP_T && opA != TIERMM_OP_N) return set_error(TIERMM_EINVAL, "%s: opA %d", who, opA);
  int st = check_sizes(who, n, m, k);
  if (st) return st;
  if ((opA == TIERMM_OP_T && lda < k) || (opA == TIERMM_OP_N && lda < m) || ldb < k || ldc < m)
    return set_error(TIERMM_EINVAL, "%s: lda, ldb or ldc too small", who);
  if (m == 0 || n == 0) return TIERMM_OK;
  if (!A || !B || !C) return set_error(TIERMM_EINVAL, "%s: null buffer", who);
  void* w = nullptr;
  st = get_workspace(ws, ws_bytes, tiermm_sgemm_ws_bytes(opA, m, n, k), &w, who);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  const int kp = pad32(k);
  uint8_t* b = (uint8_t*)w;
  uint16_t* ahi = (uint16_t*)b; b += al256((size_t)m * kp * 2);
  uint16_t* alo = (uint16_t*)b; b += al256((size_t)m * kp * 2);
  int32_t* aexp = (int32_t*)b;  b += al256((size_t)m * 4);
  uint16_t* bhi = (uint16_t*)b; b += al256((size_t)n * kp * 2);
  uint16_t* blo = (uint16_t*)b; b += al256((size_t)n * kp * 2);
  int32_t* bexp = (int32_t*)b;  b += al256((size_t)n * 4);
  // rows [rows][ld] into rows of kp: the register-resident split when they are packed
  // rows of a whole number of K steps, else the general one
  auto split_rows = [&](const float* src, int ld, int rows, uint16_t* hi, uint16_t* lo, int32_t* ex) {
    if (ld == kp && kp == k) x3s_split_launch(src, hi, lo, ex, rows, k, s);
    else x3s_split_ld_kernel<<<rows, 256, 0, s>>>(src, (size_t)ld, k, kp, hi, lo, ex);
  };
  if (opA == TIERMM_OP_T) {  // op(A) rows are A's rows: [m][lda]
    split_rows(A, lda, m, ahi, alo, aexp);
    TM_LAUNCH_CHECK("tiermm_sgemm: split A");
  } else {  // op(A) rows are A's columns: A is [k][lda] in memory (linear_dx, tier.cpp:1226)
    uint32_t* amax = (uint32_t*)b;
    zero32_kernel<<<(unsigned)((m + 255) / 256), 256, 0, s>>>(amax, (size_t)m);
    TM_LAUNCH_CHECK("tiermm_sgemm: column maxima");
    col_absmax_kernel<<<dim3((unsigned)((m + 255) / 256), (unsigned)((k + 255) / 256)), 256, 0, s>>>(A, (size_t)lda, k,
                                                                                                  m, amax);
    TM_LAUNCH_CHECK("tiermm_sgemm: column maxima");
    x3s_split_t_kernel<<<dim3((unsigned)((m + 63) / 64), (unsigned)((kp + 63) / 64)), 256, 0, s>>>(
        A, (size_t)lda, k, m, kp, amax, ahi, alo, aexp);
    TM_LAUNCH_CHECK("tiermm_sgemm: split A");
  }
  split_rows(B, ldb, n, bhi, blo, bexp);
  TM_LAUNCH_CHECK("tiermm_sgemm: split B");
  // column-major C(m x n) with ldc == row-major out[n][ldc] = B^T[n][k] * op(A)^T
  X3Args a{};
  a.A[0] = bhi; a.A[1] = blo; a.B[0] = ahi; a.B[1] = alo;
  a.lda = kp; a.ldb = kp; a.C = C; a.ldc = ldc; a.M = n; a.N = m; a.K = kp;
  a.aexp = bexp; a.bexp = aexp; a.beta = beta;
  if (big_tiles(n, m) >= 192) return launch_x3_big<X3_2X2>(a, s, who);
  return launch_x3<128, 128, X3_2X2>(a, s, who);
}

size_t tiermm_qgemm_ws_bytes(int qtype, int M, int N, int K, int mode) {
  if (K % BK) {  // dense rows of an odd length: W and x padded to rows of Kp
    const size_t kp = (size_t)pad32(K);
    if (mode == TIERMM_MODE_F32) {  // a chunk of padded fp32 W rows, padded fp32 x, their two-part splits
      const size_t nc = (size_t)f32_rows(N, (int)kp, M);
      return al256(nc * kp * 4) + 2 * al256(nc * kp * 2) + al256(nc * 4) + al256((size_t)M * kp * 4) +
             2 * al256((size_t)M * kp * 2) + al256((size_t)M * 4);
    }
    return al256((size_t)N * kp * 2) + (size_t)3 * M * kp * sizeof(uint16_t);  // padded W16, x planes
  }
  if (mode == TIERMM_MODE_F32) {
    if (qgemm_fusable(qtype, &M, 1, N, K, true, true))  // x's two-part split, both exponent rows; split-K partials
      return 2 * al256((size_t)M * K * 2) + al256((size_t)M * 4) + al256((size_t)N * 4) +
             qgemm_fused_partials_bytes(qtype, M, N, K, true);
    // a chunk of fp32 W rows, their two-part split, and x's
    const size_t nc = (size_t)f32_rows(N, K, M);
    return al256(nc * K * 4) + 2 * al256(nc * K * 2) + al256(nc * 4) + 2 * al256((size_t)M * K * 2) +
           al256((size_t)M * 4);
  }
  const size_t parts = (size_t)3 * M * K * sizeof(uint16_t);  // x split in three fp16 planes
  if (qgemm_fusable(qtype, &M, 1, N, K, true))
    return al256(parts) + qgemm_fused_partials_bytes(qtype, M, N, K);  // W decoded inside the GEMM; split-K partials
  return (size_t)N * K * sizeof(uint16_t) + parts;                   // W16 staged in the workspace
}

int tiermm_qgemm(const void* W, int qtype, size_t rb, const float* X, float* Y, int M, int N, int K, int ldy,
                 int mode, float beta, void* ws, size_t ws_bytes, tiermm_stream_t stream) {
  const char* who = "tiermm_qgemm";
  int st = check_qweight(who, W, qtype, rb, K, 1);
  if (st) return st;
  if (mode != TIERMM_MODE_X3REF && mode != TIERMM_MODE_F32) return set_error(TIERMM_EINVAL, "%s: mode %d", who, mode);
  st = check_sizes(who, M, N, K);
  if (st) return st;
  if (ldy < N) return set_error(TIERMM_EINVAL, "%s: ldy < N", who);
  if (M == 0 || N == 0) return TIERMM_OK;
  if (!X || !Y) return set_error(TIERMM_EINVAL, "%s: null buffer", who);
  void* w = nullptr;
  st = get_workspace(ws, ws_bytes, tiermm_qgemm_ws_bytes(qtype, M, N, K, mode), &w, who);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  if (K % BK) return qgemm_padded(W, qtype, rb, X, Y, M, N, K, ldy, mode, beta, w, s, who);
  const size_t mk = (size_t)M * K;
  if (mode == TIERMM_MODE_F32 && qgemm_fusable(qtype, &M, 1, N, K, true, true)) {
    // the same semantics with W decoded inside the GEMM: no fp32 or fp16 copy of W
    // in memory; one pass over the weight's block scales for its row exponents first
    uint8_t* b = (uint8_t*)w;
    uint16_t* xhi = (uint16_t*)b;             b += al256(mk * 2);
    b += al256(mk * 2);                       // xlo, one plane stride after xhi
    int32_t* xexp = (int32_t*)b;              b += al256((size_t)M * 4);
    int32_t* wexp = (int32_t*)b;              b += al256((size_t)N * 4);
    float* partials = (float*)b;
    const size_t xs = al256(mk * 2) / 2;
    st = f32_prep(X, xhi, xhi + xs, xexp, M, K, W, qtype, rb, N, wexp, s);  // both passes in one launch
    if (st == TIERMM_UNSUPPORTED) {
      x3s_split_launch(X, xhi, xhi + xs, xexp, M, K, s);
      TM_LAUNCH_CHECK("tiermm_qgemm: split x");
      st = qrow_exps(W, qtype, rb, N, K, wexp, s);
    }
    if (st) return st;
    int cus = 0;
    st = device_cus(&cus);
    if (st) return st;
    return qgemm_fused(W, qtype, rb, xhi, xs, 0, Y, ldy, M, N, K, beta, cus, s, who, partials, xexp, wexp);
  }
  if (mode == TIERMM_MODE_F32) {
    // chat prefill semantics (tier.cpp:2358-2359): fp32 dequant, fp32-accurate
    // product -- here the two-part split GEMM (relative error ~2^-21 of fp64) over
    // chunks of f32_rows weight rows, each expanded to fp32 and split in the
    // workspace (the reference expands a bounded chunk too, tier.cpp:2225-2227)
    const int nc = f32_rows(N, K, M);
    uint8_t* b = (uint8_t*)w;
    float* wf = (float*)b;                    b += al256((size_t)nc * K * 4);
    uint16_t* whi = (uint16_t*)b;             b += al256((size_t)nc * K * 2);
    uint16_t* wlo = (uint16_t*)b;             b += al256((size_t)nc * K * 2);
    int32_t* wexp = (int32_t*)b;              b += al256((size_t)nc * 4);
    uint16_t* xhi = (uint16_t*)b;             b += al256(mk * 2);
    uint16_t* xlo = (uint16_t*)b;             b += al256(mk * 2);
    int32_t* xexp = (int32_t*)b;
    x3s_split_launch(X, xhi, xlo, xexp, M, K, s);
    TM_LAUNCH_CHECK("tiermm_qgemm: split x");
    for (int n0 = 0; n0 < N; n0 += nc) {
      const int nr = std::min(nc, N - n0);
      st = tiermm_dequant(W, qtype, rb, K, (size_t)n0, (size_t)nr, wf, TIERMM_OUT_F32, stream);
      if (st) return st;
      x3s_split_launch(wf, whi, wlo, wexp, nr, K, s);
      TM_LAUNCH_CHECK("tiermm_qgemm: split W");
      X3Args a{};
      a.A[0] = xhi; a.A[1] = xlo; a.B[0] = whi; a.B[1] = wlo;
      a.lda = K; a.ldb = K; a.C = Y + n0; a.ldc = ldy; a.M = M; a.N = nr; a.K = K;
      a.aexp = xexp; a.bexp = wexp; a.beta = beta;
      st = big_tiles(M, nr) >= 192 ? launch_x3_big<X3_2X2>(a, s, who) : launch_x3<128, 128, X3_2X2>(a, s, who);
      if (st) return st;
    }
    return TIERMM_OK;
  }
  // The types the fused kernel decodes, at every M: W is decoded inside the GEMM (at
  // M = 4096 the wide-tile plans beat fp16 staging + the big-tile GEMM by 5-25 %).
  if (qgemm_fusable(qtype, &M, 1, N, K, true)) {
    uint16_t* parts = (uint16_t*)w;
    float* partials = (float*)((uint8_t*)w + al256(3 * mk * sizeof(uint16_t)));
    // K-tiled planes where x allows (a fragment load is then one contiguous kilobyte)
    const size_t xt = ((uintptr_t)X & 15) == 0 ? (size_t)M : 0;
    st = split3_launch(X, parts, mk, mk, TIERMM_HML, s, false, xt, K);
    if (st) return st;
    int cus = 0;
    st = device_cus(&cus);
    if (st) return st;
    return qgemm_fused(W, qtype, rb, parts, mk, xt, Y, ldy, M, N, K, beta, cus, s, who, partials);
  }
  uint16_t* w16 = (uint16_t*)w;
  uint16_t* parts = w16 + (size_t)N * K;
  // The big-tile kernel reads the planes K-tiled (one contiguous kilobyte per load,
  // ~4 % faster); the small-tile kernel reads them row-major.
  const bool tiled = big_tiles(M, N) >= 192 && K % 32 == 0 && ((uintptr_t)X & 15) == 0;
  st = dequant_f16_rows(W, qtype, rb, K, (size_t)N, w16, s, tiled);
  if (st) return st;
  st = split3_launch(X, parts, mk, mk, TIERMM_HML, s, false, tiled ? (size_t)M : 0, K);
  if (st) return st;
  if (!tiled) return x3ref_nt(parts, mk, w16, K, Y, ldy, M, N, K, beta, s, who);
  X3Args a{};
  a.A[0] = parts; a.A[1] = parts + mk; a.A[2] = parts + 2 * mk;
  a.B[0] = w16;
  a.lda = K; a.ldb = K; a.atile = M; a.btile = N;
  a.C = Y; a.ldc = ldy; a.M = M; a.N = N; a.K = K; a.beta = beta;
  return launch_x3_big<X3_REF>(a, s, who);
}

size_t tiermm_qgemm_x3parts_ws_bytes(int qtype, int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % BK) return 0;
  if (qgemm_fusable(qtype, &M, 1, N, K, true)) return qgemm_fused_partials_bytes(qtype, M, N, K);
  return (size_t)N * K * sizeof(uint16_t);  // the fp16 weight
}

int tiermm_qgemm_x3parts(const void* W, int qtype, size_t rb, const uint16_t* xparts, size_t part_stride,
                         int layout, float* Y, int M, int N, int K, int ldy, float beta, void* ws, size_t ws_bytes,
                         tiermm_stream_t stream) {
  const char* who = "tiermm_qgemm_x3parts";
  int st = check_qweight(who, W, qtype, rb, K, 1);
  if (st) return st;
  st = check_nt(who, M, N, K);
  if (st) return st;
  if (ldy < N) return set_error(TIERMM_EINVAL, "%s: ldy < N", who);
  if (layout != TIERMM_PARTS_ROWS && layout != TIERMM_PARTS_KTILED)
    return set_error(TIERMM_EINVAL, "%s: layout %d", who, layout);
  const bool tiled = layout == TIERMM_PARTS_KTILED;
  if (M == 0 || N == 0) return TIERMM_OK;
  if (!xparts || !Y || !aligned16(xparts) || part_stride < (size_t)M * K || part_stride % 8)
    return set_error(TIERMM_EINVAL, "%s: x planes must be 16-byte aligned, part_stride >= M*K and a multiple of 8",
                     who);
  void* w = nullptr;
  st = get_workspace(ws, ws_bytes, tiermm_qgemm_x3parts_ws_bytes(qtype, M, N, K), &w, who);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  if (qgemm_fusable(qtype, &M, 1, N, K, true)) {
    int cus = 0;
    st = device_cus(&cus);
    if (st) return st;
    return qgemm_fused(W, qtype, rb, xparts, part_stride, tiled ? (size_t)M : 0, Y, ldy, M, N, K, beta, cus, s, who,
                       (float*)w);
  }
  uint16_t* w16 = (uint16_t*)w;
  st = dequant_f16_rows(W, qtype, rb, K, (size_t)N, w16, s, tiled);
  if (st) return st;
  if (!tiled) return x3ref_nt(xparts, part_stride, w16, K, Y, ldy, M, N, K, beta, s, who);
  X3Args a{};  // both operands K-tiled: the big-tile kernel (rows past M or N read clamped)
  a.A[0] = xparts; a.A[1] = xparts + part_stride; a.A[2] = xparts + 2 * part_stride;
  a.B[0] = w16;
  a.lda = K; a.ldb = K; a.atile = M; a.btile = N;
  a.C = Y; a.ldc = ldy; a.M = M; a.N = N; a.K = K; a.beta = beta;
  return launch_x3_big<X3_REF>(a, s, who);
}

size_t tiermm_qgemm_grouped_ws_bytes(const int* qtype_e, const int* expert_offsets, int n_experts, int N, int K,
                                     int mode) {
  size_t need = 0;
  if (mode == TIERMM_MODE_F32) {  // expert by expert through tiermm_qgemm
    for (int e = 0; e < n_experts; ++e) {
      const int Me = expert_offsets[e + 1] - expert_offsets[e];
      if (Me > 0) need = std::max(need, tiermm_qgemm_ws_bytes(qtype_e[e], Me, N, K, mode));
    }
    return need;
  }
  // x3-ref: the three fp16 planes of all routed rows, plus the fp16 weights of a
  // chunk of experts (grouped 256x320 launch) or of one expert at a time (the
  // experts that are not decoded inside the GEMM)
  const size_t P = n_experts > 0 ? (size_t)expert_offsets[n_experts] : 0;
  const auto types = routed_types(qtype_e, expert_offsets, n_experts, N, K);
  bool staged = false;
  for (auto& t : types) staged = staged || !t.second;
  const int chunk = staged && n_experts > 0 ? big_group_chunk(expert_offsets, n_experts, N, K) : 0;
  if (chunk) return al256(3 * P * K * sizeof(uint16_t)) + chunk * al256((size_t)N * K * sizeof(uint16_t));
  return al256(3 * P * K * sizeof(uint16_t)) + (staged ? (size_t)N * K * sizeof(uint16_t) : 0);
}

int tiermm_qgemm_grouped(const void* const* W_e, const int* qtype_e, const size_t* rb_e, const float* X_sorted,
                         const int* expert_offsets, int n_experts, float* Y_sorted, int N, int K, int mode, void* ws,
                         size_t ws_bytes, tiermm_stream_t stream) {
  const char* who = "tiermm_qgemm_grouped";
  if (n_experts < 0 || !expert_offsets || (n_experts && (!W_e || !qtype_e || !rb_e)))
    return set_error(TIERMM_EINVAL, "%s: null expert tables", who);
  if (n_experts && expert_offsets[0] != 0) return set_error(TIERMM_EINVAL, "%s: expert_offsets[0] != 0", who);
  for (int e = 0; e < n_experts; ++e)
    if (expert_offsets[e + 1] < expert_offsets[e]) return set_error(TIERMM_EINVAL, "%s: offsets decrease at %d", who, e);
  if (mode != TIERMM_MODE_X3REF && mode != TIERMM_MODE_F32) return set_error(TIERMM_EINVAL, "%s: mode %d", who, mode);
  int st = check_nt(who, 1, N, K);
  if (st) return st;
  for (int e = 0; e < n_experts; ++e) {
    if (expert_offsets[e + 1] == expert_offsets[e]) continue;
    st = check_qweight(who, W_e[e], qtype_e[e], rb_e[e], K, 8);
    if (st) return st;
  }
  if (n_experts == 0 || expert_offsets[n_experts] == 0 || N == 0) return TIERMM_OK;
  if (!X_sorted || !Y_sorted) return set_error(TIERMM_EINVAL, "%s: null buffer", who);
  const size_t wsb = tiermm_qgemm_grouped_ws_bytes(qtype_e, expert_offsets, n_experts, N, K, mode);
  void* w = nullptr;
  st = get_workspace(ws, ws_bytes, wsb, &w, who);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  if (mode == TIERMM_MODE_F32) {  // one stream: the experts run in order and share the workspace
    for (int e = 0; e < n_experts; ++e) {
      const int o = expert_offsets[e], Me = expert_offsets[e + 1] - o;
      if (Me == 0) continue;
      st = tiermm_qgemm(W_e[e], qtype_e[e], rb_e[e], X_sorted + (size_t)o * K, Y_sorted + (size_t)o * N, Me, N, K, N,
                        mode, 0.f, w, wsb, stream);
      if (st) return st;
    }
    return TIERMM_OK;
  }
  // x3-ref: split every routed row once; each expert multiplies its slice of the planes
  const size_t P = (size_t)expert_offsets[n_experts], pk = P * K;
  uint16_t* parts = (uint16_t*)w;
  uint16_t* w16 = (uint16_t*)((uint8_t*)w + al256(3 * pk * sizeof(uint16_t)));
  // Every routed type one the fused kernel decodes: one fused launch per type (no fp16
  // decode pass), which beats decode + the grouped big-tile launch (config 5's gate/up,
  // 64 q4_K experts of ~512 rows, N = 1408, K = 2048: the MoE line 2.72 ms against
  // 2.86 ms).  Otherwise, where the experts' 256-row tiles fill the chip, every expert
  // goes through fp16 staging and the grouped big-tile launch.
  const auto types = routed_types(qtype_e, expert_offsets, n_experts, N, K);
  bool all_fused = !types.empty();
  for (auto& t : types) all_fused = all_fused && t.second;
  const int chunk = all_fused ? 0 : big_group_chunk(expert_offsets, n_experts, N, K);
  // the grouped big-tile launch and the all-fused launches read K-tiled planes; the
  // per-expert paths row-major ones
  const bool tiled = (chunk || all_fused) && K % 32 == 0 && ((uintptr_t)X_sorted & 15) == 0;
  st = split3_launch(X_sorted, parts, pk, pk, TIERMM_HML, s, false, tiled ? P : 0, K);
  if (st) return st;
  if (chunk) {  // fp16 weights of up to `chunk` experts, then one grouped launch over their tiles
    const size_t per = al256((size_t)N * K * sizeof(uint16_t));
    X3Args a{};
    a.A[0] = parts; a.A[1] = parts + pk; a.A[2] = parts + 2 * pk;
    a.lda = K; a.ldb = K; a.C = Y_sorted; a.ldc = N; a.N = N; a.K = K;
    if (tiled) {
      a.atile = (int)P;
      a.btile = N;
    }
    std::vector<int> ex;
    for (int e = 0; e < n_experts; ++e)
      if (expert_offsets[e + 1] > expert_offsets[e]) ex.push_back(e);
    for (size_t c0 = 0; c0 < ex.size(); c0 += chunk) {
      const int n = (int)std::min<size_t>(chunk, ex.size() - c0);
      X3Groups g{};
      g.n = n;
      for (int i = 0; i < n; ++i) {
        const int e = ex[c0 + i];
        g.row0[i] = expert_offsets[e];
        g.rows[i] = expert_offsets[e + 1] - expert_offsets[e];
        g.B[i] = (const uint16_t*)((uint8_t*)w16 + i * per);
        g.tile0[i + 1] = g.tile0[i] + (int)big_tiles(g.rows[i], N);
      }
      // one decode launch per weight type in the chunk
      std::vector<char> done(n, 0);
      for (int i = 0; i < n; ++i) {
        if (done[i]) continue;
        const int qt = qtype_e[ex[c0 + i]];
        std::vector<const void*> src;
        std::vector<uint16_t*> dst;
        for (int j = i; j < n; ++j)
          if (!done[j] && qtype_e[ex[c0 + j]] == qt) {
            done[j] = 1;
            src.push_back(W_e[ex[c0 + j]]);
            dst.push_back((uint16_t*)g.B[j]);
          }
        st = dequant_f16_group(src.data(), dst.data(), (int)src.size(), qt, rb_e[ex[c0 + i]], K, (size_t)N, s, tiled);
        if (st) return st;
      }
      st = big_tn(N) == 352 ? launch_x3_big_grouped<X3_REF, 352>(a, g, s, who)
                            : launch_x3_big_grouped<X3_REF, 320>(a, g, s, who);
      if (st) return st;
    }
    return TIERMM_OK;
  }
  int cus = 0;
  st = device_cus(&cus);
  if (st) return st;
  // experts of each fused type: one launch (per 64 experts) whose workgroups cover every
  // expert's tiles
  for (auto& t : types) {
    if (!t.second) continue;
    std::vector<const void*> gw;
    std::vector<int> g0, gr;
    size_t grb = 0;
    for (int e = 0; e < n_experts; ++e) {
      const int o = expert_offsets[e], Me = expert_offsets[e + 1] - o;
      if (Me == 0 || qtype_e[e] != t.first) continue;
      if (grb && rb_e[e] != grb) return set_error(TIERMM_EINVAL, "%s: experts of one type with different row bytes", who);
      grb = rb_e[e];
      gw.push_back(W_e[e]);
      g0.push_back(o);
      gr.push_back(Me);
    }
    st = qgemm_fused_groups(gw.data(), t.first, g0.data(), gr.data(), (int)gw.size(), grb, parts, pk,
                            tiled ? P : 0, Y_sorted, N, N, K, 0.f, cus, s, who, nullptr);
    if (st) return st;
  }
  // other types: fp16 W staged per expert, then the x3-ref GEMM on the expert's rows
  for (int e = 0; e < n_experts; ++e) {
    const int o = expert_offsets[e], Me = expert_offsets[e + 1] - o;
    if (Me == 0 || type_fused(types, qtype_e[e])) continue;
    st = dequant_f16_rows(W_e[e], qtype_e[e], rb_e[e], K, (size_t)N, w16, s);
    if (!st) st = x3ref_nt(parts + (size_t)o * K, pk, w16, K, Y_sorted + (size_t)o * N, N, Me, N, K, 0.f, s, who);
    if (st) return st;
  }
  return TIERMM_OK;
}

int tiermm_moe_combine(const float* Y_sorted, const int* token_pairs, const float* pair_weight, float* out, int T,
                       int topk, int N, tiermm_stream_t stream) {
  if (T < 0 || topk < 0 || N < 0) return set_error(TIERMM_EINVAL, "tiermm_moe_combine: negative size");
  if (T == 0 || N == 0) return TIERMM_OK;
  if (!Y_sorted || !token_pairs || !pair_weight || !out) return set_error(TIERMM_EINVAL, "tiermm_moe_combine: null buffer");
  if (N % 4 == 0 && topk <= 16 && ((uintptr_t)Y_sorted & 15) == 0 && ((uintptr_t)out & 15) == 0)
    moe_combine4_kernel<<<T, 256, 0, (hipStream_t)stream>>>(Y_sorted, token_pairs, pair_weight, out, topk, N);
  else
    moe_combine_kernel<<<T, 256, 0, (hipStream_t)stream>>>(Y_sorted, token_pairs, pair_weight, out, topk, N);
  TM_LAUNCH_CHECK("tiermm_moe_combine: launch");
  return TIERMM_OK;
}

}  // extern "C"

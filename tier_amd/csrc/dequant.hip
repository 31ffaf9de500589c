// dequant.hip -- tiermm_dequant: quantized or dense rows -> fp32 / fp16 / bf16 (dq_k<T>,
// tier.cpp:293-298).
//
// One thread decodes 8 consecutive outputs of a row and writes them with one
// 16-byte store (fp16/bf16) or two (fp32): the kernel is bound by the output
// writes (2 B/element for fp16 against 0.56 B/element read for Q4_K).
#include "tm_device.h"

namespace tiermm {
namespace {

// trows > 0: fp16 output in the K-tiled layout of a plane of trows rows (ktile_index),
// written in unit order.
template <int QT, int OUT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ W, size_t rb, int cols, size_t r0,
                                                      size_t n8, void* __restrict__ out, size_t trows = 0) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n8; t += stride) {
    const size_t e = t * 8;  // output offset: unit t in row-major or K-tiled order
    size_t row;
    int col;
    if (trows) {
      ktile_unit(t, trows, row, col);
    } else {
      row = e / (size_t)cols;
      col = (int)(e - row * (size_t)cols);
    }
    float v[8];
    Dec<QT>::run(W + (r0 + row) * rb, col, v);
    if (OUT == TIERMM_OUT_F32) {
      float4* o = (float4*)((float*)out + e);
      o[0] = make_float4(v[0], v[1], v[2], v[3]);
      o[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint32_t p[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = OUT == TIERMM_OUT_F16 ? f2h(v[2 * k]) : f2bf(v[2 * k]);
        const uint32_t hi = OUT == TIERMM_OUT_F16 ? f2h(v[2 * k + 1]) : f2bf(v[2 * k + 1]);
        p[k] = lo | (hi << 16);
      }
      *(uint4*)((uint16_t*)out + e) = make_uint4(p[0], p[1], p[2], p[3]);
    }
  }
}

template <int QT>
int launch_dequant(const void* W, size_t rb, int cols, size_t r0, size_t nrows, void* out, int out_dtype,
                   hipStream_t s) {
  const size_t n8 = nrows * (size_t)cols / 8;
  if (n8 == 0) return TIERMM_OK;
  const size_t want = (n8 + 255) / 256;
  const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
  const uint8_t* w = (const uint8_t*)W;
  switch (out_dtype) {
    case TIERMM_OUT_F32: dequant_kernel<QT, TIERMM_OUT_F32><<<grid, 256, 0, s>>>(w, rb, cols, r0, n8, out); break;
    case TIERMM_OUT_F16: dequant_kernel<QT, TIERMM_OUT_F16><<<grid, 256, 0, s>>>(w, rb, cols, r0, n8, out); break;
    default: dequant_kernel<QT, TIERMM_OUT_BF16><<<grid, 256, 0, s>>>(w, rb, cols, r0, n8, out); break;
  }
  TM_LAUNCH_CHECK("tiermm_dequant: launch");
  return TIERMM_OK;
}

// Dense rows (F32 / F16 / BF16) one element per thread: out[i] = T(q_val(row, col)),
// i < n = nrows * cols, for row lengths that are not whole 8-element chunks.
template <int QT, int OUT>
__global__ __launch_bounds__(256) void dequant_elem_kernel(const uint8_t* __restrict__ W, size_t rb, int cols,
                                                           size_t r0, size_t n, void* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const size_t row = i / (size_t)cols;
    const float v = dense_val<QT>(W + (r0 + row) * rb, i - row * (size_t)cols);
    if (OUT == TIERMM_OUT_F32) ((float*)out)[i] = v;
    else ((uint16_t*)out)[i] = OUT == TIERMM_OUT_F16 ? f2h(v) : f2bf(v);
  }
}

template <int QT>
int launch_dequant_elems(const void* W, size_t rb, int cols, size_t r0, size_t nrows, void* out, int out_dtype,
                         hipStream_t s) {
  const size_t n = nrows * (size_t)cols;
  if (n == 0) return TIERMM_OK;
  const size_t want = (n + 255) / 256;
  const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
  const uint8_t* w = (const uint8_t*)W;
  switch (out_dtype) {
    case TIERMM_OUT_F32: dequant_elem_kernel<QT, TIERMM_OUT_F32><<<grid, 256, 0, s>>>(w, rb, cols, r0, n, out); break;
    case TIERMM_OUT_F16: dequant_elem_kernel<QT, TIERMM_OUT_F16><<<grid, 256, 0, s>>>(w, rb, cols, r0, n, out); break;
    default: dequant_elem_kernel<QT, TIERMM_OUT_BF16><<<grid, 256, 0, s>>>(w, rb, cols, r0, n, out); break;
  }
  TM_LAUNCH_CHECK("tiermm_dequant: launch");
  return TIERMM_OK;
}

// f(std::integral_constant<int, QT>{}) for a dense type F32 / F16 / BF16.
template <class F>
auto with_dense(int qtype, F&& f) {
  if (qtype == QT_F32) return f(std::integral_constant<int, QT_F32>{});
  if (qtype == QT_F16) return f(std::integral_constant<int, QT_F16>{});
  return f(std::integral_constant<int, QT_BF16>{});
}

// Several weights of one type and shape to fp16 in one launch: blockIdx.y picks
// the weight (routed experts before their grouped GEMM).
constexpr int DQ_GROUP = 64;
struct DqGroup {
  const uint8_t* W[DQ_GROUP];
  uint16_t* out[DQ_GROUP];
};

template <int QT>
__global__ __launch_bounds__(256) void dequant_f16_group_kernel(const DqGroup g, size_t rb, int cols, size_t n8,
                                                                size_t trows) {
  const uint8_t* W = g.W[blockIdx.y];
  uint16_t* out = g.out[blockIdx.y];
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n8; t += stride) {
    const size_t e = t * 8;  // output offset: unit t in row-major or K-tiled order
    size_t row;
    int col;
    if (trows) {
      ktile_unit(t, trows, row, col);
    } else {
      row = e / (size_t)cols;
      col = (int)(e - row * (size_t)cols);
    }
    float v[8];
    Dec<QT>::run(W + row * rb, col, v);
    uint32_t p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) p[k] = f2h(v[2 * k]) | (f2h(v[2 * k + 1]) << 16);
    *(uint4*)(out + e) = make_uint4(p[0], p[1], p[2], p[3]);
  }
}

}  // namespace

// Shared argument checks for a quantized weight: type handled, rb consistent,
// alignment of the row bytes the decoders assume.
bool gpu_type(int qtype) {
  switch (qtype) {
    case QT_F32: case QT_F16: case QT_BF16: case QT_Q4_0: case QT_Q4_1: case QT_Q5_0: case QT_Q5_1:
    case QT_Q8_0: case QT_Q2_K: case QT_Q3_K: case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: case QT_IQ4_NL:
    case QT_IQ4_XS: case QT_TQ1_0: case QT_TQ2_0: case QT_MXFP4: case QT_NF4: case QT_FP4:
    case QT_IQ2_XXS: case QT_IQ2_XS: case QT_IQ2_S: case QT_IQ3_XXS: case QT_IQ3_S: case QT_IQ1_S:
    case QT_IQ1_M: return true;
    default: return false;
  }
}

// dense_unit: the column granularity the caller needs for dense rows (F32 / F16 /
// BF16): 8 where its kernels decode 8 consecutive elements at a time, 1 where it
// has an element-wise path for other lengths.
int check_qweight(const char* who, const void* W, int qtype, size_t rb, int cols, int dense_unit) {
  const BlockInfo* bi = block_info(qtype);
  if (!bi || !gpu_type(qtype)) return set_error(TIERMM_UNSUPPORTED, "%s: type %d is not handled on the GPU", who, qtype);
  const int whole = bi->elems > 1 ? (bi->elems > 8 ? bi->elems : 8) : dense_unit;
  if (cols <= 0 || cols % whole)
    return set_error(TIERMM_UNSUPPORTED, "%s: %d columns are not whole %s blocks of %d", who, cols, bi->name, whole);
  if (rb != (size_t)cols / bi->elems * bi->bytes)
    return set_error(TIERMM_EINVAL, "%s: rb %zu does not match %d %s columns", who, rb, cols, bi->name);
  const size_t align = (qtype == QT_Q4_K || qtype == QT_Q5_K)                          ? 16
                       : (qtype == QT_F32 || qtype == QT_Q2_K || qtype == QT_NF4 || qtype == QT_FP4) ? 4
                       : qtype == QT_MXFP4                                                    ? 1
                                                                                             : 2;
  if (!W || ((uintptr_t)W % align) || (rb % align))
    return set_error(TIERMM_EINVAL, "%s: weight rows must be %zu-byte aligned", who, align);
  return TIERMM_OK;
}

// Whole rows to fp16 for the quantized GEMM (dq_launch<tier_fp16>, tier.cpp:515),
// row-major or (tiled, cols a multiple of 32) in the K-tiled layout.
int dequant_f16_rows(const void* W, int qtype, size_t rb, int cols, size_t nrows, uint16_t* out, hipStream_t s,
                     bool tiled) {
  if (!tiled)
    return with_qtype(qtype, [&](auto qt) {
      return launch_dequant<decltype(qt)::value>(W, rb, cols, 0, nrows, out, TIERMM_OUT_F16, s);
    });
  const size_t n8 = nrows * (size_t)cols / 8;
  if (n8 == 0) return TIERMM_OK;
  const size_t want = (n8 + 255) / 256;
  const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
  return with_qtype(qtype, [&](auto qt) -> int {
    dequant_kernel<decltype(qt)::value, TIERMM_OUT_F16><<<grid, 256, 0, s>>>((const uint8_t*)W, rb, cols, 0, n8, out,
                                                                            nrows);
    TM_LAUNCH_CHECK("dequant_f16_rows: launch");
    return TIERMM_OK;
  });
}

// n (<= 64) weights of one type, each nrows x cols, to fp16 at out[i], row-major or
// (tiled) in the K-tiled layout.
int dequant_f16_group(const void* const* W, uint16_t* const* out, int n, int qtype, size_t rb, int cols,
                      size_t nrows, hipStream_t s, bool tiled) {
  if (n <= 0) return TIERMM_OK;
  if (n > DQ_GROUP) return set_error(TIERMM_EINVAL, "dequant_f16_group: %d weights (max %d)", n, DQ_GROUP);
  const size_t n8 = nrows * (size_t)cols / 8;
  if (n8 == 0) return TIERMM_OK;
  DqGroup g{};
  for (int i = 0; i < n; ++i) {
    g.W[i] = (const uint8_t*)W[i];
    g.out[i] = out[i];
  }
  const size_t want = (n8 + 255) / 256;
  const dim3 grid((unsigned)(want < 2048 ? want : 2048), (unsigned)n);
  return with_qtype(qtype, [&](auto qt) -> int {
    dequant_f16_group_kernel<decltype(qt)::value><<<grid, 256, 0, s>>>(g, rb, cols, n8, tiled ? nrows : 0);
    TM_LAUNCH_CHECK("dequant_f16_group: launch");
    return TIERMM_OK;
  });
}

}  // namespace tiermm

using namespace tiermm;

extern "C" int tiermm_dequant(const void* W, int qtype, size_t rb, int cols, size_t r0, size_t nrows, void* out,
                              int out_dtype, tiermm_stream_t stream) {
  int st = check_qweight("tiermm_dequant", W, qtype, rb, cols, 1);
  if (st) return st;
  if (out_dtype != TIERMM_OUT_F32 && out_dtype != TIERMM_OUT_F16 && out_dtype != TIERMM_OUT_BF16)
    return set_error(TIERMM_EINVAL, "tiermm_dequant: unknown output dtype %d", out_dtype);
  hipStream_t s = (hipStream_t)stream;
  const bool dense = qtype == QT_F32 || qtype == QT_F16 || qtype == QT_BF16;
  if (dense && nrows && (cols % 8 || ((uintptr_t)out % 16))) {
    // dq_k's one element per thread (tier.cpp:294-296) for rows that are not whole
    // 8-element chunks, or an output that is not 16-byte aligned
    const size_t align = out_dtype == TIERMM_OUT_F32 ? 4 : 2;
    if (!out || ((uintptr_t)out % align))
      return set_error(TIERMM_EINVAL, "tiermm_dequant: output must be %zu-byte aligned", align);
    return with_dense(qtype, [&](auto qt) {
      return launch_dequant_elems<decltype(qt)::value>(W, rb, cols, r0, nrows, out, out_dtype, s);
    });
  }
  if (nrows && (!out || ((uintptr_t)out % 16)))
    return set_error(TIERMM_EINVAL, "tiermm_dequant: output must be 16-byte aligned");
  return with_qtype(qtype, [&](auto qt) {
    return launch_dequant<decltype(qt)::value>(W, rb, cols, r0, nrows, out, out_dtype, s);
  });
}

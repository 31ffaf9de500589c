// host_dequant.hip -- tiermm_dequant_host: q_val (quant.h:59-121) on the host, for
// the tools that compare a quantized base with its source (tier --tq-check,
// tier.cpp:2749-2765) without a GPU.
//
// It runs the same decoders as the kernels (Dec<> in tm_decode.h, compiled
// here for the host), so the host and device values come from one decode
// source.  Each row is first copied into a 16-byte aligned buffer with zero
// padding: the decoders read whole 16-byte headers and 8-element chunks, and
// host rows may start anywhere and (dense rows) end inside a chunk.
#include <cstring>
#include <vector>

#include "tm_decode.h"

namespace tiermm {
bool gpu_type(int qtype);
}

using namespace tiermm;

extern "C" int tiermm_dequant_host(const void* W, int qtype, size_t rb, int cols, size_t nrows, float* out) {
  const char* who = "tiermm_dequant_host";
  const BlockInfo* b = block_info(qtype);
  if (!b || !gpu_type(qtype)) return set_error(TIERMM_UNSUPPORTED, "%s: type %d", who, qtype);
  if (cols <= 0 || cols % b->elems || rb != (size_t)(cols / b->elems) * b->bytes)
    return set_error(TIERMM_EINVAL, "%s: rb %zu does not match %d columns", who, rb, cols);
  if (nrows && (!W || !out)) return set_error(TIERMM_EINVAL, "%s: null buffer", who);
  const int c8 = (cols + 7) / 8 * 8;
  return with_qtype(qtype, [&](auto qt) {
    constexpr int QT = decltype(qt)::value;
    std::vector<uint8_t> buf(rb + 64 + 16, 0);
    uint8_t* row = buf.data() + ((16 - ((uintptr_t)buf.data() & 15)) & 15);
    std::vector<float> vals((size_t)c8);
    for (size_t r = 0; r < nrows; ++r) {
      std::memcpy(row, (const uint8_t*)W + r * rb, rb);
      for (int c = 0; c < c8; c += 8) Dec<QT>::run(row, c, vals.data() + c);
      std::memcpy(out + r * (size_t)cols, vals.data(), (size_t)cols * sizeof(float));
    }
    return (int)TIERMM_OK;
  });
}

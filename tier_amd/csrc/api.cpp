// api.cpp -- library state, error reporting, block-format registry, workspace
// pool and the host quantizer entry point of libtiermm.so.
#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "tm_host.h"

namespace tiermm {
namespace {

// Block geometry table (quant.h:26-30): type id, name, elements, bytes.
const BlockInfo kBlocks[] = {
  {QT_F32, "F32", 1, 4}, {QT_F16, "F16", 1, 2}, {QT_BF16, "BF16", 1, 2}, {QT_Q4_0, "Q4_0", 32, 18},
  {QT_Q4_1, "Q4_1", 32, 20}, {QT_Q5_0, "Q5_0", 32, 22}, {QT_Q5_1, "Q5_1", 32, 24},
  {QT_Q8_0, "Q8_0", 32, 34}, {QT_Q2_K, "Q2_K", 256, 84}, {QT_Q3_K, "Q3_K", 256, 110},
  {QT_Q4_K, "Q4_K", 256, 144}, {QT_Q5_K, "Q5_K", 256, 176}, {QT_Q6_K, "Q6_K", 256, 210},
  {16, "IQ2_XXS", 256, 66}, {17, "IQ2_XS", 256, 74}, {22, "IQ2_S", 256, 82}, {18, "IQ3_XXS", 256, 98},
  {21, "IQ3_S", 256, 110}, {19, "IQ1_S", 256, 50}, {29, "IQ1_M", 256, 56}, {20, "IQ4_NL", 32, 18},
  {23, "IQ4_XS", 256, 136}, {34, "TQ1_0", 256, 54}, {35, "TQ2_0", 256, 66}, {39, "MXFP4", 32, 17},
  {200, "NF4", 64, 36}, {201, "FP4", 64, 36},
};

thread_local char g_err[512] = "";

struct Pool {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_mu;
std::vector<Pool> g_pools;  // indexed by device

}  // namespace

const BlockInfo* block_info(int qtype) {
  for (const auto& b : kBlocks)
    if (b.type == qtype) return &b;
  return nullptr;
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(int hip_err, const char* what) {
  set_error(-hip_err, "%s: %s", what, hipGetErrorString((hipError_t)hip_err));
  return -hip_err;
}

int get_workspace(void* ws, size_t ws_bytes, size_t need, void** out, const char* who) {
  if (need == 0) {
    *out = ws;
    return TIERMM_OK;
  }
  if (ws) {
    if (ws_bytes < need)
      return set_error(TIERMM_EINVAL, "%s: workspace of %zu bytes, %zu needed", who, ws_bytes, need);
    *out = ws;
    return TIERMM_OK;
  }
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, who);
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_pools.size() <= dev) g_pools.resize(dev + 1);
  Pool& p = g_pools[dev];
  if (p.bytes < need) {
    if (p.ptr) {
      // the previous pool may still be read by queued work: drain before freeing
      e = hipDeviceSynchronize();
      if (e != hipSuccess) return hip_fail(e, who);
      (void)hipFree(p.ptr);
      p.ptr = nullptr;
      p.bytes = 0;
    }
    size_t grow = need + need / 4;
    e = hipMalloc(&p.ptr, grow);
    if (e != hipSuccess) {
      p.ptr = nullptr;
      return hip_fail(e, who);
    }
    p.bytes = grow;
  }
  *out = p.ptr;
  return TIERMM_OK;
}

// Compute units of the current device, read once per device.
int device_cus(int* cus) {
  static std::atomic<int> cache[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "device_cus: hipGetDevice");
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *cus = c;
      return TIERMM_OK;
    }
  }
  int c = 0;
  e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_fail(e, "device_cus: hipDeviceGetAttribute");
  if (dev >= 0 && dev < 64) cache[dev].store(c, std::memory_order_relaxed);
  *cus = c;
  return TIERMM_OK;
}

}  // namespace tiermm

using namespace tiermm;

extern "C" {

int tiermm_init(int device) {
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "tiermm_init: hipSetDevice");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "tiermm_init: hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(TIERMM_UNSUPPORTED, "tiermm_init: device %d is %s; this library is built for gfx950", device,
                     prop.gcnArchName);
  return noalloc_scratch_init();  // the device address of tiermm_x3_rows_noalloc's scratch
}

void tiermm_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  int cur = 0;
  (void)hipGetDevice(&cur);
  for (size_t d = 0; d < g_pools.size(); ++d) {
    if (!g_pools[d].ptr) continue;
    (void)hipSetDevice((int)d);
    (void)hipDeviceSynchronize();
    (void)hipFree(g_pools[d].ptr);
    g_pools[d] = Pool{};
  }
  (void)hipSetDevice(cur);
}

const char* tiermm_last_error(void) { return g_err; }

const char* tiermm_version(void) { return "tiermm 0.1 (gfx950)"; }

int tiermm_q_info(int qtype, int* blk_elems, int* blk_bytes) {
  const BlockInfo* b = block_info(qtype);
  if (!b) return set_error(TIERMM_UNSUPPORTED, "tiermm_q_info: unknown type %d", qtype);
  if (blk_elems) *blk_elems = b->elems;
  if (blk_bytes) *blk_bytes = b->bytes;
  return TIERMM_OK;
}

int tiermm_q_row_bytes(int qtype, int cols, size_t* rb) {
  const BlockInfo* b = block_info(qtype);
  if (!b) return set_error(TIERMM_UNSUPPORTED, "tiermm_q_row_bytes: unknown type %d", qtype);
  if (cols < 0 || cols % b->elems)
    return set_error(TIERMM_UNSUPPORTED, "tiermm_q_row_bytes: %d columns are not whole %s blocks", cols, b->name);
  if (rb) *rb = (size_t)cols / b->elems * b->bytes;
  return TIERMM_OK;
}

int tiermm_quantize(int qtype, const float* x, void* out, size_t rows, int cols, int nthreads) {
  return quantize_rows(qtype, x, out, rows, cols, nthreads);
}

}  // extern "C"

// noalloc.hip -- tiermm_x3_rows_noalloc: chat_fp3's product (tier.cpp:2195-2219)
// for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// It runs the kernels of tiermm_x3_rows -- the three-part split of x, then the
// x3-ref GEMM -- with the fp16 planes of x in a static device scratch instead
// of a workspace argument or the library's pool.  No allocation happens on any
// call: the scratch is a file-scope __device__ array, one copy per GPU, held
// until the process ends.  Its size bounds the activations: 3 * M * K * 2
// bytes <= TIERMM_NOALLOC_SCRATCH_BYTES (32 MiB: M = 256 rows at K = 14336,
// M = 1024 at K = 5120).
#include <atomic>

#include "tm_device.h"

namespace tiermm {

int x3ref_nt(const uint16_t* xparts, size_t stride, const uint16_t* W, int ldw, float* C, int ldc, int M, int N,
             int K, float beta, hipStream_t s, const char* who, bool bf16);
int split3_launch(const float* x, uint16_t* parts, size_t n, size_t stride, int order, hipStream_t s, bool bf16,
                  size_t trows, int cols);

// The scratch.  In host code its name is only a stand-in, never a device
// address: the address on each device comes from hipGetSymbolAddress, taken
// once per device with that device current (tiermm_init, else the first call
// on the device) and kept in g_scratch_dev.  Calls that overlap on one device
// share it and race.
static __device__ __align__(256) uint8_t scratch[TIERMM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_dev[kMaxDevices];
}  // namespace

int noalloc_scratch_init() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "tiermm: scratch set-up");
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(TIERMM_UNSUPPORTED, "tiermm: device %d is past the %d the scratch table holds", dev, kMaxDevices);
  if (g_scratch_dev[dev].load(std::memory_order_acquire)) return TIERMM_OK;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_fail(e, "tiermm: scratch address");
  if (!p) return set_error(TIERMM_EINVAL, "tiermm: scratch address is null");
  g_scratch_dev[dev].store(p, std::memory_order_release);
  return TIERMM_OK;
}

namespace {

// The current device's scratch address.
int noalloc_scratch(void** out, const char* who) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, who);
  if (dev < 0 || dev >= kMaxDevices) return set_error(TIERMM_UNSUPPORTED, "%s: device %d", who, dev);
  void* p = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (!p) {
    const int st = noalloc_scratch_init();
    if (st) return st;
    p = g_scratch_dev[dev].load(std::memory_order_acquire);
  }
  *out = p;
  return TIERMM_OK;
}

}  // namespace
}  // namespace tiermm

using namespace tiermm;

extern "C" int tiermm_x3_rows_noalloc(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo,
                                      tiermm_stream_t stream) {
  const char* who = "tiermm_x3_rows_noalloc";
  if (M < 0 || N < 0 || K < 0) return set_error(TIERMM_EINVAL, "%s: negative size", who);
  if (K % 32) return set_error(TIERMM_UNSUPPORTED, "%s: K=%d is not a multiple of 32", who, K);
  if (ldo < N) return set_error(TIERMM_EINVAL, "%s: ldo < N", who);
  if (M == 0 || N == 0) return TIERMM_OK;
  if (!W || ((uintptr_t)W & 15) || !x || !y) return set_error(TIERMM_EINVAL, "%s: W must be 16-byte aligned", who);
  const size_t mk = (size_t)M * K, need = 3 * mk * sizeof(uint16_t);
  if (need > TIERMM_NOALLOC_SCRATCH_BYTES)
    return set_error(TIERMM_UNSUPPORTED, "%s: x of %d x %d needs %zu bytes of planes, the scratch holds %zu", who, M,
                     K, need, (size_t)TIERMM_NOALLOC_SCRATCH_BYTES);
  void* w = nullptr;
  int st = noalloc_scratch(&w, who);
  if (st) return st;
  // the split writes every plane element the GEMM reads: nothing needs clearing
  hipStream_t s = (hipStream_t)stream;
  st = split3_launch(x, (uint16_t*)w, mk, mk, TIERMM_HML, s, false, 0, 0);
  if (st) return st;
  return x3ref_nt((const uint16_t*)w, mk, W, K, y, ldo, M, N, K, 0.f, s, who, false);
}

// ref_gemv.cpp -- CPU baseline built on the reference's own q_val.
//
// TEST INFRASTRUCTURE ONLY (timed by bench.py's cpu_baseline leg, never the
// product).  gemv_q (tier.cpp:300-306) evaluated on host threads: each output
// row is sum_k q_val(row,type,k)*x[k] in fp32; rows are split into contiguous
// ranges, one per thread, as pool_run splits rows (tier.cpp:1029, 1041-1046).
// Built with -O3 -march=x86-64-v3 so the compiler may vectorise what it can.
#include "quant.h"

#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

extern "C" void ref_gemv_threads(const uint8_t* W, int t, size_t rb, const float* x, float* y, int N,
                                 int K, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  auto work = [&](int w) {
    const int r0 = (int)((long long)N * w / nthreads), r1 = (int)((long long)N * (w + 1) / nthreads);
    for (int r = r0; r < r1; ++r) {
      const uint8_t* row = W + (size_t)r * rb;
      float acc = 0.f;
      for (int k = 0; k < K; ++k) acc += q_val(row, t, k) * x[k];
      y[r] = acc;
    }
  };
  if (nthreads == 1) { work(0); return; }
  std::vector<std::thread> th;
  for (int w = 0; w < nthreads; ++w) th.emplace_back(work, w);
  for (auto& h : th) h.join();
}

// qgemm_q4k.hip -- fused q4_K dequant + x3-ref GEMM for prefill (M > 1).
//
// Y[M][ldy] (beta)= sum over the parts p of x (lo, mid, hi) of X_p[M][K] * W16[N][K]^T,
// W16 = fp16(q_val(W_n, k)) -- the training path's dq_k<tier_fp16> (tier.cpp:515,
// 293-298) followed by fp3gemm (tier.cpp:922-943) -- without writing W16 to
// memory: the q4_K rows are decoded into an LDS B tile as the K loop needs them.
//
// Tiling: a workgroup owns BM=128 rows of X x BN rows of W (BN in 64..160, a
// multiple of 16), one K step of 32 (one q4_K sub-block) per stage,
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
//     stages in LDS.  It works a sub-block pair at a time (two K steps share
//     their 32 qs bytes: low nibbles, then high nibbles), loading each row's
//     super-block header and qs bytes into registers four pairs ahead, and
//     decodes each element exactly as q_val (d*sc*q - dmin*m, one rounding),
//     rounded to fp16 (RNE, two elements per v_cvt_pk_f16_f32).  Bytes widen
//     with one mask and convert with v_cvt_f32_ubyte<n>: 2.75 VALU ops per
//     element.
// LDS rows hold 32 halfs as four 16-byte chunks, chunk c at slot
// c ^ ((row >> 2) & 3), so the fragment reads (16 rows x 4 chunks) hit
// distinct bank groups.  x comes in K-tiled planes (ktile_index) where the
// caller's x allows it, so a fragment load is one contiguous kilobyte.
//
// Measured, M = 512 (bench.py lines; x split and split-K reduce included):
// 5120x5120 81 us, 14336x5120 195 us, 5120x14336 204 us, against 97-100,
// 224-234 and 246-254 us when the producers streamed raw bytes through an LDS
// ring by DMA and decoded a stage at a time (one lane per half row, two passes
// at BN = 160).  Cycle counters in a timing copy showed that decoder at ~1450
// cycles per K step, 70 % of the producer's time, with the consumers waiting
// on it for 26 % of theirs; with the register-fed pair decoder the consumers
// wait 9 % and the MFMA issue is the larger part of their K step.
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
  const uint16_t* X;  // parts at X, X + xs, X + 2 xs (hi, mid, lo), rows of K halfs
  size_t xs;
  size_t xt;          // > 0: the planes are K-tiled (ktile_index) over xt rows
  float* Y;
  size_t rb;
  int ldy, N, K;
  float beta;
  float* P;   // split K: partial sums of split kz at P + kz * ps, rows of N floats
  size_t ps;
  int ngroups;
  int tile0[QG + 1];
  int row0[QG];
  int rows[QG];
  const uint8_t* W[QG];
};

__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 64 + ((chunk ^ ((row >> 2) & 3)) * 16)); }

__device__ __forceinline__ void lds_rel(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits until the four flags at f (16-byte aligned, LDS) are all >= v: one
// 16-byte read per try.  The flags only grow, and the data they publish is read
// after this returns (the empty asm keeps those reads below the loop).
__device__ __forceinline__ void poll4(const int* f, int v) {
  typedef int i4 __attribute__((ext_vector_type(4)));
  const volatile __attribute__((address_space(3))) i4* fl =
      (const volatile __attribute__((address_space(3))) i4*)(size_t)lds_addr(f);
  for (;;) {
    const i4 t = *fl;
    if (min(min(t[0], t[1]), min(t[2], t[3])) >= v) break;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
}

// Flags (stage numbers, slot-major so that one poll reads all four):
//   ready[q % FL][p] = q -- producer p's B rows of stage q are stored;
//   done[q % FL][c] = q  -- consumer c has read stage q's B tile.
// Stage q's B tile is slot q % NBR.  Producer p decodes the pair of stages q,
// q + 1 once every consumer has read stage q + 1 - NBR (the later slot's
// previous user, and so the earlier's too).  That stage is below q, its ready
// published by every producer, so each wait ends; a consumer waits only for
// its own loads and for ready.
template <int BN, int KS>
__global__ __launch_bounds__(512) void qgemm_q4k_x3ref(const QArgs p) {
  constexpr int NB = BN / 16;
  constexpr int NBR = QNBR, FL = 4, XR = 4, DP = 4;
  constexpr int PR = BN / 4;
  constexpr int LPR = 2 * PR <= 64 ? 2 : 1, HPL = 2 / LPR;  // decode: lanes per row, halves per lane
  constexpr int NL = 1 + HPL;                                // producer loads per sub-block pair
  constexpr int BPART = BN * 64;
  constexpr int FLAGOFF = NBR * BPART;
  static_assert(BN % 16 == 0 && BN <= 160, "tile width");
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
  const int nk = p.K / QBK / KS, kq0 = kz * nk;  // this split's K steps (a multiple of 8)
  __syncthreads();  // flags initialised

  if (wave >= 4) {
    // ------------------------------------------------------------ producer
    // LPR lanes per row of the producer's PR, each decoding HPL halves of 16
    // elements.  A sub-block pair (K steps q, q + 1 with q even) shares its 32 qs
    // bytes: low nibbles for q, high nibbles for q + 1.  Per pair a lane loads the
    // super-block header and its qs half (or halves) into registers, DP pairs ahead.
    const int pw = wave - 4;
    const bool act = lane < LPR * PR;
    const int dr = min(lane / LPR, PR - 1), h0 = (lane % LPR) * HPL;
    const int r = pw * PR + dr;
    const uint8_t* rowp = Wg + (size_t)min(n0 + r, p.N - 1) * p.rb;
    const int np = nk / 2;  // pairs of this split (a multiple of 4)
    u32x4 Hr[DP], Qr[DP][HPL];
    // pair j into register slot u (j >= np: pair np - 1 again, so every pair issues NL loads)
    auto issue = [&](int j, u32x4& h, u32x4 (&qv)[HPL]) __attribute__((always_inline)) {
      const int qq = kq0 + 2 * min(j, np - 1);
      const uint8_t* b = rowp + (size_t)(qq >> 3) * 144;
      h = gload16(b);
#pragma unroll
      for (int i = 0; i < HPL; ++i) qv[i] = gload16(b + 16 + 32 * ((qq & 7) >> 1) + 16 * (h0 + i));
    };
#pragma unroll
    for (int u = 0; u < DP; ++u) issue(u, Hr[u], Qr[u]);
    for (int j0 = 0; j0 < np; j0 += DP) {
#pragma unroll
      for (int u = 0; u < DP; ++u) {
        const int j = j0 + u, q = 2 * j;
        vm_wait<NL * (DP - 1)>();  // pair j is in registers
        asm volatile("" : "+v"(Hr[u]));
#pragma unroll
        for (int i = 0; i < HPL; ++i) asm volatile("" : "+v"(Qr[u][i]));
        // B slots of stages q, q + 1: their previous users, q + 1 - NBR and before, read by all
        if (q + 1 >= NBR) poll4(done + 4 * ((q + 1 - NBR) % FL), q + 1 - NBR);
        if (act) {
          const u32x4 H = Hr[u];
          const float d = h2f(H[0] & 0xffffu), dmin = h2f(H[0] >> 16);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            int sc, mn;
            kq_scale_min(((kq0 + q) & 7) + t, H[1], H[2], H[3], sc, mn);
            const float dsc = d * (float)sc, dm = dmin * (float)mn;
            uint8_t* bt = lds + ((q + t) % NBR) * BPART;
#pragma unroll
            for (int i = 0; i < HPL; ++i) {
              uint32_t o[8];
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
                asm volatile("" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
                const h2v p0 = {(_Float16)f[0], (_Float16)f[1]}, p1 = {(_Float16)f[2], (_Float16)f[3]};
                o[2 * w] = __builtin_bit_cast(uint32_t, p0);
                o[2 * w + 1] = __builtin_bit_cast(uint32_t, p1);
              }
              *(u32x4*)(bt + swz(r, 2 * (h0 + i))) = u32x4{o[0], o[1], o[2], o[3]};
              *(u32x4*)(bt + swz(r, 2 * (h0 + i) + 1)) = u32x4{o[4], o[5], o[6], o[7]};
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
    vm_wait<0>();  // drain the re-loads past the end
    return;
  }

  // -------------------------------------------------------------- consumer
  const int c = wave;
  const int fr = lane & 15, fc = lane >> 4;
  const uint32_t fo = swz(fr, fc);
  // A fragment (part, i): row c*32 + 16i + fr of the tile, halfs 8fc.. of stage q
  // K-tiled planes: K step qq of row r at (qq * xt + r) * 32, so a fragment's 16
  // rows are one contiguous kilobyte; row-major: row r at r * K + qq * 32
  const uint16_t* xa[3][2];
  const size_t kstep = p.xt ? p.xt * QBK : (size_t)QBK;
#pragma unroll
  for (int part = 0; part < 3; ++part)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const size_t r = (size_t)min(m0 + c * 32 + i * 16 + fr, M - 1);
      xa[part][i] = p.xt ? p.X + part * p.xs + ((size_t)p.row0[grp] + r) * QBK + 8 * fc
                         : Xg + part * p.xs + r * p.K + 8 * fc;
    }
  u32x4 A[XR][3][2];
  auto loadA = [&](int q, u32x4 (&dst)[3][2]) __attribute__((always_inline)) {
    const int qq = kq0 + min(q, nk - 1);  // past the end: a re-read, so every stage issues 6 loads
#pragma unroll
    for (int part = 0; part < 3; ++part)
#pragma unroll
      for (int i = 0; i < 2; ++i) dst[part][i] = gload16(xa[part][i] + (size_t)qq * kstep);
  };
  float4v acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < XR - 1; ++d) loadA(d, A[d]);
  for (int q0 = 0; q0 < nk; q0 += XR) {  // nk is a multiple of 8
#pragma unroll
    for (int u = 0; u < XR; ++u) {
      const int q = q0 + u;
      loadA(q + XR - 1, A[(u + XR - 1) % XR]);
      vm_wait<6 * (XR - 1)>();  // stage q's fragments are in registers
#pragma unroll
      for (int part = 0; part < 3; ++part)
#pragma unroll
        for (int i = 0; i < 2; ++i) asm volatile("" : "+v"(A[u][part][i]));
      const int sl = q % FL;
      poll4(ready + 4 * sl, q);
      const uint8_t* bs = lds + (q % NBR) * BPART;
      half8 bf[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) bf[j] = *(const half8*)(bs + j * 1024 + fo);
      // parts lo, mid, hi (tier.cpp:940) into one fp32 accumulator
#pragma unroll
      for (int part = 2; part >= 0; --part)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int i = 0; i < 2; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, A[u][part][i]), bf[j],
                                                               acc[i][j], 0, 0, 0);
      if (lane == 0) lds_rel(&done[4 * sl + c], q);
    }
  }
  vm_wait<0>();  // drain the re-reads past the end

  // epilogue: register i of lane l holds row 4*(l/16) + i, column l%16 of a 16x16 block
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
          float v = acc[i][j][r];
          if (p.beta != 0.f) v = fmaf(p.beta, *cp, v);
          *cp = v;
        } else {
          p.P[(size_t)kz * p.ps + (size_t)row * p.N + col] = acc[i][j][r];  // split K: one group
        }
      }
  }
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

template <int BN, int KS>
int launch_q(const QArgs& a, hipStream_t s, const char* who) {
  constexpr size_t lds = QNBR * (size_t)BN * 64 + 2 * 4 * 4 * 4;
  static_assert(lds <= 160 * 1024, "LDS budget");
  static std::atomic<uint64_t> attr{0};
  int st = lds_attr_once(attr, (const void*)qgemm_q4k_x3ref<BN, KS>, (int)lds, who);
  if (st) return st;
  qgemm_q4k_x3ref<BN, KS><<<(unsigned)a.tile0[a.ngroups] * KS, 512, lds, s>>>(a);
  TM_LAUNCH_CHECK(who);
  return TIERMM_OK;
}

template <int KS>
int launch_q_bn(int bn, const QArgs& a, hipStream_t s, const char* who) {
  switch (bn) {
    case 160: return launch_q<160, KS>(a, s, who);
    case 128: return launch_q<128, KS>(a, s, who);
    case 112: return launch_q<112, KS>(a, s, who);
    case 96: return launch_q<96, KS>(a, s, who);
    case 80: return launch_q<80, KS>(a, s, who);
    default: return launch_q<64, KS>(a, s, who);
  }
}

// Tiles of one BN over the groups' row counts.
long q_tiles(const int* rows, int n, int N, int bn) {
  long t = 0;
  for (int g = 0; g < n; ++g) t += (long)((rows[g] + QBM - 1) / QBM) * ((N + bn - 1) / bn);
  return t;
}

constexpr int kBns[6] = {160, 128, 112, 96, 80, 64};
// Per-workgroup time model, us: kRound + kUnit[BN] * BN * (K steps of the split), fitted to
// 512x{5120,14336,4096,1024,2048,1408}x{5120,14336,4096,2048} and {256,1024,2048}x5120x5120
// on MI355X (every (BN, KS) of the sweep; the model picks the measured best in each).
constexpr double kRound = 12.0;
constexpr double kUnit[6] = {6.25e-3, 6.8e-3, 7.0e-3, 8.0e-3, 8.7e-3, 10.5e-3};
constexpr size_t kMaxPartials = (size_t)256 << 20;  // bytes of split-K partial sums

struct QPlan {
  int bn, ks;
};

bool plan_ok(int bn, int ks, int K, size_t rows_total, int N, bool split) {
  if (ks > 1 && (!split || (K / 256) % ks || (size_t)ks * rows_total * N * 4 > kMaxPartials)) return false;
  if (ks < acc_chunks(K)) return false;  // each split's accumulator sums at most the chunk of the x3 GEMMs
  for (int b : kBns)
    if (b == bn) return ks == 1 || ks == 2 || ks == 4;
  return false;
}

// (BN, KS) for the fused kernel.  TIERMM_QGEMM_TILE="BN,KS" overrides the model when
// the pair is valid for the shape (tests and tuning).
QPlan q_plan(const int* rows, int n, int N, int K, int cus, bool split) {
  size_t rows_total = 0;
  for (int g = 0; g < n; ++g) rows_total += (size_t)rows[g];
  if (const char* e = getenv("TIERMM_QGEMM_TILE")) {
    int bn = 0, ks = 0;
    if (sscanf(e, "%d,%d", &bn, &ks) == 2 && plan_ok(bn, ks, K, rows_total, N, split)) return {bn, ks};
  }
  const int nk = K / QBK;
  QPlan best{0, 0};  // none: the shape does not take the fused kernel
  double best_t = -1;
  for (int i = 0; i < 6; ++i)
    for (int ks = 1; ks <= 4; ks *= 2) {
      if (!plan_ok(kBns[i], ks, K, rows_total, N, split)) continue;
      const long wg = q_tiles(rows, n, N, kBns[i]) * ks;
      double t = (double)((wg + cus - 1) / cus) * (kRound + kUnit[i] * kBns[i] * nk / ks);
      if (ks > 1) t += (double)rows_total * N * 4 * (ks + 1) / 4e6;  // the reduce, ~4 TB/s
      if (best_t < 0 || t < best_t) {
        best_t = t;
        best = {kBns[i], ks};
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
size_t qgemm_q4k_partials_bytes(int M, int N, int K) {
  const QPlan pl = q_plan(&M, 1, N, K, cus_or_default(), true);
  return pl.ks > 1 ? (size_t)pl.ks * M * N * sizeof(float) : 0;
}

// Whether the fused kernel takes n groups of these row counts: some (BN, KS) fits,
// KS > 1 only when `split` (one group with a partial-sum workspace), and every
// split short enough for one fp32 accumulator (acc_chunks).
bool qgemm_q4k_fusable(const int* rows, int n, int N, int K, bool split) {
  return q_plan(rows, n, N, K, cus_or_default(), split && n == 1).bn != 0;
}

// Fused q4_K x3-ref GEMM over n groups (rows[g] rows of x from row0[g], weight W[g]);
// the x planes hold every group's rows (plane stride xs).  A single group may split K,
// with `partials` (qgemm_q4k_partials_bytes) holding the partial sums.
int qgemm_q4k_fused_groups(const void* const* W, const int* row0, const int* rows, int n, size_t rb,
                           const uint16_t* xparts, size_t xs, size_t xt, float* Y, int ldy, int N, int K, float beta,
                           int cus, hipStream_t s, const char* who, float* partials) {
  const QPlan pl = q_plan(rows, n, N, K, cus, n == 1 && partials != nullptr);
  if (pl.bn == 0) return set_error(TIERMM_UNSUPPORTED, "%s: no fused q4_K plan for N=%d K=%d", who, N, K);
  for (int g0 = 0; g0 < n; g0 += QG) {
    QArgs a{};
    a.X = xparts; a.xs = xs; a.xt = xt; a.Y = Y; a.rb = rb; a.ldy = ldy; a.N = N; a.K = K; a.beta = beta;
    a.P = partials; a.ps = n == 1 ? (size_t)rows[0] * N : 0;
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
    switch (pl.ks) {
      case 4: st = launch_q_bn<4>(pl.bn, a, s, who); break;
      case 2: st = launch_q_bn<2>(pl.bn, a, s, who); break;
      default: st = launch_q_bn<1>(pl.bn, a, s, who); break;
    }
    if (st) return st;
    if (pl.ks > 1) {  // n == 1: rows row0[0].. of Y
      const size_t cnt = (size_t)rows[0] * N;
      qgemm_splitk_reduce<<<(unsigned)((cnt + 255) / 256), 256, 0, s>>>(partials, a.ps, pl.ks,
                                                                       Y + (size_t)row0[0] * ldy, ldy, rows[0], N,
                                                                       beta);
      TM_LAUNCH_CHECK(who);
    }
  }
  return TIERMM_OK;
}

int qgemm_q4k_fused(const void* W, size_t rb, const uint16_t* xparts, size_t xs, size_t xt, float* Y, int ldy, int M,
                    int N, int K, float beta, int cus, hipStream_t s, const char* who, float* partials) {
  const int row0 = 0;
  return qgemm_q4k_fused_groups(&W, &row0, &M, 1, rb, xparts, xs, xt, Y, ldy, N, K, beta, cus, s, who, partials);
}

}  // namespace tiermm

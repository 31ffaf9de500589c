// qgemm_q4k.hip -- fused q4_K dequant + x3-ref GEMM for prefill (M > 1).
//
// Y[M][ldy] (beta)= sum over the parts p of x (lo, mid, hi) of X_p[M][K] * W16[N][K]^T,
// W16 = fp16(q_val(W_n, k)) -- the training path's dq_k<tier_fp16> (tier.cpp:515,
// 293-298) followed by fp3gemm (tier.cpp:922-943) -- without writing W16 to
// memory: the q4_K rows are decoded into the LDS B tile as the K loop needs
// them.
//
// Tiling: a workgroup owns BM=128 rows of X x BN rows of W (BN in 64..128, a
// multiple of 16 picked per shape so the tile count fills the CUs); 8 waves, two
// per SIMD: wave w the X rows [32(w%4), 32(w%4)+32) against the 16-column blocks
// j = 2jj + w/4 (every other block), on v_mfma_f32_16x16x32_f16.  K advances 32
// per stage (one q4_K sub-block):
//   * the three x parts (pre-split, HML planes) and the raw weight bytes reach
//     LDS by global_load_lds_dwordx4;
//   * thread (r, h) of waves 4..7 decodes elements [16h, 16h+16) of the
//     sub-block of W row r from the raw bytes, exactly as q_val (d*sc*q -
//     dmin*m, one rounding), rounds to fp16 (v_cvt, RNE) and stores them in the
//     other B buffer while the current stage's MFMAs run.  Waves 0..3 only
//     multiply, so each SIMD has one wave with MFMAs to issue while the other
//     decodes or waits on LDS.
// LDS rows hold 32 halfs as four 16-byte chunks, chunk c at slot
// c ^ ((row >> 2) & 3), so the fragment reads (16 rows x 4 chunks) hit
// distinct bank groups.
#include "tm_device.h"

namespace tiermm {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int QBM = 128, QBK = 32;
constexpr int XPART = QBM * 64;  // bytes of one x part per stage
constexpr int XRING = 4;         // x stages in LDS: three in flight while one is multiplied

// A launch covers up to QG groups (one plain GEMM, or the experts of a routed
// batch): group g multiplies rows [row0[g], row0[g] + rows[g]) of X and Y with
// weight W[g]; its tiles are workgroups [tile0[g], tile0[g+1]).
constexpr int QG = 64;
struct QArgs {
  const uint16_t* X;  // parts at X, X + xs, X + 2 xs (hi, mid, lo), rows of K halfs
  size_t xs;
  float* Y;
  size_t rb;
  int ldy, N, K;
  float beta;
  int ngroups;
  int tile0[QG + 1];
  int row0[QG];
  int rows[QG];
  const uint8_t* W[QG];
};

__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 64 + ((chunk ^ ((row >> 2) & 3)) * 16)); }

template <int BN>
__global__ __launch_bounds__(512) void qgemm_q4k_x3ref(const QArgs p) {
  constexpr int NB = BN / 16, NBW = (NB + 1) / 2;  // blocks in the tile, per wave
  constexpr int BPART = BN * 64;
  constexpr int XSTAGE = 3 * XPART;
  constexpr int BOFF = XRING * XSTAGE;                 // the two B buffers follow the x ring
  constexpr int RAWB = BN * 48, NRI = (RAWB + 1023) / 1024, RAWS = NRI * 1024;
  constexpr int RAWOFF = BOFF + 2 * BPART;             // then the raw weight ring
  constexpr int JUNK = RAWOFF + XRING * RAWS;          // then a KiB for loads past the raw image
  extern __shared__ __attribute__((aligned(16))) uint16_t lds_h[];
  uint8_t* lds = (uint8_t*)lds_h;
  const uint32_t lds0 = lds_addr(lds);

  int grp = 0;  // the group of this workgroup (uniform scan over the tile prefix)
  // One GEMM: workgroups go round-robin over the 8 XCDs, so XCD x is given the
  // x-th eighth of the tile sequence (M-block major), a few M-blocks whose x rows
  // stay in that XCD's L2 while its N tiles stream past.
  int b = (int)blockIdx.x;
  const int nt_all = p.tile0[p.ngroups];
  if (p.ngroups == 1 && (nt_all & 7) == 0) b = (b & 7) * (nt_all >> 3) + (b >> 3);
  while (grp + 1 < p.ngroups && b >= p.tile0[grp + 1]) ++grp;
  const int tile = b - p.tile0[grp];
  const int ntn = (p.N + BN - 1) / BN;
  const int tm = tile / ntn, tn = tile % ntn;
  const int m0 = tm * QBM, n0 = tn * BN;
  const int M = p.rows[grp];
  const uint16_t* Xg = p.X + (size_t)p.row0[grp] * p.K;
  float* Yg = p.Y + (size_t)p.row0[grp] * p.ldy;
  const uint8_t* Wg = p.W[grp];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, wn = wave >> 2;

  // x DMA: 3 parts x 8 loads of 16 rows per stage, 3 per wave
  const uint16_t* xsrc[3];
  uint32_t xoff[3];
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int t = wave + 8 * u, part = t >> 3, ch = t & 7;
    const int row = ch * 16 + (lane >> 2), slot = lane & 3;
    xsrc[u] = Xg + part * p.xs + (size_t)min(m0 + row, M - 1) * p.K + 8 * (slot ^ ((row >> 2) & 3));
    xoff[u] = (uint32_t)(part * XPART + ch * 1024);
  }
  auto issue_x = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 3; ++u) dma16(xsrc[u] + kt * QBK, lds0 + (kt % XRING) * XSTAGE + xoff[u]);
  };

  // Raw weight bytes of a stage, per W row r: the super-block header and the two
  // 16-byte qs chunks holding the sub-block ([r][3][16 bytes], RAWB bytes in a
  // slot of RAWS).  They arrive by DMA like x, one stage ahead of x, so that
  // stage kt's loads bring x(kt) and raw(kt+1).  A load writes 1 KiB at a
  // wave-uniform LDS address: its lanes past RAWB land in the slot's padding,
  // and whole loads past the image write a junk KiB, so that every wave issues
  // the same number of loads.
  constexpr int RAWI = (NRI + 7) / 8;  // raw loads per wave per stage
  constexpr int GRPL = 3 + RAWI;       // loads per wave per stage
  const int nk = p.K / QBK;
  const uint8_t* rsrc[RAWI];
  int rkind[RAWI];
#pragma unroll
  for (int u = 0; u < RAWI; ++u) {
    const int f = (wave + 8 * u) * 1024 + lane * 16;
    const int r = min(f / 48, BN - 1), c = (f % 48) >> 4;
    rsrc[u] = Wg + (size_t)min(n0 + r, p.N - 1) * p.rb;
    rkind[u] = c;
  }
  auto issue_raw = [&](int kt) __attribute__((always_inline)) {
    kt = min(kt, nk - 1);
    const int sb = kt >> 3, s = kt & 7;
#pragma unroll
    for (int u = 0; u < RAWI; ++u) {
      const int ii = wave + 8 * u, c = rkind[u];
      const uint8_t* g = rsrc[u] + (size_t)sb * 144 + (c == 0 ? 0 : 16 + 32 * (s >> 1) + 16 * (c - 1));
      const uint32_t dst = ii < NRI ? (uint32_t)(RAWOFF + (kt % XRING) * RAWS + ii * 1024) : (uint32_t)JUNK;
      dma16(g, lds0 + dst);
    }
  };

  // decode: thread (r, h) of waves 4..7 turns elements [16h, 16h+16) of W row r
  // into fp16 (threads past 2*BN repeat row BN-1 and store to the junk KiB, so a
  // decoding wave has no divergent branch)
  const int dt = tid - 256;
  const int dr = min(max(dt, 0) >> 1, BN - 1), dh = tid & 1;
  const bool dwave = wave >= 4;  // wave-uniform
  const bool dec = dt >= 0 && dt < 2 * BN;
  auto decode = [&](int kt, uint32_t (&o)[8]) __attribute__((always_inline)) {
    const int s = kt & 7;
    const uint8_t* raw = lds + RAWOFF + (kt % XRING) * RAWS + dr * 48;
    const u32x4 H = *(const u32x4*)raw;
    const u32x4 Q = *(const u32x4*)(raw + 16 + 16 * dh);
    int sc, mn;
    kq_scale_min(s, H[1], H[2], H[3], sc, mn);
    const float dsc = h2f(H[0] & 0xffffu) * (float)sc, dm = h2f(H[0] >> 16) * (float)mn;
    const int sh = 4 * (s & 1);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t v = Q[w] >> sh;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        // q_val (quant.h:83-84): both products exact, one rounding; then fp16 RNE
        const float lo = fmaf(dsc, (float)((v >> (16 * b)) & 15u), -dm);
        const float hi = fmaf(dsc, (float)((v >> (16 * b + 8)) & 15u), -dm);
        o[2 * w + b] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
      }
    }
  };
  auto store_b = [&](int buf, const uint32_t (&o)[8]) __attribute__((always_inline)) {
    uint8_t* bt = dec ? lds + BOFF + buf * BPART : lds + JUNK;
    const int r = dec ? dr : 0;
    *(u32x4*)(bt + swz(r, 2 * dh)) = u32x4{o[0], o[1], o[2], o[3]};
    *(u32x4*)(bt + swz(r, 2 * dh + 1)) = u32x4{o[4], o[5], o[6], o[7]};
  };

  float4v acc[2][NBW];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int jj = 0; jj < NBW; ++jj) acc[i][jj] = float4v{0.f, 0.f, 0.f, 0.f};

  // fragment offsets: lane l reads row (l%16) of a 16-row block, chunk l/16
  const int fr = lane & 15, fc = lane >> 4;
  const uint32_t fo = swz(fr, fc);

  // Loads (every wave, in issue order): raw(0), then per stage q = 0, 1, 2, ...
  // the group {raw(q+1), x(q)}; group q+3 is issued in stage q (past the end,
  // the last stage is re-loaded into the free slots).  At the top of stage kt
  // groups kt+1 and kt+2 are younger than group kt: 2*GRPL loads.
  issue_raw(0);
  for (int q = 0; q < XRING - 1; ++q) {
    issue_raw(q + 1);
    issue_x(min(q, nk - 1));
  }
  vm_wait<(XRING - 1) * GRPL>();  // raw(0)
  __syncthreads();
  if (dwave) {
    uint32_t o[8];
    decode(0, o);
    store_b(0, o);
  }
  for (int kt = 0; kt < nk; ++kt) {
    vm_wait<2 * GRPL>();  // group kt: x(kt), raw(kt+1)
    __syncthreads();      // ... for every wave, and B(kt) is written; slot (kt-1) % XRING and B(kt-1) are free
    issue_raw(kt + XRING);
    issue_x(min(kt + XRING - 1, nk - 1));
    uint32_t o[8];
    if (dwave) decode(min(kt + 1, nk - 1), o);  // stage kt+1 (its raw bytes came with group kt)
    const uint8_t* xs = lds + (kt % XRING) * XSTAGE;
    const uint8_t* bs = lds + BOFF + (kt & 1) * BPART;
    // every fragment of the stage first (one LDS latency per stage), then the MFMAs
    half8 bf[NBW], af[3][2];
#pragma unroll
    for (int jj = 0; jj < NBW; ++jj) bf[jj] = *(const half8*)(bs + min(2 * jj + wn, NB - 1) * 1024 + fo);
#pragma unroll
    for (int part = 0; part < 3; ++part)
#pragma unroll
      for (int i = 0; i < 2; ++i) af[part][i] = *(const half8*)(xs + part * XPART + (wm * 32 + i * 16) * 64 + fo);
    // parts lo, mid, hi (tier.cpp:940) into one fp32 accumulator
#pragma unroll
    for (int part = 2; part >= 0; --part) {
#pragma unroll
      for (int jj = 0; jj < NBW; ++jj)
        if ((NB & 1) == 0 || jj < NBW - 1 || wn == 0)  // odd NB: the last block is wave-column 0's
#pragma unroll
          for (int i = 0; i < 2; ++i)
            acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[part][i], bf[jj], acc[i][jj], 0, 0, 0);
    }
    if (dwave) store_b((kt + 1) & 1, o);
  }
  vm_wait<0>();  // drain the re-loads past the end

  // epilogue: register i of lane l holds row 4*(l/16) + i, column l%16 of a 16x16 block
#pragma unroll
  for (int jj = 0; jj < NBW; ++jj) {
    const int j = 2 * jj + wn;
    const int col = n0 + j * 16 + (lane & 15);
    if (j >= NB || col >= p.N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
        if (row >= M) continue;
        float* c = Yg + (size_t)row * p.ldy + col;
        float v = acc[i][jj][r];
        if (p.beta != 0.f) v = fmaf(p.beta, *c, v);
        *c = v;
      }
  }
}

template <int BN>
int launch_q(const QArgs& a, hipStream_t s, const char* who) {
  constexpr size_t lds = (size_t)XRING * 3 * XPART + 2 * (size_t)BN * 64 + (size_t)XRING * ((BN * 48 + 1023) / 1024) * 1024 + 1024;
  static_assert(lds <= 160 * 1024, "LDS budget");
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)qgemm_q4k_x3ref<BN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return hip_fail(e, who);
    attr_set = true;
  }
  qgemm_q4k_x3ref<BN><<<(unsigned)a.tile0[a.ngroups], 512, lds, s>>>(a);
  TM_LAUNCH_CHECK(who);
  return TIERMM_OK;
}

// Tiles of one BN over the groups' row counts.
long q_tiles(const int* rows, int n, int N, int bn) {
  long t = 0;
  for (int g = 0; g < n; ++g) t += (long)((rows[g] + QBM - 1) / QBM) * ((N + bn - 1) / bn);
  return t;
}

}  // namespace

// Fused q4_K x3-ref GEMM over n groups (rows[g] rows of x from row0[g], weight W[g]);
// the x planes hold every group's rows (plane stride xs).  BN is the one with the
// shortest critical path: rounds of workgroups over the CUs times the work of a
// tile (proportional to BN), larger BN on ties.
int qgemm_q4k_fused_groups(const void* const* W, const int* row0, const int* rows, int n, size_t rb,
                           const uint16_t* xparts, size_t xs, float* Y, int ldy, int N, int K, float beta, int cus,
                           hipStream_t s, const char* who) {
  const int cand[5] = {128, 112, 96, 80, 64};
  int best = 128;
  long best_t = -1;
  for (int c : cand) {
    const long t = (q_tiles(rows, n, N, c) + cus - 1) / cus * c;
    if (best_t < 0 || t < best_t) {
      best_t = t;
      best = c;
    }
  }
  for (int g0 = 0; g0 < n; g0 += QG) {
    QArgs a{};
    a.X = xparts; a.xs = xs; a.Y = Y; a.rb = rb; a.ldy = ldy; a.N = N; a.K = K; a.beta = beta;
    a.ngroups = 0;
    a.tile0[0] = 0;
    for (int g = g0; g < n && g < g0 + QG; ++g) {
      if (rows[g] == 0) continue;
      const int j = a.ngroups++;
      a.row0[j] = row0[g];
      a.rows[j] = rows[g];
      a.W[j] = (const uint8_t*)W[g];
      a.tile0[j + 1] = a.tile0[j] + (int)q_tiles(&rows[g], 1, N, best);
    }
    if (a.ngroups == 0) continue;
    int st;
    switch (best) {
      case 128: st = launch_q<128>(a, s, who); break;
      case 112: st = launch_q<112>(a, s, who); break;
      case 96: st = launch_q<96>(a, s, who); break;
      case 80: st = launch_q<80>(a, s, who); break;
      default: st = launch_q<64>(a, s, who); break;
    }
    if (st) return st;
  }
  return TIERMM_OK;
}

int qgemm_q4k_fused(const void* W, size_t rb, const uint16_t* xparts, size_t xs, float* Y, int ldy, int M, int N, int K,
                    float beta, int cus, hipStream_t s, const char* who) {
  const int row0 = 0;
  return qgemm_q4k_fused_groups(&W, &row0, &M, 1, rb, xparts, xs, Y, ldy, N, K, beta, cus, s, who);
}

}  // namespace tiermm

// qgemv_q4k_ws.hip -- Q4_K (and Q5_K) decode GEMV from 1024 rows up (qgemv_ws_takes):
// a workgroup streams one 16-row tile at a time through producer waves.
//
// Same arithmetic and x digit layout as qgemv_q4k.hip (gemv_q, tier.cpp:299-306;
// q_val Q4_K, quant.h:83-84); q4k_mfma.h holds the shared pieces.
//
// Work split.  Workgroup w takes the row tiles w, w + G, w + 2G, ... (G = the
// grid, R tiles each), so at any moment the chip reads a compact window of
// consecutive tiles, and it streams them one after another.  A tile is cut
// into stages of GS super-blocks: each of the 4 producer waves (one per SIMD)
// brings 4 of the 16 rows (4 row segments of GS*144 bytes) into a ring of NS
// slots of its own with global_load_lds_dwordx4; while it waits for stage q - D
// to land, stages q - D .. q are in flight.  16-byte pads after the row segments
// and after each producer's slots (ws_pad) put the 16 rows a consumer reads at one
// column on distinct groups of LDS banks: without them up to four rows met in one
// group.  That halved the bank-conflict cycles (13824x5120: 0.47 -> 0.25 M;
// 16384x8192: 1.94 -> 0.59 M) without moving the time: the consumers of this
// kernel are not LDS-bound.  Long row segments and few
// concurrent tiles measured faster than 16 short segments per wave from 864
// tiles at once (13824x5120: 8.9 against 9.2 us; 10240x8192: 10.4 against
// 11.8 us).  Up to K = 5120 a stage is the whole tile (a contiguous 16-row
// span) with one more tile in flight: 13824x5120 8.55-8.57 against 8.86-9.02 us
// for 12-super-block stages two deep, 14336x4096 7.71 against 8.34 us.  Deeper
// rings measured slower in every geometry tried (whole tiles two ahead: 9.74 us).
// The loads carry the non-temporal hint: every weight byte is read once
// (13824x5120: 8.9-9.2 against 9.3-9.5 us; 10240x8192: 10.2 against 10.7 us).
//
// Consumers.  Consumer c owns super-block columns c, c + NC, ... < GS of every
// stage (CPS of them), so the x digits and the x metadata it needs sit in its
// registers from the start (MS columns) and its LDS reads are the weight bytes
// alone.  8 consumers with 4 producers (3 waves per SIMD) measured faster than
// 4-12 consumers in other counts (13824x5120, whole-tile stages: 8.54 against
// 8.63-9.11 us).  With 3 or 4 tiles per workgroup its partial sum of each tile
// goes to an LDS area of its own as the tile ends, and after one barrier the
// workgroup adds the NC partials of each row in a fixed order (13824x5120 8.51
// against 8.57-8.64 us, 16384x8192 13.74-13.81 against 13.85-13.93); otherwise
// the sums stay in registers until every stage is consumed and then go to the
// ring, behind a second barrier.  Up to K = 8192 the q4_K consumers take the high
// nibbles as 16 (q - 8) through one v_bitop3 per word (q4k_sb_hb), the offset folded
// into each column's accumulator start: 8 fewer VALU instructions per column of ~59,
// bit-identical (13824x5120 8.31-8.32 against 8.22-8.24 us; 16384x8192 within noise).
//
// Hand-off through LDS flags holding stage numbers, which only grow:
//   full[slot][p] = q  -- producer p's rows of stage q have landed (its own
//                         vmcnt wait: loads retire in order);
//   done[slot][c] = q  -- consumer c is past stage q (set without waiting
//                         when the stage holds no column of c).
// A producer refills a slot with stage q once every done[slot][.] >= q - NS;
// a consumer reads stage q once every full[slot][.] >= q.  Every wait ends: a
// producer has marked stage q - D full before it issues q, and it waits only
// for stages <= q - NS < q - D, which all consumers can finish; consumers wait
// only for stages that are issued and are marked full in order.
#include <climits>
#include <utility>

#include "q4k_mfma.h"

namespace tiermm {
namespace {

constexpr int NP = 4;      // producer waves
constexpr int PROWS = 4;   // rows of a tile per producer
constexpr int GTILE = 256; // target grid: tiles per workgroup R = ceil(tiles / GTILE)

constexpr int pad4(int n) { return (n + 3) / 4 * 4; }

__device__ __forceinline__ void lds_rel(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits until the NF (a multiple of 4) flags at f (16-byte aligned, LDS) are
// all >= v, reading them 16 bytes at a time.  The data they publish is read
// after this returns (the empty asm keeps those reads below the loop).
template <int NF>
__device__ __forceinline__ void poll_ge(const int* f, int v) {
  typedef int i4 __attribute__((ext_vector_type(4)));
  const volatile __attribute__((address_space(3))) i4* fl =
      (const volatile __attribute__((address_space(3))) i4*)(size_t)lds_addr(f);
  for (;;) {
    int m = INT_MAX;
#pragma unroll
    for (int j = 0; j < NF / 4; ++j) {
      const i4 t = fl[j];
      m = min(m, min(min(t[0], t[1]), min(t[2], t[3])));
    }
    if (m >= v) break;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
}

// LDS bank conflicts of the consumers' 16-byte reads (8 lanes a pass over 32
// banks: rows 0-7, then 8-15, at one column) for row segments `pitch` bytes apart
// in a slot and producer regions `region` bytes apart: the sum over both passes
// of the most rows that meet in one group of four banks (2 = none).
constexpr int ws_conflicts(int pitch, int region) {
  int cost = 0;
  for (int pass = 0; pass < 2; ++pass) {
    int cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0}, worst = 0;
    for (int n = 8 * pass; n < 8 * pass + 8; ++n) {
      const long dw = ((long)(n / PROWS) * region + (long)(n % PROWS) * pitch) / 4;
      const int grp = (int)(dw % 32) / 4;
      worst = ++cnt[grp] > worst ? cnt[grp] : worst;
    }
    cost += worst;
  }
  return cost;
}
// Padding of a ring: 16-byte pads after each row segment (k) and after each
// producer's region of ns slots (m), the fewest (k + m, up to 7 each) that spread
// the 16 rows over the banks (13824x5120: one pad per row, 2896-byte rows).
struct WsPad {
  int k, m;
};
constexpr WsPad ws_pad(int grp, int ns) {
  WsPad best{0, 0};
  int bc = ws_conflicts(grp, ns * PROWS * grp);
  for (int t = 1; t < 15; ++t)
    for (int k = 0; k <= t && k < 8; ++k) {
      const int m = t - k, pitch = grp + 16 * k;
      if (m < 8 && ws_conflicts(pitch, ns * PROWS * pitch + 16 * m) < bc) {
        bc = ws_conflicts(pitch, ns * PROWS * pitch + 16 * m);
        best = WsPad{k, m};
      }
    }
  return best;
}

// Stages issued before the x barrier (at most the ring's NS slots).  At K = 14336 the x
// preparation takes ~2.7 us, and with 3 stages (D) requested the loads ran dry before it
// ended: 4 stages measured 4096x14336 8.04 against 8.41 us (5 stages: 8.37).  At K = 5120
// a second whole tile up front lost (13824x5120 8.43 against 8.24 us).
constexpr int ws_pre(int XK, int NS, int D) { return XK == 14336 ? 4 : D; }

// Marks stages 0 .. PRE - D - 1 full as they land, after PRE stages of NLD loads each went out.
template <int NLD, int PRE, int D, int... M>
__device__ __forceinline__ void ws_mark_pre(std::integer_sequence<int, M...>, int* full, int p, int lane) {
  (
      [&] {
        vm_wait<NLD * (PRE - 1 - M)>();
        if (lane == 0) lds_rel(&full[NP * M + p], M);
      }(),
      ...);
}

template <int QT, int GS_, int NC, int NS, int R>
struct WsLayout {
  static constexpr int GS = GS_;                                // super-blocks per stage
  static constexpr int CPS = (GS + NC - 1) / NC;                // columns per consumer per stage
  static constexpr int GRP = GS * MfmaFmt<QT>::SBB;             // one row's segment
  static constexpr WsPad PAD = ws_pad(GRP, NS);
  static constexpr int PITCH = GRP + 16 * PAD.k;                // its place in a slot (with the pad)
  static constexpr int SLOT = PROWS * PITCH;                    // one producer's part of a stage
  static constexpr int REGION = NS * SLOT + 16 * PAD.m;         // one producer's slots (with the pad)
  static constexpr int NLD = (SLOT + 1023) / 1024;              // 1 KiB loads per part
  static constexpr int LAST = (SLOT - (NLD - 1) * 1024) / 16;   // lanes of the last load
  static constexpr int NCP = pad4(NC);
  static constexpr size_t RING = (size_t)NP * REGION;
  static constexpr size_t LDS = RING + NS * NP * 4 + NS * NCP * 4;
  // the per-tile partial sums reuse the ring once every stage has been consumed
  static_assert((size_t)R * NC * 16 * 4 <= RING, "partial sums fit in the ring");
};

// Several matrices with the same K and block type in one launch (tiermm_qgemv_batch):
// matrix i owns tiles [t0[i], t0[i+1]) of the concatenated tile sequence, with rows
// N[i], weight W[i] and output y[i]; entries past the batch have t0 = the tile count.
// NB = 0: one matrix, given by the kernel's own arguments.
constexpr int WS_BATCH = 4;
template <int NB>
struct WsMats {
  const uint8_t* W[NB];
  float* y[NB];
  int t0[NB + 1];
  int N[NB];
};
template <>
struct WsMats<0> {};

// Split stages (SK): with more row tiles than workgroups but fewer than two per
// workgroup, whole tiles per workgroup leave CUs idle or load some workgroups with one
// tile more than others.  Instead workgroup b takes the stages [T b / G, T (b + 1) / G)
// of the tile-major stage sequence (T = tiles x stages per tile), so every workgroup
// streams the same bytes to within one stage.  G <= tiles makes every range at least a
// tile long, so a tile is shared by at most two workgroups, split at the boundary
// between them.  Each of the two adds its part of the tile's rows; per row they meet in
// one 64-bit slot of ws_pair (boundary b's 16 rows): each swaps its part in, and the one
// that gets the other's part back writes y = lower part + upper part (a fixed order) and
// empties the slot.  Nobody waits for anybody.  A slot carries the launch's epoch (a host
// counter) beside the part's bits; an entry of another epoch (left by a call that
// overlapped this one on the device) counts as empty.  Overlapping calls on one device
// that take this path race (rows left unwritten, no hang); calls that do not overlap
// always leave the slots empty.
constexpr int WS_SK_GRID = GTILE;
// How a workgroup's work is cut: R whole tiles (WS_TILES) or a range of stages (WS_STAGES).
constexpr int WS_TILES = 0, WS_STAGES = 1;
__device__ unsigned long long ws_pair[(WS_SK_GRID + 1) * 16];
// a stored part is its bits ^ WS_SENT, never 0: a computed float is never the
// signalling NaN 0x7fbadbad (arithmetic yields quiet NaNs)
constexpr uint32_t WS_SENT = 0x7fbadbadu;
std::atomic<unsigned> ws_epoch{0};  // one count for every launch in split stages
template <bool SK>
struct WsSplit {
  unsigned epoch;
};
template <>
struct WsSplit<false> {};

// Leaves `part` (row n of boundary b's tile) in the slot or, when the other workgroup's
// part was there, returns true with the row's sum in *sum: lower + upper.  One swap (a
// compare-and-swap and then a take cost a second round trip to memory: 5120x14336
// 11.69 against 11.35 us).
__device__ __forceinline__ bool ws_pair_meet(int b, int n, unsigned epoch, bool upper, float part, float* sum) {
  unsigned long long* p = ws_pair + b * 16 + n;
  const unsigned long long mine = ((unsigned long long)epoch << 32) | (__float_as_uint(part) ^ WS_SENT);
  const unsigned long long old = __hip_atomic_exchange(p, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old == 0 || (unsigned)(old >> 32) != epoch) return false;  // the first here: the other takes it
  __hip_atomic_store(p, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float o = __uint_as_float((uint32_t)old ^ WS_SENT);
  *sum = upper ? o + part : part + o;
  return true;
}

template <int QT, int R, int GS_, int NC, int NS, int D, int XP, int XK, int NB, int SPLIT = WS_TILES>
__global__ __launch_bounds__(64 * (NC + NP)) void qgemv_q4k_ws(const uint8_t* __restrict__ W, size_t rb,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int N, int K, int G, const WsMats<NB> mats,
                                                            const WsSplit<SPLIT == WS_STAGES> sk) {
  // G = gridDim.x, passed as an argument: without a read of the grid size the kernel
  // needs none of the implicit arguments, so its argument segment is 44 bytes, not 296
  constexpr bool SK = SPLIT == WS_STAGES;
  static_assert(!SK || NB == 0, "split stages serve one matrix");
  // q4_K in split stages: the split tiles' parts meet early (the first tile's part is left
  // as soon as it is summed, the last tile's partner part taken while the consumers finish):
  // 5120x14336 11.12 -> 10.90 us.  q5_K keeps both meetings at the end (the early ones
  // spilled 4 more registers there: 12.97 -> 13.79 us).
  constexpr bool EARLY = SK && QT == QT_Q4_K;
  using L = WsLayout<QT, GS_, NC, NS, R>;
  constexpr int SBB = MfmaFmt<QT>::SBB;
  constexpr int GS = L::GS, CPS = L::CPS, GRP = L::GRP, PITCH = L::PITCH, SLOT = L::SLOT, NLD = L::NLD,
                NCP = L::NCP;
  constexpr int MG = (XK / 256 + GS - 1) / GS;  // stages per tile, at most
  constexpr int MS = MG * CPS;                  // super-block columns per consumer
  static_assert(NLD * D <= 63, "vmcnt counts at most 63 loads");
  static_assert(D >= 0 && NS > D, "ring deeper than the stages in flight");
  static_assert(NC + NP <= 16, "at most 1024 threads per workgroup");
  static_assert(SLOT % 16 == 0, "16-byte aligned slots");
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // L::LDS bytes
  __shared__ __attribute__((aligned(16))) uint8_t xlds[xq_bytes(XK) - ZERO_BYTES];  // no zero rows: A is set once
  __shared__ int nf[NC];               // per consumer: x held a non-finite value
  int* full = (int*)(ring + L::RING);  // [NS][NP]
  int* done = full + NS * NP;          // [NS][NCP]
  // [R][NC][16]: for 3 or 4 tiles an area of their own, written as each tile ends;
  // otherwise the ring, once every stage has been consumed
  constexpr bool OWN = R == 3 || R == 4;
  __shared__ float red_own[OWN ? R * NC * 16 : 1];
  float* red = OWN ? red_own : (float*)ring;
  // SK: consumers past the first tile's partial sums; what the early swaps of the split
  // tiles got back ([0, 16): the last tile's take, [16, 32): the first tile's deposit)
  __shared__ int first_in[1];
  __shared__ unsigned long long met[SK ? 32 : 1];
  const int nsb = K >> 8, ngrp = (nsb + GS - 1) / GS;
  int tiles;
  if constexpr (NB == 0)
    tiles = (N + 15) >> 4;
  else
    tiles = mats.t0[NB];
  // this workgroup's stages: R whole tiles blockIdx.x, blockIdx.x + G, ...; or (SK) the
  // range [s0, s1) of the stage sequence, whose first stage lies in tile t0
  int total = R * ngrp, s0 = 0, s1 = 0, t0 = 0;
  if constexpr (SK) {
    // 32-bit: T * G <= 512 tiles x 56 stages x 256 workgroups
    const unsigned T = (unsigned)(tiles * ngrp);
    s0 = (int)(T * blockIdx.x / (unsigned)G);
    s1 = (int)(T * (blockIdx.x + 1) / (unsigned)G);
    t0 = s0 / ngrp;
    total = s1 - s0;
  }
  // tile t of the sequence: its matrix's weight, output, rows and tile index there
  struct TileRef {
    const uint8_t* W;
    float* y;
    int N, tile;
  };
  auto locate = [&](int t) __attribute__((always_inline)) {
    if constexpr (NB == 0) {
      return TileRef{W, y, N, t};
    } else {
      int m = 0;
#pragma unroll
      for (int i = 1; i < NB; ++i) m += t >= mats.t0[i] ? 1 : 0;
      return TileRef{mats.W[m], mats.y[m], mats.N[m], t - mats.t0[m]};
    }
  };
  uint8_t* xq = xlds;
  float* meta = (float*)(xq + nsb * XQ_SB);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // x holds NaN or +-Inf: read once the x preparation is published where registers allow
  // (up to K = 8192), at the end otherwise
  constexpr bool XEARLY = MS <= 4;
  bool xbad = false;

  if (wave >= NC) {
    // ------------------------------------------------------------ producer
    const int p = wave - NC;
    // up to K = 5120 the producers issue ahead of the consumers' VALU work on their SIMD
    // (13824x5120 8.20 -> 8.15 us, 5120x5120 5.36 -> 5.28); above it this lost 6-8 %
    // (4096x14336 8.01 -> 8.66 us)
    if constexpr (XK <= 5120) __builtin_amdgcn_s_setprio(1);
    if (lane < NS) full[NP * lane + p] = -1;
    if (p == 0 && lane == 0) first_in[0] = 0;
    if (p == 0)  // consumer flags; padding entries never hold a wait back
      for (int i = lane; i < NS * NCP; i += 64) done[i] = (i % NCP) < NC ? -1 : INT_MAX;
    // byte f of a slot: row f / PITCH of the producer's 4, byte f % PITCH of its
    // segment (the pad past GRP takes a re-read of the segment's last 16 bytes)
    int roff[NLD], coff[NLD];
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int f = min(j * 1024 + lane * 16, SLOT - 16);
      roff[j] = f / PITCH;
      coff[j] = f % PITCH;
    }
    const uint32_t ring_lds = lds_addr(ring + p * L::REGION);
    auto issue = [&](int q) __attribute__((always_inline)) {
      int tile, gi;
      if constexpr (SK) {
        tile = (s0 + q) / ngrp;
        gi = s0 + q - tile * ngrp;
      } else {
        const int r = q / ngrp;
        gi = q - r * ngrp;
        // a tile past the last one (its workgroup has fewer) re-reads the last tile
        tile = min((int)blockIdx.x + r * G, tiles - 1);
      }
      const TileRef tr = locate(tile);
      const int rbase = min(tr.tile * 16 + PROWS * p, tr.N - 1), rmax = min(PROWS - 1, tr.N - 1 - rbase);
      // bytes past the row's last super-block re-read the last valid 16 bytes
      const int lastb = min(GS, nsb - GS * gi) * SBB - 16;
      const uint8_t* b = tr.W + (size_t)rbase * rb + (size_t)gi * GRP;
      const uint32_t dst = ring_lds + (q % NS) * SLOT;
#pragma unroll
      for (int j = 0; j < NLD; ++j)
        if (j < NLD - 1 || L::LAST == 64 || lane < L::LAST)
          dma16_nt(b + (size_t)min(roff[j], rmax) * rb + min(coff[j], lastb), dst + j * 1024);
    };
    // PRE stages go out before the x barrier when the workgroup has that many (the ring
    // is empty), D otherwise; the steady loop keeps D in flight
    constexpr int PRE = ws_pre(XK, NS, D);
    const bool deep = PRE > D && total >= PRE;
    const int pro = deep ? PRE : min(D, total);
    for (int q = 0; q < pro; ++q) issue(q);
    __syncthreads();  // flags initialised; consumers have prepared x
    if constexpr (XEARLY) xbad = flags_any(nf, NC);
    int marked = 0;   // stages marked full so far
    if constexpr (PRE > D) {
      if (deep) {  // stage m has landed once at most PRE - 1 - m stages' loads are pending
        ws_mark_pre<NLD, PRE, D>(std::make_integer_sequence<int, PRE - D>{}, full, p, lane);
        marked = PRE - D;
      }
    }
    for (int q = deep ? PRE : D; q < total; ++q) {
      if (q >= NS) poll_ge<NCP>(done + (q % NS) * NCP, q - NS);
      issue(q);
      vm_wait<NLD * D>();  // stage q - D has landed
      if (lane == 0) lds_rel(&full[NP * (marked % NS) + p], marked);
      ++marked;
    }
    vm_wait<0>();
    for (; marked < total; ++marked)
      if (lane == 0) lds_rel(&full[NP * (marked % NS) + p], marked);
    if constexpr (EARLY) {
      // the last tile goes on into the next workgroup, which left its part of it early
      // (its first tile): take it now, while the consumers finish, so that the round trip
      // is not at the end
      const int tl = (s1 - 1) / ngrp;
      if (p == 0 && (tl + 1) * ngrp > s1 && lane < 16 && tl * 16 + lane < N)
        met[lane] = __hip_atomic_exchange(ws_pair + ((int)blockIdx.x + 1) * 16 + lane, 0ull, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (!OWN) __syncthreads();  // every stage consumed: the ring is free
    __syncthreads();                         // partial sums are in red[]
  } else {
    // -------------------------------------------------------------- consumers
    const int c = wave, n = lane & 15, g = lane >> 4;
    constexpr int NT = 64 * NC;
    // x: one thread per 16 elements (threads past K/16 load a clamped copy and skip)
    u32x4 xr[XP][4];
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int hh = min(tid + j * NT, (K >> 4) - 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) xr[j][i] = *(const u32x4*)(x + hh * 16 + 4 * i);
    }
    bool bad = false;
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int hh = tid + j * NT;
      if (hh < (K >> 4)) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int w = 0; w < 4; ++w) v[4 * i + w] = __uint_as_float(xr[j][i][w]);
        bad |= nonfinite16(v);
        prep_half(hh >> 1, hh & 1, v, xq, meta);
      }
    }
    publish_nonfinite(bad, nf, c, lane);
    __syncthreads();
    if constexpr (XEARLY) xbad = flags_any(nf, NC);
    // this lane's A operands of its columns GS*gi + c + NC*i, m = gi*CPS + i
    // (zeros where it carries no digit)
    i32x4 A[MS][4];
    float4 mt[MS];
#pragma unroll
    for (int m = 0; m < MS; ++m) {
      const int sb = min(GS * (m / CPS) + c + NC * (m % CPS), nsb - 1);
      const uint8_t* ap = xlds + sb * XQ_SB + g * 64 + (n & 3) * 16;
      const bool live0 = (n >> 2) == 2 * (g >> 1), live1 = (n >> 2) == 2 * (g >> 1) + 1;
      const i32x4 z4 = {0, 0, 0, 0};
      A[m][0] = live0 ? *(const i32x4*)(ap) : z4;
      A[m][1] = live1 ? *(const i32x4*)(ap + XQ_T) : z4;
      A[m][2] = live0 ? *(const i32x4*)(ap + 2 * XQ_T) : z4;
      A[m][3] = live1 ? *(const i32x4*)(ap + 3 * XQ_T) : z4;
      mt[m] = *(const float4*)(meta + sb * 16 + g * 4);
    }
    // q4_K up to K = 8192: high nibbles through q4k_sb_hb (its accumulator starts per column)
    constexpr bool HB = QT == QT_Q4_K && MS <= 4;
    i32x4 hi0[HB ? MS : 1][2];
    if constexpr (HB) {
#pragma unroll
      for (int m = 0; m < MS; ++m) {
        q4k_hi_init(A[m], hi0[m][0], hi0[m][1]);
        mt[m] = q4k_hi_scale(mt[m], g);
      }
    }
    // row n of a stage: producer n / 4's slot, row n % 4 of it; column c
    const uint8_t* rowbase = ring + (n / PROWS) * L::REGION + (n % PROWS) * PITCH + c * SBB;
    float part[OWN ? 1 : R];  // (!OWN) this consumer's sum of row n of each tile (lanes g == 0)
    unsigned long long upswap = 0;  // SK: what the deposit of the first tile's part got back
    bool upmine = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int gi = 0; gi < MG; ++gi) {
        // q: this stage's place in the workgroup's sequence
        const int q = SK ? (t0 + r) * ngrp + gi - s0 : r * ngrp + gi;
        if (gi < ngrp && (!SK || (q >= 0 && q < total))) {
          const int slot = q % NS;
          if (GS * gi + c < nsb) {
            poll_ge<NP>(full + NP * slot, q);
#pragma unroll
            for (int i = 0; i < CPS; ++i)
              if (c + NC * i < GS && GS * gi + c + NC * i < nsb) {
                if constexpr (HB)
                  acc = q4k_sb_hb(rowbase + slot * SLOT + NC * i * SBB, g, A[gi * CPS + i], mt[gi * CPS + i],
                                  hi0[gi * CPS + i][0], hi0[gi * CPS + i][1], acc);
                else
                  acc = MfmaFmt<QT>::step_reg(rowbase + slot * SLOT + NC * i * SBB, g, A[gi * CPS + i],
                                              mt[gi * CPS + i], acc);
              }
          }
          if (lane == 0) lds_rel(&done[slot * NCP + c], q);
        }
      }
      acc = row_sum4(acc);
      if constexpr (OWN) {
        if (g == 0) red[(r * NC + c) * 16 + n] = acc;
      } else {
        part[r] = acc;
      }
      if constexpr (EARLY) {
        if (r == 0 && t0 * ngrp < s0) {
          // the first tile began in the previous workgroup: the last consumer done with it
          // leaves its part (the sum of the consumers' partials, in the final loop's order)
          // for that workgroup now, long before the end
          int old = 0;
          if (lane == 0) old = __hip_atomic_fetch_add(first_in, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
          old = __shfl(old, 0, 64);
          if (old == NC - 1 && lane < 16 && t0 * 16 + lane < N) {
            float sp = 0.f;
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) sp += red[cc * 16 + lane];
            const unsigned long long mine = ((unsigned long long)sk.epoch << 32) | (__float_as_uint(sp) ^ WS_SENT);
            upswap = __hip_atomic_exchange(ws_pair + (int)blockIdx.x * 16 + lane, mine, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            upmine = true;
          }
        }
      }
    }
    if constexpr (EARLY)
      if (upmine) met[16 + lane] = upswap;
    if constexpr (!OWN) {
      __syncthreads();  // every stage consumed: the ring is free
      if (g == 0)
#pragma unroll
        for (int r = 0; r < R; ++r) red[(r * NC + c) * 16 + n] = part[r];
    }
    __syncthreads();  // partial sums are in red[]
  }
  // the output row of row n of this workgroup's tile r (false: none), its tile in t
  auto out_row = [&](int r, int n, int& t, TileRef& tr, int& row) __attribute__((always_inline)) {
    t = SK ? t0 + r : (int)blockIdx.x + r * G;
    if (SK ? t * ngrp >= s1 : t >= tiles) return false;  // (SK: the tile holds a stage of the range)
    tr = locate(t);
    row = tr.tile * 16 + n;
    return row < tr.N;
  };
  // SK: the split tiles' meetings end here, before both branches below, so that every call
  // leaves the table empty.  EARLY: the first tile's part was deposited already (a part
  // the other workgroup had left first means this one sums the row), and the last tile's
  // partner part taken (met[n]), else it is deposited now (ws_pair_meet).  Otherwise
  // both parts meet here (ws_pair_meet).
  float ssum = 0.f;
  bool split = false, swrite = false;
  if constexpr (SK) {
    if (tid < R * 16) {
      const int r = tid >> 4, n = tid & 15;
      int t, row;
      TileRef tr;
      if (out_row(r, n, t, tr, row)) {
        const bool upper = t * ngrp < s0, lower = (t + 1) * ngrp > s1;
        if (upper || lower) {
          split = true;
          float sp = 0.f;
#pragma unroll
          for (int c = 0; c < NC; ++c) sp += red[(r * NC + c) * 16 + n];
          const unsigned long long o = EARLY ? met[upper ? 16 + n : n] : 0ull;
          const bool theirs = o != 0 && (unsigned)(o >> 32) == sk.epoch;
          const float other = __uint_as_float((uint32_t)o ^ WS_SENT);
          if (!EARLY) {
            swrite = ws_pair_meet((int)blockIdx.x + (upper ? 0 : 1), n, sk.epoch, upper, sp, &ssum);
          } else if (upper) {
            if (theirs) {  // the other part was there before this one: take it off the table
              __hip_atomic_store(ws_pair + (int)blockIdx.x * 16 + n, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              ssum = other + sp;  // lower + upper
              swrite = true;
            }
          } else if (theirs) {
            ssum = sp + other;
            swrite = true;
          } else {
            swrite = ws_pair_meet((int)blockIdx.x + 1, n, sk.epoch, false, sp, &ssum);
          }
        }
      }
    }
  }
  if (XEARLY ? xbad : flags_any(nf, NC)) {  // NaN or +-Inf in x: the rows take gemv_q's non-finite sums
    // (a tile two workgroups share gets the same whole-row value from both)
    for (int i = wave; i < R * 16; i += NC + NP) {
      const int r = i >> 4, n = i & 15;
      int t, row;
      TileRef tr;
      if (out_row(r, n, t, tr, row)) {
        const float s = nonfinite_terms<QT>(tr.W + (size_t)row * rb, x, 0, K, lane);
        if (lane == 0) tr.y[row] = s;
      }
    }
    return;
  }
  for (int i = tid; i < R * 16; i += 64 * (NC + NP)) {
    const int r = i >> 4, n = i & 15;
    int t, row;
    TileRef tr;
    if (out_row(r, n, t, tr, row)) {
      if (SK && split) {  // a split tile's row: written by the workgroup that met the other part
        if (swrite) tr.y[row] = ssum;
        continue;
      }
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) s += red[(r * NC + c) * 16 + n];
      tr.y[row] = s;
    }
  }
}

template <int QT, int R, int GS, int NC, int NS, int D, int XP, int XK, int NB, int SPLIT = WS_TILES>
int launch_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, const WsMats<NB>& mats, int tiles,
              hipStream_t s) {
  // WS_STAGES: WS_SK_GRID workgroups (no more than the tiles)
  constexpr bool SK = SPLIT == WS_STAGES;
  const unsigned grid = SK ? (unsigned)min(tiles, WS_SK_GRID) : (unsigned)(tiles + R - 1) / R;
  WsSplit<SK> sk;
  if constexpr (SK) sk.epoch = ws_epoch.fetch_add(1, std::memory_order_relaxed);
  using L = WsLayout<QT, GS, NC, NS, R>;
  static_assert(xq_bytes(XK) - ZERO_BYTES + 4 * NC + (R == 3 || R == 4 ? R * NC * 64 : 0) + L::LDS <= 160 * 1024,
                "LDS budget (x digits, flags, partial sums, ring)");
  static_assert(XK / 16 <= 64 * NC * XP, "x preparation: one thread per 16 elements");
  static std::atomic<uint64_t> attr{0};
  int st = lds_attr_once(attr, (const void*)qgemv_q4k_ws<QT, R, GS, NC, NS, D, XP, XK, NB, SPLIT>, (int)L::LDS,
                         "tiermm_qgemv: q4_K LDS attribute");
  if (st) return st;
  qgemv_q4k_ws<QT, R, GS, NC, NS, D, XP, XK, NB, SPLIT>
      <<<grid, 64 * (NC + NP), L::LDS, s>>>((const uint8_t*)W, rb, x, y, N, K, (int)grid, mats, sk);
  TM_LAUNCH_CHECK("tiermm_qgemv: q4_K launch");
  return TIERMM_OK;
}

// R = ceil(tiles / GTILE) tiles per workgroup (instantiated for 1-4, 6 and 8), so
// the grid, ceil(tiles / R), stays at or below 256 workgroups up to 2048 tiles.
template <int QT, int GS, int NC, int NS, int D, int XP, int XK, int NB = 0>
int launch_ws_r(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s,
                const WsMats<NB>& mats = {}) {
  int tiles;
  if constexpr (NB == 0)
    tiles = (N + 15) / 16;
  else
    tiles = mats.t0[NB];
  const int r = (tiles + GTILE - 1) / GTILE;
  switch (r <= 4 ? r : r <= 6 ? 6 : 8) {
    case 1: return launch_ws<QT, 1, GS, NC, NS, D, XP, XK, NB>(W, rb, x, y, N, K, mats, tiles, s);
    case 2: return launch_ws<QT, 2, GS, NC, NS, D, XP, XK, NB>(W, rb, x, y, N, K, mats, tiles, s);
    case 3: return launch_ws<QT, 3, GS, NC, NS, D, XP, XK, NB>(W, rb, x, y, N, K, mats, tiles, s);
    case 4: return launch_ws<QT, 4, GS, NC, NS, D, XP, XK, NB>(W, rb, x, y, N, K, mats, tiles, s);
    case 6: return launch_ws<QT, 6, GS, NC, NS, D, XP, XK, NB>(W, rb, x, y, N, K, mats, tiles, s);
    default: return launch_ws<QT, 8, GS, NC, NS, D, XP, XK, NB>(W, rb, x, y, N, K, mats, tiles, s);
  }
}

}  // namespace

// Which GEMVs take this kernel.  q4_K: from 64 row tiles up to K = 5120, from 640
// up to 8192, 64..256 tiles up to 14336, and 257..512 tiles above 8192 (per-wave
// kernel against this one: 5120x14336 12.1 against 11.1 us in split stages, 8192x14336
// 14.4 against 13.7 us in two tiles a workgroup).  q5_K: from 64 row tiles up to
// K = 5120, from 640 up to 8192, and 64..512 tiles above 8192 up to 14336.
bool qgemv_ws_takes(int qtype, int N, int K) {
  const int tiles = (N + 15) / 16;
  if (qtype == QT_Q4_K)
    return (K <= 5120 && tiles >= 64) || (K <= 8192 && tiles >= 640) || (K <= 14336 && tiles >= 64 && tiles <= 256) ||
           (K > 8192 && K <= 14336 && tiles > 256 && tiles <= 512);
  if (qtype == QT_Q5_K)
    return (K <= 5120 && tiles >= 64) || (K <= 8192 && tiles >= 640) || (K > 8192 && K <= 14336 && tiles >= 64 && tiles <= 512);
  return false;
}

// Tiles per workgroup: the grid lands at or below 256 workgroups (a uniform count
// per workgroup measured faster than a ragged one: 13824x5120 8.90 against 9.16 us,
// 5120x5120 5.89 against 6.26 us).  Up to K = 5120 whole-tile stages of 20
// super-blocks (shorter rows re-read their last 16 bytes to fill the fixed load
// count; still the fastest at K = 4096), 8 consumers with up to 3 columns each; up
// to 8192 and up to 14336 stages of 8 super-blocks (whole-tile and 16-super-block
// stages measured slower at 10240x8192: 10.8 against 10.1 us).  Up to 14336, where the
// kernel takes 64..256 tiles, a ring of 5 slots with 3 stages in flight (the LDS the
// 60 KB of x digits leave): 4096x14336 8.39 against 8.66 us for 4 slots and 2 in
// flight, 1024 and 2048 rows within 1 %; 4 in flight lost (8.13 against 7.62 us at
// 1024 rows).  Four of the stages go out before the x barrier (ws_pre).  From 257 to 384
// tiles split stages (WS_STAGES): 5120x14336 11.1 us against 12.1 on the per-wave
// kernel, 14.7 for 160 workgroups of two tiles; above that two tiles a workgroup.  At
// K <= 5120 split stages need shorter stages and lost (5120x5120: 6.0-6.5 against
// 5.4 us for 160 workgroups of two whole tiles).
int qgemv_q4k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  const int tiles = (N + 15) / 16;
  if (K <= 5120) return launch_ws_r<QT_Q4_K, 20, 8, 3, 1, 1, 5120>(W, rb, x, y, N, K, s);
  if (K <= 8192) return launch_ws_r<QT_Q4_K, 8, 8, 4, 2, 1, 8192>(W, rb, x, y, N, K, s);
  if (K <= 14336 && tiles > WS_SK_GRID && tiles <= 384)  // ranges of 1-1.5 tiles' stages: at most 3 tiles each
    return launch_ws<QT_Q4_K, 3, 8, 8, 5, 3, 2, 14336, 0, WS_STAGES>(W, rb, x, y, N, K, {}, tiles, s);
  if (K <= 14336) return launch_ws_r<QT_Q4_K, 8, 8, 5, 3, 2, 14336>(W, rb, x, y, N, K, s);
  return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemv: q4_K K=%d above %d", K, 14336);
}

// The same kernel on Q5_K (176-byte super-blocks; stages of 10 super-blocks up
// to K = 5120 keep the ring within the LDS).  Against the per-wave kernel:
// 13824x5120 10.8 against 12.5 us, 10240x8192 12.0 against 15.4 us, 5120x5120
// 7.2 against 7.8 us.  Above K = 8192 a 4-slot ring of 8-super-block stages, 2 in flight
// (60 KB of x digits leave room for 4 slots; stages of 6 super-blocks spilled): 5120x14336
// 12.7 against 14.0 us (split stages), 4096x14336 9.8 against 10.8, 8192x14336 15.7
// against 17.0, 1024x14336 8.9 against 9.0.  Q8_0 (272-byte groups) gained nothing this way (a 3-slot
// ring: 17.5 against 17.1 us at 13824x5120, 36.6 against 22.2 us at 10240x8192;
// 4096x4096 whole-tile stages: 8.4 against 5.9 us) and keeps the per-wave kernel.
int qgemv_q5k_ws(const void* W, size_t rb, const float* x, float* y, int N, int K, hipStream_t s) {
  const int tiles = (N + 15) / 16;
  if (K <= 5120) return launch_ws_r<QT_Q5_K, 10, 10, 4, 2, 1, 5120>(W, rb, x, y, N, K, s);
  if (K <= 8192) return launch_ws_r<QT_Q5_K, 8, 8, 4, 2, 1, 8192>(W, rb, x, y, N, K, s);
  if (K <= 14336 && tiles > WS_SK_GRID && tiles <= 384)
    return launch_ws<QT_Q5_K, 3, 8, 8, 4, 2, 2, 14336, 0, WS_STAGES>(W, rb, x, y, N, K, {}, tiles, s);
  if (K <= 14336) return launch_ws_r<QT_Q5_K, 8, 8, 4, 2, 2, 14336>(W, rb, x, y, N, K, s);
  return set_error(TIERMM_UNSUPPORTED, "tiermm_qgemv: q5_K K=%d above %d", K, 14336);
}

// Whether the whole-tile kernel takes a batch of `count` (2..WS_BATCH) q4_K or q5_K
// matrices of K <= 5120 columns in one launch: it must take each matrix on its own, so
// that each gets the arithmetic of its own call (a tile's sums do not depend on how
// many tiles a workgroup streams).
bool qgemv_ws_batch_takes(int qtype, const int* N, int count, int K) {
  if ((qtype != QT_Q4_K && qtype != QT_Q5_K) || count < 2 || count > WS_BATCH || K > 5120) return false;
  for (int i = 0; i < count; ++i)
    if (!qgemv_ws_takes(qtype, N[i], K)) return false;
  return true;
}

// The matrices of a batch (N[i] > 0, count <= WS_BATCH, qgemv_ws_batch_takes) in one
// launch: each tile, its rows and its sums are those of a launch on its matrix alone,
// so every y[i] is the same, bit for bit, as qgemv_q4k_ws / qgemv_q5k_ws on W[i].
int qgemv_ws_batch(const void* const* W, int qtype, size_t rb, const float* x, float* const* y, const int* N,
                   int count, int K, hipStream_t s) {
  WsMats<WS_BATCH> m{};
  int t = 0;
  for (int i = 0; i < WS_BATCH; ++i) {
    m.t0[i] = t;
    if (i < count) {
      m.W[i] = (const uint8_t*)W[i];
      m.y[i] = y[i];
      m.N[i] = N[i];
      t += (N[i] + 15) / 16;
    } else {
      m.W[i] = (const uint8_t*)W[0];
      m.y[i] = y[0];
      m.N[i] = N[0];
    }
  }
  m.t0[WS_BATCH] = t;
  if (qtype == QT_Q4_K) return launch_ws_r<QT_Q4_K, 20, 8, 3, 1, 1, 5120, WS_BATCH>(W[0], rb, x, y[0], N[0], K, s, m);
  return launch_ws_r<QT_Q5_K, 10, 10, 4, 2, 1, 5120, WS_BATCH>(W[0], rb, x, y[0], N[0], K, s, m);
}

}  // namespace tiermm

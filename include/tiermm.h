/*
 * tiermm.h -- C ABI of libtiermm.so, the MI355X (gfx950) frozen-weight matmul
 * path of tierlm: GGUF block dequantization fused into GEMV/GEMM, and the
 * "x3" split-precision fp16 GEMM.
 *
 * The reference engine (tier/tier.cpp) has no shared library: these entry
 * points replace the engine-internal functions cited on each one, keeping their
 * argument meaning so a tier.cpp-like engine can call them in place of the
 * originals.
 *
 * Conventions
 *  - Matrices are row-major.  A weight is W[N][K] (N = out_features rows,
 *    K = in_features cols); a quantized row is rb = K/blk*blk_bytes bytes,
 *    rows contiguous (quant.h:33, tier.cpp:288).  Activations X[M][K] fp32,
 *    outputs Y[M][ldy] fp32.
 *  - Every tensor argument is a DEVICE pointer allocated by the caller, except
 *    for tiermm_quantize (host memory).  Nothing here frees caller memory.
 *  - Calls are stream-ordered and asynchronous: no host synchronisation, no
 *    device allocation on the hot path.  A NULL stream is the null stream.
 *  - Status: TIERMM_OK (0); TIERMM_UNSUPPORTED (1) when a shape/type/layout is
 *    not handled (the caller falls back, as the engine does when
 *    tw::launch() returns false, tier_wmma.h:81, or chat_fp3() returns false,
 *    tier.cpp:2368); TIERMM_EINVAL (2) for a bad argument; a negative value is
 *    -(hipError_t) of a failed HIP call.  No call exits the process (the
 *    reference's HIP_CHECK does, tier.cpp:63-64); tiermm_last_error() gives the
 *    text of the last failure on the calling thread.
 *  - Workspace (ws, ws_bytes): entry points that need scratch take it
 *    explicitly; *_ws_bytes() returns the size.  ws == NULL selects a pool the
 *    library grows per device (allocation happens on that call, outside any
 *    graph capture) and frees in tiermm_shutdown(); calls that share the pool
 *    must be ordered on one stream.
 */
#ifndef TIERMM_H
#define TIERMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tiermm_stream_t; /* a hipStream_t */

enum {
  TIERMM_OK = 0,
  TIERMM_UNSUPPORTED = 1,
  TIERMM_EINVAL = 2
};

/* ggml type ids, as quant.h:21-24 numbers them. */
enum {
  TIERMM_F32 = 0,
  TIERMM_F16 = 1,
  TIERMM_Q4_0 = 2,
  TIERMM_Q4_1 = 3,
  TIERMM_Q5_0 = 6,
  TIERMM_Q5_1 = 7,
  TIERMM_Q8_0 = 8,
  TIERMM_Q2_K = 10,
  TIERMM_Q3_K = 11,
  TIERMM_Q4_K = 12,
  TIERMM_Q5_K = 13,
  TIERMM_Q6_K = 14,
  TIERMM_IQ2_XXS = 16,
  TIERMM_IQ2_XS = 17,
  TIERMM_IQ3_XXS = 18,
  TIERMM_IQ1_S = 19,
  TIERMM_IQ4_NL = 20,
  TIERMM_IQ3_S = 21,
  TIERMM_IQ2_S = 22,
  TIERMM_IQ4_XS = 23,
  TIERMM_IQ1_M = 29,
  TIERMM_BF16 = 30,
  TIERMM_TQ1_0 = 34,
  TIERMM_TQ2_0 = 35,
  TIERMM_MXFP4 = 39,
  TIERMM_NF4 = 200,
  TIERMM_FP4 = 201
};

/* element type of a dequantized output (dq_k<T>, tier.cpp:294: float, tier_fp16, hip_bfloat16) */
enum { TIERMM_OUT_F32 = 0, TIERMM_OUT_F16 = 1, TIERMM_OUT_BF16 = 2 };

/* split layouts: TIERMM_HML = planes hi,mid,lo at 0, s, 2s (fp3gemm, tier.cpp:925);
 * TIERMM_LMH = lo,mid,hi (split3s_fp16, tier.cpp:2193-2194) */
enum { TIERMM_HML = 0, TIERMM_LMH = 1 };

/* BLAS operation of the weight operand in tiermm_x3_gemm (hipblasOperation_t values) */
enum { TIERMM_OP_N = 111, TIERMM_OP_T = 112 };

/* quantized-GEMM semantics: X3REF = fp16 dequant then x3 (training path,
 * tier.cpp:515 + 922); F32 = fp32 dequant then fp32 GEMM (chat prefill path,
 * tier.cpp:2358-2359). */
enum { TIERMM_MODE_X3REF = 0, TIERMM_MODE_F32 = 1 };

/* ------------------------------------------------------------------ library */
/* Select `device` (hipSetDevice) and set up per-device state.  Replaces the
 * engine's lazy global set-up (g_lt/g_lt_ws/g_own_tmp, tier.cpp:923-924). */
int tiermm_init(int device);
/* Free the library's pools on every device it used. */
void tiermm_shutdown(void);
/* Text of the last error raised on the calling thread ("" if none). */
const char* tiermm_last_error(void);
const char* tiermm_version(void);

/* ---------------------------------------------------- block-format registry */
/* quant.h:25-31 q_info: elements and bytes per block of `qtype`.
 * TIERMM_UNSUPPORTED for an unknown id. */
int tiermm_q_info(int qtype, int* blk_elems, int* blk_bytes);
/* quant.h:33-34 q_row_bytes + q_cols_ok: *rb = cols/blk*blk_bytes.
 * TIERMM_UNSUPPORTED if cols is not a whole number of blocks. */
int tiermm_q_row_bytes(int qtype, int cols, size_t* rb);

/* ----------------------------------------------------------------- dequant */
/* dq_k<T> / dq_launch (tier.cpp:293-298): for i < nrows*cols,
 * out[i] = T(q_val(W + (r0 + i/cols)*rb, qtype, i%cols)), T = fp32, fp16
 * (round to nearest even, subnormals kept, as tier_fp16) or bf16 (RNE, as
 * hip_bfloat16).  qtype: every q_val type -- F32, F16, BF16, Q4_0, Q4_1, Q5_0,
 * Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S,
 * IQ1_S, IQ1_M, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NF4, FP4; cols a multiple of
 * the block (dense rows: any cols).
 * Bit-exact with the reference's q_val for finite block scales. */
int tiermm_dequant(const void* W, int qtype, size_t rb, int cols, size_t r0, size_t nrows,
                   void* out, int out_dtype, tiermm_stream_t stream);

/* --------------------------------------------------------------- decode GEMV */
/* gemv_q (tier.cpp:299-306, launched at 2357): y[r] = sum_k q_val(W_r, k) * x[k]
 * for r < N, fp32 accumulation.  W: N rows of rb bytes; x: K fp32, 16-byte
 * aligned, any K; y: N fp32.  qtype: the GPU types of tiermm_dequant; dense
 * rows (F32/F16/BF16) go to tiermm_gemv's kernel and must start 16-byte
 * aligned.  Non-finite x: y takes gemv_q's fp32 result classes exactly -- NaN
 * everywhere for a NaN in x, and for +-Inf at column k, +-Inf or NaN per row
 * from the signs (and zeros) of q_val(W_r, k).  q4_K / q5_K with 257..384 row tiles
 * above K = 8192 pair workgroups through a small device-global table that every
 * call leaves empty: such calls on one GPU must not overlap (order them on one
 * stream), or rows of theirs may go unwritten. */
int tiermm_qgemv(const void* W, int qtype, size_t rb, const float* x, float* y, int N, int K,
                 tiermm_stream_t stream);
/* No counterpart in the reference as an entry point (chat_lin calls gemv_q once per
 * matrix, tier.cpp:2357): gemv_q of count (1..TIERMM_QGEMV_BATCH) matrices that share
 * x, K and the block type, e.g. the q and k projections of a layer, or gate and up.
 * W, y and N are HOST arrays (W[i], y[i] device pointers; rows N[i] >= 0, y[i] may be
 * null where N[i] == 0); rb, alignment and errors as tiermm_qgemv.  Where the whole-tile
 * kernel takes the concatenated rows (q4_K / q5_K, K <= 5120) the matrices run as one
 * launch, which saves a launch and a kernel tail per extra matrix (q4_K 4096x5120 +
 * 1024x5120: 5.4 against 8.5 us); otherwise one tiermm_qgemv each.  Every y[i] is the
 * same, bit for bit, as tiermm_qgemv on W[i]. */
#define TIERMM_QGEMV_BATCH 4
int tiermm_qgemv_batch(const void* const* W, int qtype, size_t rb, const float* x, float* const* y,
                       const int* N, int count, int K, tiermm_stream_t stream);

/* --------------------------------------------------------------- x3 splits */
/* split3_fp_k (tier.cpp:869-870) / split3s_fp16 (tier.cpp:2192-2194):
 * h = fp16(v); m = fp16(v - h); l = fp16(v - h - m) (fp32 subtractions), for
 * i < n; written as planes at parts + {0, part_stride, 2*part_stride} in the
 * given order (TIERMM_HML or TIERMM_LMH).  part_stride >= n. */
int tiermm_split3_f16(const float* x, uint16_t* parts, size_t n, size_t part_stride, int order,
                      tiermm_stream_t stream);

/* ------------------------------------------------------- dense-row GEMV */
/* gemv<T> (tier.cpp:2261-2268, launched at 2345, 2363, 2616 for the fp16/bf16
 * frozen matrices and the LM head): y[r] = sum_k float(W[r][k]) * x[k], fp32
 * accumulation.  wtype in {TIERMM_F32, TIERMM_F16 (tier_fp16 bits),
 * TIERMM_BF16}; W: N rows of K elements, 16-byte aligned; any K. */
int tiermm_gemv(const void* W, int wtype, const float* x, float* y, int N, int K, tiermm_stream_t stream);

/* split3_k (tier.cpp:866-867) / split3s (tier.cpp:2159-2161): the same split
 * in bf16 parts (hip_bfloat16 rounding: nearest even), layouts as above. */
int tiermm_split3_bf16(const float* x, uint16_t* parts, size_t n, size_t part_stride, int order,
                       tiermm_stream_t stream);

/* ------------------------------------------------------------ x3-ref GEMM */
/* fp3gemm (tier.cpp:922-943) in its BLAS column-major contract:
 * C(m x n) = op(A)(m x k) * B(k x n) + beta * C, A fp16 (the frozen weight,
 * exact), B fp32 split into three fp16 parts; the three products run on fp16
 * MFMA with fp32 accumulation.  With opA = TIERMM_OP_T and lda = k this is the
 * forward linear out[n][m] = x[n][k] * W[m][k]^T (low3_linear, tier.cpp:1212);
 * with opA = TIERMM_OP_N and lda = m it is the dX product of linear_dx /
 * linear_dx_acc (tier.cpp:1226, 1234): A is m x k column-major (W[k][m] in
 * memory).  The large-tile kernel reads that layout in place (the reference's
 * TR operand, tier_wmma.h:34-37) when k is a multiple of 32, m and lda multiples
 * of 8 and A 16-byte aligned; otherwise A is transposed into the workspace first
 * (same result, bit for bit).  ldc >= m.  Accuracy: rel. Frobenius error <= 2^-20
 * against fp64(A * B). */
int tiermm_x3_gemm(int opA, int m, int n, int k, const uint16_t* A, int lda, const float* B,
                   float beta, float* C, int ldc, void* ws, size_t ws_bytes,
                   tiermm_stream_t stream);
size_t tiermm_x3_gemm_ws_bytes(int m, int n, int k);

/* bf3gemm (tier.cpp:900-921): tiermm_x3_gemm with the weight in bf16 and x split
 * in three bf16 parts, on bf16 MFMA (the engine's fallback when fp16 x3 is not
 * available).  Same arguments, workspace size and accuracy bar. */
int tiermm_x3_gemm_bf16(int opA, int m, int n, int k, const uint16_t* A, int lda, const float* B,
                        float beta, float* C, int ldc, void* ws, size_t ws_bytes,
                        tiermm_stream_t stream);

/* chat_fp3 (tier.cpp:2195-2219): y[M][ldo] = x[M][K] * W[N][K]^T with x split
 * into three fp16 parts and W fp16, fp32 accumulation (the reference sums the
 * parts as (lo + mid) + hi, add3ld tier.cpp:2162-2164). ldo >= N. */
int tiermm_x3_rows(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo,
                   void* ws, size_t ws_bytes, tiermm_stream_t stream);
size_t tiermm_x3_rows_ws_bytes(int M, int K, int N);
/* chat_bf3 (tier.cpp:2165-2189): tiermm_x3_rows with a bf16 weight and bf16 parts. */
int tiermm_x3_rows_bf16(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo,
                        void* ws, size_t ws_bytes, tiermm_stream_t stream);

/* No counterpart in the reference: tiermm_x3_rows for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same product, kernels and accuracy; no
 * workspace argument and no allocation on any call: the three fp16 planes of x
 * live in a static device scratch of TIERMM_NOALLOC_SCRATCH_BYTES per GPU, held
 * until the process ends (its device address is looked up by tiermm_init, or by
 * the first call on a device).  TIERMM_UNSUPPORTED when 3 * M * K * 2 bytes
 * exceed it, or K is not a multiple of 32.  Calls that overlap on one GPU share
 * the scratch and race: order them on one stream. */
#define TIERMM_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int tiermm_x3_rows_noalloc(const uint16_t* W, const float* x, float* y, int M, int K, int N, int ldo,
                           tiermm_stream_t stream);

/* ------------------------------------------------------------ x3-2x2 GEMM */
/* Two-part split with a power-of-two exponent per row (the storage of the 2x2
 * x3 GEMM; README.md:21 describes it, no reference function exists):
 * e_r = 14 - floor(log2(max_k |src[r][k]|)) (0 for an all-zero row, clamped
 * to [-100, 100]); hi = fp16(src * 2^e_r); lo = fp16(src * 2^e_r - hi).
 * exps[r] = e_r.  Scaling keeps lo out of the fp16 subnormal range. */
int tiermm_x3s_split(const float* src, uint16_t* hi, uint16_t* lo, int32_t* exps, int rows,
                     int cols, tiermm_stream_t stream);
/* Y[M][ldy] = 2^-(xexp[m] + wexp[n]) * (Xhi*Whi^T + Xhi*Wlo^T + Xlo*Whi^T), the
 * three products on fp16 MFMA accumulated in fp32.  X*: [M][K], W*: [N][K].
 * Accuracy: rel. Frobenius error <= 2^-20 against fp64(X * W^T). */
int tiermm_x3s_gemm(const uint16_t* Xhi, const uint16_t* Xlo, const int32_t* xexp,
                    const uint16_t* Whi, const uint16_t* Wlo, const int32_t* wexp, float* Y,
                    int M, int N, int K, int ldy, tiermm_stream_t stream);

/* sgemm (tier.cpp:773-865) with opB = N in its BLAS column-major contract, on fp32
 * operands: C(m x n) = op(A)(m x k) * B(k x n) + beta * C.  It is the x3-off fallback
 * of low3_linear / linear / linear_dx / linear_dx_acc (tier.cpp:1196-1200, 1213,
 * 1229-1230, 1235-1236) on the expanded fp32 weight.  opA = TIERMM_OP_T, lda >= k: A
 * is [m][lda] row-major (the forward out[n][m] = x[n][k] * W[m][k]^T); opA =
 * TIERMM_OP_N, lda >= m: A is [k][lda] row-major (the dX product dX[n][m] = dY[n][k] *
 * W[k][m]).  B is [n][ldb] (ldb >= k), C is [n][ldc] (ldc >= m).  The rows of op(A)
 * and of B are split into fp16 hi/lo parts scaled by a power of two per row, and
 * hi*hi + hi*lo + lo*hi run on fp16 MFMA with fp32 accumulation (any k: rows are
 * zero-padded to a multiple of 32 in the workspace): rel. Frobenius error <= 2^-20
 * against fp64(op(A) * B). */
int tiermm_sgemm(int opA, int m, int n, int k, const float* A, int lda, const float* B, int ldb, float beta,
                 float* C, int ldc, void* ws, size_t ws_bytes, tiermm_stream_t stream);
size_t tiermm_sgemm_ws_bytes(int opA, int m, int n, int k);

/* -------------------------------------------------------- quantized GEMM */
/* The M > 1 quantized linear: Y[M][ldy] = X[M][K] * dequant(W)^T + beta * Y.
 * mode TIERMM_MODE_X3REF: W is dequantized to fp16 (bit-exact with dq_k<tier_fp16>,
 * tier.cpp:515) inside the kernel and multiplied with x split in three fp16
 * parts (fp3gemm semantics, tier.cpp:922): rel. Frobenius error <= 2^-20
 * against fp64(fp16deq(W) * X).  mode TIERMM_MODE_F32: the chat prefill
 * semantics (fp32 dequant, then an fp32 GEMM, tier.cpp:2358-2359): rel.
 * Frobenius error <= 2^-20 against fp64(deq(W) * X).  qtype: the GPU types of
 * tiermm_dequant.  The workspace (tiermm_qgemm_ws_bytes) holds the x parts and,
 * for q8_0 / q4_K / q5_K / q6_K / q5_0 (decoded inside the GEMM), the split-K partial
 * sums, or for the other types the fp16 weight; the environment variable
 * TIERMM_QGEMM_TILE="BN,KS[,KC]" overrides the fused kernel's tile width, split count
 * and accumulation chunks (read at each call, and by the size query; ignored when
 * invalid for the shape). */
int tiermm_qgemm(const void* W, int qtype, size_t rb, const float* X, float* Y, int M, int N,
                 int K, int ldy, int mode, float beta, void* ws, size_t ws_bytes,
                 tiermm_stream_t stream);
size_t tiermm_qgemm_ws_bytes(int qtype, int M, int N, int K, int mode);
/* No counterpart in the reference (an introspection aid for tuning and tests): the tile
 * plan that tiermm_qgemm's fused dequant kernel takes for a TIERMM_MODE_X3REF product of
 * this shape -- tile width *bn, K splits *ks, accumulation chunks *kc -- after
 * TIERMM_QGEMM_TILE; TIERMM_UNSUPPORTED when the type or shape does not take it. */
int tiermm_qgemm_plan(int qtype, int M, int N, int K, int* bn, int* ks, int* kc);
/* No counterpart in the reference as an entry point (fp3gemm, tier.cpp:922-943, splits
 * its B operand on every call): tiermm_qgemm's TIERMM_MODE_X3REF product with x
 * already split, so products that read the same activations (the q / k / v
 * projections, gate / up) split them once.  xparts: the three fp16 planes of x[M][K]
 * in TIERMM_HML order, 16-byte aligned, part_stride (a multiple of 8, >= M*K)
 * elements apart, laid out as `layout` says:
 *   TIERMM_PARTS_ROWS   -- row-major, as tiermm_split3_f16 writes them;
 *   TIERMM_PARTS_KTILED -- K-tiled, as tiermm_split3_f16_ktiled writes them (element
 *                          (r, c) at ((c/32)*M + r)*32 + c%32): each MFMA operand load
 *                          is one contiguous kilobyte, the layout tiermm_qgemm uses
 *                          itself, and the faster one.
 * K a multiple of 32 (TIERMM_UNSUPPORTED otherwise).  Same result, bit for bit, as
 * tiermm_qgemm on the unsplit x.  Workspace (tiermm_qgemm_x3parts_ws_bytes): the fused
 * kernel's split-K partial sums, or the fp16 weight for the types it does not decode. */
#define TIERMM_PARTS_ROWS 0
#define TIERMM_PARTS_KTILED 1
int tiermm_qgemm_x3parts(const void* W, int qtype, size_t rb, const uint16_t* xparts, size_t part_stride,
                         int layout, float* Y, int M, int N, int K, int ldy, float beta, void* ws,
                         size_t ws_bytes, tiermm_stream_t stream);
size_t tiermm_qgemm_x3parts_ws_bytes(int qtype, int M, int N, int K);
/* split3_fp_k (tier.cpp:869-870) of x[M][K] (16-byte aligned, K a multiple of 32) into
 * the K-tiled planes of TIERMM_PARTS_KTILED, in TIERMM_HML order, part_stride (a
 * multiple of 8, >= M*K) elements apart: the same values as tiermm_split3_f16. */
int tiermm_split3_f16_ktiled(const float* x, uint16_t* parts, int M, int K, size_t part_stride,
                             tiermm_stream_t stream);

/* ------------------------------------------------- grouped (MoE) GEMM */
/* No reference function (the reference refuses MoE models, arch.py:158-159):
 * the experts' matmuls of a routed batch.  Rows [expert_offsets[e],
 * expert_offsets[e+1]) of X_sorted[.][K] are the tokens routed to expert e
 * (sorted by expert); Y_sorted[r][N] = X_sorted[r] * dequant(W_e[e])^T with
 * tiermm_qgemm's semantics per expert (`mode`).  W_e, qtype_e, rb_e and
 * expert_offsets (n_experts + 1 entries) are HOST arrays; W_e[e] are device
 * pointers.  Expert down-projections whose K is not a multiple of 256 use a
 * 32-element type (q5_0, as llama.cpp falls back). */
int tiermm_qgemm_grouped(const void* const* W_e, const int* qtype_e, const size_t* rb_e,
                         const float* X_sorted, const int* expert_offsets, int n_experts,
                         float* Y_sorted, int N, int K, int mode, void* ws, size_t ws_bytes,
                         tiermm_stream_t stream);
size_t tiermm_qgemm_grouped_ws_bytes(const int* qtype_e, const int* expert_offsets, int n_experts,
                                     int N, int K, int mode);
/* Per-token weighted combine of the routed outputs: out[t][n] =
 * sum_{j<topk} pair_weight[p] * Y_sorted[p][n], p = token_pairs[t*topk + j],
 * summed in j order.  token_pairs, pair_weight: device arrays. */
int tiermm_moe_combine(const float* Y_sorted, const int* token_pairs, const float* pair_weight,
                       float* out, int T, int topk, int N, tiermm_stream_t stream);

/* ------------------------------------------------------ host quantizer */
/* q_row (quant.h:201-204) over `rows` rows of `cols` host floats, writing
 * rows*rb bytes of blocks to host memory `out`: Q8_0 (quant.h:134-136),
 * Q4_K/Q5_K (qk_minmax_row, quant.h:138-173), Q6_K (q6_k_row, quant.h:175-199);
 * byte-identical with the reference.  Rows are split over `nthreads` host
 * threads (<= 0: all hardware threads). */
int tiermm_quantize(int qtype, const float* x, void* out, size_t rows, int cols, int nthreads);

/* ------------------------------------------------------- .tq container */
/* A quantized base on disk (reader tq_load/tq_of, tier.cpp:273-292; writers
 * tier.cpp:2716-2744 and quant.py:60-105): a NUL-padded text header of hb
 * bytes -- "TQB1 <hb> <n>", "#key value" meta lines, and one line per matrix
 * "<name> <type> <rows> <cols> <offset> <bytes> [err]" -- then the matrices at
 * 4096-aligned offsets, rows of q_row_bytes(type, cols) bytes back to back.
 * Host-side only; the rows a caller reads go to device memory with its own
 * copies (see tiermm_qgemv and friends for the layout they expect). */
typedef struct tiermm_tq tiermm_tq;
/* Parse the header; TIERMM_EINVAL for a file that is not a .tq or a matrix
 * line that does not parse (unknown type, columns not whole blocks, byte count
 * other than rows * q_row_bytes).  A repeated name replaces the earlier one. */
int tiermm_tq_open(const char* path, tiermm_tq** out);
void tiermm_tq_close(tiermm_tq* tq);
int tiermm_tq_count(const tiermm_tq* tq);
/* Index of the matrix called `name`, or -1 (tq_of, tier.cpp:292). */
int tiermm_tq_find(const tiermm_tq* tq, const char* name);
/* Fields of matrix i (any pointer may be NULL); err is -1 when the file has none. */
int tiermm_tq_info(const tiermm_tq* tq, int i, const char** name, int* qtype, int* rows, int* cols,
                   uint64_t* offset, uint64_t* bytes, size_t* rb, double* err);
int tiermm_tq_meta_count(const tiermm_tq* tq);
int tiermm_tq_meta(const tiermm_tq* tq, int i, const char** key, const char** value);
/* Copy rows [r0, r0 + nrows) of matrix i (nrows * rb bytes) to host memory dst. */
int tiermm_tq_read_rows(const tiermm_tq* tq, int i, size_t r0, size_t nrows, void* dst);
/* Write n matrices (host data, rows * q_row_bytes bytes each) and nmeta meta
 * pairs to `path` through "<path>.part" and a rename, as the reference writers
 * do; errs (may be NULL: "-1") are written with 6 decimals. */
int tiermm_tq_write(const char* path, int n, const char* const* names, const int* qtypes, const int* rows,
                    const int* cols, const void* const* data, const double* errs, int nmeta,
                    const char* const* keys, const char* const* values);

/* q_val (quant.h:59-121) on the host: out[r*cols + c] for nrows rows of rb bytes
 * of any GPU type of tiermm_dequant (host memory; the comparison behind
 * tier --tq-check, tier.cpp:2749-2765). */
int tiermm_dequant_host(const void* W, int qtype, size_t rb, int cols, size_t nrows, float* out);

/* Type of one projection under a quantization recipe (tier.cpp:2701-2713, the
 * same rule as recipe_types in tierlm.py:1858-1874).  recipe: "Q8_0", "Q6_K",
 * "Q5_K_M", "Q5_K_S", "Q4_K_M" or "Q4_K_S"; slot 0..6 = q, k, v, o, gate, up,
 * down projection; for slot 2 (index, count) = the v_proj's rank among the
 * layers that have one and their number, for slot 6 the layer index and the
 * number of layers (ignored for other slots).  Returns the type id, or
 * TIERMM_EINVAL for an unknown recipe. */
int tiermm_recipe_type(const char* recipe, int slot, int index, int count);

/* ------------------------------------------ chat linears with weight streaming */
/* The chat engine's per-linear dispatch, chat_lin (tier.cpp:2351-2378), and its
 * double-buffered weight streaming (g_chat_SQ / chat_slot / chat_issue,
 * tier.cpp:2283-2285; placement tier.cpp:2549-2555).  A set holds the
 * matrices of a model's linears.  Each is resident in device memory or
 * streamed from pinned host memory through `nslots` device slots on a copy
 * stream of its own, overlapped with compute on the set's compute stream.
 * Streamed matrices must be used in registration order, cyclically (the
 * engine's layer order); a use out of that order is refused (TIERMM_EINVAL)
 * and tiermm_chat_restart(c, 1) rewinds.  A set is used from one host thread
 * with the device it was created on current. */
typedef struct tiermm_chat tiermm_chat;
/* New set; nslots in 2..8 (the engine uses 2), compute_stream as chat_lin's g_chat_cs. */
int tiermm_chat_create(int nslots, tiermm_stream_t compute_stream, tiermm_chat** out);
/* Waits for the set's work, frees what it allocated (not the caller's rows). */
void tiermm_chat_destroy(tiermm_chat* c);
/* Register a matrix (rows x cols of qtype, row bytes rb) before tiermm_chat_place.
 * dev != NULL: resident in the caller's device memory (16-byte aligned).
 * dev == NULL: host rows, placed by tiermm_chat_place (pinned when streamed).
 * *id is its handle for tiermm_chat_lin.  qtype: the GPU types of tiermm_dequant. */
int tiermm_chat_add(tiermm_chat* c, int qtype, size_t rb, int rows, int cols, const void* host, void* dev, int* id);
/* Placement (tier.cpp:2549-2555): in registration order a matrix is copied to
 * device memory while (resident bytes + its bytes) <= budget and
 * (resident bytes + its bytes + reserve) < free memory less the slots; after
 * the first that is not, every later one is streamed.  Allocates the slots and
 * issues their first copies (tier.cpp:2569).  On failure the set is as before. */
int tiermm_chat_place(tiermm_chat* c, size_t budget, size_t reserve, size_t* resident_bytes,
                      size_t* streamed_bytes);
/* chat_lin: y[M][rows] = x[M][cols] * W^T on the compute stream.  M == 1:
 * gemv_q / gemv<T> (tiermm_qgemv, tiermm_gemv); M > 1: quantized rows through
 * tiermm_qgemm(mode), fp16 / bf16 rows through tiermm_x3_rows(_bf16) when
 * mode is TIERMM_MODE_X3REF (chat_fp3 / chat_bf3) and else, as fp32 rows always,
 * through tiermm_qgemm(TIERMM_MODE_F32) (the engine's expand + SGEMM).  x, y:
 * device fp32, x 16-byte aligned.  A streamed matrix waits for its copy and
 * then refills its slot with the use nslots ahead (tier.cpp:2377). */
int tiermm_chat_lin(tiermm_chat* c, int id, const float* x, float* y, int M, int mode);
/* Trained rows over matrix id's output (chat_heads, tier.cpp:2339-2350; set up at
 * tier.cpp:2514-2526): after the base product, hr rows of htype (TIERMM_F16 or
 * TIERMM_BF16, the engine's storage type) at hd -- device memory, 16-byte aligned,
 * [hr][cols], kept by the caller -- replace output rows ri[j] (a device int array
 * of hr row indices), or rows 0..hr-1 when ri is NULL.  They are computed as
 * gemv<T> at M = 1 and with fp32 semantics (expand + SGEMM) above.  hr = 0 or
 * hd = NULL removes them. */
int tiermm_chat_set_heads(tiermm_chat* c, int id, int hr, int htype, const void* hd, const int* ri);
/* Apply the trained rows (on != 0, the default) or not: the engine's g_chat_heads,
 * switched with the trained/base mode (tier.cpp:2338, 2669). */
int tiermm_chat_heads(tiermm_chat* c, int on);
/* LoRA adapter of matrix id (chat_lora, tier.cpp:2333-2337; loaded at 2420-2429,
 * 2476-2477): after the base product and the trained rows, y += s * (x A^T) B^T
 * with A [r][cols] and B [rows][r] fp32 device arrays kept by the caller, both
 * products fp32-accurate.  r = 0 or a NULL array removes it. */
int tiermm_chat_set_lora(tiermm_chat* c, int id, int r, const float* A, const float* B);
/* The adapters' scale s = on ? k * alpha / r : 0 (g_chat_lalpha, g_chat_lk and
 * g_chat_lon, tier.cpp:2332, 2651, 2668); s == 0 skips them.  Defaults: alpha 0
 * (adapters off until set), k 1, on. */
int tiermm_chat_lora_scale(tiermm_chat* c, float alpha, float k, int on);
/* After the host rows of streamed matrices changed (or to rewind the cyclic
 * order, rewind != 0): wait for the set's streams and issue the pending copies
 * again (the engine's chat_issue(qi), chat_issue(qi+1), tier.cpp:2666-2676). */
int tiermm_chat_restart(tiermm_chat* c, int rewind);
/* *streamed: 1 if matrix id is streamed, 0 if resident (-1 for id < 0); the
 * set's resident and streamed bytes and the streamed uses so far. */
int tiermm_chat_info(const tiermm_chat* c, int id, int* streamed, size_t* resident_bytes, size_t* streamed_bytes,
                     long long* uses);
/* Pinned host memory for streamed rows (hipHostMalloc). */
int tiermm_host_alloc(size_t bytes, void** out);
int tiermm_host_free(void* p);

#ifdef __cplusplus
}
#endif
#endif /* TIERMM_H */

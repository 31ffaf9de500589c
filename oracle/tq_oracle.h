/*
 * tq_oracle.h -- CPU restatement of the reference's frozen-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker.
 * The product (tier_amd / libtiermm.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference checkout, tier/ directory).
 *
 * Parity pinning (what checks each function against something other than
 * itself) is listed per function below.
 */
#ifndef TQ_ORACLE_H
#define TQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (quant.h:21-24). */
enum {
  ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7,
  ORC_Q8_0 = 8, ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13,
  ORC_Q6_K = 14, ORC_IQ4_NL = 20, ORC_IQ4_XS = 23, ORC_BF16 = 30, ORC_TQ1_0 = 34,
  ORC_TQ2_0 = 35, ORC_MXFP4 = 39, ORC_NF4 = 200, ORC_FP4 = 201,
  ORC_IQ2_XXS = 16, ORC_IQ2_XS = 17, ORC_IQ3_XXS = 18, ORC_IQ1_S = 19, ORC_IQ3_S = 21, ORC_IQ2_S = 22,
  ORC_IQ1_M = 29
};
/* output dtypes of the dequant (dq_k<T>, tier.cpp:294): float, tier_fp16, hip_bfloat16 */
enum { ORC_OUT_F32 = 0, ORC_OUT_F16 = 1, ORC_OUT_BF16 = 2 };

/* Block geometry (quant.h:25-34).  Returns 0 when the type is unknown.
 * Pinned: tests compare against oracle/_ref q_row_bytes for every type id. */
int orc_q_block(int type, int* blk_elems, int* blk_bytes);
size_t orc_q_row_bytes(int type, int cols);

/* fp16 <-> fp32.  orc_h2f restates q_h2f (quant.h:37-42) / tier_fp16::to_float
 * (gpu_compat.h:175-190); orc_f2h restates tier_fp16::from_float
 * (gpu_compat.h:151-174): RNE with subnormals, overflow -> inf,
 * NaN -> sign|0x7e00.  Pinned: all 65536 fp16 encodings and 2^32 fp32 inputs
 * against _ref q_f2h/q_h2f (finite inputs) and numpy astype(float16). */
float orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
/* Array forms of the conversions (for exhaustive checks). */
void orc_f2h_n(const float* x, uint16_t* h, size_t n);
void orc_h2f_n(const uint16_t* h, float* x, size_t n);
void orc_f2bf_n(const float* x, uint16_t* b, size_t n);
/* hip_bfloat16(float) rounding (RNE, used by dq_k<hip_bfloat16>).
 * Pinned: numpy reference rounding in tests (random + boundary inputs). */
uint16_t orc_f2bf(float f);

/* Scalar dequant of one element, quant.h:59-121, for every type q_val handles:
 * Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS,
 * TQ1_0, TQ2_0, MXFP4, NF4, FP4, F32, F16, BF16, and the lattice-grid IQ2_XXS,
 * IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S and IQ1_M, whose grids come from the
 * library's tier_amd/csrc/iq_grids.h (the same tables the GPU decoders read); 0
 * for other ids.  Pinned: the reference's golden vectors (Q4_0..Q6_K and the
 * lattice types) and closed-form special cases in tests/test_oracle.py; every type
 * on random blocks, the types without golden vectors on every payload byte value,
 * and the lattice types on every grid point, against oracle/_ref (the reference's
 * own q_val); MXFP4's levels against E2M1 by definition. */
float orc_q_val(const uint8_t* row, int type, int col);

/* dq_k<T> / dq_launch (tier.cpp:293-298): out[i] = T(q_val(W+(r0+i/cols)*rb, type, i%cols))
 * for i < nrows*cols, T chosen by out_dtype. */
void orc_dequant(const uint8_t* W, int type, size_t rb, int cols, size_t r0, size_t nrows,
                 void* out, int out_dtype);

/* gemv_q (tier.cpp:299-306) computed in fp64: y[r] = sum_k (double)q_val * (double)x[k].
 * This is the ideal result every GPU GEMV is compared against. */
void orc_gemv_f64(const uint8_t* W, int type, size_t rb, const float* x, double* y, int N, int K);

/* gemv_q as the reference GPU kernel evaluates it (tier.cpp:300-306) for a given
 * wave width: lane-strided fp32 fused multiply-add, then the __shfl_down tree.
 * Used to state how far the reference's own result sits from fp64. */
void orc_gemv_lanes(const uint8_t* W, int type, size_t rb, const float* x, float* y, int N, int K,
                    int wave);

/* split3_fp_k (tier.cpp:869-870) and split3s_fp16 (tier.cpp:2192-2194):
 * h=fp16(v); r=v-h; m=fp16(r); l=fp16(r-m).  order 0 ("HML", fp3gemm planes
 * at 0,n,2n = hi,mid,lo); order 1 ("LMH", chat layout d[i]=lo, d[i+s]=mid,
 * d[i+2s]=hi).  Pinned: reconstruction closed form (Sterbenz: v-h exact) and
 * the relative bound of cpu_gpu_sim.py:142-153 in tests. */
void orc_split3_f16(const float* x, uint16_t* parts, size_t n, size_t stride, int order);

/* Two-part split with a per-row power-of-two exponent, the storage of the 2x2
 * "x3" GEMM (README.md:21 prose; no reference function).  For row r:
 * e_r = 14 - floor(log2(max_k |v[r][k]|)) (0 for an all-zero row), clamped to
 * [-100, 100]; v' = v * 2^e_r; hi = fp16(v'); lo = fp16(v' - hi).
 * Pinned: exact reconstruction bound |v' - hi - lo| <= ulp_fp16(lo)/2 and the
 * fp64 product bound 2^-20 (tests). */
void orc_x3s_split(const float* v, uint16_t* hi, uint16_t* lo, int32_t* exps, int rows, int cols);
int32_t orc_x3s_row_exp(const float* v, int cols);

#ifdef __cplusplus
}
#endif
#endif

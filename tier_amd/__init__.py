"""tier_amd -- MI355X (gfx950) frozen-weight matmul path of tierlm, behind a C ABI.

``libtiermm.so`` (built in-tree by ``tier_amd.build``) holds hand-written HIP
kernels for gfx950 and exports the C ABI declared in ``include/tiermm.h``.
This module binds that ABI with ctypes and mirrors, under the reference's own
names, the engine functions the ABI replaces:

=====================  ====================================  ==============================
reference function     meaning                               here
=====================  ====================================  ==============================
q_row_bytes/q_cols_ok  quant.h:31-34                         ``q_row_bytes``
dq_launch / dq_k<T>    tier.cpp:293-298                      ``dq_launch``
gemv_q                 tier.cpp:299-306                      ``gemv_q``
split3_fp_k/split3s    tier.cpp:869-870, 2192-2194           ``split3``
fp3gemm                tier.cpp:922-943                      ``fp3gemm``
chat_fp3               tier.cpp:2195-2219                    ``chat_fp3`` (returns False when unsupported)
chat_lin (quantized)   tier.cpp:2351-2378                    ``qlinear``
q_row                  quant.h:201-204                       ``q_row`` (host)
=====================  ====================================  ==============================

Device tensors are passed as integer device addresses (``tier_amd.hip`` gives
them).  There is no CPU fallback: if the library is missing, importing this
package raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtiermm.so")

OK, UNSUPPORTED, EINVAL = 0, 1, 2
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NF4, FP4 = 10, 11, 20, 23, 34, 35, 39, 200, 201
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M = 16, 17, 18, 19, 21, 22, 29
# the types the GPU kernels decode (dq_k / gemv_q over q_val): every type of quant.h:21-24
GPU_TYPES = (F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, TQ1_0,
             TQ2_0, MXFP4, NF4, FP4, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M)
OUT_F32, OUT_F16, OUT_BF16 = 0, 1, 2
HML, LMH = 0, 1
OP_N, OP_T = 111, 112
MODE_X3REF, MODE_F32 = 0, 1
TYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1",
              Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K",
              IQ4_NL: "iq4_nl", IQ4_XS: "iq4_xs", TQ1_0: "tq1_0", TQ2_0: "tq2_0", MXFP4: "mxfp4", NF4: "nf4",
              FP4: "fp4", IQ2_XXS: "iq2_xxs", IQ2_XS: "iq2_xs", IQ2_S: "iq2_s", IQ3_XXS: "iq3_xxs",
              IQ3_S: "iq3_s", IQ1_S: "iq1_s", IQ1_M: "iq1_m"}

# every symbol include/tiermm.h declares
EXPORTS = (
    "tiermm_init", "tiermm_shutdown", "tiermm_last_error", "tiermm_version", "tiermm_q_info",
    "tiermm_q_row_bytes", "tiermm_dequant", "tiermm_qgemv", "tiermm_split3_f16", "tiermm_x3_gemm",
    "tiermm_x3_gemm_ws_bytes", "tiermm_x3_rows", "tiermm_x3_rows_ws_bytes", "tiermm_x3s_split",
    "tiermm_x3s_gemm", "tiermm_qgemm", "tiermm_qgemm_ws_bytes", "tiermm_quantize", "tiermm_gemv",
    "tiermm_qgemm_grouped", "tiermm_qgemm_grouped_ws_bytes", "tiermm_moe_combine", "tiermm_recipe_type",
    "tiermm_split3_bf16", "tiermm_x3_gemm_bf16", "tiermm_x3_rows_bf16", "tiermm_tq_open", "tiermm_tq_close",
    "tiermm_tq_count", "tiermm_tq_find", "tiermm_tq_info", "tiermm_tq_meta_count", "tiermm_tq_meta",
    "tiermm_tq_read_rows", "tiermm_tq_write", "tiermm_dequant_host", "tiermm_chat_create", "tiermm_chat_destroy",
    "tiermm_chat_add", "tiermm_chat_place", "tiermm_chat_lin", "tiermm_chat_restart", "tiermm_chat_info",
    "tiermm_host_alloc", "tiermm_host_free", "tiermm_x3_rows_noalloc", "tiermm_chat_set_heads",
    "tiermm_chat_heads", "tiermm_chat_set_lora", "tiermm_chat_lora_scale", "tiermm_sgemm", "tiermm_sgemm_ws_bytes",
    "tiermm_qgemm_plan",
    "tiermm_qgemm_x3parts",
    "tiermm_qgemm_x3parts_ws_bytes",
    "tiermm_split3_f16_ktiled",
    "tiermm_qgemv_batch",
)


class TiermmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class TiermmUnsupported(TiermmError):
    pass


if not os.path.isfile(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built: run `python -m tier_amd.build` (no CPU fallback exists)")

_L = ctypes.CDLL(LIB_PATH)
_vp, _sz, _i, _f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float


def _sig(name, args, res=ctypes.c_int):
    fn = getattr(_L, name)
    fn.argtypes = args
    fn.restype = res
    return fn


_sig("tiermm_init", [_i])
_sig("tiermm_shutdown", [], None)
_sig("tiermm_last_error", [], ctypes.c_char_p)
_sig("tiermm_version", [], ctypes.c_char_p)
_sig("tiermm_q_info", [_i, ctypes.POINTER(_i), ctypes.POINTER(_i)])
_sig("tiermm_q_row_bytes", [_i, _i, ctypes.POINTER(_sz)])
_sig("tiermm_dequant", [_vp, _i, _sz, _i, _sz, _sz, _vp, _i, _vp])
_sig("tiermm_qgemv", [_vp, _i, _sz, _vp, _vp, _i, _i, _vp])
_sig("tiermm_qgemv_batch", [_vp, _i, _sz, _vp, _vp, _vp, _i, _i, _vp])
_sig("tiermm_split3_f16", [_vp, _vp, _sz, _sz, _i, _vp])
_sig("tiermm_x3_gemm", [_i, _i, _i, _i, _vp, _i, _vp, _f, _vp, _i, _vp, _sz, _vp])
_sig("tiermm_x3_gemm_ws_bytes", [_i, _i, _i], _sz)
_sig("tiermm_x3_rows", [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp])
_sig("tiermm_x3_rows_ws_bytes", [_i, _i, _i], _sz)
_sig("tiermm_x3s_split", [_vp, _vp, _vp, _vp, _i, _i, _vp])
_sig("tiermm_x3s_gemm", [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp])
_sig("tiermm_qgemm", [_vp, _i, _sz, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp])
_sig("tiermm_sgemm", [_i, _i, _i, _i, _vp, _i, _vp, _i, _f, _vp, _i, _vp, _sz, _vp])
_sig("tiermm_sgemm_ws_bytes", [_i, _i, _i, _i], _sz)
_sig("tiermm_qgemm_plan", [_i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)])
_sig("tiermm_qgemm_ws_bytes", [_i, _i, _i, _i, _i], _sz)
_sig("tiermm_qgemm_x3parts", [_vp, _i, _sz, _vp, _sz, _i, _vp, _i, _i, _i, _i, _f, _vp, _sz, _vp])
_sig("tiermm_split3_f16_ktiled", [_vp, _vp, _i, _i, _sz, _vp])
_sig("tiermm_qgemm_x3parts_ws_bytes", [_i, _i, _i, _i], _sz)
_sig("tiermm_quantize", [_i, _vp, _vp, _sz, _i, _i])
_sig("tiermm_gemv", [_vp, _i, _vp, _vp, _i, _i, _vp])
_pi = ctypes.POINTER(_i)
_sig("tiermm_qgemm_grouped", [ctypes.POINTER(_vp), _pi, ctypes.POINTER(_sz), _vp, _pi, _i, _vp, _i, _i, _i, _vp,
                              _sz, _vp])
_sig("tiermm_qgemm_grouped_ws_bytes", [_pi, _pi, _i, _i, _i, _i], _sz)
_sig("tiermm_moe_combine", [_vp, _vp, _vp, _vp, _i, _i, _i, _vp])
_sig("tiermm_recipe_type", [ctypes.c_char_p, _i, _i, _i])
_sig("tiermm_split3_bf16", [_vp, _vp, _sz, _sz, _i, _vp])
_sig("tiermm_x3_gemm_bf16", [_i, _i, _i, _i, _vp, _i, _vp, _f, _vp, _i, _vp, _sz, _vp])
_sig("tiermm_x3_rows_bf16", [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp])
_cp, _u64 = ctypes.c_char_p, ctypes.c_uint64
_sig("tiermm_tq_open", [_cp, ctypes.POINTER(_vp)])
_sig("tiermm_tq_close", [_vp], None)
_sig("tiermm_tq_count", [_vp])
_sig("tiermm_tq_find", [_vp, _cp])
_sig("tiermm_tq_info", [_vp, _i, ctypes.POINTER(_cp), _pi, _pi, _pi, ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                        ctypes.POINTER(_sz), ctypes.POINTER(ctypes.c_double)])
_sig("tiermm_tq_meta_count", [_vp])
_sig("tiermm_tq_meta", [_vp, _i, ctypes.POINTER(_cp), ctypes.POINTER(_cp)])
_sig("tiermm_tq_read_rows", [_vp, _i, _sz, _sz, _vp])
_sig("tiermm_dequant_host", [_vp, _i, _sz, _i, _sz, _vp])
_sig("tiermm_tq_write", [_cp, _i, ctypes.POINTER(_cp), _pi, _pi, _pi, ctypes.POINTER(_vp),
                         ctypes.POINTER(ctypes.c_double), _i, ctypes.POINTER(_cp), ctypes.POINTER(_cp)])

_sig("tiermm_chat_create", [_i, _vp, ctypes.POINTER(_vp)])
_sig("tiermm_chat_destroy", [_vp], None)
_sig("tiermm_chat_add", [_vp, _i, _sz, _i, _i, _vp, _vp, _pi])
_sig("tiermm_chat_place", [_vp, _sz, _sz, ctypes.POINTER(_sz), ctypes.POINTER(_sz)])
_sig("tiermm_chat_lin", [_vp, _i, _vp, _vp, _i, _i])
_sig("tiermm_chat_restart", [_vp, _i])
_sig("tiermm_chat_info", [_vp, _i, _pi, ctypes.POINTER(_sz), ctypes.POINTER(_sz), ctypes.POINTER(ctypes.c_longlong)])
_sig("tiermm_chat_set_heads", [_vp, _i, _i, _i, _vp, _vp])
_sig("tiermm_chat_heads", [_vp, _i])
_sig("tiermm_chat_set_lora", [_vp, _i, _i, _vp, _vp])
_sig("tiermm_chat_lora_scale", [_vp, _f, _f, _i])
_sig("tiermm_host_alloc", [_sz, ctypes.POINTER(_vp)])
_sig("tiermm_host_free", [_vp])
_sig("tiermm_x3_rows_noalloc", [_vp, _vp, _vp, _i, _i, _i, _i, _vp])
NOALLOC_SCRATCH_BYTES = 32 << 20  # TIERMM_NOALLOC_SCRATCH_BYTES


def chat_fp3_noalloc(W: int, x: int, y: int, M: int, K: int, N: int, ldo: int, stream=None) -> bool:
    """chat_fp3 without any device allocation (static scratch): False when x does not fit it."""
    code = _L.tiermm_x3_rows_noalloc(W, x, y, M, K, N, ldo, _s(stream))
    if code == UNSUPPORTED:
        return False
    _check(code)
    return True


def lib():
    return _L


def last_error() -> str:
    return (_L.tiermm_last_error() or b"").decode()


def _check(code: int) -> None:
    if code == OK:
        return
    cls = TiermmUnsupported if code == UNSUPPORTED else TiermmError
    raise cls(code, last_error())


def _s(stream) -> int | None:
    if stream is None:
        return None
    return getattr(stream, "handle", stream)


def init(device: int = 0) -> None:
    _check(_L.tiermm_init(device))


def shutdown() -> None:
    _L.tiermm_shutdown()


def version() -> str:
    return _L.tiermm_version().decode()


# ---------------------------------------------------------------- registry
def q_info(qtype: int) -> tuple[int, int]:
    be, bb = _i(), _i()
    _check(_L.tiermm_q_info(qtype, ctypes.byref(be), ctypes.byref(bb)))
    return be.value, bb.value


def q_row_bytes(qtype: int, cols: int) -> int:
    rb = _sz()
    _check(_L.tiermm_q_row_bytes(qtype, cols, ctypes.byref(rb)))
    return rb.value


def q_cols_ok(qtype: int, cols: int) -> bool:
    rb = _sz()
    return _L.tiermm_q_row_bytes(qtype, cols, ctypes.byref(rb)) == OK


# ------------------------------------------------------------- host quantizer
def q_row(qtype: int, x: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """Quantize rows of a host fp32 matrix [rows][cols] (quant.h:201-204); returns [rows][rb] bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, cols = x.shape
    out = np.empty((rows, q_row_bytes(qtype, cols)), dtype=np.uint8)
    _check(_L.tiermm_quantize(qtype, x.ctypes.data_as(_vp), out.ctypes.data_as(_vp), rows, cols, nthreads))
    return out


# ------------------------------------------------------------- device entry points
def dq_launch(W: int, qtype: int, rb: int, cols: int, r0: int, nrows: int, out: int, out_dtype: int = OUT_F16,
              stream=None) -> None:
    """dq_launch (tier.cpp:297): dequantize rows r0..r0+nrows of W into out."""
    _check(_L.tiermm_dequant(W, qtype, rb, cols, r0, nrows, out, out_dtype, _s(stream)))


def gemv_q(W: int, qtype: int, rb: int, x: int, y: int, N: int, K: int, stream=None) -> None:
    """gemv_q (tier.cpp:300): y[N] = dequant(W)[N][K] * x[K]."""
    _check(_L.tiermm_qgemv(W, qtype, rb, x, y, N, K, _s(stream)))


QGEMV_BATCH = 4


def gemv_q_batch(Ws, qtype: int, rb: int, x: int, ys, Ns, K: int, stream=None) -> None:
    """gemv_q (tier.cpp:300) of up to QGEMV_BATCH matrices sharing x, K and the block type,
    in one launch where the whole-tile kernel takes them (tiermm_qgemv_batch): ys[i][Ns[i]]
    = dequant(Ws[i])[Ns[i]][K] * x[K], bit for bit as gemv_q on each."""
    n = len(Ws)
    if not (len(ys) == len(Ns) == n):
        raise ValueError("gemv_q_batch: Ws, ys and Ns differ in length")
    w = (ctypes.c_void_p * max(n, 1))(*Ws)
    y = (ctypes.c_void_p * max(n, 1))(*ys)
    ns = (ctypes.c_int * max(n, 1))(*Ns)
    _check(_L.tiermm_qgemv_batch(w, qtype, rb, x, y, ns, n, K, _s(stream)))


def split3(x: int, parts: int, n: int, stride: int | None = None, order: int = HML, stream=None) -> None:
    """split3_fp_k / split3s_fp16 (tier.cpp:869, 2192)."""
    _check(_L.tiermm_split3_f16(x, parts, n, n if stride is None else stride, order, _s(stream)))


def fp3gemm(opA: int, m: int, n: int, k: int, A: int, lda: int, B: int, beta: float, C: int, ldc: int,
            ws: int | None = None, ws_bytes: int = 0, stream=None) -> None:
    """fp3gemm (tier.cpp:922) in its BLAS column-major contract."""
    _check(_L.tiermm_x3_gemm(opA, m, n, k, A, lda, B, beta, C, ldc, ws, ws_bytes, _s(stream)))


def split3_bf16(x: int, parts: int, n: int, stride: int | None = None, order: int = HML, stream=None) -> None:
    """split3_k / split3s (tier.cpp:866, 2159): bf16 parts."""
    _check(_L.tiermm_split3_bf16(x, parts, n, n if stride is None else stride, order, _s(stream)))


def bf3gemm(opA: int, m: int, n: int, k: int, A: int, lda: int, B: int, beta: float, C: int, ldc: int,
            ws: int | None = None, ws_bytes: int = 0, stream=None) -> None:
    """bf3gemm (tier.cpp:900): fp3gemm's contract with a bf16 weight and bf16 parts."""
    _check(_L.tiermm_x3_gemm_bf16(opA, m, n, k, A, lda, B, beta, C, ldc, ws, ws_bytes, _s(stream)))


def chat_bf3(W: int, x: int, y: int, M: int, K: int, N: int, ldo: int, ws: int | None = None, ws_bytes: int = 0,
             stream=None) -> bool:
    """chat_bf3 (tier.cpp:2165): False when the shape is not handled (the caller falls back)."""
    code = _L.tiermm_x3_rows_bf16(W, x, y, M, K, N, ldo, ws, ws_bytes, _s(stream))
    if code == UNSUPPORTED:
        return False
    _check(code)
    return True


def x3_gemm_ws_bytes(m: int, n: int, k: int) -> int:
    return _L.tiermm_x3_gemm_ws_bytes(m, n, k)


def chat_fp3(W: int, x: int, y: int, M: int, K: int, N: int, ldo: int, ws: int | None = None, ws_bytes: int = 0,
             stream=None) -> bool:
    """chat_fp3 (tier.cpp:2195): False when the shape is not handled (the caller falls back)."""
    code = _L.tiermm_x3_rows(W, x, y, M, K, N, ldo, ws, ws_bytes, _s(stream))
    if code == UNSUPPORTED:
        return False
    _check(code)
    return True


def x3_rows_ws_bytes(M: int, K: int, N: int) -> int:
    return _L.tiermm_x3_rows_ws_bytes(M, K, N)


def x3s_split(src: int, hi: int, lo: int, exps: int, rows: int, cols: int, stream=None) -> None:
    _check(_L.tiermm_x3s_split(src, hi, lo, exps, rows, cols, _s(stream)))


def x3s_gemm(Xhi: int, Xlo: int, xexp: int, Whi: int, Wlo: int, wexp: int, Y: int, M: int, N: int, K: int,
             ldy: int | None = None, stream=None) -> None:
    _check(_L.tiermm_x3s_gemm(Xhi, Xlo, xexp, Whi, Wlo, wexp, Y, M, N, K, N if ldy is None else ldy, _s(stream)))


def sgemm(opA: int, m: int, n: int, k: int, A: int, lda: int, B: int, ldb: int, beta: float, C: int, ldc: int,
          ws: int | None = None, ws_bytes: int = 0, stream=None) -> None:
    """sgemm (tier.cpp:773) with opB = N in its BLAS column-major contract: the x3-off
    fallback's fp32 product (tier.cpp:1196-1200, 1229-1230, 1235-1236)."""
    _check(_L.tiermm_sgemm(opA, m, n, k, A, lda, B, ldb, beta, C, ldc, ws, ws_bytes, _s(stream)))


def sgemm_ws_bytes(opA: int, m: int, n: int, k: int) -> int:
    return _L.tiermm_sgemm_ws_bytes(opA, m, n, k)


def qgemm(W: int, qtype: int, rb: int, X: int, Y: int, M: int, N: int, K: int, ldy: int | None = None,
          mode: int = MODE_X3REF, beta: float = 0.0, ws: int | None = None, ws_bytes: int = 0, stream=None) -> None:
    _check(_L.tiermm_qgemm(W, qtype, rb, X, Y, M, N, K, N if ldy is None else ldy, mode, beta, ws, ws_bytes,
                           _s(stream)))


def qgemm_plan(qtype: int, M: int, N: int, K: int):
    """(BN, KS, KC) of the fused dequant GEMM for this shape, or None when it does not take it."""
    bn, ks, kc = _i(), _i(), _i()
    code = _L.tiermm_qgemm_plan(qtype, M, N, K, ctypes.byref(bn), ctypes.byref(ks), ctypes.byref(kc))
    if code == UNSUPPORTED:
        return None
    _check(code)
    return bn.value, ks.value, kc.value


def qgemm_ws_bytes(qtype: int, M: int, N: int, K: int, mode: int = MODE_X3REF) -> int:
    return _L.tiermm_qgemm_ws_bytes(qtype, M, N, K, mode)


PARTS_ROWS, PARTS_KTILED = 0, 1


def qgemm_x3parts(W: int, qtype: int, rb: int, xparts: int, part_stride: int, Y: int, M: int, N: int, K: int,
                  ldy: int | None = None, beta: float = 0.0, ws: int | None = None, ws_bytes: int = 0,
                  stream=None, layout: int = PARTS_KTILED) -> None:
    """tiermm_qgemm (x3-ref) on x already split: HML planes part_stride apart, row-major
    (split3) or K-tiled (split3_ktiled)."""
    _check(_L.tiermm_qgemm_x3parts(W, qtype, rb, xparts, part_stride, layout, Y, M, N, K,
                                   N if ldy is None else ldy, beta, ws, ws_bytes, _s(stream)))


def split3_ktiled(x: int, parts: int, M: int, K: int, stride: int | None = None, stream=None) -> None:
    """split3_fp_k of x[M][K] into K-tiled HML planes (the layout qgemm_x3parts reads fastest)."""
    _check(_L.tiermm_split3_f16_ktiled(x, parts, M, K, M * K if stride is None else stride, _s(stream)))


def qgemm_x3parts_ws_bytes(qtype: int, M: int, N: int, K: int) -> int:
    return _L.tiermm_qgemm_x3parts_ws_bytes(qtype, M, N, K)


def gemv(W: int, wtype: int, x: int, y: int, N: int, K: int, stream=None) -> None:
    """gemv<T> (tier.cpp:2261-2268): y = W x for fp32 / fp16 / bf16 rows (wtype F32, F16, BF16)."""
    _check(_L.tiermm_gemv(W, wtype, x, y, N, K, _s(stream)))


def _grouped_tables(W_e, qtype_e, rb_e, offsets):
    n = len(W_e)
    if not (len(qtype_e) == len(rb_e) == n and len(offsets) == n + 1):
        raise ValueError("expert tables must have n_experts entries and offsets n_experts + 1")
    return (n, (_vp * n)(*W_e), (_i * n)(*qtype_e), (_sz * n)(*rb_e), (_i * (n + 1))(*offsets))


def qgemm_grouped_ws_bytes(qtype_e, offsets, N: int, K: int, mode: int = MODE_X3REF) -> int:
    n = len(qtype_e)
    return _L.tiermm_qgemm_grouped_ws_bytes((_i * n)(*qtype_e), (_i * (n + 1))(*offsets), n, N, K, mode)


def qgemm_grouped(W_e, qtype_e, rb_e, X_sorted: int, offsets, Y_sorted: int, N: int, K: int,
                  mode: int = MODE_X3REF, ws: int | None = None, ws_bytes: int = 0, stream=None) -> None:
    """Experts' quantized matmuls of a routed batch (host tables; device W_e, X, Y)."""
    n, w, q, r, o = _grouped_tables(W_e, qtype_e, rb_e, offsets)
    _check(_L.tiermm_qgemm_grouped(w, q, r, X_sorted, o, n, Y_sorted, N, K, mode, ws, ws_bytes, _s(stream)))


SLOTS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
         "mlp.up_proj", "mlp.down_proj")


def recipe_types(rec: str, mats) -> list[str]:
    """tierlm.py:1858-1874 recipe_types: the type name of each matrix (layer, key, rows, cols)
    under recipe `rec`, by the library's rule (tier.cpp:2701-2713)."""
    mats = list(mats)
    n_layers = 1 + max((l for l, k, *_ in mats if k == "mlp.down_proj"), default=-1)
    n_v = sum(1 for _, k, *_ in mats if k == "self_attn.v_proj")
    out, v_rank = [], 0
    for layer, key, *_ in mats:
        slot = SLOTS.index(key) if key in SLOTS else 0
        if slot == 2:
            index, count = v_rank, n_v
            v_rank += 1
        else:
            index, count = layer, n_layers
        t = _L.tiermm_recipe_type(rec.encode(), slot, index, count)
        if t < 0 or t == EINVAL:
            raise TiermmError(t, last_error())
        out.append(TYPE_NAMES[t])
    return out


def dequant_host(blocks: np.ndarray, qtype: int, cols: int) -> np.ndarray:
    """q_val of every element of host rows (quant.h:59-121), fp32 [rows][cols]."""
    b = np.ascontiguousarray(blocks, np.uint8)
    rows = b.shape[0] if b.ndim == 2 else 1
    rb = q_row_bytes(qtype, cols)
    out = np.empty((rows, cols), np.float32)
    _check(_L.tiermm_dequant_host(b.ctypes.data_as(_vp), qtype, rb, cols, rows, out.ctypes.data_as(_vp)))
    return out


def moe_combine(Y_sorted: int, token_pairs: int, pair_weight: int, out: int, T: int, topk: int, N: int,
                stream=None) -> None:
    _check(_L.tiermm_moe_combine(Y_sorted, token_pairs, pair_weight, out, T, topk, N, _s(stream)))


def qlinear(W: int, qtype: int, rb: int, x: int, y: int, M: int, N: int, K: int, ws: int | None = None,
            ws_bytes: int = 0, stream=None) -> None:
    """The quantized branch of chat_lin (tier.cpp:2356-2359): GEMV at M=1; above, fp32
    dequant and an fp32-accurate product (MODE_F32), as the engine's dequant + SGEMM."""
    if M == 1:
        gemv_q(W, qtype, rb, x, y, N, K, stream)
    else:
        qgemm(W, qtype, rb, x, y, M, N, K, N, MODE_F32, 0.0, ws, ws_bytes, stream)


# ------------------------------------------------- chat linears with streaming
class HostRows:
    """Pinned host memory from tiermm_host_alloc, viewable as a numpy byte array."""

    def __init__(self, nbytes: int):
        p = _vp()
        _check(_L.tiermm_host_alloc(max(int(nbytes), 1), ctypes.byref(p)))
        self.ptr, self.nbytes = p.value, int(nbytes)

    def array(self) -> np.ndarray:
        buf = (ctypes.c_uint8 * max(self.nbytes, 1)).from_address(self.ptr)
        return np.frombuffer(buf, np.uint8, self.nbytes)

    def free(self) -> None:
        if self.ptr:
            _check(_L.tiermm_host_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Chat:
    """A set of chat linears (chat_lin, tier.cpp:2351-2378) with the engine's weight
    streaming (chat_issue, tier.cpp:2283-2285; placement tier.cpp:2549-2555).

    The engine streams through 2 slots; the default here is 4, which lets a large copy
    start while two shorter products are still running (a 4096-token prefill over
    config-4 layers: the streamed pass within 2 % of the resident one, against 10 % with
    2 slots)."""

    def __init__(self, nslots: int = 4, stream=None):
        h = _vp()
        _check(_L.tiermm_chat_create(nslots, _s(stream), ctypes.byref(h)))
        self._h = h

    def add(self, qtype: int, rows: int, cols: int, host: int | None = None, dev: int | None = None) -> int:
        i = _i()
        _check(_L.tiermm_chat_add(self._h, qtype, q_row_bytes(qtype, cols), rows, cols, host, dev, ctypes.byref(i)))
        return i.value

    def place(self, budget: int | None = None, reserve: int = 512 << 20) -> tuple[int, int]:
        r, s = _sz(), _sz()
        b = (1 << 64) - 1 if budget is None else budget
        _check(_L.tiermm_chat_place(self._h, b, reserve, ctypes.byref(r), ctypes.byref(s)))
        return r.value, s.value

    def lin(self, i: int, x: int, y: int, M: int, mode: int = MODE_F32) -> None:
        _check(_L.tiermm_chat_lin(self._h, i, x, y, M, mode))

    def restart(self, rewind: bool = False) -> None:
        _check(_L.tiermm_chat_restart(self._h, int(rewind)))

    def set_heads(self, i: int, hr: int, htype: int, hd: int | None, ri: int | None = None) -> None:
        """chat_heads (tier.cpp:2339-2350): hr trained rows (device, F16 or BF16) over output
        rows ri (device int array) or rows 0..hr-1."""
        _check(_L.tiermm_chat_set_heads(self._h, i, hr, htype, hd, ri))

    def heads(self, on: bool) -> None:
        _check(_L.tiermm_chat_heads(self._h, int(on)))

    def set_lora(self, i: int, r: int, A: int | None, B: int | None) -> None:
        """chat_lora (tier.cpp:2333-2337): y += s (x A^T) B^T, A [r][cols], B [rows][r] fp32."""
        _check(_L.tiermm_chat_set_lora(self._h, i, r, A, B))

    def lora_scale(self, alpha: float, k: float = 1.0, on: bool = True) -> None:
        _check(_L.tiermm_chat_lora_scale(self._h, alpha, k, int(on)))

    def info(self, i: int = -1) -> dict:
        st, r, s, u = _i(), _sz(), _sz(), ctypes.c_longlong()
        _check(_L.tiermm_chat_info(self._h, i, ctypes.byref(st), ctypes.byref(r), ctypes.byref(s), ctypes.byref(u)))
        return {"streamed": st.value, "resident_bytes": r.value, "streamed_bytes": s.value, "uses": u.value}

    def close(self) -> None:
        if self._h:
            _L.tiermm_chat_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""CPU oracle for the frozen-weight matmul path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(``tier_amd``) never imports it.

Two libraries back it:

* ``_build/libtqoracle.so`` -- the plain-C restatement in ``tq_oracle.c``
  (see ``tq_oracle.h`` for the reference file:line each function follows and
  for what pins it);
* ``_ref/libtqref.so`` -- the reference's own ``quant.h`` compiled from the
  reference checkout by ``Makefile`` (target ``ref``).  Optional: present where
  it was built, absent otherwise (``ref_available()``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libtqoracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libtqref.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = (
    0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 30)
IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NF4, FP4 = 20, 23, 34, 35, 39, 200, 201
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M = 16, 17, 18, 19, 21, 22, 29
OUT_F32, OUT_F16, OUT_BF16 = 0, 1, 2

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)

_lib = None
_ref = None


def build(with_ref: bool | None = None) -> None:
    """Compile the oracle (and, where the reference checkout exists, _ref)."""
    targets = ["all"]
    ref_dir = os.environ.get("TIER_REF_DIR", "/root/reference/tier")
    if with_ref is None:
        with_ref = os.path.isfile(os.path.join(ref_dir, "quant.h"))
    if with_ref:
        targets.append("ref")
    subprocess.run(["make", "-s", "-B", "-C", HERE, f"REF_DIR={ref_dir}"] + targets, check=True)


def _ptr(a, t):
    return a.ctypes.data_as(t)


def lib():
    global _lib
    if _lib is None:
        if not os.path.isfile(LIB_PATH):
            build(with_ref=False)
        L = ctypes.CDLL(LIB_PATH)
        L.orc_q_row_bytes.restype = ctypes.c_size_t
        L.orc_q_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
        L.orc_q_block.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        L.orc_h2f.restype = ctypes.c_float
        L.orc_h2f.argtypes = [ctypes.c_uint16]
        L.orc_f2h.restype = ctypes.c_uint16
        L.orc_f2h.argtypes = [ctypes.c_float]
        L.orc_f2bf.restype = ctypes.c_uint16
        L.orc_f2bf.argtypes = [ctypes.c_float]
        for nm, a, b in (("orc_f2h_n", _f32p, _u16p), ("orc_h2f_n", _u16p, _f32p), ("orc_f2bf_n", _f32p, _u16p)):
            getattr(L, nm).argtypes = [a, b, ctypes.c_size_t]
        L.orc_q_val.restype = ctypes.c_float
        L.orc_q_val.argtypes = [_u8p, ctypes.c_int, ctypes.c_int]
        L.orc_dequant.argtypes = [_u8p, ctypes.c_int, ctypes.c_size_t, ctypes.c_int, ctypes.c_size_t,
                                  ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int]
        L.orc_gemv_f64.argtypes = [_u8p, ctypes.c_int, ctypes.c_size_t, _f32p, _f64p, ctypes.c_int, ctypes.c_int]
        L.orc_gemv_lanes.argtypes = [_u8p, ctypes.c_int, ctypes.c_size_t, _f32p, _f32p, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int]
        L.orc_split3_f16.argtypes = [_f32p, _u16p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int]
        L.orc_x3s_split.argtypes = [_f32p, _u16p, _u16p, _i32p, ctypes.c_int, ctypes.c_int]
        L.orc_x3s_row_exp.restype = ctypes.c_int32
        L.orc_x3s_row_exp.argtypes = [_f32p, ctypes.c_int]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.isfile(REF_PATH)


def ref():
    """The reference's own quant.h, compiled (see Makefile target ``ref``)."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_PATH)
        R.ref_q_row_bytes.restype = ctypes.c_size_t
        R.ref_q_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
        R.ref_q_cols_ok.argtypes = [ctypes.c_int, ctypes.c_int]
        R.ref_q_h2f.restype = ctypes.c_float
        R.ref_q_h2f.argtypes = [ctypes.c_uint16]
        R.ref_q_f2h.restype = ctypes.c_uint16
        R.ref_q_f2h.argtypes = [ctypes.c_float]
        R.ref_dequant_rows.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, ctypes.c_size_t, _f32p]
        R.ref_quantize_rows.argtypes = [ctypes.c_int, _f32p, ctypes.c_size_t, ctypes.c_int, _u8p]
        R.ref_gemv_threads.argtypes = [_u8p, ctypes.c_int, ctypes.c_size_t, _f32p, _f32p, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int]
        _ref = R
    return _ref


# ---------------------------------------------------------------- numpy API
def block(qtype: int):
    be, bb = ctypes.c_int(), ctypes.c_int()
    if not lib().orc_q_block(qtype, ctypes.byref(be), ctypes.byref(bb)):
        raise ValueError(f"unknown type {qtype}")
    return be.value, bb.value


def row_bytes(qtype: int, cols: int) -> int:
    return int(lib().orc_q_row_bytes(qtype, cols))


def dequant(W: np.ndarray, qtype: int, cols: int, out_dtype: int = OUT_F32, r0: int = 0, nrows=None):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    rb = row_bytes(qtype, cols)
    total_rows = W.size // rb
    nrows = total_rows - r0 if nrows is None else nrows
    out = np.empty(nrows * cols, dtype=np.float32 if out_dtype == OUT_F32 else np.uint16)
    lib().orc_dequant(_ptr(W, _u8p), qtype, rb, cols, r0, nrows, out.ctypes.data_as(ctypes.c_void_p), out_dtype)
    return out.reshape(nrows, cols)


def gemv_f64(W: np.ndarray, qtype: int, x: np.ndarray, N: int, K: int) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(N, dtype=np.float64)
    lib().orc_gemv_f64(_ptr(W, _u8p), qtype, row_bytes(qtype, K), _ptr(x, _f32p), _ptr(y, _f64p), N, K)
    return y


def gemv_lanes(W: np.ndarray, qtype: int, x: np.ndarray, N: int, K: int, wave: int = 64) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(N, dtype=np.float32)
    lib().orc_gemv_lanes(_ptr(W, _u8p), qtype, row_bytes(qtype, K), _ptr(x, _f32p), _ptr(y, _f32p), N, K, wave)
    return y


def f2h(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits, round to nearest even (tier_fp16::from_float)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    h = np.empty(x.size, np.uint16)
    lib().orc_f2h_n(_ptr(x, _f32p), _ptr(h, _u16p), x.size)
    return h


def h2f(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    x = np.empty(h.size, np.float32)
    lib().orc_h2f_n(_ptr(h, _u16p), _ptr(x, _f32p), h.size)
    return x


def f2bf(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (hip_bfloat16(float))."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    b = np.empty(x.size, np.uint16)
    lib().orc_f2bf_n(_ptr(x, _f32p), _ptr(b, _u16p), x.size)
    return b


def split3(x: np.ndarray, order: int = 0, stride: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    stride = x.size if stride is None else stride
    parts = np.zeros(2 * stride + x.size, dtype=np.uint16)
    lib().orc_split3_f16(_ptr(x, _f32p), _ptr(parts, _u16p), x.size, stride, order)
    return parts


def x3s_split(v: np.ndarray):
    v = np.ascontiguousarray(v, dtype=np.float32)
    rows, cols = v.shape
    hi = np.empty((rows, cols), np.uint16)
    lo = np.empty((rows, cols), np.uint16)
    ex = np.empty(rows, np.int32)
    lib().orc_x3s_split(_ptr(v, _f32p), _ptr(hi, _u16p), _ptr(lo, _u16p), _ptr(ex, _i32p), rows, cols)
    return hi, lo, ex


def h2f_array(h: np.ndarray) -> np.ndarray:
    """fp16 bit patterns -> fp32 values (exact; numpy's float16 widening is exact)."""
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------- fp64 product references
def x3s_product_f64(xh, xl, ex, wh, wl, ew):
    """Exact-in-fp64 value of the 2x2 split product Y = 2^-(ex+ew) (Xh Wh^T + Xh Wl^T + Xl Wh^T)."""
    f = lambda a: h2f_array(a).astype(np.float64)
    acc = f(xh) @ f(wh).T + f(xh) @ f(wl).T + f(xl) @ f(wh).T
    return acc * np.exp2(-(ex[:, None].astype(np.float64) + ew[None, :].astype(np.float64)))


def rel_fro(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.sqrt((want * want).sum())
    return float(np.sqrt(((got - want) ** 2).sum()) / den) if den > 0 else float(np.abs(got).max())


# -------------------------------------------------- reference (quant.h) access
def ref_dequant(W: np.ndarray, qtype: int, cols: int) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    rb = int(ref().ref_q_row_bytes(qtype, cols))
    rows = W.size // rb
    out = np.empty((rows, cols), np.float32)
    ref().ref_dequant_rows(_ptr(W, _u8p), qtype, cols, rows, _ptr(out, _f32p))
    return out


def ref_quantize(x: np.ndarray, qtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    rb = int(ref().ref_q_row_bytes(qtype, cols))
    out = np.zeros(rows * rb, np.uint8)
    if not ref().ref_quantize_rows(qtype, _ptr(x, _f32p), rows, cols, _ptr(out, _u8p)):
        raise ValueError("reference quantizer refused the type")
    return out.reshape(rows, rb)


def ref_gemv_threads(W: np.ndarray, qtype: int, x: np.ndarray, N: int, K: int, nthreads: int) -> np.ndarray:
    y = np.empty(N, np.float32)
    ref().ref_gemv_threads(_ptr(W, _u8p), qtype, int(ref().ref_q_row_bytes(qtype, K)), _ptr(x, _f32p),
                           _ptr(y, _f32p), N, K, nthreads)
    return y


def random_blocks(rng: np.random.Generator, qtype: int, nblocks: int, moderate: bool = False) -> np.ndarray:
    """Random block bytes with finite fp16 scale fields ~N(0,0.02), as check_quant.py:31-48 builds them;
    NF4/FP4 get an fp32 absmax ~N(0,0.02).  MXFP4's exponent byte is any byte (2^127 * 12 overflows, as
    in the reference), or with moderate=True one in [110, 130] for products that must stay finite."""
    be, bb = block(qtype)
    b = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    halfs = {Q4_0: [0], Q4_1: [0, 2], Q5_0: [0], Q5_1: [0, 2], Q8_0: [0], Q2_K: [80, 82], Q3_K: [108],
             Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208], IQ4_NL: [0], IQ4_XS: [0], TQ1_0: [52],
             TQ2_0: [64], IQ2_XXS: [0], IQ2_XS: [0], IQ2_S: [0], IQ3_XXS: [0], IQ3_S: [0],
             IQ1_S: [0]}.get(qtype, [])
    for o in halfs:
        h = (rng.standard_normal(nblocks) * 0.02).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
        b[:, o:o + 2] = h
    if qtype == IQ1_M:  # the fp16 d sits in the top nibbles of the four u16 scale words at 48
        h = (rng.standard_normal(nblocks) * 0.02).astype(np.float16).view(np.uint16).astype(np.uint32)
        for j in range(4):
            w = b[:, 48 + 2 * j].astype(np.uint32) | (b[:, 49 + 2 * j].astype(np.uint32) << 8)
            w = (w & 0x0fff) | (((h >> (4 * j)) & 15) << 12)
            b[:, 48 + 2 * j] = (w & 255).astype(np.uint8)
            b[:, 49 + 2 * j] = (w >> 8).astype(np.uint8)
    if qtype in (NF4, FP4):
        b[:, 0:4] = (rng.standard_normal(nblocks) * 0.02).astype(np.float32).view(np.uint8).reshape(nblocks, 4)
    if qtype == MXFP4 and moderate:
        b[:, 0] = rng.integers(110, 131, size=nblocks, dtype=np.uint8)
    return b

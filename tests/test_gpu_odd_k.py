"""GPU parity for operand lengths that are not whole steps of the kernels.

fp3gemm / chat_fp3 / bf3gemm / chat_bf3 (tier.cpp:900-943, 2165-2219) hand every
shape to hipBLASLt, which takes any k; the quantized GEMM takes dense rows of any
length (chat_lin's fp16/bf16/fp32 rows, tier.cpp:2360-2374).  Here K is not a
multiple of the 32-wide K step (K = 1000, 1001, 77), so the operands are padded
with zeros in the workspace.  Bars as the rest of the x3 tests: relative
Frobenius error <= 2^-20 against fp64 of fp16(W) * x (x3-ref; fp32 rows for
MODE_F32; bf16 weight values for the bf16 twins).

dq_k (tier.cpp:293-298) works one element per thread, so dense rows of any
length and any naturally aligned output are taken: bit-exact with the oracle.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20


def _w16(N, K, seed):
    w = (np.random.default_rng(seed).standard_normal((N, K)) * 0.02).astype(np.float32)
    bits = oracle.f2h(w).reshape(N, K)
    return bits, oracle.h2f_array(bits).reshape(N, K).astype(np.float64)


@pytest.mark.parametrize("K", [1000, 1001, 77])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_fp3gemm_forward_odd_k(gpu, K, beta):
    """fp3gemm(OP_T, m=N, n=M, k=K, W16, lda=K, x, beta, out, ldc=N)."""
    M, N = 300, 700
    bits, wf = _w16(N, K, K)
    x = activations(M, K, seed=K + 1)
    y0 = activations(M, N, seed=K + 2)
    A, B, C = hip.to_device(bits), hip.to_device(x), hip.to_device(y0)
    tier_amd.fp3gemm(tier_amd.OP_T, N, M, K, A.ptr, K, B.ptr, beta, C.ptr, N)
    hip.synchronize()
    got = C.download(np.float32, M * N).reshape(M, N)
    want = x.astype(np.float64) @ wf.T + beta * y0.astype(np.float64)
    assert oracle.rel_fro(got, want) <= BAR


@pytest.mark.parametrize("K", [1000, 999])
def test_fp3gemm_dx_odd_k(gpu, K):
    """fp3gemm(OP_N, m=K, n=M, k=N, W16 [N][K] with lda=K, dY [M][N]) -> dX [M][K], N odd."""
    M, N = 256, K
    Kx = 640  # the dX width (the weight's in_features)
    bits, wf = _w16(N, Kx, N)
    dy = activations(M, N, seed=N + 3)
    A, B, C = hip.to_device(bits), hip.to_device(dy), hip.DeviceBuffer(M * Kx * 4)
    tier_amd.fp3gemm(tier_amd.OP_N, Kx, M, N, A.ptr, Kx, B.ptr, 0.0, C.ptr, Kx)
    hip.synchronize()
    got = C.download(np.float32, M * Kx).reshape(M, Kx)
    assert oracle.rel_fro(got, dy.astype(np.float64) @ wf) <= BAR


@pytest.mark.parametrize("K", [1000, 1001])
def test_chat_fp3_odd_k(gpu, K):
    M, N, ldo = 40, 333, 340
    bits, wf = _w16(N, K, K + 5)
    x = activations(M, K, seed=K + 6)
    W, X, Y = hip.to_device(bits), hip.to_device(x), hip.DeviceBuffer(M * ldo * 4)
    Y.fill_bytes(0x3f)
    assert tier_amd.chat_fp3(W.ptr, X.ptr, Y.ptr, M, K, N, ldo)
    hip.synchronize()
    got = Y.download(np.float32, M * ldo).reshape(M, ldo)
    assert oracle.rel_fro(got[:, :N], x.astype(np.float64) @ wf.T) <= BAR
    assert np.all(got[:, N:].view(np.uint32) == 0x3f3f3f3f)


def test_bf16_twins_odd_k(gpu):
    """bf3gemm / chat_bf3 with K = 1000: bf16 weight, bf16 parts."""
    M, N, K = 64, 200, 1000
    w = (np.random.default_rng(9).standard_normal((N, K)) * 0.02).astype(np.float32)
    bits = oracle.f2bf(w).reshape(N, K)
    wf = (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = activations(M, K, seed=10)
    W, X = hip.to_device(bits), hip.to_device(x)
    Y1, Y2 = hip.DeviceBuffer(M * N * 4), hip.DeviceBuffer(M * N * 4)
    tier_amd.bf3gemm(tier_amd.OP_T, N, M, K, W.ptr, K, X.ptr, 0.0, Y1.ptr, N)
    assert tier_amd.chat_bf3(W.ptr, X.ptr, Y2.ptr, M, K, N, N)
    hip.synchronize()
    want = x.astype(np.float64) @ wf.T
    for Y in (Y1, Y2):
        assert oracle.rel_fro(Y.download(np.float32, M * N).reshape(M, N), want) <= BAR


@pytest.mark.parametrize("wtype", [tier_amd.F32, tier_amd.F16, tier_amd.BF16])
@pytest.mark.parametrize("mode", [tier_amd.MODE_X3REF, tier_amd.MODE_F32])
@pytest.mark.parametrize("K", [1000, 1001])
def test_qgemm_dense_rows_odd_k(gpu, wtype, mode, K):
    M, N = 200, 384
    rng = np.random.default_rng(K + wtype + mode)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bits = {tier_amd.F32: w, tier_amd.F16: oracle.f2h(w).reshape(N, K),
            tier_amd.BF16: oracle.f2bf(w).reshape(N, K)}[wtype]
    raw = np.ascontiguousarray(bits).view(np.uint8).reshape(N, -1)
    x = activations(M, K, seed=K + 7)
    W, X, Y = hip.to_device(raw), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, wtype, tier_amd.q_row_bytes(wtype, K), X.ptr, Y.ptr, M, N, K, mode=mode)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    if mode == tier_amd.MODE_F32:
        wref = oracle.dequant(raw, wtype, K).astype(np.float64)
    else:
        wref = oracle.h2f_array(oracle.dequant(raw, wtype, K, oracle.OUT_F16)).reshape(N, K).astype(np.float64)
    assert oracle.rel_fro(got, x.astype(np.float64) @ wref.T) <= BAR


@pytest.mark.parametrize("wtype", [tier_amd.F32, tier_amd.F16, tier_amd.BF16])
@pytest.mark.parametrize("out", [tier_amd.OUT_F32, tier_amd.OUT_F16, tier_amd.OUT_BF16])
@pytest.mark.parametrize("cols,offset", [(12, 0), (1001, 0), (1000, 4)])
def test_dequant_dense_any_length(gpu, wtype, out, cols, offset):
    """dq_k on dense rows of 12 and 1001 columns, and on 1000 columns into an output
    4 bytes past a 16-byte boundary: bit-exact, and nothing written outside the rows."""
    nrows, r0 = 9, 2
    rng = np.random.default_rng(cols + wtype * 10 + out)
    w = (rng.standard_normal((nrows + r0, cols)) * 3).astype(np.float32)
    bits = {tier_amd.F32: w, tier_amd.F16: oracle.f2h(w).reshape(-1, cols),
            tier_amd.BF16: oracle.f2bf(w).reshape(-1, cols)}[wtype]
    raw = np.ascontiguousarray(bits).view(np.uint8).reshape(nrows + r0, -1)
    esz = 4 if out == tier_amd.OUT_F32 else 2
    n = nrows * cols
    W = hip.to_device(raw)
    O = hip.DeviceBuffer(n * esz + 64)
    O.fill_bytes(0x5a)
    tier_amd.dq_launch(W.ptr, wtype, raw.shape[1], cols, r0, nrows, O.ptr + offset, out)
    hip.synchronize()
    got = O.download(np.uint8, n * esz + 64)
    want = oracle.dequant(raw, wtype, cols, out, r0, nrows).ravel()
    assert np.array_equal(got[offset:offset + n * esz].view(want.dtype), want)
    assert np.all(got[:offset] == 0x5a) and np.all(got[offset + n * esz:] == 0x5a)

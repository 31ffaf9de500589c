"""GPU parity of tiermm_sgemm, the fp32 product of the x3-off fallback (sgemm,
tier.cpp:773-865, called by low3_linear / linear / linear_dx / linear_dx_acc,
tier.cpp:1196-1200, 1213, 1229-1230, 1235-1236): relative Frobenius error <= 2^-20
against fp64(op(A) * B), in the BLAS column-major contract with opB = N."""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20


def run(opA, m, n, k, A, lda, B, ldb, C0, ldc, beta):
    dA, dB, dC = hip.to_device(A), hip.to_device(B), hip.to_device(C0)
    tier_amd.sgemm(opA, m, n, k, dA.ptr, lda, dB.ptr, ldb, beta, dC.ptr, ldc)
    hip.synchronize()
    return dC.download(np.float32, C0.size).reshape(C0.shape)


@pytest.mark.parametrize("beta", [0.0, 1.0])
@pytest.mark.parametrize("k", [200, 256])
def test_sgemm_forward_contract(gpu, beta, k):
    """sgemm(OP_T, OP_N, m=N, n=M, k=K, W, lda, x, ldb, beta, out, ldc): out[M][ldc] = x W^T (+ beta out),
    the forward linear on the expanded weight (tier.cpp:1213), strided A, B and C."""
    rng = np.random.default_rng(3)
    M, N, lda, ldb, ldc = 96, 320, k + 8, k + 4, 330
    w = (rng.standard_normal((N, lda)) * 0.02).astype(np.float32)
    x = activations(M, ldb, seed=4)
    c0 = rng.standard_normal((M, ldc)).astype(np.float32)
    got = run(tier_amd.OP_T, N, M, k, w, lda, x, ldb, c0, ldc, beta)
    ref = x[:, :k].astype(np.float64) @ w[:, :k].astype(np.float64).T + beta * c0[:, :N].astype(np.float64)
    assert oracle.rel_fro(got[:, :N], ref) <= BAR
    assert np.array_equal(got[:, N:], c0[:, N:])  # columns past m untouched


@pytest.mark.parametrize("beta", [0.0, 1.0])
@pytest.mark.parametrize("k", [320, 333])
def test_sgemm_dx_contract(gpu, beta, k):
    """sgemm(OP_N, OP_N, m=K, n=M, k=N, W, lda=K, dY, ldb=N, beta, dX, ldc=K): dX[M][K] = dY W (+ beta dX),
    linear_dx / linear_dx_acc on the expanded weight (tier.cpp:1229-1230, 1235-1236)."""
    rng = np.random.default_rng(5)
    M, K = 96, 200
    N = k
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    dy = activations(M, N, seed=6)
    dx0 = rng.standard_normal((M, K)).astype(np.float32)
    got = run(tier_amd.OP_N, K, M, N, w, K, dy, N, dx0, K, beta)
    ref = dy.astype(np.float64) @ w.astype(np.float64) + beta * dx0.astype(np.float64)
    assert oracle.rel_fro(got, ref) <= BAR


def test_sgemm_dx_column_scales(gpu):
    """OP_N with columns of the weight at very different scales, an all-zero column and a
    column past lda's used part: each output column (one exponent per weight column) is
    checked on its own."""
    rng = np.random.default_rng(7)
    M, N, K, lda = 64, 256, 192, 200
    w = (rng.standard_normal((N, lda)) * 0.02).astype(np.float32)
    w[:, 3] *= np.float32(1e-30)
    w[:, 5] *= np.float32(1e20)
    w[:, 7] = 0.0
    w[:, K:] = np.nan  # never read
    dy = activations(M, N, seed=8)
    got = run(tier_amd.OP_N, K, M, N, w, lda, dy, N, np.zeros((M, K), np.float32), K, 0.0)
    ref = dy.astype(np.float64) @ w[:, :K].astype(np.float64)
    for col in range(K):
        if col == 7:
            assert np.all(got[:, col] == 0.0)
        else:
            assert oracle.rel_fro(got[:, col], ref[:, col]) <= BAR, col


@pytest.mark.parametrize("name,N,K", [("q", 4096, 5120), ("kv", 1024, 5120), ("o", 5120, 4096),
                                      ("gate_up", 14336, 5120), ("down", 5120, 14336)])
def test_sgemm_config4_dx_shapes(gpu, name, N, K):
    """The dX products of BASELINE config 4's projections (W [N][K]) for 512 tokens, beta = 1 (the
    accumulate variant): dX = dY W + dX, 16 token rows checked in full against fp64."""
    rng = np.random.default_rng(N + K)
    M = 512
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    dy = activations(M, N, seed=9)
    dx0 = rng.standard_normal((M, K)).astype(np.float32)
    got = run(tier_amd.OP_N, K, M, N, w, K, dy, N, dx0, K, 1.0)
    rows = rng.choice(M, 16, replace=False)
    ref = dy[rows].astype(np.float64) @ w.astype(np.float64) + dx0[rows].astype(np.float64)
    assert oracle.rel_fro(got[rows], ref) <= BAR

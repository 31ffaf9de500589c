"""tiermm_qgemm_x3parts: tiermm_qgemm's x3-ref product (fp3gemm's three fp16 parts
of x, tier.cpp:922-943, against the fp16 dequant of W) on x split beforehand by
tiermm_split3_f16 (row-major planes) or tiermm_split3_f16_ktiled (K-tiled planes), so
that products reading the same activations share one split.

The fused kernel and the staged kernel sum the same MFMA products in the same order
whatever layout the x planes come in, so each result must equal tiermm_qgemm's on
the unsplit x bit for bit; one case is also held to 2^-20 against the fp64 product.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu


def _split(X, M, K, stride, layout):
    P = hip.DeviceBuffer(3 * stride * 2)
    if layout == tier_amd.PARTS_ROWS:
        tier_amd.split3(X.ptr, P.ptr, M * K, stride, tier_amd.HML)
    else:
        tier_amd.split3_ktiled(X.ptr, P.ptr, M, K, stride)
    return P


def _qgemm(W, t, X, M, N, K, y0=None, beta=0.0):
    Y = hip.to_device(y0) if y0 is not None else hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, beta=beta)
    return Y


def _parts(W, t, P, stride, M, N, K, layout, y0=None, beta=0.0):
    Y = hip.to_device(y0) if y0 is not None else hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm_x3parts(W.ptr, t, tier_amd.q_row_bytes(t, K), P.ptr, stride, Y.ptr, M, N, K, beta=beta,
                           layout=layout)
    return Y


def test_ktiled_split_is_a_permutation(gpu):
    """tiermm_split3_f16_ktiled writes tiermm_split3_f16's values, element (r, c) of each
    plane at ((c/32)*M + r)*32 + c%32."""
    M, K = 37, 96
    x = activations(M, K, seed=94)
    x[0, :4] = [0.0, -0.0, 1e-30, 7.0e4]
    X = hip.to_device(x)
    rows, tiled = _split(X, M, K, M * K + 8, tier_amd.PARTS_ROWS), _split(X, M, K, M * K + 8, tier_amd.PARTS_KTILED)
    hip.synchronize()
    a = rows.download(np.uint16).reshape(3, -1)[:, :M * K].reshape(3, M, K // 32, 32)
    b = tiled.download(np.uint16).reshape(3, -1)[:, :M * K].reshape(3, K // 32, M, 32)
    assert np.array_equal(a.transpose(0, 2, 1, 3), b)


@pytest.mark.parametrize("layout", [tier_amd.PARTS_ROWS, tier_amd.PARTS_KTILED])
@pytest.mark.parametrize("t", [tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K, tier_amd.Q8_0, tier_amd.Q5_0,
                               tier_amd.Q4_0, tier_amd.IQ4_XS])
def test_parts_equal_qgemm(gpu, t, layout):
    """Fused types (a split-K plan at this shape) and staged ones (q4_0, iq4_xs: the
    row-major planes on the small-tile kernel, the K-tiled ones on the big-tile kernel,
    with partial row and column tiles), beta = 1, planes padded apart (part_stride > M*K).
    Bit-identical with tiermm_qgemm, whose kernels sum the same products in the same
    order; the K-tiled staged case is a different kernel, so it is held to 2^-20."""
    M, N, K = 300, 1000, 1024
    rng = np.random.default_rng(90 + t)
    if t in (tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K, tier_amd.Q8_0):
        blocks = quantized_weight(t, N, K, seed=91 + t)
    else:
        blocks = oracle.random_blocks(rng, t, N * K // oracle.block(t)[0]).reshape(N, -1)
    x = activations(M, K, seed=92)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    W, X = hip.to_device(blocks), hip.to_device(x)
    stride = M * K + 40
    P = _split(X, M, K, stride, layout)
    a = _qgemm(W, t, X, M, N, K, y0, 1.0)
    b = _parts(W, t, P, stride, M, N, K, layout, y0, 1.0)
    hip.synchronize()
    ga, gb = a.download(np.float32, M * N), b.download(np.float32, M * N)
    staged_tiled = layout == tier_amd.PARTS_KTILED and t in (tier_amd.Q4_0, tier_amd.IQ4_XS)
    if not staged_tiled:
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))
    if t == tier_amd.Q4_K or staged_tiled:
        w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K).astype(np.float64)
        ref = x.astype(np.float64) @ w16.T + y0.astype(np.float64)
        assert oracle.rel_fro(gb.reshape(M, N), ref) <= 2.0 ** -20


def test_parts_shared_by_qkv(gpu):
    """Config 4's q, k and v projections (q4_K, q4_K, q5_K) from one K-tiled split of x."""
    M, K = 512, 5120
    x = activations(M, K, seed=93)
    X = hip.to_device(x)
    P = _split(X, M, K, M * K, tier_amd.PARTS_KTILED)
    for t, N in ((tier_amd.Q4_K, 4096), (tier_amd.Q4_K, 1024), (tier_amd.Q5_K, 1024)):
        W = hip.to_device(quantized_weight(t, N, K, seed=N + t))
        a, b = _qgemm(W, t, X, M, N, K), _parts(W, t, P, M * K, M, N, K, tier_amd.PARTS_KTILED)
        hip.synchronize()
        assert np.array_equal(a.download(np.uint32, M * N), b.download(np.uint32, M * N)), (t, N)

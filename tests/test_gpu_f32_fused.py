"""tiermm_qgemm's TIERMM_MODE_F32 (the chat prefill semantics, tier.cpp:2358-2359:
fp32 dequant of W, an fp32-accurate product) with the weight decoded inside the GEMM
for q4_K / q5_K / q6_K / q8_0 / q5_0, and the bounded-chunk expansion for the rest.

Each result is checked against the fp64 product of x with the oracle's fp32 dequant
(oracle.dequant(..., OUT_F32), pinned on the reference's golden vectors) to a relative
Frobenius error of 2^-20.  A product that dropped the lo parts (fp16 W or fp16 x)
misses that bar by orders of magnitude, so it separates the two-part split from a
plain fp16 GEMM.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20
FUSED = [("q4_K", tier_amd.Q4_K), ("q5_K", tier_amd.Q5_K), ("q6_K", tier_amd.Q6_K), ("q8_0", tier_amd.Q8_0),
         ("q5_0", tier_amd.Q5_0)]


def al256(n):
    return (n + 255) // 256 * 256


def fused_ws(M, N, K, ks):
    """Workspace of the fused fp32 path: x's hi and lo planes, both exponent rows, split-K partials."""
    return 2 * al256(M * K * 2) + al256(M * 4) + al256(N * 4) + (ks * M * N * 4 if ks > 1 else 0)


def run_f32(blocks, t, x, N, K, beta=0.0, y0=None):
    M = x.shape[0]
    W, X = hip.to_device(blocks), hip.to_device(x)
    Y = hip.to_device(y0) if y0 is not None else hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, mode=tier_amd.MODE_F32, beta=beta)
    hip.synchronize()
    return Y.download(np.float32, M * N).reshape(M, N)


def f32_weight(blocks, t, N, K):
    return oracle.dequant(blocks, t, K, oracle.OUT_F32).reshape(N, K).astype(np.float64)


@pytest.mark.parametrize("name,t", FUSED)
@pytest.mark.parametrize("bn,ks", [(160, 1), (128, 1), (64, 1), (160, 2), (128, 2), (64, 2), (160, 4), (128, 4),
                                   (64, 4)])
def test_f32_fused_plans(gpu, monkeypatch, name, t, bn, ks):
    """Every plan of the fp32 kernels on every fused type: partial M and N tiles, beta = 1,
    the split-K reduce, and the workspace query without any copy of W."""
    monkeypatch.setenv("TIERMM_QGEMM_TILE", f"{bn},{ks}")
    M, N, K = 300, 1000, 1024
    assert tier_amd.qgemm_ws_bytes(t, M, N, K, tier_amd.MODE_F32) == fused_ws(M, N, K, ks)
    blocks = quantized_weight(t, N, K, seed=bn + ks + t)
    x = activations(M, K, seed=7 + t)
    y0 = np.random.default_rng(bn * ks).standard_normal((M, N)).astype(np.float32)
    got = run_f32(blocks, t, x, N, K, beta=1.0, y0=y0)
    ref = x.astype(np.float64) @ f32_weight(blocks, t, N, K).T + y0.astype(np.float64)
    assert oracle.rel_fro(got, ref) <= BAR


# config 4's projections (q/k/o/gate/up q4_K, v q6_K, down q5_K or q6_K)
CONFIG4 = [("q", tier_amd.Q4_K, 5120, 5120), ("k", tier_amd.Q4_K, 1024, 5120), ("v", tier_amd.Q6_K, 1024, 5120),
           ("o", tier_amd.Q4_K, 5120, 4096), ("gate", tier_amd.Q4_K, 14336, 5120),
           ("down_q5", tier_amd.Q5_K, 5120, 14336), ("down_q6", tier_amd.Q6_K, 5120, 14336)]


@pytest.mark.parametrize("M", [256, 4096])
@pytest.mark.parametrize("name,t,N,K", CONFIG4)
def test_f32_config4(gpu, M, name, t, N, K):
    """The chat prefill product at its chunk size (M = 256, tier.cpp:2538) and at the
    config's 4096-token batch: decoded inside the GEMM (no fp32 W in the workspace),
    fp64-checked on every row at M = 256 and on 64 sampled rows at M = 4096."""
    # x's planes, both exponent rows and at most four K splits' partial sums: no copy of W
    assert tier_amd.qgemm_ws_bytes(t, M, N, K, tier_amd.MODE_F32) <= fused_ws(M, N, K, 4)
    blocks = quantized_weight(t, N, K, seed=N + K + t)
    x = activations(M, K, seed=M + t)
    got = run_f32(blocks, t, x, N, K)
    rows = np.arange(M) if M <= 256 else np.random.default_rng(3).choice(M, 64, replace=False)
    ref = x[rows].astype(np.float64) @ f32_weight(blocks, t, N, K).T
    assert oracle.rel_fro(got[rows], ref) <= BAR


def test_f32_unfused_chunks(gpu):
    """K beyond the fused fp32 kernels (q4_K, K = 32768) and a type they do not decode
    (q4_0): fp32 rows expanded 960 at a time (256 MiB of expansion), three chunks with
    the last one partial, written at their column offsets of Y."""
    M, K = 40, 32768
    for t, N in ((tier_amd.Q4_K, 2000), (tier_amd.Q4_0, 2000)):
        assert tier_amd.qgemm_plan(t, M, N, K) is None or t == tier_amd.Q4_K
        ws = tier_amd.qgemm_ws_bytes(t, M, N, K, tier_amd.MODE_F32)
        assert ws < 960 * K * 8 + 2 * al256(M * K * 2) + 2 * 4096  # one chunk of W rows, not N of them
        rng = np.random.default_rng(t)
        blocks = oracle.random_blocks(rng, t, N * K // oracle.block(t)[0]).reshape(N, -1)
        x = activations(M, K, seed=50 + t)
        got = run_f32(blocks, t, x, N, K)
        ref = x.astype(np.float64) @ f32_weight(blocks, t, N, K).T
        assert oracle.rel_fro(got, ref) <= BAR, t


def test_f32_padded_chunks(gpu):
    """Dense fp32 rows of an odd length (K = 33001, padded to 33024) over two chunks of
    rows: the padded path's bounded expansion."""
    M, N, K = 24, 1000, 33001
    rng = np.random.default_rng(61)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = activations(M, K, seed=62)
    got = run_f32(np.ascontiguousarray(w).view(np.uint8).reshape(N, -1), tier_amd.F32, x, N, K)
    assert oracle.rel_fro(got, x.astype(np.float64) @ w.astype(np.float64).T) <= BAR

"""GPU parity of tiermm_qgemv_batch: gemv_q (tier.cpp:299-306) of several matrices that
share x, K and the block type in one call.

Bar: bit for bit the outputs of tiermm_qgemv on each matrix alone (the batch runs the
same per-tile arithmetic, or falls back to those calls), and the usual GEMV bar of
relative Frobenius error <= 1e-5 against the fp64 product of the oracle's dequantization.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _alone(blocks, t, X, N, K):
    W = hip.to_device(blocks)
    Y = hip.DeviceBuffer(max(N, 1) * 4)
    Y.fill_bytes(0xff)
    tier_amd.gemv_q(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, N, K)
    hip.synchronize()
    return Y.download(np.float32, N)


def _batch(blist, t, X, Ns, K):
    Ws = [hip.to_device(b) for b in blist]
    Ys = [hip.DeviceBuffer(max(n, 1) * 4) for n in Ns]
    for y in Ys:
        y.fill_bytes(0xff)
    tier_amd.gemv_q_batch([w.ptr for w in Ws], t, tier_amd.q_row_bytes(t, K), X.ptr, [y.ptr for y in Ys], Ns, K)
    hip.synchronize()
    return [y.download(np.float32, n) for y, n in zip(Ys, Ns)]


CASES = [
    ("q4_K q+k", tier_amd.Q4_K, (4096, 1024), 5120),        # one layer's q and k projections
    ("q4_K gate+up", tier_amd.Q4_K, (14336, 14336), 5120),  # gate and up
    ("q4_K four", tier_amd.Q4_K, (1024, 2048, 1040, 3000), 4096),  # ragged rows, K = 4096
    ("q4_K one", tier_amd.Q4_K, (1032,), 5120),
    ("q5_K two", tier_amd.Q5_K, (1024, 1024), 5120),
    ("q4_K small (falls back)", tier_amd.Q4_K, (512, 4096), 5120),  # 32 tiles alone: per-wave kernel
    ("q4_K long rows (falls back)", tier_amd.Q4_K, (2048, 1024), 14336),
    ("q6_K (falls back)", tier_amd.Q6_K, (1024, 1024), 5120),
    ("q8_0 (falls back)", tier_amd.Q8_0, (1024, 4096), 4096),
]


@pytest.mark.parametrize("name,t,Ns,K", CASES, ids=[c[0] for c in CASES])
def test_batch_bit_identical_with_single_calls(gpu, name, t, Ns, K):
    blist = [quantized_weight(t, n, K, seed=K + 17 * i + n) for i, n in enumerate(Ns)]
    x = activations(1, K, seed=5)[0]
    X = hip.to_device(x)
    got = _batch(blist, t, X, list(Ns), K)
    for i, (b, n) in enumerate(zip(blist, Ns)):
        one = _alone(b, t, X, n, K)
        assert np.array_equal(got[i].view(np.uint32), one.view(np.uint32)), (name, i)
        assert oracle.rel_fro(got[i], oracle.gemv_f64(b, t, x, n, K)) <= TOL, (name, i)


def test_batch_rows_zero_and_nonfinite_x(gpu):
    """A matrix without rows takes no part (its null output is not touched); NaN and Inf in
    x give each matrix the rows tiermm_qgemv gives it alone (gemv_q's non-finite sums)."""
    t, K = tier_amd.Q4_K, 5120
    Ns = [2048, 0, 1024]
    blist = [quantized_weight(t, max(n, 16), K, seed=90 + i)[:n] for i, n in enumerate(Ns)]
    x = activations(1, K, seed=6)[0]
    x[7] = np.nan
    x[4000] = np.inf
    X = hip.to_device(x)
    live = [b for b, n in zip(blist, Ns) if n]
    Ws = [hip.to_device(b) for b in live]
    Ys = [hip.DeviceBuffer(n * 4) for n in Ns if n]
    tier_amd.gemv_q_batch([Ws[0].ptr, 0, Ws[1].ptr], t, tier_amd.q_row_bytes(t, K), X.ptr, [Ys[0].ptr, 0, Ys[1].ptr],
                          Ns, K)
    hip.synchronize()
    for b, n, Y in zip(live, [n for n in Ns if n], Ys):
        got = Y.download(np.float32, n)
        one = _alone(b, t, X, n, K)
        assert np.array_equal(got.view(np.uint32), one.view(np.uint32))


def test_batch_argument_checks(gpu):
    t, K = tier_amd.Q4_K, 5120
    X = hip.to_device(np.zeros(K, np.float32))
    W = hip.to_device(quantized_weight(t, 64, K, seed=1))
    Y = hip.DeviceBuffer(64 * 4)
    rb = tier_amd.q_row_bytes(t, K)
    with pytest.raises(tier_amd.TiermmError):  # more matrices than the batch holds
        tier_amd.gemv_q_batch([W.ptr] * 5, t, rb, X.ptr, [Y.ptr] * 5, [64] * 5, K)
    with pytest.raises(tier_amd.TiermmError):  # negative rows
        tier_amd.gemv_q_batch([W.ptr, W.ptr], t, rb, X.ptr, [Y.ptr, Y.ptr], [64, -1], K)
    with pytest.raises(tier_amd.TiermmError):  # rb of another K
        tier_amd.gemv_q_batch([W.ptr, W.ptr], t, rb + 144, X.ptr, [Y.ptr, Y.ptr], [64, 64], K)

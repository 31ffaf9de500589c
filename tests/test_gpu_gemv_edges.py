"""GPU parity of tiermm_qgemv / tiermm_gemv at the edges of gemv_q's contract
(tier.cpp:299-306, 2261-2268): non-finite activations and K above 16384.

Non-finite x.  gemv_q sums q_val * x in fp32, so a NaN anywhere in x makes every
y NaN, and +-Inf at column k makes row r +-Inf (sign of q_val(r, k) * x[k]) or
NaN (q_val(r, k) == 0, or terms of both signs).  The int8-digit kernels carry
finite x only and must still give that pattern; every kernel family is driven
here (whole-tile q4_K/q5_K, per-wave q4_K/q5_K/q8_0, q6_K, the staged 32-element
block kernel, the generic kernel).  Expected: the oracle's restatement of
gemv_q's own lane-order fp32 sum (orc_gemv_lanes), whose NaN / +Inf / -Inf
pattern must match exactly; the fp64 closed form (orc_gemv_f64) must agree with
it, which pins the pattern independently of the summation order.

Long K.  The reference loop has no K bound.  q4_K, q5_K and q8_0 rows up to
K = 28672 run on the int8-MFMA kernel (x digits of the whole row in 121 KiB of
LDS); q6_K above 14336 and the other types above 16384 on the generic kernel,
which reads x from global memory.  Bar: relative Frobenius error <= 1e-5 against
fp64.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _gemv(blocks, t, x, N, K):
    rb = tier_amd.q_row_bytes(t, K)
    assert blocks.nbytes == N * rb, (blocks.nbytes, N * rb)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(N * 4)
    Y.fill_bytes(0x3f)  # 0x3f3f3f3f is finite: a row left unwritten cannot pass for NaN
    tier_amd.gemv_q(W.ptr, t, rb, X.ptr, Y.ptr, N, K)
    hip.synchronize()
    return Y.download(np.float32, N)


def _classes(y):
    return np.isnan(y), np.isposinf(y), np.isneginf(y)


# (type, N, K): the kernel that serves each shape is named in the id
KERNELS = [
    (tier_amd.Q4_K, 13824, 5120, "q4K-whole-tile-4-tiles"),
    (tier_amd.Q4_K, 5120, 5120, "q4K-whole-tile-2-tiles"),
    (tier_amd.Q4_K, 1024, 14336, "q4K-whole-tile-k14336"),
    (tier_amd.Q4_K, 10240, 8192, "q4K-whole-tile-k8192"),
    (tier_amd.Q4_K, 512, 5120, "q4K-per-wave-1x4"),
    (tier_amd.Q4_K, 5120, 14336, "q4K-whole-tile-split-stages"),
    (tier_amd.Q4_K, 8192, 14336, "q4K-whole-tile-k14336-2-tiles"),
    (tier_amd.Q4_K, 9000, 14336, "q4K-per-wave-2x4"),
    (tier_amd.Q4_K, 512, 14336, "q4K-per-wave-1x8"),
    (tier_amd.Q5_K, 13824, 5120, "q5K-whole-tile"),
    (tier_amd.Q5_K, 1024, 5120, "q5K-whole-tile-1-tile"),
    (tier_amd.Q5_K, 512, 5120, "q5K-per-wave"),
    (tier_amd.Q5_K, 5120, 14336, "q5K-whole-tile-split-stages"),
    (tier_amd.Q5_K, 4096, 14336, "q5K-whole-tile-k14336"),
    (tier_amd.Q8_0, 4096, 4096, "q8_0-per-wave"),
    (tier_amd.Q8_0, 10240, 8192, "q8_0-per-wave-tall"),
    (tier_amd.Q6_K, 1024, 5120, "q6K"),
    (tier_amd.Q6_K, 5120, 14336, "q6K-long"),
    (tier_amd.Q4_0, 300, 4096, "q4_0-staged"),
    (tier_amd.Q5_1, 300, 4096, "q5_1-staged-min"),
    (tier_amd.Q2_K, 200, 1024, "q2K-generic"),
]


def _patterns(K):
    return {
        "nan": {7: np.nan},
        "pinf": {K // 3: np.inf},
        "pinf_ninf": {5: np.inf, K // 2 + 3: -np.inf},
        "ninf_nan": {K - 1: -np.inf, 100: np.nan},
    }


@pytest.mark.parametrize("t,N,K,kern", KERNELS, ids=[k[3] for k in KERNELS])
@pytest.mark.parametrize("pat", ["nan", "pinf", "pinf_ninf", "ninf_nan"])
def test_gemv_nonfinite_x(gpu, t, N, K, kern, pat):
    rng = np.random.default_rng(N + K + t)
    be, _ = oracle.block(t)
    if t in (tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K, tier_amd.Q8_0):
        blocks = quantized_weight(t, N, K, seed=N + K + t)
    else:
        blocks = oracle.random_blocks(rng, t, N * (K // be), moderate=True).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    for k, v in _patterns(K)[pat].items():
        x[k] = np.float32(v)
    y = _gemv(blocks, t, x, N, K)
    # the reference's own fp32 lane-order sum and the fp64 closed form agree on the classes
    want = oracle.gemv_lanes(blocks, t, x, N, K)
    closed = oracle.gemv_f64(blocks, t, x, N, K)
    for a, b in zip(_classes(want), _classes(closed)):
        assert np.array_equal(a, b)
    assert not np.any(np.isfinite(want))
    for name, a, b in zip(("nan", "+inf", "-inf"), _classes(y), _classes(want)):
        bad = np.nonzero(a != b)[0]
        assert bad.size == 0, f"{name} pattern differs at rows {bad[:8]} (of {bad.size})"


def test_gemv_nonfinite_single_column_signs(gpu):
    """+Inf in one column: each row takes the sign of its q_val there, NaN where q_val is 0
    (q8_0 codes of 0 give exact zeros); the three classes all occur."""
    t, N, K = tier_amd.Q8_0, 2048, 4096
    blocks = quantized_weight(t, N, K, seed=77)
    rng = np.random.default_rng(77)
    x = rng.standard_normal(K).astype(np.float32)
    c = 1234
    x[c] = np.float32(np.inf)
    y = _gemv(blocks, t, x, N, K)
    col = oracle.dequant(blocks, t, K)[:, c]
    assert np.array_equal(np.isposinf(y), col > 0)
    assert np.array_equal(np.isneginf(y), col < 0)
    assert np.array_equal(np.isnan(y), col == 0)
    assert (col == 0).any() and (col > 0).any() and (col < 0).any()


LONG = [(tier_amd.Q4_K, 1000, 20480), (tier_amd.Q4_K, 3000, 28672), (tier_amd.Q5_K, 1000, 28672),
        (tier_amd.Q6_K, 700, 20480), (tier_amd.Q8_0, 1000, 28672), (tier_amd.Q4_0, 600, 20480),
        (tier_amd.Q5_0, 300, 17408)]


@pytest.mark.parametrize("t,N,K", LONG, ids=[f"{tier_amd.TYPE_NAMES[c[0]]}-{c[1]}x{c[2]}" for c in LONG])
def test_gemv_k_above_16384(gpu, t, N, K):
    rng = np.random.default_rng(K + t)
    if t in (tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K, tier_amd.Q8_0):
        blocks = quantized_weight(t, N, K, seed=N + K)
    else:  # no quantizer in the reference: random blocks with finite fp16 scales
        blocks = oracle.random_blocks(rng, t, N * (K // oracle.block(t)[0]), moderate=True).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    assert np.all(np.isfinite(y))
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("wtype", [tier_amd.F32, tier_amd.F16, tier_amd.BF16])
@pytest.mark.parametrize("K", [20480, 28672, 16392])
def test_gemv_dense_k_above_16384(gpu, wtype, K):
    """gemv<T> rows longer than the LDS copy of x; K = 16392 also through gemv_q."""
    N = 333
    rng = np.random.default_rng(K + wtype)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bits = {tier_amd.F32: w, tier_amd.F16: oracle.f2h(w).reshape(N, K),
            tier_amd.BF16: oracle.f2bf(w).reshape(N, K)}[wtype]
    wf = oracle.dequant(np.ascontiguousarray(bits).view(np.uint8).reshape(N, -1), wtype, K).astype(np.float64)
    x = rng.standard_normal(K).astype(np.float32)
    W, X, Y = hip.to_device(bits), hip.to_device(x), hip.DeviceBuffer(N * 4)
    tier_amd.gemv(W.ptr, wtype, X.ptr, Y.ptr, N, K)
    hip.synchronize()
    want = wf @ x.astype(np.float64)
    assert oracle.rel_fro(Y.download(np.float32, N), want) <= TOL
    y2 = _gemv(np.ascontiguousarray(bits).view(np.uint8).reshape(N, -1), wtype, x, N, K)
    assert oracle.rel_fro(y2, want) <= TOL

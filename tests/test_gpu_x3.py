"""GPU parity of the split kernels and the x3 GEMMs.

Splits are bit-exact with the oracle.  GEMMs: relative Frobenius error <= 2^-20
against fp64 -- of X*W^T for the 2x2 variant, of
fp16(W)*X for x3-ref (fp3gemm / chat_fp3 / the quantized GEMM, whose weight is
the bit-exact fp16 dequantization).
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20


@pytest.mark.parametrize("tail", [5, 3])  # 70005 elements: per-element kernel; 70000: 8 per thread
def test_split3_bit_exact(gpu, tail):
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.uniform(-60000, 60000, 50000),
                        np.ldexp(rng.uniform(-1, 1, 20000), rng.integers(-40, 10, 20000)),
                        [0.0, -0.0, 65504.0, 65520.0, 1e-30]]).astype(np.float32)[:70000 + (tail == 5) * 5]
    n = x.size
    X = hip.to_device(x)
    for order, stride in ((tier_amd.HML, n), (tier_amd.LMH, n + 40)):
        P = hip.DeviceBuffer((2 * stride + n) * 2)
        P.fill_bytes(0)
        tier_amd.split3(X.ptr, P.ptr, n, stride, order)
        hip.synchronize()
        got = P.download(np.uint16, 2 * stride + n)
        want = oracle.split3(x, order, stride)
        for i in range(3):
            assert np.array_equal(got[i * stride:i * stride + n], want[i * stride:i * stride + n]), (order, i)


@pytest.mark.parametrize("cols", [1000, 1001, 5120, 8192, 14336, 20000])
def test_x3s_split_bit_exact(gpu, cols):
    """Rows held in registers (cols a multiple of 4, up to 16384) and the two-pass kernel."""
    rng = np.random.default_rng(12)
    v = (rng.standard_normal((9, cols)) * np.array([0.02, 1, 1e-6, 300, 0, 1e4, 2e-5, 5, 1e-30])[:, None])
    v = v.astype(np.float32)
    rows, cols = v.shape
    S = hip.to_device(v)
    H, L, E = hip.DeviceBuffer(v.size * 2), hip.DeviceBuffer(v.size * 2), hip.DeviceBuffer(rows * 4)
    tier_amd.x3s_split(S.ptr, H.ptr, L.ptr, E.ptr, rows, cols)
    hip.synchronize()
    hi, lo, ex = oracle.x3s_split(v)
    assert np.array_equal(E.download(np.int32, rows), ex)
    assert np.array_equal(H.download(np.uint16, v.size), hi.ravel())
    assert np.array_equal(L.download(np.uint16, v.size), lo.ravel())


def _x3s_gemm(X, W):
    M, K = X.shape
    N = W.shape[0]
    dX, dW = hip.to_device(X), hip.to_device(W)
    xh, xl, wh, wl = (hip.DeviceBuffer(a * K * 2) for a in (M, M, N, N))
    xe, we = hip.DeviceBuffer(M * 4), hip.DeviceBuffer(N * 4)
    Y = hip.DeviceBuffer(M * N * 4)
    tier_amd.x3s_split(dX.ptr, xh.ptr, xl.ptr, xe.ptr, M, K)
    tier_amd.x3s_split(dW.ptr, wh.ptr, wl.ptr, we.ptr, N, K)
    tier_amd.x3s_gemm(xh.ptr, xl.ptr, xe.ptr, wh.ptr, wl.ptr, we.ptr, Y.ptr, M, N, K)
    hip.synchronize()
    return Y.download(np.float32, M * N).reshape(M, N)


@pytest.mark.parametrize("M,N,K", [(256, 384, 1024), (130, 70, 320), (1, 5, 32), (512, 640, 5120)])
def test_x3s_gemm_vs_fp64(gpu, M, N, K):
    W = (np.random.default_rng(8).standard_normal((N, K)) * 0.02).astype(np.float32)
    X = activations(M, K, seed=9)
    Y = _x3s_gemm(X, W)
    ref = X.astype(np.float64) @ W.astype(np.float64).T
    assert oracle.rel_fro(Y, ref) <= BAR


def test_x3s_gemm_config2_sampled(gpu):
    """BASELINE config 2 at full size: W 5120x5120 ~N(0,0.02), X 4096x5120 ~N(0,1); fp64 on 192 sampled rows."""
    M, N, K = 4096, 5120, 5120
    W = (np.random.default_rng(8).standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float32)
    X = activations(M, K, seed=9)
    Y = _x3s_gemm(X, W)
    rows = np.random.default_rng(1).choice(M, 192, replace=False)
    ref = X[rows].astype(np.float64) @ W.astype(np.float64).T
    assert np.all(np.isfinite(Y))
    assert oracle.rel_fro(Y[rows], ref) <= BAR


def test_x3s_gemm_big_tiles_ragged(gpu):
    """Large enough for the 256x320-tile kernel, with partial tiles along M and N."""
    M, N, K = 4100, 5000, 640
    W = (np.random.default_rng(10).standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float32)
    X = activations(M, K, seed=11)
    Y = _x3s_gemm(X, W)
    rows = np.concatenate([np.arange(8), np.arange(M - 8, M), np.random.default_rng(2).choice(M, 112, replace=False)])
    ref = X[rows].astype(np.float64) @ W.astype(np.float64).T
    assert np.all(np.isfinite(Y))
    assert oracle.rel_fro(Y[rows], ref) <= BAR
    assert oracle.rel_fro(Y[rows][:, -7:], ref[:, -7:]) <= BAR


def _fp16(w):
    return oracle.h2f(oracle.f2h(w)).reshape(w.shape)


@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_fp3gemm_forward_contract(gpu, beta):
    """fp3gemm(OP_T, m=N, n=M, k=K, W16, lda=K, x, beta, C, ldc): out[M][ldc] = x W^T (+ beta*out)."""
    rng = np.random.default_rng(13)
    M, N, K, ldc = 192, 320, 768, 336
    w16 = oracle.f2h((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).reshape(N, K)
    x = activations(M, K, seed=14)
    c0 = rng.standard_normal((M, ldc)).astype(np.float32)
    A, B, C = hip.to_device(w16), hip.to_device(x), hip.to_device(c0)
    tier_amd.fp3gemm(tier_amd.OP_T, N, M, K, A.ptr, K, B.ptr, beta, C.ptr, ldc)
    hip.synchronize()
    got = C.download(np.float32, M * ldc).reshape(M, ldc)
    ref = x.astype(np.float64) @ oracle.h2f(w16).reshape(N, K).astype(np.float64).T + beta * c0[:, :N]
    assert oracle.rel_fro(got[:, :N], ref) <= BAR
    assert np.array_equal(got[:, N:], c0[:, N:])  # columns past m untouched


def test_chat_fp3_rows(gpu):
    rng = np.random.default_rng(15)
    M, N, K, ldo = 100, 200, 1024, 256
    w16 = oracle.f2h((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).reshape(N, K)
    x = activations(M, K, seed=16)
    A, B, Y = hip.to_device(w16), hip.to_device(x), hip.DeviceBuffer(M * ldo * 4)
    assert tier_amd.chat_fp3(A.ptr, B.ptr, Y.ptr, M, K, N, ldo)
    hip.synchronize()
    got = Y.download(np.float32, M * ldo).reshape(M, ldo)[:, :N]
    ref = x.astype(np.float64) @ oracle.h2f(w16).reshape(N, K).astype(np.float64).T
    assert oracle.rel_fro(got, ref) <= BAR


QG = [("q4_K", tier_amd.Q4_K, 96, 640, 1024), ("q8_0", tier_amd.Q8_0, 64, 256, 512),
      ("q5_K", tier_amd.Q5_K, 64, 128, 768), ("q6_K", tier_amd.Q6_K, 33, 100, 512),
      ("q5_0", tier_amd.Q5_0, 40, 64, 1408)]


@pytest.mark.parametrize("name,t,M,N,K", QG, ids=[c[0] for c in QG])
def test_qgemm_x3ref(gpu, name, t, M, N, K):
    blocks = quantized_weight(t, N, K, seed=20 + t)
    x = activations(M, K, seed=21)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T
    assert oracle.rel_fro(got, ref) <= BAR


@pytest.mark.parametrize("t,beta,M", [(tier_amd.Q4_0, 0.0, 4096), (tier_amd.Q3_K, 1.0, 4000),
                                      (tier_amd.IQ4_XS, 0.0, 4096), (tier_amd.Q4_K, 0.0, 4096),
                                      (tier_amd.Q5_K, 1.0, 4000), (tier_amd.Q6_K, 0.0, 4096)])
def test_qgemm_big_tiles_k_tiled_planes(gpu, t, beta, M):
    """Large M: a partial last column tile, beta = 1; an x that is only 4-byte aligned
    takes row-major planes instead of K-tiled ones, and both give the same bits (M = 4000:
    a partial last row tile too).  q4_0, q3_K and IQ4_XS go through fp16 staging and the
    big-tile x3-ref GEMM; q4_K, q5_K and q6_K through the fused kernel's wide tiles."""
    N, K = 4000, 512
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(np.random.default_rng(40 + t), t, N * (K // be)).reshape(N, -1)
    x = activations(M, K, seed=41)
    y0 = np.random.default_rng(42).standard_normal((M, N)).astype(np.float32)
    W = hip.to_device(blocks)
    X = hip.to_device(x)
    Xu = hip.DeviceBuffer(x.nbytes + 16).upload(x, offset=4)
    Y, Yu = hip.to_device(y0), hip.to_device(y0)
    rb = tier_amd.q_row_bytes(t, K)
    tier_amd.qgemm(W.ptr, t, rb, X.ptr, Y.ptr, M, N, K, beta=beta)
    tier_amd.qgemm(W.ptr, t, rb, Xu.ptr + 4, Yu.ptr, M, N, K, beta=beta)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    got_u = Yu.download(np.float32, M * N).reshape(M, N)
    assert np.array_equal(got.view(np.uint32), got_u.view(np.uint32))
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T + beta * y0.astype(np.float64)
    assert oracle.rel_fro(got, ref) <= BAR


@pytest.mark.parametrize("M,N,K,beta", [(130, 100, 768, 0.0), (1, 50, 256, 0.0), (257, 1000, 2048, 1.0),
                                         (512, 5120, 1024, 0.0)])
def test_qgemm_q4k_fused_shapes(gpu, M, N, K, beta):
    """The fused q4_K kernel: partial tiles along M and N, one-row and one-super-block
    cases, beta = 1 accumulation, random blocks with extreme scale fields."""
    t = tier_amd.Q4_K
    rng = np.random.default_rng(M + N + K)
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = activations(M, K, seed=22)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.to_device(y0)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, beta=beta)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T + beta * y0.astype(np.float64)
    assert np.all(np.isfinite(got))
    assert oracle.rel_fro(got, ref) <= BAR


# Types the fused kernel decodes, with a K whose rows are only 2-byte aligned where the
# block size allows it (q6_K 768: 630-byte rows; q8_0 / q5_0 480: 510 / 330-byte rows).
FUSED = [("q4_K", tier_amd.Q4_K, 512), ("q5_K", tier_amd.Q5_K, 512), ("q6_K", tier_amd.Q6_K, 768),
         ("q8_0", tier_amd.Q8_0, 480), ("q5_0", tier_amd.Q5_0, 480)]


@pytest.mark.parametrize("name,t,K", FUSED, ids=[f[0] for f in FUSED])
@pytest.mark.parametrize("bn", [160, 128, 64])
@pytest.mark.parametrize("scale", ["0.02", "60", "tiny"])
def test_qgemm_fused_decode_bit_exact(gpu, monkeypatch, name, t, K, bn, scale):
    """One-hot rows of x read the fused kernel's fp16 weights back: row m of x is e_m, so
    Y[m][n] = W16[n][m] exactly (one non-zero product per sum).  This pins the in-kernel
    decode -- q_val, then fp16 round-to-nearest-even -- bit for bit against the oracle,
    for each type and decode layout (one lane per row at BN = 160, two at BN <= 128),
    with weights from fp16 subnormals up to values in the thousands (q5_0, which has no
    quantizer: random blocks with d ~N(0, 0.02))."""
    monkeypatch.setenv("TIERMM_QGEMM_TILE", f"{bn},1")
    N = 352
    # tiny: mostly fp16 subnormal weights (q6_K's fp16 d would itself underflow at 2e-6)
    sigma = {"0.02": 0.02, "60": 60.0, "tiny": 5e-5 if t == tier_amd.Q6_K else 2e-6}[scale]
    blocks = quantized_weight(t, N, K, seed=46, sigma=sigma)
    x = np.eye(K, dtype=np.float32)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(K * N * 4)
    rb = tier_amd.q_row_bytes(t, K)
    assert tier_amd.qgemm_ws_bytes(t, K, N, K) == 3 * K * K * 2  # the fused plan: no fp16 W in the workspace
    tier_amd.qgemm(W.ptr, t, rb, X.ptr, Y.ptr, K, N, K)
    hip.synchronize()
    got = Y.download(np.float32, K * N).reshape(K, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    assert np.all(np.isfinite(w16)) and np.count_nonzero(w16) > 0
    assert np.array_equal(got, w16.T)  # +0 and -0 compare equal: a zero weight sums to +0


TYPE_PLANS = [(256, 1), (224, 2), (160, 1), (160, 2), (128, 4), (64, 1), (64, 4)]


@pytest.mark.parametrize("name,t", [(f[0], f[1]) for f in FUSED[1:]], ids=[f[0] for f in FUSED[1:]])
@pytest.mark.parametrize("bn,ks", TYPE_PLANS)
def test_qgemm_fused_type_plans(gpu, monkeypatch, name, t, bn, ks):
    """The fused kernel on q5_K, q6_K, q8_0 and q5_0 weights at every tile width and
    split-K factor it takes: partial M and N tiles, beta = 1, K split into units of
    each type's producer (q6_K: quarter super-blocks)."""
    monkeypatch.setenv("TIERMM_QGEMM_TILE", f"{bn},{ks}")
    M, N, K, beta = 300, 1000, 1024, 1.0
    assert tier_amd.qgemm_ws_bytes(t, M, N, K) == 3 * M * K * 2 + (ks * M * N * 4 if ks > 1 else 0)
    rng = np.random.default_rng(M + N + K + bn + ks + t)
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(rng, t, N * (K // be)).reshape(N, -1)
    x = activations(M, K, seed=25)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.to_device(y0)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, beta=beta)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T + beta * y0.astype(np.float64)
    assert np.all(np.isfinite(got))
    assert oracle.rel_fro(got, ref) <= BAR


@pytest.mark.parametrize("plan", ["128,1,2", "256,2", "160,1,2", "default"])
@pytest.mark.parametrize("t", [tier_amd.Q4_K, tier_amd.Q6_K])
def test_qgemm_fused_k_chunks(gpu, monkeypatch, t, plan):
    """K = 8192, beyond one accumulator's 6144: two K chunks, either launched in turn with
    the second adding into Y (BN,1,2) or as two splits with partial sums (BN,2); beta = 1
    on top of both."""
    if plan != "default":
        monkeypatch.setenv("TIERMM_QGEMM_TILE", plan)
    M, N, K, beta = 300, 1000, 8192, 1.0
    ks = int(plan.split(",")[1]) if plan != "default" else None
    if ks is not None:
        assert tier_amd.qgemm_ws_bytes(t, M, N, K) == 3 * M * K * 2 + (ks * M * N * 4 if ks > 1 else 0)
        want = tuple(int(v) for v in plan.split(",")) + ((1,) if plan.count(",") == 1 else ())
        assert tier_amd.qgemm_plan(t, M, N, K) == want  # the forced plan is the one run
    rng = np.random.default_rng(K + t + len(plan))
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = activations(M, K, seed=27)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.to_device(y0)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, beta=beta)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T + beta * y0.astype(np.float64)
    assert oracle.rel_fro(got, ref) <= BAR


@pytest.mark.parametrize("name,t,K", [("q8_0", tier_amd.Q8_0, 1408), ("q5_0", tier_amd.Q5_0, 1408),
                                      ("q8_0_k96", tier_amd.Q8_0, 96), ("q6_K_k256", tier_amd.Q6_K, 256)],
                         ids=lambda v: v if isinstance(v, str) else None)
@pytest.mark.parametrize("M", [1, 257])
def test_qgemm_fused_odd_k(gpu, name, t, K, M):
    """K that is not a multiple of 256 (the MoE down projection's 1408; three q8_0
    blocks) or a single q6_K super-block with 2-byte aligned rows, through the default
    plan: every row of x, every partial tile."""
    N = 200
    rng = np.random.default_rng(K + M + t)
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(rng, t, N * (K // be)).reshape(N, -1)
    x = activations(M, K, seed=26)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    assert oracle.rel_fro(got, x.astype(np.float64) @ w16.astype(np.float64).T) <= BAR


@pytest.mark.parametrize("M,N,K", [(130, 100, 768), (512, 1000, 2048)])
def test_qgemm_q4k_fused_x_layouts(gpu, M, N, K):
    """x at a 16-byte aligned address is split into K-tiled planes, x 4 bytes past one
    into row-major planes: the fused q4_K kernel gives bit-identical results from both,
    within the fp64 bar."""
    t = tier_amd.Q4_K
    rng = np.random.default_rng(3 * M + N)
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = activations(M, K, seed=24)
    W, X = hip.to_device(blocks), hip.to_device(x)
    Xu = hip.DeviceBuffer(M * K * 4 + 16)
    Xu.upload(x, offset=4)
    Y, Yu = hip.DeviceBuffer(M * N * 4), hip.DeviceBuffer(M * N * 4)
    rb = tier_amd.q_row_bytes(t, K)
    tier_amd.qgemm(W.ptr, t, rb, X.ptr, Y.ptr, M, N, K)
    tier_amd.qgemm(W.ptr, t, rb, Xu.ptr + 4, Yu.ptr, M, N, K)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    got_u = Yu.download(np.float32, M * N).reshape(M, N)
    assert np.array_equal(got.view(np.uint32), got_u.view(np.uint32))
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    assert oracle.rel_fro(got, x.astype(np.float64) @ w16.astype(np.float64).T) <= BAR


@pytest.mark.parametrize("bn,ks", [(256, 1), (256, 4), (224, 2), (192, 1), (160, 1), (160, 2), (160, 4), (128, 2),
                                   (112, 4), (96, 2), (80, 4), (64, 2), (64, 1)])
@pytest.mark.parametrize("M,N,K,beta", [(300, 1000, 1024, 1.0), (512, 352, 2048, 0.0), (130, 998, 1024, 1.0)])
def test_qgemm_q4k_tile_plans(gpu, monkeypatch, bn, ks, M, N, K, beta):
    """Every tile width and split-K factor of the fused q4_K kernel, forced through
    TIERMM_QGEMM_TILE: partial M and N tiles, the split-K reduce with beta = 1 (four
    columns a thread, and one at N = 998), and the workspace query sized for the partial
    sums."""
    monkeypatch.setenv("TIERMM_QGEMM_TILE", f"{bn},{ks}")
    t = tier_amd.Q4_K
    assert tier_amd.qgemm_ws_bytes(t, M, N, K) == 3 * M * K * 2 + (ks * M * N * 4 if ks > 1 else 0)
    rng = np.random.default_rng(M + N + K + bn + ks)
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = activations(M, K, seed=23)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.to_device(y0)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, beta=beta)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T + beta * y0.astype(np.float64)
    assert np.all(np.isfinite(got))
    assert oracle.rel_fro(got, ref) <= BAR


def test_qgemm_split_k_padded_rows(gpu, monkeypatch):
    """Split-K into an output with padded rows (ldy > N) and beta = 1: the reduce keeps
    the padding untouched and accumulates into the rows."""
    monkeypatch.setenv("TIERMM_QGEMM_TILE", "160,4")
    t, M, N, K, ldy = tier_amd.Q4_K, 200, 336, 1024, 352
    rng = np.random.default_rng(44)
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = activations(M, K, seed=45)
    y0 = rng.standard_normal((M, ldy)).astype(np.float32)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.to_device(y0)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, ldy=ldy, beta=1.0)
    hip.synchronize()
    got = Y.download(np.float32, M * ldy).reshape(M, ldy)
    assert np.array_equal(got[:, N:], y0[:, N:])
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x.astype(np.float64) @ w16.astype(np.float64).T + y0[:, :N].astype(np.float64)
    assert oracle.rel_fro(got[:, :N], ref) <= BAR


@pytest.mark.parametrize("N,K", [(5120, 5120), (5120, 14336)])
def test_qgemm_m512_split_k_sampled(gpu, N, K):
    """Config 3 shapes whose default plan splits K (wide tiles, two splits and the reduce);
    fp64 check on sampled output rows."""
    t, M = tier_amd.Q4_K, 512
    blocks = quantized_weight(t, N, K, seed=35)
    x = activations(M, K, seed=36)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    rows = np.random.default_rng(3).choice(M, 48, replace=False)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x[rows].astype(np.float64) @ w16.astype(np.float64).T
    assert np.all(np.isfinite(got))
    assert oracle.rel_fro(got[rows], ref) <= BAR


def test_qgemm_config3_m512_sampled(gpu):
    """Config 3 prefill: q4_K 14336x5120 at M=512; fp64 check on sampled output rows."""
    t, M, N, K = tier_amd.Q4_K, 512, 14336, 5120
    blocks = quantized_weight(t, N, K, seed=33)
    x = activations(M, K, seed=34)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    rows = np.random.default_rng(2).choice(M, 48, replace=False)
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K)
    ref = x[rows].astype(np.float64) @ w16.astype(np.float64).T
    assert oracle.rel_fro(got[rows], ref) <= BAR


@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_fp3gemm_dx_contract(gpu, beta):
    """fp3gemm(OP_N, m=K, n=M, k=N, W16, lda=K, dY, beta, dX, ldc=K): dX[M][K] = dY W16 (+ beta*dX),
    the linear_dx / linear_dx_acc products (tier.cpp:1226, 1234)."""
    rng = np.random.default_rng(17)
    M, N, K = 96, 320, 200
    w16 = oracle.f2h((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).reshape(N, K)
    dy = activations(M, N, seed=18)
    dx0 = rng.standard_normal((M, K)).astype(np.float32)
    A, B, C = hip.to_device(w16), hip.to_device(dy), hip.to_device(dx0)
    tier_amd.fp3gemm(tier_amd.OP_N, K, M, N, A.ptr, K, B.ptr, beta, C.ptr, K)
    hip.synchronize()
    got = C.download(np.float32, M * K).reshape(M, K)
    ref = dy.astype(np.float64) @ oracle.h2f(w16).reshape(N, K).astype(np.float64) + beta * dx0.astype(np.float64)
    assert oracle.rel_fro(got, ref) <= BAR


@pytest.mark.parametrize("name,t,M,N,K", [("q4_K", tier_amd.Q4_K, 70, 300, 1024), ("q6_K", tier_amd.Q6_K, 33, 64, 512),
                                          ("q8_0", tier_amd.Q8_0, 300, 640, 1024)])
def test_qgemm_f32_mode(gpu, name, t, M, N, K):
    """TIERMM_MODE_F32 (chat prefill, tier.cpp:2358-2359): fp32 dequant times x, against fp64."""
    blocks = quantized_weight(t, N, K, seed=40 + t)
    x = activations(M, K, seed=41)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, mode=tier_amd.MODE_F32)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    wf = oracle.dequant(blocks, t, K, oracle.OUT_F32).reshape(N, K)
    assert oracle.rel_fro(got, x.astype(np.float64) @ wf.astype(np.float64).T) <= BAR


@pytest.mark.parametrize("t", [tier_amd.Q4_0, tier_amd.Q4_1, tier_amd.Q5_1, tier_amd.F32, tier_amd.F16, tier_amd.BF16,
                               tier_amd.Q3_K, tier_amd.IQ4_XS, tier_amd.NF4, tier_amd.IQ2_XS, tier_amd.IQ3_S,
                               tier_amd.IQ1_M])
@pytest.mark.parametrize("mode", [tier_amd.MODE_X3REF, tier_amd.MODE_F32])
def test_qgemm_more_types(gpu, t, mode):
    """The legacy 32-blocks and dense rows through tiermm_qgemm, both semantics, against fp64."""
    rng = np.random.default_rng(80 + t)
    M, N, K = 45, 160, 768
    if t in (tier_amd.F32, tier_amd.F16, tier_amd.BF16):
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        bits = {tier_amd.F32: w, tier_amd.F16: oracle.f2h(w), tier_amd.BF16: oracle.f2bf(w)}[t]
        blocks = np.ascontiguousarray(bits).view(np.uint8).reshape(N, -1)
    else:
        blocks = oracle.random_blocks(rng, t, N * K // oracle.block(t)[0]).reshape(N, -1)
    x = activations(M, K, seed=81)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, M, N, K, mode=mode)
    hip.synchronize()
    got = Y.download(np.float32, M * N).reshape(M, N)
    out = oracle.OUT_F16 if mode == tier_amd.MODE_X3REF else oracle.OUT_F32
    wd = oracle.dequant(blocks, t, K, out)
    wd = (oracle.h2f(wd) if out == oracle.OUT_F16 else wd).reshape(N, K)
    assert oracle.rel_fro(got, x.astype(np.float64) @ wd.astype(np.float64).T) <= BAR


def _bf16(w):
    return oracle.f2bf(np.ascontiguousarray(w, np.float32)).reshape(w.shape)


def _bf16_to_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_split3_bf16_bit_exact(gpu):
    """split3_k / split3s (tier.cpp:866-867, 2159-2161): hip_bfloat16 rounding of v, v - h, v - h - m."""
    rng = np.random.default_rng(23)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 1e-30, -7.5e4, 3.0e38], np.float32)])
    _split3_bf16_case(x)                         # 5005 elements: the per-element kernel
    _split3_bf16_case(np.concatenate([x[:4995], x[-5:]]))  # 5000: eight elements per thread


def _split3_bf16_case(x):
    n = x.size
    X, P = hip.to_device(x), hip.DeviceBuffer(3 * n * 2)
    for order in (tier_amd.HML, tier_amd.LMH):
        tier_amd.split3_bf16(X.ptr, P.ptr, n, n, order)
        hip.synchronize()
        got = P.download(np.uint16, 3 * n).reshape(3, n)
        h = _bf16(x)
        r = x - (h.astype(np.uint32) << 16).view(np.float32)
        m = _bf16(r)
        l = _bf16(r - (m.astype(np.uint32) << 16).view(np.float32))
        want = np.stack([h, m, l]) if order == tier_amd.HML else np.stack([l, m, h])
        assert np.array_equal(got, want)


@pytest.mark.parametrize("opA", [tier_amd.OP_T, tier_amd.OP_N])
def test_bf3gemm_contract(gpu, opA):
    """bf3gemm (tier.cpp:900-921): the fp3gemm contract with bf16 storage, forward (OP_T) and dX (OP_N)."""
    rng = np.random.default_rng(29)
    M, N, K = 130, 256, 320
    w16 = _bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    if opA == tier_amd.OP_T:  # out[M][N] = x W^T
        x = activations(M, K, seed=30)
        A, B, C = hip.to_device(w16), hip.to_device(x), hip.DeviceBuffer(M * N * 4)
        tier_amd.bf3gemm(opA, N, M, K, A.ptr, K, B.ptr, 0.0, C.ptr, N)
        ref = x.astype(np.float64) @ _bf16_to_f64(w16).T
        shape = (M, N)
    else:  # dX[M][K] = dY W
        dy = activations(M, N, seed=31)
        A, B, C = hip.to_device(w16), hip.to_device(dy), hip.DeviceBuffer(M * K * 4)
        tier_amd.bf3gemm(opA, K, M, N, A.ptr, K, B.ptr, 0.0, C.ptr, K)
        ref = dy.astype(np.float64) @ _bf16_to_f64(w16)
        shape = (M, K)
    hip.synchronize()
    got = C.download(np.float32, shape[0] * shape[1]).reshape(shape)
    assert oracle.rel_fro(got, ref) <= BAR


def test_chat_bf3_rows(gpu):
    rng = np.random.default_rng(33)
    M, N, K, ldo = 64, 200, 1024, 208
    w16 = _bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x = activations(M, K, seed=34)
    A, B, Y = hip.to_device(w16), hip.to_device(x), hip.DeviceBuffer(M * ldo * 4)
    assert tier_amd.chat_bf3(A.ptr, B.ptr, Y.ptr, M, K, N, ldo)
    hip.synchronize()
    got = Y.download(np.float32, M * ldo).reshape(M, ldo)[:, :N]
    assert oracle.rel_fro(got, x.astype(np.float64) @ _bf16_to_f64(w16).T) <= BAR


def _dx_case(m, n, k, lda, beta, seed, bf16=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, m)) * 0.02).astype(np.float32)
    w16 = np.zeros((k, lda), np.uint16)
    w16[:, :m] = (_bf16(w) if bf16 else oracle.f2h(w).reshape(k, m))
    dy = activations(n, k, seed=seed + 1)
    dx0 = rng.standard_normal((n, m)).astype(np.float32)
    A, B, C = hip.to_device(w16), hip.to_device(dy), hip.to_device(dx0)
    (tier_amd.bf3gemm if bf16 else tier_amd.fp3gemm)(tier_amd.OP_N, m, n, k, A.ptr, lda, B.ptr, beta, C.ptr, m)
    hip.synchronize()
    return C.download(np.float32, n * m).reshape(n, m), w16, dy, dx0


@pytest.mark.parametrize("beta", [0.0, 1.0])
@pytest.mark.parametrize("name,m,k,bf16", [("q", 5120, 4096, False), ("gate", 5120, 14336, False),
                                           ("down", 14336, 5120, False), ("ragged", 4104, 2080, False),
                                           ("q_bf16", 5120, 4096, True)])
def test_x3_gemm_dx_in_place(gpu, name, m, k, bf16, beta):
    """The dX product (linear_dx / linear_dx_acc, tier.cpp:1226, 1234) at config 4's shapes
    (4096 tokens; W[k][m] in memory), fp16 (fp3gemm) and bf16 (bf3gemm): the big-tile kernel
    reads W in place (TR), with K in accumulation chunks at k = 14336 and partial column
    tiles at m = 4104.  Bit-identical with the transpose-first path (the same W with
    lda = m + 4, which the in-place read does not take), and within 2^-20 of fp64 on 64
    sampled rows."""
    n = 4096
    got, w16, dy, dx0 = _dx_case(m, n, k, m, beta, m + k, bf16)
    ref_t, _, _, _ = _dx_case(m, n, k, m + 4, beta, m + k, bf16)
    assert np.array_equal(got.view(np.uint32), ref_t.view(np.uint32))
    rows = np.random.default_rng(5).choice(n, 64, replace=False)
    wm = np.ascontiguousarray(w16[:, :m])
    wf = (_bf16_to_f64(wm) if bf16 else oracle.h2f(wm.ravel()).reshape(k, m).astype(np.float64))
    ref = dy[rows].astype(np.float64) @ wf + beta * dx0[rows].astype(np.float64)
    assert oracle.rel_fro(got[rows], ref) <= BAR

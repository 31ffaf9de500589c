"""GPU parity of tiermm_qgemv (gemv_q, tier.cpp:299-306).

Bar: relative Frobenius error <= 1e-5 against the fp64 product of the oracle's
fp32 dequantization with x (BASELINE config 1 states y rel-err <= 1e-5; the
reference's own lane-strided fp32 GEMV sits near 1e-7 of fp64).
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _gemv(blocks, t, x, N, K):
    rb = tier_amd.q_row_bytes(t, K)
    # the kernel reads N * rb bytes: a short host array is a test bug, stopped before the launch
    assert blocks.nbytes == N * rb, (blocks.nbytes, N * rb)
    W = hip.to_device(blocks)
    X = hip.to_device(x)
    Y = hip.DeviceBuffer(N * 4)
    Y.fill_bytes(0xff)
    tier_amd.gemv_q(W.ptr, t, rb, X.ptr, Y.ptr, N, K)
    hip.synchronize()
    return Y.download(np.float32, N)


CASES = [
    ("q8_0", tier_amd.Q8_0, 4096, 4096),      # config 1
    ("q4_K", tier_amd.Q4_K, 13824, 5120),     # north-star GEMV
    ("q4_K", tier_amd.Q4_K, 5120, 5120),      # config 3 shapes
    ("q4_K", tier_amd.Q4_K, 14336, 5120),
    ("q4_K", tier_amd.Q4_K, 5120, 14336),
    ("q5_K", tier_amd.Q5_K, 1024, 5120),      # config 4 v_proj / down_proj types
    ("q5_K", tier_amd.Q5_K, 5120, 14336),
    ("q6_K", tier_amd.Q6_K, 1024, 5120),
    ("q6_K", tier_amd.Q6_K, 5120, 14336),
    ("q5_0", tier_amd.Q5_0, 2048, 1408),      # MoE down_proj fallback type
]


@pytest.mark.parametrize("name,t,N,K", CASES, ids=[f"{c[0]}-{c[2]}x{c[3]}" for c in CASES])
def test_gemv_config_shapes(gpu, name, t, N, K):
    blocks = quantized_weight(t, N, K, seed=N + K + t)
    x = activations(1, K, seed=2)[0]
    y = _gemv(blocks, t, x, N, K)
    want = oracle.gemv_f64(blocks, t, x, N, K)
    assert np.all(np.isfinite(y))
    assert oracle.rel_fro(y, want) <= TOL


@pytest.mark.parametrize("t", [tier_amd.Q8_0, tier_amd.Q5_0, tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K,
                               tier_amd.Q4_0, tier_amd.Q4_1, tier_amd.Q5_1, tier_amd.Q2_K, tier_amd.Q3_K,
                               tier_amd.IQ4_NL, tier_amd.IQ4_XS, tier_amd.TQ1_0, tier_amd.TQ2_0, tier_amd.MXFP4,
                               tier_amd.NF4, tier_amd.FP4, tier_amd.IQ2_XXS, tier_amd.IQ2_XS, tier_amd.IQ2_S,
                               tier_amd.IQ3_XXS, tier_amd.IQ3_S, tier_amd.IQ1_S, tier_amd.IQ1_M])
@pytest.mark.parametrize("N,K", [(1, 256), (13, 512), (7, 768), (65, 2304)])
def test_gemv_ragged_shapes(gpu, t, N, K):
    """Row counts that do not fill a wave or a block; one super-block rows; K not a multiple of 512."""
    rng = np.random.default_rng(N * 1000 + K + t)
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(rng, t, N * (K // be), moderate=True).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("t", [tier_amd.Q8_0, tier_amd.Q4_0, tier_amd.Q4_1, tier_amd.Q5_0, tier_amd.Q5_1])
@pytest.mark.parametrize("N,K", [(300, 14336), (9, 16384), (1029, 8192), (4100, 4096)])
def test_gemv_block32_rows_in_lds(gpu, t, N, K):
    """The 32-element block types staged whole in LDS: one row per wave above 80 KiB a
    workgroup (K = 8192 .. 16384), two below; a partial last workgroup."""
    rng = np.random.default_rng(N + K + t)
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(rng, t, N * (K // be)).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("N,K", [(8, 256), (24, 768), (40, 5120), (1000, 2304), (1024, 4096), (10240, 5120),
                                 (2000, 14336), (4096, 14336), (4100, 14336), (10240, 8192), (10240, 14336)])
def test_gemv_q6k_mfma(gpu, N, K):
    """Q6_K on int8 MFMA: 210-byte super-blocks leave rows at every even shift in
    their 16-byte window; one to four K parts per row tile; every launch shape."""
    rng = np.random.default_rng(N + K)
    t = tier_amd.Q6_K
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL
    # per row as well: a row read at a wrong shift stands out
    want = oracle.gemv_f64(blocks, t, x, N, K)
    err = np.abs(y - want) / np.maximum(np.abs(want), 1e-3 * np.abs(want).max())
    assert err.max() <= 1e-4


@pytest.mark.parametrize("N,K", [(64, 4096), (4100, 14336), (13824, 5120)])
def test_gemv_q6k_extremes(gpu, N, K):
    """Q6_K rows at the ends of the value range: every scale -128 and every q6 0 or 63
    (the weights -32 and 31, so the digit dots of q6 and the digit sums taken off them
    both reach their largest sizes), x over 2^-30 .. 2^30 in every 32-element block.
    Rows are checked one by one: a row read at a wrong dword phase or a wrong digit
    sum stands out."""
    rng = np.random.default_rng(N + K + 66)
    t = tier_amd.Q6_K
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    b = blocks.reshape(-1, 210)
    b[:, 192:208] = 0x80
    b[:, :192] = rng.choice(np.array([0x00, 0xFF], np.uint8), size=(b.shape[0], 192))
    x = (rng.standard_normal(K) * np.float32(2.0) ** rng.integers(-30, 31, K)).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    want = oracle.gemv_f64(blocks, t, x, N, K)
    assert oracle.rel_fro(y, want) <= TOL
    err = np.abs(y - want) / np.maximum(np.abs(want), 1e-3 * np.abs(want).max())
    assert err.max() <= 1e-4


@pytest.mark.parametrize("t", [tier_amd.Q8_0, tier_amd.Q5_1])
def test_gemv_block32_unaligned_rows(gpu, t):
    """Weights at an address that is not 16-byte aligned take the per-element kernel;
    both kernels meet the bar on the same rows."""
    N, K = 200, 4096
    rng = np.random.default_rng(t)
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(rng, t, N * (K // be)).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    rb = tier_amd.q_row_bytes(t, K)
    W = hip.DeviceBuffer(blocks.nbytes + 16).upload(blocks, offset=2)
    X, Y = hip.to_device(x), hip.DeviceBuffer(N * 4)
    tier_amd.gemv_q(W.ptr + 2, t, rb, X.ptr, Y.ptr, N, K)
    hip.synchronize()
    want = oracle.gemv_f64(blocks, t, x, N, K)
    y_off = Y.download(np.float32, N)
    assert oracle.rel_fro(y_off, want) <= TOL
    assert oracle.rel_fro(_gemv(blocks, t, x, N, K), want) <= TOL


@pytest.mark.parametrize("t", [tier_amd.Q5_K, tier_amd.Q8_0])
@pytest.mark.parametrize("N,K", [(10250, 5120), (10256, 8192), (10240, 14336), (5000, 7936), (3000, 14336)])
def test_gemv_mfma_tall(gpu, t, N, K):
    """q5_K / q8_0 on the int8-MFMA kernel with more row tiles than CUs (eight waves a
    workgroup) and ragged row counts, at each K class."""
    rng = np.random.default_rng(N + K + t)
    be, _ = oracle.block(t)
    blocks = oracle.random_blocks(rng, t, N * (K // be)).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("N,K", [(10250, 4352), (10240, 256), (10256, 8192), (10240, 1280), (10250, 14336)])
def test_gemv_q4k_tall_ragged(gpu, N, K):
    """Tall q4_K matrices (the producer-wave kernel): a partial last row tile, K halves of
    unequal super-block counts (17 = 8 + 9), a half with no super-block (K = 256)."""
    t = tier_amd.Q4_K
    rng = np.random.default_rng(N + K)
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    x[::131] *= np.float32(300.0)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("t", [tier_amd.Q4_K, tier_amd.Q5_K])
@pytest.mark.parametrize("N,K", [(2000, 5120), (5000, 3072), (10256, 2048), (13824, 5120), (16390, 2048),
                                 (20000, 768), (28700, 1024), (40000, 512), (14000, 8192)])
def test_gemv_tall_tiles_per_workgroup(gpu, t, N, K):
    """The whole-tile kernel (q4_K, q5_K) at each count of row tiles per workgroup it is
    built for (1, 2, 3, 4, 6 and 8; 40000 rows need more workgroups than CUs), with
    workgroups whose last tiles lie past the matrix and partial last row tiles (5000,
    16390, 28700)."""
    rng = np.random.default_rng(7 * N + K + t)
    blocks = oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    want = oracle.gemv_f64(blocks, t, x, N, K)
    assert oracle.rel_fro(y, want) <= TOL
    # every row written, none left at the 0xff fill
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("t", [tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q8_0])
@pytest.mark.parametrize("N", [1000, 1024, 4096, 4100, 6144, 6160, 8192, 8200])
def test_gemv_long_k_launch_shapes(gpu, t, N):
    """K = 14336 around the launch-shape boundaries: q4_K takes the whole-tile kernel from
    64 to 256 row tiles (1024 and 4096 rows), in split stages from 257 to 384 (4100,
    6144), two tiles a workgroup from 385 to 512 (6160, 8192), and the per-wave kernel
    outside (1000, 8200); q5_K the same from 64 tiles; q8_0 switches at 256 tiles between
    one tile x eight K parts and two tiles x four K parts per workgroup."""
    K = 14336
    rng = np.random.default_rng(N + t)
    blocks = oracle.random_blocks(rng, t, N * (K // oracle.block(t)[0])).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("N,K", [(17, 256), (1000, 768), (4096, 4096), (4096, 5120), (4100, 5120)])
def test_gemv_q8_0_eight_k_parts(gpu, N, K):
    """q8_0 at most 256 row tiles: one tile x eight K parts, down to K parts with no
    group of eight blocks (K = 256, 768)."""
    t = tier_amd.Q8_0
    blocks = quantized_weight(t, N, K, seed=N + K)
    x = activations(1, K, seed=K)[0]
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


def test_gemv_zero_and_extreme_inputs(gpu):
    t, N, K = tier_amd.Q4_K, 64, 1024
    blocks = quantized_weight(t, N, K, seed=5)
    y = _gemv(blocks, t, np.zeros(K, np.float32), N, K)
    assert np.all(y == 0)
    x = activations(1, K, seed=6)[0] * np.float32(1e4)
    x[::97] = np.float32(3e4)
    y = _gemv(blocks, t, x, N, K)
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


def test_gemv_on_a_stream(gpu):
    """Stream-ordered: the call returns before the result is ready; a stream sync makes it visible."""
    t, N, K = tier_amd.Q6_K, 300, 4096
    blocks = quantized_weight(t, N, K, seed=8)
    x = activations(1, K, seed=9)[0]
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(N * 4)
    s = hip.Stream()
    tier_amd.gemv_q(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, N, K, stream=s)
    s.synchronize()
    y = Y.download(np.float32, N)
    s.destroy()
    assert oracle.rel_fro(y, oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


@pytest.mark.parametrize("wtype", [tier_amd.F32, tier_amd.F16, tier_amd.BF16])
@pytest.mark.parametrize("N,K", [(1000, 4096), (33, 1001), (5, 16)])
def test_gemv_dense_rows(gpu, wtype, N, K):
    """gemv<T> (tier.cpp:2261-2268) on fp32 / fp16 / bf16 rows; K = 1001 takes the element-wise path."""
    rng = np.random.default_rng(N + K + wtype)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    if wtype == tier_amd.F32:
        bits, wf = w, w
    elif wtype == tier_amd.F16:
        bits = oracle.f2h(w).reshape(N, K)
        wf = oracle.h2f(bits).reshape(N, K)
    else:
        bits = oracle.f2bf(w).reshape(N, K)
        wf = (bits.astype(np.uint32) << 16).view(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    W, X, Y = hip.to_device(bits), hip.to_device(x), hip.DeviceBuffer(N * 4)
    tier_amd.gemv(W.ptr, wtype, X.ptr, Y.ptr, N, K)
    hip.synchronize()
    y = Y.download(np.float32, N)
    assert oracle.rel_fro(y, wf.astype(np.float64) @ x.astype(np.float64)) <= TOL


@pytest.mark.parametrize("wtype", [tier_amd.F32, tier_amd.F16, tier_amd.BF16])
def test_gemv_q_on_dense_rows(gpu, wtype):
    """gemv_q over q_val's dense cases takes the dense-row kernel: the same bits as tiermm_gemv."""
    rng = np.random.default_rng(70 + wtype)
    N, K = 77, 1032
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    bits = {tier_amd.F32: w, tier_amd.F16: oracle.f2h(w), tier_amd.BF16: oracle.f2bf(w)}[wtype].reshape(N, K)
    x = rng.standard_normal(K).astype(np.float32)
    W, X, Y1, Y2 = hip.to_device(bits), hip.to_device(x), hip.DeviceBuffer(N * 4), hip.DeviceBuffer(N * 4)
    tier_amd.gemv_q(W.ptr, wtype, tier_amd.q_row_bytes(wtype, K), X.ptr, Y1.ptr, N, K)
    tier_amd.gemv(W.ptr, wtype, X.ptr, Y2.ptr, N, K)
    hip.synchronize()
    y1, y2 = Y1.download(np.float32, N), Y2.download(np.float32, N)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    wf = oracle.dequant(np.ascontiguousarray(bits).view(np.uint8).reshape(N, -1), wtype, K)
    assert oracle.rel_fro(y1, wf.reshape(N, K).astype(np.float64) @ x.astype(np.float64)) <= TOL


def test_gemv_from_a_tq_base(gpu, tmp_path):
    """A quantized base written to .tq, opened by name, its rows uploaded and multiplied."""
    from tier_amd import tq
    t, N, K = tier_amd.Q4_K, 300, 2048
    blocks = quantized_weight(t, N, K, seed=12)
    p = str(tmp_path / "base.tq")
    tq.write_tq_arrays(p, [("model.layers.0.mlp.up_proj.weight", t, N, K, blocks)], {"from": "test"})
    with tq.TqFile(p) as f:
        i = f.find("model.layers.0.mlp.up_proj.weight")
        e = f.entry(i)
        rows = f.read_rows(i)
    x = activations(1, K, seed=13)[0]
    W, X, Y = hip.to_device(rows), hip.to_device(x), hip.DeviceBuffer(N * 4)
    tier_amd.gemv_q(W.ptr, e["qtype"], e["rb"], X.ptr, Y.ptr, e["rows"], e["cols"])
    hip.synchronize()
    assert oracle.rel_fro(Y.download(np.float32, N), oracle.gemv_f64(blocks, t, x, N, K)) <= TOL


SPLIT = [(4100, 14336), (5120, 14336), (6000, 14336), (6144, 14336), (5000, 9216), (4500, 12800)]


@pytest.mark.parametrize("t", [tier_amd.Q4_K, tier_amd.Q5_K])
@pytest.mark.parametrize("N,K", SPLIT)
def test_gemv_split_stages(gpu, t, N, K):
    """q4_K and q5_K with 257..384 row tiles above K = 8192: each workgroup streams an equal range of
    stages, and a tile split between two workgroups gets its rows from the two parts
    (lower + upper) through the pairing slots.  Partial last tiles (4100, 6000, 5000, 4500
    rows), a last stage shorter than the others (K = 9216: 36 super-blocks in stages of 8;
    12800: 50).  Bar: 1e-5 against fp64 over the matrix and 1e-3 per row (a row that missed
    its other part is off by about half its value), every row written (NaN fill), and the
    same bits on repeated calls, also with another split shape in between (the slots are
    left empty by every call)."""
    blocks = quantized_weight(t, N, K, seed=N + K)
    x = activations(1, K, seed=N)[0]
    want = oracle.gemv_f64(blocks, t, x, N, K)
    rb = tier_amd.q_row_bytes(t, K)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(N * 4)
    o_blocks = quantized_weight(tier_amd.Q4_K, 5120, 14336, seed=3)
    o_x = activations(1, 14336, seed=4)[0]
    OW, OX, OY = hip.to_device(o_blocks), hip.to_device(o_x), hip.DeviceBuffer(5120 * 4)
    runs = []
    for i in range(3):
        Y.fill_bytes(0xff)
        tier_amd.gemv_q(W.ptr, t, rb, X.ptr, Y.ptr, N, K)
        if i == 1:  # another split shape between the second and third call
            tier_amd.gemv_q(OW.ptr, tier_amd.Q4_K, tier_amd.q_row_bytes(tier_amd.Q4_K, 14336), OX.ptr, OY.ptr, 5120,
                            14336)
        hip.synchronize()
        runs.append(Y.download(np.float32, N))
    y = runs[0]
    assert np.all(np.isfinite(y))
    assert oracle.rel_fro(y, want) <= TOL
    err = np.abs(y - want) / np.maximum(np.abs(want), 1e-3 * np.abs(want).max())
    assert err.max() <= 1e-3
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), y.view(np.uint32))
    oy = OY.download(np.float32, 5120)
    assert oracle.rel_fro(oy, oracle.gemv_f64(o_blocks, tier_amd.Q4_K, o_x, 5120, 14336)) <= TOL

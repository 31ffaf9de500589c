"""tiermm_x3_rows_noalloc against tiermm_x3_rows (chat_fp3, tier.cpp:2195-2219).

The allocation-free variant runs the same kernels with the fp16 planes of x in a
static device scratch, so its output must equal tiermm_x3_rows' bit for bit; both
are also held to the x3-ref bar (relative Frobenius error <= 2^-20 against fp64
of fp16(W) * x).  Two calls in a row, the second smaller, show that the scratch
keeps no state that a later call depends on.  Sizes past the scratch are refused
before any launch.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20


def _fp16_weight(N, K, seed):
    w = (np.random.default_rng(seed).standard_normal((N, K)) * 0.02).astype(np.float32)
    bits = oracle.f2h(w).reshape(N, K)
    return bits, oracle.h2f_array(bits).reshape(N, K).astype(np.float64)


def _both(M, K, N, ldo, seed):
    bits, wf = _fp16_weight(N, K, seed)
    x = activations(M, K, seed=seed + 1)
    W, X = hip.to_device(bits), hip.to_device(x)
    Y1, Y2 = hip.DeviceBuffer(M * ldo * 4), hip.DeviceBuffer(M * ldo * 4)
    Y1.fill_bytes(0x3f)
    Y2.fill_bytes(0x3f)
    code = tier_amd.lib().tiermm_x3_rows_noalloc(W.ptr, X.ptr, Y1.ptr, M, K, N, ldo, None)
    assert code == tier_amd.OK, tier_amd.last_error()
    assert tier_amd.chat_fp3(W.ptr, X.ptr, Y2.ptr, M, K, N, ldo)
    hip.synchronize()
    y1 = Y1.download(np.float32, M * ldo).reshape(M, ldo)
    y2 = Y2.download(np.float32, M * ldo).reshape(M, ldo)
    return y1, y2, x, wf


def test_noalloc_matches_x3_rows_two_calls(gpu):
    for M, K, N, ldo, seed in ((256, 14336, 3000, 3008, 1), (37, 1024, 500, 500, 2)):
        y1, y2, x, wf = _both(M, K, N, ldo, seed)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), (M, K, N)
        assert np.array_equal(y1[:, N:].view(np.uint32), np.full((M, ldo - N), 0x3f3f3f3f, np.uint32))
        assert oracle.rel_fro(y1[:, :N], x.astype(np.float64) @ wf.T) <= BAR


def test_noalloc_big_tiles_then_small(gpu):
    """A call that takes the 256-row big-tile kernel (>= 192 tiles), then a small one."""
    for M, K, N, ldo, seed in ((1024, 5120, 20480, 20480, 3), (5, 256, 64, 64, 4)):
        y1, y2, x, wf = _both(M, K, N, ldo, seed)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), (M, K, N)
        rows = np.random.default_rng(seed).choice(M, min(M, 48), replace=False)
        assert oracle.rel_fro(y1[rows, :N], x[rows].astype(np.float64) @ wf.T) <= BAR


def test_noalloc_refuses_past_the_scratch(gpu):
    M, K, N = 4096, 5120, 64
    assert 3 * M * K * 2 > tier_amd.NOALLOC_SCRATCH_BYTES
    B = hip.DeviceBuffer(1024)  # never read: the size is refused on the host first
    code = tier_amd.lib().tiermm_x3_rows_noalloc(B.ptr, B.ptr, B.ptr, M, K, N, N, None)
    assert code == tier_amd.UNSUPPORTED
    assert "scratch" in tier_amd.last_error()
    assert not tier_amd.chat_fp3_noalloc(B.ptr, B.ptr, B.ptr, M, K, N, N)


def test_noalloc_refuses_k_not_a_multiple_of_32(gpu):
    """tiermm_x3_rows pads any K; the allocation-free form has no room for padded copies and
    refuses K % 32 != 0 on the host, before any launch, so a caller can fall back."""
    B = hip.DeviceBuffer(1024)  # never read
    code = tier_amd.lib().tiermm_x3_rows_noalloc(B.ptr, B.ptr, B.ptr, 4, 1000, 8, 8, None)
    assert code == tier_amd.UNSUPPORTED
    assert "multiple of 32" in tier_amd.last_error()

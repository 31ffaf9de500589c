"""Decode GEMVs (gemv_q, tier.cpp:299-306) captured in a HIP graph and replayed.

A serving loop captures a decode step once and replays it, so tiermm_qgemv must record
only kernel launches (no allocation, no memset node) and give the same rows on every
replay.  The whole-tile kernel in split stages keeps state between its workgroups in a
device-global table that each launch leaves empty; replays carry the captured epoch,
so this also checks that every replay finds the table empty.  Bar: every replay bit for
bit equal to the same calls issued eagerly, with eager work (fills, another split-stage
call) between the replays.
"""
import numpy as np
import pytest

import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu

# (type, N, K): the headline's whole tiles, split stages (q4_K, q5_K), per-wave q8_0, q6_K
CASES = [(tier_amd.Q4_K, 13824, 5120), (tier_amd.Q4_K, 5120, 14336), (tier_amd.Q5_K, 5120, 14336),
         (tier_amd.Q8_0, 4096, 4096), (tier_amd.Q6_K, 5120, 14336)]


def test_qgemv_graph_replays_match_eager(gpu):
    s = hip.Stream()
    mats = []
    for i, (t, N, K) in enumerate(CASES):
        W = hip.to_device(quantized_weight(t, N, K, seed=40 + i))
        X = hip.to_device(activations(1, K, seed=50 + i)[0])
        mats.append((t, N, K, tier_amd.q_row_bytes(t, K), W, X, hip.DeviceBuffer(N * 4), hip.DeviceBuffer(N * 4)))
    for t, N, K, rb, W, X, Ye, _ in mats:
        tier_amd.gemv_q(W.ptr, t, rb, X.ptr, Ye.ptr, N, K, s)
    s.synchronize()
    eager = [Ye.download(np.float32, N) for t, N, K, rb, W, X, Ye, _ in mats]

    def record(st):
        for t, N, K, rb, W, X, _, Yg in mats:
            tier_amd.gemv_q(W.ptr, t, rb, X.ptr, Yg.ptr, N, K, st)

    g = hip.Graph(s, record)
    try:
        other = mats[1]
        for rep in range(3):
            for *_, Yg in mats:
                Yg.fill_bytes(0xff)
            g.launch(s)
            s.synchronize()
            for (t, N, K, rb, W, X, Ye, Yg), want in zip(mats, eager):
                got = Yg.download(np.float32, N)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rep, t, N, K)
            # an eager split-stage call between replays (another epoch on the same table)
            t, N, K, rb, W, X, Ye, _ = other
            tier_amd.gemv_q(W.ptr, t, rb, X.ptr, Ye.ptr, N, K, s)
            s.synchronize()
            assert np.array_equal(Ye.download(np.float32, N).view(np.uint32), eager[1].view(np.uint32))
    finally:
        g.destroy()
        s.destroy()

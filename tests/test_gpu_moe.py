"""GPU parity of the grouped (MoE) quantized GEMM and the weighted combine.

There is no reference function (the reference refuses MoE models,
arch.py:158-159): the bar is the per-expert decomposition into dense products
(fp64 of the oracle's fp16 dequantization times x) and an fp64 weighted sum,
relative Frobenius error <= 2^-20.
"""
import ctypes

import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20


def _route(rng, T, E, topk):
    """Router logits ~N(0,1) -> softmax -> top-k; pairs sorted by expert (stable)."""
    logits = rng.standard_normal((T, E))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    top = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    pair_tok = np.repeat(np.arange(T), topk)
    pair_exp = top.ravel()
    pair_w = p[np.arange(T)[:, None], top].ravel().astype(np.float32)
    order = np.argsort(pair_exp, kind="stable")
    offsets = np.zeros(E + 1, np.int32)
    np.add.at(offsets, pair_exp + 1, 1)
    offsets = np.cumsum(offsets).astype(np.int32)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    token_pairs = inv.reshape(T, topk).astype(np.int32)  # sorted-pair index of token t's j-th expert
    return pair_tok[order], pair_exp[order], pair_w[order], offsets, token_pairs


@pytest.mark.parametrize("t,N,K", [(tier_amd.Q4_K, 256, 512), (tier_amd.Q5_0, 192, 1408)])
def test_grouped_gemm_and_combine(gpu, t, N, K):
    rng = np.random.default_rng(N + K)
    T, E, topk = 96, 8, 2
    pair_tok, pair_exp, pair_w, offsets, token_pairs = _route(rng, T, E, topk)
    be, _ = oracle.block(t)
    blocks = [oracle.random_blocks(rng, t, N * (K // be)).reshape(N, -1) for _ in range(E)]
    x = activations(T, K, seed=5)
    xs = np.ascontiguousarray(x[pair_tok])
    # an expert with no tokens: move expert 5's pairs to expert 6
    sel = pair_exp == 5
    pair_exp = np.where(sel, 6, pair_exp)
    order = np.argsort(pair_exp, kind="stable")
    pair_tok, pair_exp, pair_w, xs = pair_tok[order], pair_exp[order], pair_w[order], xs[order]
    counts = np.bincount(pair_exp, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    token_pairs = inv[token_pairs.ravel()].reshape(T, topk).astype(np.int32)
    assert counts[5] == 0

    dW = [hip.to_device(b) for b in blocks]
    rb = tier_amd.q_row_bytes(t, K)
    X = hip.to_device(xs)
    Y = hip.DeviceBuffer(xs.shape[0] * N * 4)
    tier_amd.qgemm_grouped([w.ptr for w in dW], [t] * E, [rb] * E, X.ptr, offsets.tolist(), Y.ptr, N, K)
    TP, PW, OUT = hip.to_device(token_pairs), hip.to_device(pair_w), hip.DeviceBuffer(T * N * 4)
    tier_amd.moe_combine(Y.ptr, TP.ptr, PW.ptr, OUT.ptr, T, topk, N)
    hip.synchronize()
    ys = Y.download(np.float32, xs.shape[0] * N).reshape(-1, N)
    out = OUT.download(np.float32, T * N).reshape(T, N)

    w16 = [oracle.h2f(oracle.dequant(b, t, K, oracle.OUT_F16)).reshape(N, K).astype(np.float64) for b in blocks]
    ref_s = np.empty((xs.shape[0], N))
    for e in range(E):
        a, b = offsets[e], offsets[e + 1]
        ref_s[a:b] = xs[a:b].astype(np.float64) @ w16[e].T
    assert oracle.rel_fro(ys, ref_s) <= BAR
    ref = np.zeros((T, N))
    for tt in range(T):
        for j in range(topk):
            p = token_pairs[tt, j]
            ref[tt] += float(pair_w[p]) * ref_s[p]
    assert oracle.rel_fro(out, ref) <= BAR


MIXED = {"fused": [tier_amd.Q4_K, tier_amd.Q5_0, tier_amd.Q8_0, tier_amd.Q6_K],
         "staged": [tier_amd.Q4_K, tier_amd.Q4_0, tier_amd.Q8_0, tier_amd.Q3_K]}


@pytest.mark.parametrize("with_ws", [False, True])
@pytest.mark.parametrize("kind", ["fused", "staged"])
def test_grouped_big_tiles_mixed_types(gpu, with_ws, kind):
    """Routed rows that fill the chip with 256-row tiles: 70 experts (two groups of at
    most 64 per launch), four weight types in one call, an empty expert, a one-row
    expert and ragged row counts.  "fused": every type is decoded inside the GEMM, one
    fused launch per type; "staged": one type (q4_0, q3_K) is not, so every expert goes
    through fp16 staging and the grouped 256x320 launch."""
    rng = np.random.default_rng(70)
    E, N, K = 70, 640, 256
    types = MIXED[kind]
    counts = rng.integers(260, 330, E)
    counts[3], counts[11], counts[40] = 0, 1, 257
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    P = int(offsets[-1])
    qt = [types[e % 4] for e in range(E)]
    blocks = [oracle.random_blocks(rng, qt[e], N * (K // oracle.block(qt[e])[0])).reshape(N, -1) for e in range(E)]
    xs = activations(P, K, seed=71)
    dW = [hip.to_device(b) for b in blocks]
    X, Y = hip.to_device(xs), hip.DeviceBuffer(P * N * 4)
    rbs = [tier_amd.q_row_bytes(q, K) for q in qt]
    ws = wsb = None
    if with_ws:
        wsb = tier_amd.qgemm_grouped_ws_bytes(qt, offsets.tolist(), N, K)
        # planes, plus one chunk of fp16 experts when staged
        assert wsb == 3 * P * K * 2 if kind == "fused" else wsb >= 3 * P * K * 2 + 64 * N * K * 2
        ws = hip.DeviceBuffer(wsb)
    tier_amd.qgemm_grouped([w.ptr for w in dW], qt, rbs, X.ptr, offsets.tolist(), Y.ptr, N, K,
                           ws=ws.ptr if ws else None, ws_bytes=wsb or 0)
    hip.synchronize()
    ys = Y.download(np.float32, P * N).reshape(P, N)
    ref = np.empty((P, N))
    for e in range(E):
        a, b = offsets[e], offsets[e + 1]
        w16 = oracle.h2f(oracle.dequant(blocks[e], qt[e], K, oracle.OUT_F16)).reshape(N, K).astype(np.float64)
        ref[a:b] = xs[a:b].astype(np.float64) @ w16.T
    for e in (11, 40, 69):  # per expert as well: a misplaced row or group shows here
        a, b = offsets[e], offsets[e + 1]
        assert oracle.rel_fro(ys[a:b], ref[a:b]) <= BAR, e
    assert oracle.rel_fro(ys, ref) <= BAR


def test_grouped_stacked_gate_up_bit_identical(gpu):
    """Each expert's gate and up rows stored stacked (one 2N-row weight, as MoE engines keep
    w1 / w3) give, in one grouped call, exactly the two separate grouped products: every
    output column is summed over K in the same order whatever the tile width."""
    rng = np.random.default_rng(2816)
    E, N, K = 16, 1408, 2048
    counts = rng.integers(440, 590, E)
    counts[2], counts[9] = 0, 3
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    P = int(offsets[-1])
    t = tier_amd.Q4_K
    gate = [oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1) for _ in range(E)]
    up = [oracle.random_blocks(rng, t, N * (K // 256)).reshape(N, -1) for _ in range(E)]
    xs = activations(P, K, seed=72)
    X = hip.to_device(xs)
    rb = tier_amd.q_row_bytes(t, K)
    outs = {}
    for name, ws_, n in (("gate", gate, N), ("up", up, N), ("gu", [np.concatenate([g, u]) for g, u in zip(gate, up)], 2 * N)):
        dW = [hip.to_device(b) for b in ws_]
        Y = hip.DeviceBuffer(P * n * 4)
        tier_amd.qgemm_grouped([w.ptr for w in dW], [t] * E, [rb] * E, X.ptr, offsets.tolist(), Y.ptr, n, K)
        hip.synchronize()
        outs[name] = Y.download(np.float32, P * n).reshape(P, n)
    assert np.array_equal(outs["gu"][:, :N].view(np.uint32), outs["gate"].view(np.uint32))
    assert np.array_equal(outs["gu"][:, N:].view(np.uint32), outs["up"].view(np.uint32))
    a, b = offsets[9], offsets[10]
    w16 = oracle.h2f(oracle.dequant(gate[9], t, K, oracle.OUT_F16)).reshape(N, K).astype(np.float64)
    assert oracle.rel_fro(outs["gate"][a:b], xs[a:b].astype(np.float64) @ w16.T) <= BAR


@pytest.mark.parametrize("N,topk", [(2048, 8), (8, 1), (6, 8), (1024, 17), (4, 16)])
def test_moe_combine_shapes(gpu, N, topk):
    """The combine on both of its kernels (four columns a thread when N % 4 == 0 and
    topk <= 16, one column otherwise): each token's weighted sum of its top-k rows
    against fp64."""
    rng = np.random.default_rng(N * 31 + topk)
    T = 37
    P = T * topk
    ys = rng.standard_normal((P, N)).astype(np.float32)
    tp = rng.permutation(P).astype(np.int32).reshape(T, topk)
    pw = rng.random(P).astype(np.float32)
    Y, TP, PW, OUT = hip.to_device(ys), hip.to_device(tp), hip.to_device(pw), hip.DeviceBuffer(T * N * 4)
    tier_amd.moe_combine(Y.ptr, TP.ptr, PW.ptr, OUT.ptr, T, topk, N)
    hip.synchronize()
    out = OUT.download(np.float32, T * N).reshape(T, N)
    ref = np.einsum("tj,tjn->tn", pw[tp].astype(np.float64), ys[tp].astype(np.float64))
    assert oracle.rel_fro(out, ref) <= BAR


def _grouped_case(rng, types, counts, N, K, seed):
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    P = int(offsets[-1])
    E = len(types)
    blocks = [oracle.random_blocks(rng, types[e], N * (K // oracle.block(types[e])[0])).reshape(N, -1) for e in range(E)]
    xs = activations(P, K, seed=seed)
    return offsets, P, blocks, xs


def _grouped_run(types, blocks, xs, offsets, N, K, with_ws=False):
    P = xs.shape[0]
    dW = [hip.to_device(b) for b in blocks]
    X, Y = hip.to_device(xs), hip.DeviceBuffer(P * N * 4)
    ws = wsb = None
    if with_ws:
        wsb = tier_amd.qgemm_grouped_ws_bytes(types, offsets.tolist(), N, K)
        ws = hip.DeviceBuffer(wsb)
    tier_amd.qgemm_grouped([w.ptr for w in dW], types, [tier_amd.q_row_bytes(q, K) for q in types], X.ptr,
                           offsets.tolist(), Y.ptr, N, K, ws=ws.ptr if ws else None, ws_bytes=wsb or 0)
    hip.synchronize()
    return Y.download(np.float32, P * N).reshape(P, N)


def _expert_ref(blocks, t, xs, N, K):
    w16 = oracle.h2f(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(N, K).astype(np.float64)
    return xs.astype(np.float64) @ w16.T


def test_grouped_fused_long_k_bit_identical_per_expert(gpu, monkeypatch):
    """All-q4_K experts at K = 8192, beyond one accumulator's 6144: the grouped call takes the
    fused kernel over several expert groups with two accumulation chunks (it may not split
    K).  Each expert against fp64, and bit for bit against tiermm_qgemm on that expert alone
    with the same plan forced (BN 128, one split, two chunks)."""
    monkeypatch.setenv("TIERMM_QGEMM_TILE", "128,1,2")
    rng = np.random.default_rng(8192)
    N, K = 320, 8192
    counts = np.array([41, 0, 57, 1, 64, 38])
    types = [tier_amd.Q4_K] * len(counts)
    offsets, P, blocks, xs = _grouped_case(rng, types, counts, N, K, seed=73)
    assert tier_amd.qgemm_plan(tier_amd.Q4_K, int(counts.max()), N, K) == (128, 1, 2)
    ys = _grouped_run(types, blocks, xs, offsets, N, K)
    for e in range(len(counts)):
        a, b = offsets[e], offsets[e + 1]
        if a == b:
            continue
        assert oracle.rel_fro(ys[a:b], _expert_ref(blocks[e], types[e], xs[a:b], N, K)) <= BAR, e
        W, X, Y = hip.to_device(blocks[e]), hip.to_device(np.ascontiguousarray(xs[a:b])), hip.DeviceBuffer((b - a) * N * 4)
        tier_amd.qgemm(W.ptr, types[e], tier_amd.q_row_bytes(types[e], K), X.ptr, Y.ptr, b - a, N, K)
        hip.synchronize()
        one = Y.download(np.float32, (b - a) * N).reshape(b - a, N)
        assert np.array_equal(one.view(np.uint32), ys[a:b].view(np.uint32)), e


def test_grouped_staged_long_k_fills_chip(gpu):
    """q4_0 experts (staged through fp16, not decoded in the GEMM) at K = 8192 with enough
    routed rows for the grouped 256-row big-tile launch, whose K chunks shift each expert's
    weight pointer: three experts (the first, one in the middle, the last) in full against
    fp64, and the whole output with and without a caller workspace bit for bit."""
    rng = np.random.default_rng(8193)
    E, N, K = 24, 1280, 8192
    counts = rng.integers(257, 320, E)
    types = [tier_amd.Q4_0] * E
    offsets, P, blocks, xs = _grouped_case(rng, types, counts, N, K, seed=74)
    ys = _grouped_run(types, blocks, xs, offsets, N, K)
    ys_ws = _grouped_run(types, blocks, xs, offsets, N, K, with_ws=True)
    assert np.array_equal(ys.view(np.uint32), ys_ws.view(np.uint32))
    for e in (0, 11, E - 1):
        a, b = offsets[e], offsets[e + 1]
        assert oracle.rel_fro(ys[a:b], _expert_ref(blocks[e], types[e], xs[a:b], N, K)) <= BAR, e


@pytest.mark.parametrize("with_ws", [False, True])
def test_grouped_sparse_mixed_types(gpu, with_ws):
    """A routed batch that does not fill the chip and mixes types the fused kernel decodes
    (q4_K, q6_K: one fused launch per type over its experts) with one it does not (q4_0:
    staged per expert), about 50 rows each: every expert against fp64."""
    rng = np.random.default_rng(50)
    N, K = 256, 1024
    types = [tier_amd.Q4_K, tier_amd.Q4_0, tier_amd.Q6_K] * 3
    counts = rng.integers(40, 60, len(types))
    counts[4] = 0
    offsets, P, blocks, xs = _grouped_case(rng, types, counts, N, K, seed=75)
    ys = _grouped_run(types, blocks, xs, offsets, N, K, with_ws=with_ws)
    for e in range(len(types)):
        a, b = offsets[e], offsets[e + 1]
        if a < b:
            assert oracle.rel_fro(ys[a:b], _expert_ref(blocks[e], types[e], xs[a:b], N, K)) <= BAR, e

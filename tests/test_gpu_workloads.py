"""GPU parity at the full workloads of BASELINE configs 4 and 5.

Config 4: the seven projections of one decoder layer (hidden 5120, 32 q / 8 kv
heads x 128, ffn 14336) on a packed 4096-token batch, in both mixed recipes of
the reference (tier.cpp:2701-2713): q4_K_S (q/k/o/gate/up q4_K, v/down q5_K)
and q4_K_M (v/down q6_K).  Weights ~N(0,0.02) through the host quantizer
(byte-identical with quant.h), activations ~N(0,1).

Config 5: the routed experts of an MoE layer: 64 experts, top-8 of softmax(router
logits ~N(0,1)), hidden 2048, expert ffn 1408, 4096 tokens sorted by expert;
gate/up q4_K, down q5_0 (K = 1408 is not a whole number of 256-element
super-blocks, so q4_K cannot hold it; q5_0 is llama.cpp's fallback), then the
per-token weighted combine.  The reference refuses MoE models (arch.py:158-159),
so the bar is the per-expert decomposition.  Expert weights are random blocks
with finite fp16 scales (every bit pattern of the format; the reference has no
q5_0 quantizer).

Bar (tiermm_qgemm's x3-ref semantics, the training path's dq_k<tier_fp16> +
fp3gemm, tier.cpp:515, 922): relative Frobenius error <= 2^-20 against fp64 of
the oracle's fp16 dequantization times x, on 48 sampled weight rows over all
tokens and on 48 sampled token rows over all outputs of every matrix, and per
expert on 48 of its rows.  MODE_F32 (the chat prefill semantics,
tier.cpp:2358-2359) is checked on the v/down types against fp64 of the fp32
dequantization.
"""
import functools

import numpy as np
import pytest

import oracle
import tier_amd
from helpers import activations, quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu
BAR = 2.0 ** -20
T, H, QD, KVD, F = 4096, 5120, 4096, 1024, 14336


@functools.lru_cache(maxsize=None)
def _weight(t, N, K, seed):
    return quantized_weight(t, N, K, seed=seed)


@functools.lru_cache(maxsize=None)
def _x(K):
    return activations(T, K, seed=100 + K)


def _w16(blocks, t, K):
    return oracle.h2f_array(oracle.dequant(blocks, t, K, oracle.OUT_F16)).reshape(-1, K).astype(np.float64)


def _check_sampled(got, x, wref, seed):
    """got [T][N] against fp64 x @ wref^T on 48 weight rows (all tokens) and 48 tokens (all rows)."""
    rng = np.random.default_rng(seed)
    N = wref.shape[0]
    cols = rng.choice(N, 48, replace=False)
    toks = rng.choice(x.shape[0], 48, replace=False)
    xd = x.astype(np.float64)
    assert np.all(np.isfinite(got))
    e1 = oracle.rel_fro(got[:, cols], xd @ wref[cols].T)
    e2 = oracle.rel_fro(got[toks], xd[toks] @ wref.T)
    assert e1 <= BAR and e2 <= BAR, (e1, e2)


# the distinct matrices of both recipes: q/k/o/gate/up are q4_K in each, v/down q5_K (S) or q6_K (M)
PROJ = {
    "q": (tier_amd.Q4_K, QD, H, 10), "k": (tier_amd.Q4_K, KVD, H, 11), "o": (tier_amd.Q4_K, H, QD, 13),
    "gate": (tier_amd.Q4_K, F, H, 14), "up": (tier_amd.Q4_K, F, H, 15),
    "v_S": (tier_amd.Q5_K, KVD, H, 12), "down_S": (tier_amd.Q5_K, H, F, 16),
    "v_M": (tier_amd.Q6_K, KVD, H, 112), "down_M": (tier_amd.Q6_K, H, F, 116),
}


@functools.lru_cache(maxsize=2)
def _wref(name, f32):
    t, N, K, seed = PROJ[name]
    blocks = _weight(t, N, K, seed)
    if f32:
        return oracle.dequant(blocks, t, K).astype(np.float64)
    return _w16(blocks, t, K)


@pytest.mark.parametrize("name", list(PROJ))
def test_decoder_layer_projection_t4096(gpu, name):
    t, N, K, seed = PROJ[name]
    blocks = _weight(t, N, K, seed)
    x = _x(K)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(T * N * 4)
    Y.fill_bytes(0xff)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, T, N, K)
    hip.synchronize()
    got = Y.download(np.float32, T * N).reshape(T, N)
    _check_sampled(got, x, _wref(name, False), seed=N + K)


@pytest.mark.parametrize("name", ["v_S", "down_S", "v_M", "down_M"])
def test_decoder_layer_f32_mode_t4096(gpu, name):
    """The chat prefill semantics on the recipes' v/down types at the layer's size."""
    t, N, K, seed = PROJ[name]
    blocks = _weight(t, N, K, seed)
    x = _x(K)
    W, X, Y = hip.to_device(blocks), hip.to_device(x), hip.DeviceBuffer(T * N * 4)
    tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), X.ptr, Y.ptr, T, N, K, mode=tier_amd.MODE_F32)
    hip.synchronize()
    got = Y.download(np.float32, T * N).reshape(T, N)
    _check_sampled(got, x, _wref(name, True), seed=N + K + 1)


def _route(seed, T_, E, topk):
    """Router logits ~N(0,1) -> softmax -> top-k; pairs sorted by expert (stable)."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T_, E))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    top = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    pair_tok = np.repeat(np.arange(T_), topk)
    pair_exp = top.ravel()
    pair_w = p[np.arange(T_)[:, None], top].ravel().astype(np.float32)
    order = np.argsort(pair_exp, kind="stable")
    offsets = np.concatenate([[0], np.cumsum(np.bincount(pair_exp, minlength=E))]).astype(np.int32)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    return pair_tok[order], pair_w[order], offsets, inv.reshape(T_, topk).astype(np.int32)


def test_moe_config5_t4096(gpu):
    E, topk, Hm, Fm = 64, 8, 2048, 1408
    pair_tok, pair_w, offsets, token_pairs = _route(18, T, E, topk)
    P = int(offsets[-1])
    assert P == T * topk
    rng = np.random.default_rng(19)
    mats = {}
    for name, t, N, K in (("gate", tier_amd.Q4_K, Fm, Hm), ("up", tier_amd.Q4_K, Fm, Hm),
                          ("down", tier_amd.Q5_0, Hm, Fm)):
        be = oracle.block(t)[0]
        mats[name] = (t, N, K, [oracle.random_blocks(rng, t, N * (K // be), moderate=True).reshape(N, -1)
                                for _ in range(E)])
    x = activations(T, Hm, seed=20)
    xs = np.ascontiguousarray(x[pair_tok])              # routed token rows, sorted by expert
    a = activations(P, Fm, seed=21)                     # the down projection's input rows
    Xs, A = hip.to_device(xs), hip.to_device(a)
    out = {}
    for name, src in (("gate", Xs), ("up", Xs), ("down", A)):
        t, N, K, blocks = mats[name]
        dW = [hip.to_device(b) for b in blocks]
        Y = hip.DeviceBuffer(P * N * 4)
        tier_amd.qgemm_grouped([w.ptr for w in dW], [t] * E, [tier_amd.q_row_bytes(t, K)] * E, src.ptr,
                               offsets.tolist(), Y.ptr, N, K)
        hip.synchronize()
        out[name] = (Y, Y.download(np.float32, P * N).reshape(P, N))
        del dW
    TP, PW, OUT = hip.to_device(token_pairs), hip.to_device(pair_w), hip.DeviceBuffer(T * Hm * 4)
    tier_amd.moe_combine(out["down"][0].ptr, TP.ptr, PW.ptr, OUT.ptr, T, topk, Hm)
    hip.synchronize()
    comb = OUT.download(np.float32, T * Hm).reshape(T, Hm)

    srng = np.random.default_rng(22)
    ref_down = {}
    for name, inp in (("gate", xs), ("up", xs), ("down", a)):
        t, N, K, blocks = mats[name]
        got = out[name][1]
        assert np.all(np.isfinite(got)), name
        for e in range(E):
            lo, hi = int(offsets[e]), int(offsets[e + 1])
            if hi == lo:
                continue
            rows = lo + srng.choice(hi - lo, min(48, hi - lo), replace=False)
            w16 = _w16(blocks[e], t, K)
            ref = inp[rows].astype(np.float64) @ w16.T
            assert oracle.rel_fro(got[rows], ref) <= BAR, (name, e)
            if name == "down":
                ref_down[e] = w16
    # combine on sampled tokens, from an fp64 recomputation of their eight routed rows
    exp_of = np.searchsorted(offsets, np.arange(P), side="right") - 1
    toks = srng.choice(T, 48, replace=False)
    want = np.zeros((48, Hm))
    for i, tt in enumerate(toks):
        for j in range(topk):
            p = token_pairs[tt, j]
            want[i] += float(pair_w[p]) * (a[p].astype(np.float64) @ ref_down[exp_of[p]].T)
    assert oracle.rel_fro(comb[toks], want) <= BAR

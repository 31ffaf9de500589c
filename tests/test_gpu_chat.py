"""GPU parity of the chat linears with weight streaming (chat_lin, tier.cpp:2351-2378;
chat_issue / chat_slot, tier.cpp:2283-2285; placement tier.cpp:2549-2555).

The streamed path runs the same kernels on the same rows as the resident one, so
every output must be bit-identical to a direct call on a resident copy, pass after
pass of the cyclic order; the direct calls are pinned to the oracle elsewhere, and
one pass is checked against the oracle here too.
"""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu

H, QD, KV, FF = 512, 512, 128, 1024
# the seven linears of a decoder layer in the engine's order (CHAT_MN, tier.cpp:2277)
SHAPES = [("q", QD, H), ("k", KV, H), ("v", KV, H), ("o", H, QD), ("gate", FF, H), ("up", FF, H), ("down", H, FF)]


def _rows(t, N, K, seed):
    """Weight rows of type t: the host quantizer for the K-quants / q8_0, random blocks for the
    legacy types, converted normals for dense rows."""
    rng = np.random.default_rng(seed)
    if t in (tier_amd.Q8_0, tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K):
        return quantized_weight(t, N, K, seed=seed)
    if t in (tier_amd.F32, tier_amd.F16, tier_amd.BF16):
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        bits = {tier_amd.F32: w, tier_amd.F16: oracle.f2h(w), tier_amd.BF16: oracle.f2bf(w)}[t]
        return np.ascontiguousarray(bits).view(np.uint8).reshape(N, -1)
    return oracle.random_blocks(rng, t, N * K // oracle.block(t)[0]).reshape(N, -1)


def _model(layers=3):
    """(type, N, K, rows) per matrix; the layers mix the types a recipe and the dense paths give."""
    mats = []
    for layer in range(layers):
        for j, (nm, N, K) in enumerate(SHAPES):
            t = {"v": tier_amd.Q6_K, "down": tier_amd.Q5_K}.get(nm, tier_amd.Q4_K)
            if layer == 1:
                t = {"v": tier_amd.F16, "o": tier_amd.BF16, "k": tier_amd.F32}.get(nm, t)
            if layer == 2:
                t = {"gate": tier_amd.Q4_1, "up": tier_amd.Q8_0, "k": tier_amd.Q5_1, "q": tier_amd.Q4_0}.get(nm, t)
            mats.append((t, N, K, _rows(t, N, K, 100 * layer + j)))
    return mats


class Rig:
    """A chat set over `mats` plus resident copies and per-matrix inputs / outputs."""

    def __init__(self, mats, M, nslots=2, budget=None, stream=None):
        self.mats, self.M = mats, M
        self.host = []
        self.chat = tier_amd.Chat(nslots, stream)
        self.ids = []
        for t, N, K, rows in mats:
            h = tier_amd.HostRows(rows.nbytes)
            h.array()[:] = rows.ravel()
            self.host.append(h)
            self.ids.append(self.chat.add(t, N, K, host=h.ptr))
        self.placed = self.chat.place(budget=budget, reserve=0)
        rng = np.random.default_rng(M)
        self.x = [rng.standard_normal((M, K)).astype(np.float32) for _, _, K, _ in mats]
        self.X = [hip.to_device(x) for x in self.x]
        self.Y = [hip.DeviceBuffer(M * N * 4) for _, N, _, _ in mats]
        self.W = [hip.to_device(rows) for *_, rows in mats]

    def run(self, order=None, mode=tier_amd.MODE_F32):
        for i in (range(len(self.mats)) if order is None else order):
            self.chat.lin(self.ids[i], self.X[i].ptr, self.Y[i].ptr, self.M, mode)
        hip.synchronize()
        return [Y.download(np.float32, self.M * N) for Y, (_, N, _, _) in zip(self.Y, self.mats)]

    def direct(self, i, mode=tier_amd.MODE_F32, rows=None):
        """The same product through the single-call entry points on a resident copy."""
        t, N, K, r = self.mats[i]
        W = self.W[i] if rows is None else hip.to_device(rows)
        Y = hip.DeviceBuffer(self.M * N * 4)
        dense = t in (tier_amd.F32, tier_amd.F16, tier_amd.BF16)
        if self.M == 1:
            if dense:
                tier_amd.gemv(W.ptr, t, self.X[i].ptr, Y.ptr, N, K)
            else:
                tier_amd.gemv_q(W.ptr, t, tier_amd.q_row_bytes(t, K), self.X[i].ptr, Y.ptr, N, K)
        elif t == tier_amd.F16 and mode == tier_amd.MODE_X3REF:
            assert tier_amd.chat_fp3(W.ptr, self.X[i].ptr, Y.ptr, self.M, K, N, N)
        elif t == tier_amd.BF16 and mode == tier_amd.MODE_X3REF:
            assert tier_amd.chat_bf3(W.ptr, self.X[i].ptr, Y.ptr, self.M, K, N, N)
        else:
            tier_amd.qgemm(W.ptr, t, tier_amd.q_row_bytes(t, K), self.X[i].ptr, Y.ptr, self.M, N, K, N,
                           tier_amd.MODE_F32 if dense else mode)
        hip.synchronize()
        return Y.download(np.float32, self.M * N)

    def close(self):
        self.chat.close()
        for h in self.host:
            h.free()


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("M,nslots,mode", [(1, 2, tier_amd.MODE_F32), (48, 2, tier_amd.MODE_F32),
                                           (48, 3, tier_amd.MODE_X3REF), (1, 4, tier_amd.MODE_X3REF)])
def test_streamed_passes_match_resident(gpu, M, nslots, mode):
    """Five matrices resident, the other sixteen streamed; three passes of the cyclic order."""
    mats = _model()
    sizes = [r.nbytes for *_, r in mats]
    rig = Rig(mats, M, nslots, budget=sum(sizes[:5]))
    try:
        assert rig.placed == (sum(sizes[:5]), sum(sizes[5:]))
        assert [rig.chat.info(i)["streamed"] for i in rig.ids] == [0] * 5 + [1] * 16
        want = [rig.direct(i, mode) for i in range(len(mats))]
        for p in range(3):
            got = rig.run(mode=mode)
            for i in range(len(mats)):
                assert _same(got[i], want[i]), (p, i)
        assert rig.chat.info()["uses"] == 3 * 16
        if M == 1:  # one pass against the oracle as well
            for i, (t, N, K, rows) in enumerate(mats):
                assert oracle.rel_fro(got[i], oracle.gemv_f64(rows, t, rig.x[i][0], N, K)) <= 1e-5, i
    finally:
        rig.close()


def test_budget_rule_streams_everything_after_the_first_miss(gpu):
    """tier.cpp:2552: after the first matrix that does not fit, later (smaller) ones stream too."""
    mats = _model(1)
    sizes = [r.nbytes for *_, r in mats]
    # q fits; k would fit on its own after q, but the budget is set so that only q does
    rig = Rig(mats, 1, budget=sizes[0] + sizes[1] - 1)
    try:
        assert [rig.chat.info(i)["streamed"] for i in rig.ids] == [0] + [1] * 6
        got = rig.run()
        for i in range(len(mats)):
            assert _same(got[i], rig.direct(i))
    finally:
        rig.close()


def test_out_of_order_use_is_refused_and_rewind_recovers(gpu):
    mats = _model(1)
    rig = Rig(mats, 1, budget=0)
    try:
        with pytest.raises(tier_amd.TiermmError, match="out of order"):
            rig.chat.lin(rig.ids[1], rig.X[1].ptr, rig.Y[1].ptr, 1)
        got = rig.run(order=[0, 1, 2])  # a pass cut short
        rig.chat.restart(rewind=True)
        got = rig.run()
        for i in range(len(mats)):
            assert _same(got[i], rig.direct(i))
    finally:
        rig.close()


def test_restart_after_host_weights_change(gpu):
    """The engine re-issues the pending copies after changing host weights (tier.cpp:2666-2676)."""
    mats = _model(1)
    rig = Rig(mats, 48, budget=0)
    try:
        rig.run()
        t, N, K, _ = mats[0]
        new = _rows(t, N, K, seed=999)
        hip.synchronize()
        rig.host[0].array()[:] = new.ravel()
        rig.chat.restart()
        got = rig.run()
        assert _same(got[0], rig.direct(0, rows=new))
        for i in range(1, len(mats)):
            assert _same(got[i], rig.direct(i))
    finally:
        rig.close()


def test_one_streamed_matrix_on_more_slots_and_a_stream(gpu):
    """Fewer streamed matrices than slots: every slot holds the same matrix in turn."""
    mats = _model(1)
    sizes = [r.nbytes for *_, r in mats]
    s = hip.Stream()
    rig = Rig(mats, 1, nslots=3, budget=sum(sizes[:6]), stream=s)
    try:
        assert [rig.chat.info(i)["streamed"] for i in rig.ids] == [0] * 6 + [1]
        for _ in range(5):
            got = rig.run()
            s.synchronize()
            for i in range(len(mats)):
                assert _same(got[i], rig.direct(i))
    finally:
        rig.close()
        s.destroy()


def test_pageable_rows_are_refused_only_when_streamed(gpu):
    t, N, K, rows = _model(1)[0]
    keep = np.ascontiguousarray(rows)
    c = tier_amd.Chat()
    c.add(t, N, K, host=keep.ctypes.data)
    with pytest.raises(tier_amd.TiermmError, match="not pinned"):
        c.place(budget=0)
    assert c.info()["resident_bytes"] == 0
    c.place(reserve=0)  # fits: copied once from pageable memory, as the engine's hipMemcpy does
    assert c.info(0)["streamed"] == 0
    X, Y = hip.to_device(np.ones(K, np.float32)), hip.DeviceBuffer(N * 4)
    c.lin(0, X.ptr, Y.ptr, 1)
    hip.synchronize()
    assert oracle.rel_fro(Y.download(np.float32, N), oracle.gemv_f64(keep, t, np.ones(K, np.float32), N, K)) <= 1e-5
    c.close()


def test_caller_resident_rows(gpu):
    """dev != NULL: the caller's device rows are used in place and never counted or freed."""
    t, N, K, rows = _model(1)[4]
    W = hip.to_device(rows)
    c = tier_amd.Chat()
    i = c.add(t, N, K, dev=W.ptr)
    assert c.place(budget=0, reserve=0) == (0, 0)
    X, Y = hip.to_device(np.arange(K, dtype=np.float32) / K), hip.DeviceBuffer(N * 4)
    c.lin(i, X.ptr, Y.ptr, 1)
    hip.synchronize()
    c.close()
    y = Y.download(np.float32, N)
    assert oracle.rel_fro(y, oracle.gemv_f64(rows, t, np.arange(K, dtype=np.float32) / K, N, K)) <= 1e-5
    assert W.download(np.uint8, rows.size).tobytes() == rows.tobytes()


@pytest.mark.parametrize("M", [1, 48])
@pytest.mark.parametrize("streamed", [False, True])
def test_trained_rows_and_lora(gpu, M, streamed):
    """chat_lin's additions after the base product (tier.cpp:2375-2376): trained fp16 rows over
    chosen output rows (chat_heads with a row index, 2339-2343) and over the first rows (no
    index, 2344-2350), then a LoRA adapter's s (x A^T) B^T (chat_lora, 2333-2337); switched off
    by the trained/base mode (g_chat_heads, g_chat_lon, 2668-2669).  fp64 references; bars:
    1e-5 at M = 1 (gemv_q / gemv<T>), 2^-20 at M = 48 (fp32 semantics)."""
    t, N, K, r, hr = tier_amd.Q4_K, 300, 512, 8, 40
    rows = quantized_weight(t, N, K, seed=41)
    mats = [(t, N, K, rows), (t, N, K, rows)]
    rig = Rig(mats, M, 2, budget=0 if streamed else None)
    rng = np.random.default_rng(42)
    hd = oracle.f2h((rng.standard_normal((2, hr, K)) * 0.02).astype(np.float32)).reshape(2, hr, K)
    hdf = oracle.h2f_array(hd).astype(np.float64)
    ri = rng.choice(N, hr, replace=False).astype(np.int32)
    A = (rng.standard_normal((r, K)) * 0.05).astype(np.float32)
    B = (rng.standard_normal((N, r)) * 0.05).astype(np.float32)
    HD, RI, DA, DB = hip.to_device(hd), hip.to_device(ri), hip.to_device(A), hip.to_device(B)
    try:
        # matrix 0: trained rows at ri; matrix 1: the first hr rows; both with the adapter
        rig.chat.set_heads(rig.ids[0], hr, tier_amd.F16, HD.ptr, RI.ptr)
        rig.chat.set_heads(rig.ids[1], hr, tier_amd.F16, HD.ptr + hr * K * 2, None)
        for i in rig.ids:
            rig.chat.set_lora(i, r, DA.ptr, DB.ptr)
        alpha, k = 16.0, 0.5
        s = k * alpha / r
        wf = oracle.dequant(rows, t, K).astype(np.float64)
        bar = 1e-5 if M == 1 else 2.0 ** -20

        def want(i, heads, lora):
            x = rig.x[i].astype(np.float64)
            y = x @ wf.T
            if heads:
                cols = ri if i == 0 else np.arange(hr)
                y[:, cols] = x @ hdf[i].T
            if lora:
                y += s * (x @ A.astype(np.float64).T) @ B.astype(np.float64).T
            return y

        for heads, lora_on in ((True, True), (False, True), (True, False)):
            rig.chat.heads(heads)
            rig.chat.lora_scale(alpha, k, lora_on)
            got = rig.run()
            for i in range(2):
                g = got[i].reshape(M, N)
                assert oracle.rel_fro(g, want(i, heads, lora_on)) <= bar, (heads, lora_on, i)
        # alpha 0 (the default before an adapter is loaded) leaves the base product alone
        rig.chat.heads(False)
        rig.chat.lora_scale(0.0)
        got = rig.run()
        for i in range(2):
            assert _same(got[i], rig.direct(i)), i
    finally:
        rig.close()

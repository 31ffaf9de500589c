#!/usr/bin/env python3
"""Benchmark of the frozen-weight matmul path on one MI355X.

Headline (BASELINE.json metric "q4_K dequant-matmul GB/s (M=1) & TFLOPS
(M=512)"): a step is one decode GEMV (tiermm_qgemv) of the north-star q4_K
weight 13824x5120 (W ~N(0,0.02) quantized by the host quantizer, x ~N(0,1)),
inputs resident in HBM.  The weight is rotated over enough copies (> 256 MiB in
total) that the 256 MiB Infinity Cache cannot hold them, so each step streams
its weight from HBM.  ``value`` is the whole-run rate: algorithmic bytes of K
steps / wall time between HIP events recorded around them on the stream the
kernels run on.  The K tiermm_qgemv calls are issued from a C loop through the C
ABI (libtiermm_probe.so's tiermm_bench_qgemv), as the engine's token loop calls
gemv_q: from Python each call costs about as much host time as a short GEMV takes
on the GPU.  They follow the W warm-up steps and, before those, ~30 ms of untimed
launches that bring the clock back from the idle of the host-side input
preparation.  ``roofline.achieved`` is the same bytes per launch over the
same events' average time per launch (it includes the gap between back-to-back
dispatches, about 1.5 us on MI355X, which a profiler's kernel duration leaves
out).

Secondary measurements in the same JSON line (``secondary``): the other config
shapes at M=1, q8_0 4096x4096 (config 1), the fused-path quantized GEMM at
M=512 (config 3, TFLOPS against fp16 peak/3), the x3-2x2 GEMM at M=4096
(config 2), the fp32 products of the x3-off fallback (tiermm_sgemm, forward and dX at
the decoder's down projection), the seven projections of a decoder layer (config 4), the routed MoE
experts (config 5), and the chat linears of four config-4 layers streamed from
pinned host memory against the host-to-device copy rate.

``cpu_baseline``: the reference's own q_val GEMV (oracle/_ref, compiled from
quant.h) on the host's threads, and on one thread, on the same weight (each timed
over a bounded number of repetitions), with the host CPU model.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6          # dense MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk
X3_PEAK_TFLOPS = FP16_PEAK_TFLOPS / 3
MALL_BYTES = 256 << 20


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_bytes(N: int, K: int, rb: int) -> int:
    return N * rb + 4 * K + 4 * N


class GemvCase:
    """A quantized weight rotated over `copies` device buffers, plus x and y."""

    def __init__(self, tier_amd, hip, qtype: int, N: int, K: int, seed: int):
        rng = np.random.default_rng(seed)
        w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        self.blocks = tier_amd.q_row(qtype, w)
        del w
        self.qtype, self.N, self.K = qtype, N, K
        self.rb = tier_amd.q_row_bytes(qtype, K)
        nbytes = N * self.rb
        self.copies = max(2, -(-(MALL_BYTES * 5 // 4) // nbytes))
        self.W = [hip.to_device(self.blocks)]
        for _ in range(self.copies - 1):
            b = hip.DeviceBuffer(nbytes)
            hip.copy_d2d(b.ptr, self.W[0].ptr, nbytes)
            self.W.append(b)
        self.x = rng.standard_normal(K).astype(np.float32)
        self.X = hip.to_device(self.x)
        self.Y = hip.DeviceBuffer(N * 4)
        self.bytes = gemv_bytes(N, K, self.rb)

    def launch(self, tier_amd, i: int, stream) -> None:
        tier_amd.gemv_q(self.W[i % self.copies].ptr, self.qtype, self.rb, self.X.ptr, self.Y.ptr, self.N, self.K,
                        stream)

    def launches(self, tier_amd, first: int, count: int, stream) -> None:
        """`count` calls of tiermm_qgemv (copies first, first + 1, ...) issued from a C loop."""
        P = probe_lib()
        ws = (ctypes.c_void_p * self.copies)(*[w.ptr for w in self.W])
        fn = ctypes.cast(tier_amd.lib().tiermm_qgemv, ctypes.c_void_p)
        st = P.tiermm_bench_qgemv(fn, ws, self.copies, first, self.qtype, self.rb, self.X.ptr, self.Y.ptr, self.N,
                                  self.K, count, stream.handle)
        if st:
            raise RuntimeError(f"tiermm_qgemv: status {st}: {tier_amd.last_error()}")


_PROBE = None


def probe_lib():
    """libtiermm_probe.so (tier_amd/csrc/probe.hip): the read floor, the MFMA ceiling and
    the C loop that issues a run of decode GEMVs."""
    global _PROBE
    if _PROBE is None:
        vp, i = ctypes.c_void_p, ctypes.c_int
        P = ctypes.CDLL(os.path.join(ROOT, "tier_amd", "libtiermm_probe.so"))
        P.tiermm_probe_read.argtypes = [vp, ctypes.c_size_t, i, i, vp, vp]
        P.tiermm_probe_mfma.argtypes = [vp, i, i, vp, vp]
        P.tiermm_bench_qgemv.argtypes = [vp, vp, i, i, i, ctypes.c_size_t, vp, vp, i, i, i, vp]
        _PROBE = P
    return _PROBE


def time_gemv(hip, stream, tier_amd, case: GemvCase, steps: int, warmup: int) -> float:
    """Milliseconds per call: `steps` back-to-back tiermm_qgemv calls, issued from a C loop
    through the C ABI, between two HIP events on `stream` (after `warmup` calls)."""
    case.launches(tier_amd, 0, warmup, stream)
    stream.synchronize()
    t0, t1 = hip.Event(), hip.Event()
    t0.record(stream)
    case.launches(tier_amd, warmup, steps, stream)
    t1.record(stream)
    t1.synchronize()
    per = t0.elapsed_ms(t1) / steps
    t0.destroy()
    t1.destroy()
    return per


def time_launches(hip, stream, launch, steps: int, warmup: int) -> float:
    """Milliseconds per launch: `steps` back-to-back launches between two HIP events on `stream`."""
    for i in range(warmup):
        launch(i)
    stream.synchronize()
    t0, t1 = hip.Event(), hip.Event()
    t0.record(stream)
    for i in range(steps):
        launch(warmup + i)
    t1.record(stream)
    t1.synchronize()
    per = t0.elapsed_ms(t1) / steps
    t0.destroy()
    t1.destroy()
    return per


def settle(hip, stream, tier_amd, case: GemvCase, ms: float = 30.0) -> None:
    """Untimed back-to-back calls (issued from the C loop) for `ms` milliseconds before a
    decode line's warm-up steps.  The host-side input preparation (quantizing the weight)
    leaves the GPU idle for seconds, and the clock controller then needs milliseconds of
    back-to-back work to return to its working clock: the 13824x5120 GEMV measured 9.05 us
    per step over the first 20 steps after idle and 8.6-8.7 us once settled, and the
    5120x5120 line 7.2 us over 50 steps after launches issued one by one from Python (which
    leave the GPU idle between them) against 5.7-5.9 us after 3000 back-to-back calls."""
    est = time_gemv(hip, stream, tier_amd, case, 4, 1)
    case.launches(tier_amd, 0, max(1, int(ms / max(est, 1e-3))), stream)
    stream.synchronize()


def time_steady(hip, stream, launch, steps: int, warm_ms: float = 60.0) -> float:
    """time_launches after at least `warm_ms` of warm-up launches.  Under a sustained MFMA
    load the clock controller overshoots for the first ~20-40 launches of a 0.5 ms GEMM
    (x3 GEMM 4096x5120x5120: 550 -> 680 -> 545 us per launch), so the MFMA-bound lines
    are timed once it has settled."""
    est = time_launches(hip, stream, launch, 2, 1)
    return time_launches(hip, stream, launch, steps, max(3, int(warm_ms / max(est, 1e-3))))


_QCACHE = {}


def _quantized(tier_amd, qtype, N, K, seed):
    """W ~N(0,0.02) through the host quantizer; q5_0 (no quantizer in the reference) as
    random 5-bit values with fp16 d ~ N(0, 0.004), the scale such W would get."""
    key = (qtype, N, K, seed)
    if key not in _QCACHE:
        _QCACHE[key] = _quantize(tier_amd, qtype, N, K, seed)
    return _QCACHE[key]


def _quantize(tier_amd, qtype, N, K, seed):
    rng = np.random.default_rng(seed)
    if qtype == tier_amd.Q5_0:
        nb = K // 32
        b = rng.integers(0, 256, size=(N * nb, 22), dtype=np.uint8)
        b[:, 0:2] = (rng.standard_normal(N * nb) * 0.004).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return b.reshape(N, nb * 22)
    return tier_amd.q_row(qtype, rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))


def bench_decoder_layer(tier_amd, hip, stream, T=4096, mode=None):
    """Config 4: the 7 projections of one decoder layer (hidden 5120, 32 q / 8 kv heads x 128,
    ffn 14336) on a packed T-token batch, q4_K_S recipe (q/k/o/gate/up q4_K, v/down q5_K),
    each a tiermm_qgemm: fp16-dequant x3 semantics (MODE_X3REF, the training forward), or
    MODE_F32 (chat_lin's prefill semantics, tier.cpp:2358-2359: fp32 dequant, fp32-accurate
    product; its chunk is 256 rows, tier.cpp:2538), whose kernels decode W inside the GEMM
    after one pass over W for its row exponents."""
    mode = tier_amd.MODE_X3REF if mode is None else mode
    H, Q, KV, F = 5120, 4096, 1024, 14336
    mats = (("q", tier_amd.Q4_K, Q, H), ("k", tier_amd.Q4_K, KV, H), ("v", tier_amd.Q5_K, KV, H),
            ("o", tier_amd.Q4_K, H, Q), ("gate", tier_amd.Q4_K, F, H), ("up", tier_amd.Q4_K, F, H),
            ("down", tier_amd.Q5_K, H, F))
    rng = np.random.default_rng(10)
    xs = {K: hip.to_device(rng.standard_normal((T, K), dtype=np.float32)) for K in (H, Q, F)}
    Y = hip.DeviceBuffer(T * F * 4)
    wsb = max(tier_amd.qgemm_ws_bytes(qt, T, N, K, mode) for _, qt, N, K in mats)
    WS = hip.DeviceBuffer(wsb)
    out, total_us, total_flop = {}, 0.0, 0.0
    for i, (name, qt, N, K) in enumerate(mats):
        log(f"bench: decoder layer {name} {N}x{K} T={T} mode={mode}")
        Wd = hip.to_device(_quantized(tier_amd, qt, N, K, 11 + i))
        rb = tier_amd.q_row_bytes(qt, K)
        f = lambda _i: tier_amd.qgemm(Wd.ptr, qt, rb, xs[K].ptr, Y.ptr, T, N, K, N,  # noqa: E731
                                      mode, 0.0, WS.ptr, wsb, stream)
        km = time_steady(hip, stream, f, 10 if T >= 1024 else 40)
        flop = 2.0 * T * N * K
        out[name] = {"type": tier_amd.TYPE_NAMES[qt], "N": N, "K": K, "us": round(km * 1e3, 1),
                     "TFLOPS": round(flop / (km * 1e-3) / 1e12, 1)}
        total_us += km * 1e3
        total_flop += flop
        del Wd
    tf = total_flop / (total_us * 1e-6) / 1e12
    return {"recipe": "q4_K_S (v, down q5_K)", "T": T, "mode": "f32" if mode == tier_amd.MODE_F32 else "x3ref",
            "workspace_bytes": wsb, "total_us": round(total_us, 1),
            "TFLOPS": round(tf, 1), "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4), "per_matrix": out}


def bench_decode_layer(tier_amd, hip, stream):
    """Chat decode (M=1) over one config-4 layer, q4_K_S recipe (q/k/o/gate/up q4_K, v/down
    q5_K): the 7 gemv_q calls chat_lin makes per layer (tier.cpp:2357), and the same with
    q + k and gate + up each as one tiermm_qgemv_batch call (5 calls).  Two copies of the
    layer's weights alternate (2 x 166 MiB > the 256 MiB MALL); x of each projection
    ~N(0,1) (5120, 4096 for o, 14336 for down)."""
    H, Q, KV, F = 5120, 4096, 1024, 14336
    mats = (("q", tier_amd.Q4_K, Q, H), ("k", tier_amd.Q4_K, KV, H), ("v", tier_amd.Q5_K, KV, H),
            ("o", tier_amd.Q4_K, H, Q), ("gate", tier_amd.Q4_K, F, H), ("up", tier_amd.Q4_K, F, H),
            ("down", tier_amd.Q5_K, H, F))
    rng = np.random.default_rng(21)
    xs = {k: hip.to_device(rng.standard_normal(k).astype(np.float32)) for k in (H, Q, F)}
    copies = []
    nbytes = 0
    for c in range(2):
        d = {}
        for name, qt, N, K in mats:
            blocks = _quantized(tier_amd, qt, N, K, 300 + len(d))
            d[name] = (hip.to_device(blocks), qt, N, K, tier_amd.q_row_bytes(qt, K), hip.DeviceBuffer(N * 4))
            if c == 0:
                nbytes += blocks.nbytes + K * 4 + N * 4
        copies.append(d)
    L = tier_amd.lib()
    vp, ip = ctypes.c_void_p, ctypes.c_int

    def single(j):
        d = copies[j % 2]
        for name, qt, N, K in mats:
            W, _, _, _, rb, Y = d[name]
            st = L.tiermm_qgemv(W.ptr, qt, rb, xs[K].ptr, Y.ptr, N, K, stream.handle)
            if st:
                raise RuntimeError(f"tiermm_qgemv {name}: {st}")

    # the batched calls' argument arrays, built once per copy
    plans = []
    for d in copies:
        calls = []
        for group in (("q", "k"), ("v",), ("o",), ("gate", "up"), ("down",)):
            qt, K, rb = d[group[0]][1], d[group[0]][3], d[group[0]][4]
            n = len(group)
            calls.append(((vp * n)(*[d[g][0].ptr for g in group]), qt, rb, xs[K].ptr,
                          (vp * n)(*[d[g][5].ptr for g in group]), (ip * n)(*[d[g][2] for g in group]), n, K))
        plans.append(calls)

    def batched(j):
        for w, qt, rb, x, y, ns, n, K in plans[j % 2]:
            st = L.tiermm_qgemv_batch(w, qt, rb, x, y, ns, n, K, stream.handle)
            if st:
                raise RuntimeError(f"tiermm_qgemv_batch: {st}")

    out = {"recipe": "q4_K_S (v, down q5_K)", "bytes_per_layer": nbytes}
    for name, fn in (("single_calls", single), ("batched_qk_gateup", batched)):
        est = time_launches(hip, stream, fn, 2, 1)
        for i in range(max(1, int(30.0 / max(est, 1e-3)))):  # settle the clock
            fn(i)
        per = float(np.median([time_launches(hip, stream, fn, 200, 10) for _ in range(3)]))
        out[name] = {"us": round(per * 1e3, 2), "GB/s": round(nbytes / (per * 1e-3) / 1e9, 1),
                     "frac_hbm": round(nbytes / (per * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def bench_decoder_layer_shared(tier_amd, hip, stream, T=4096):
    """Config 4's layer as the engine would issue it with x split once per activation
    (tiermm_split3_f16_ktiled, then tiermm_qgemm_x3parts on the K-tiled planes): one split
    for q/k/v, one for o, one for gate/up, one for down -- four splits and seven products
    per step, timed together."""
    H, Q, KV, F = 5120, 4096, 1024, 14336
    mats = (("q", tier_amd.Q4_K, Q, H), ("k", tier_amd.Q4_K, KV, H), ("v", tier_amd.Q5_K, KV, H),
            ("o", tier_amd.Q4_K, H, Q), ("gate", tier_amd.Q4_K, F, H), ("up", tier_amd.Q4_K, F, H),
            ("down", tier_amd.Q5_K, H, F))
    groups = ((H, ("q", "k", "v")), (Q, ("o",)), (H, ("gate", "up")), (F, ("down",)))
    rng = np.random.default_rng(10)
    xs = {K: hip.to_device(rng.standard_normal((T, K), dtype=np.float32)) for K in (H, Q, F)}
    P = {K: hip.DeviceBuffer(3 * T * K * 2) for K in (H, Q, F)}
    Y = hip.DeviceBuffer(T * F * 4)
    wsb = max(tier_amd.qgemm_x3parts_ws_bytes(qt, T, N, K) for _, qt, N, K in mats)
    WS = hip.DeviceBuffer(max(wsb, 256))
    W = {name: (hip.to_device(_quantized(tier_amd, qt, N, K, 11 + i)), qt, N, K)
         for i, (name, qt, N, K) in enumerate(mats)}
    log(f"bench: decoder layer, shared splits, T={T}")

    def step(_i):
        for K, names in groups:
            tier_amd.split3_ktiled(xs[K].ptr, P[K].ptr, T, K, T * K, stream)
            for nm in names:
                Wd, qt, N, Kw = W[nm]
                tier_amd.qgemm_x3parts(Wd.ptr, qt, tier_amd.q_row_bytes(qt, Kw), P[K].ptr, T * K, Y.ptr, T, N, Kw, N,
                                       0.0, WS.ptr, wsb, stream)
    km = time_steady(hip, stream, step, 10)
    flop = sum(2.0 * T * N * K for _, _, N, K in mats)
    tf = flop / (km * 1e-3) / 1e12
    del W
    return {"recipe": "q4_K_S (v, down q5_K)", "T": T, "splits": 4, "total_us": round(km * 1e3, 1),
            "TFLOPS": round(tf, 1), "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4)}


def bench_chat_stream(tier_amd, hip, stream, layers=4):
    """chat_lin with weight streaming (tier.cpp:2283-2285, 2351-2378): the 28 linears of
    `layers` config-4 decoder layers (q4_K_S, 155.6 MiB each) with every matrix streamed from
    pinned host memory through 2 device slots, against the same set resident, at M=1 (decode)
    and M=4096 (prefill, MODE_F32: chat_lin's fp32 dequant and fp32-accurate product,
    tier.cpp:2358-2359).  The roof of the streamed decode pass is the
    host-to-device copy rate, measured here as the same 28 copies back to back without
    compute.  Every figure is taken after warm-up passes (the first DMA reads of fresh
    pinned pages and a new copy queue run up to 35 % slower) and is the median over
    passes timed one at a time with a synchronisation after each, as the engine's token
    loop reads the logits back after every pass.  (Passes queued back to back without a
    synchronisation stream at ~44 GB/s: the copy queue falls behind by ~80 us per copy.)"""
    H, Q, KV, F = 5120, 4096, 1024, 14336
    shapes = ((tier_amd.Q4_K, Q, H), (tier_amd.Q4_K, KV, H), (tier_amd.Q5_K, KV, H), (tier_amd.Q4_K, H, Q),
              (tier_amd.Q4_K, F, H), (tier_amd.Q4_K, F, H), (tier_amd.Q5_K, H, F))
    log("bench: chat streaming: host rows")
    host = []
    for i, (qt, N, K) in enumerate(shapes):
        rows = _quantized(tier_amd, qt, N, K, 11 + i)
        h = tier_amd.HostRows(rows.nbytes)
        h.array()[:] = rows.ravel()
        host.append(h)
    layer_bytes = sum(h.nbytes for h in host)
    big = max(h.nbytes for h in host)
    D = [hip.DeviceBuffer(big) for _ in range(2)]
    t0, t1 = hip.Event(), hip.Event()

    def copies():  # the pass's 28 copies back to back, no compute between them
        for i in range(7 * layers):
            h = host[i % 7]
            hip.check(hip.lib().hipMemcpyAsync(ctypes.c_void_p(D[i % 2].ptr), ctypes.c_void_p(h.ptr),
                                               ctypes.c_size_t(h.nbytes), hip.H2D, ctypes.c_void_p(stream.handle)),
                      "hipMemcpyAsync")
    copies()  # first DMA touches of the pinned pages run slower
    stream.synchronize()
    per = []
    for _ in range(7):  # one pass of copies per step, synchronised, as the passes below
        t0.record(stream)
        copies()
        t1.record(stream)
        t1.synchronize()
        per.append(t0.elapsed_ms(t1))
    h2d = layers * layer_bytes / (float(np.median(per)) * 1e-3) / 1e9
    for d in D:
        d.free()
    T = 4096
    rng = np.random.default_rng(12)
    X = {K: hip.to_device(rng.standard_normal((T, K), dtype=np.float32)) for K in (H, Q, F)}
    Y = hip.DeviceBuffer(T * F * 4)
    out = {"layers": layers, "matrices": 7 * layers, "bytes_per_pass": layers * layer_bytes,
           "h2d_GBps": round(h2d, 1)}
    for placement, budget, nslots in (("streamed", 0, 2), ("streamed_4slots", 0, 4), ("resident", None, 2)):
        c = tier_amd.Chat(nslots, stream)
        ids = [c.add(qt, N, K, host=host[j].ptr) for _ in range(layers) for j, (qt, N, K) in enumerate(shapes)]
        c.place(budget=budget, reserve=0)
        for M, passes in ((1, 9), (T, 3)):
            log(f"bench: chat {placement} M={M}")

            def one_pass():
                for i, idx in enumerate(ids):
                    qt, N, K = shapes[i % 7]
                    c.lin(idx, X[K].ptr, Y.ptr, M, tier_amd.MODE_F32)
            for _ in range(3):  # the first passes over fresh host rows and a new copy queue run slower
                one_pass()
            stream.synchronize()
            per = []
            for _ in range(passes):  # one pass per step, synchronised, as the engine's token loop is
                t0.record(stream)
                one_pass()
                t1.record(stream)
                t1.synchronize()
                per.append(t0.elapsed_ms(t1))
            ms = float(np.median(per))
            key = f"{placement}_m{M}"
            out[key] = {"ms_per_pass": round(ms, 3), "GBps": round(layers * layer_bytes / (ms * 1e-3) / 1e9, 1)}
            if placement.startswith("streamed"):
                out[key]["frac_h2d"] = round(out[key]["GBps"] / h2d, 3)
        c.close()
    t0.destroy()
    t1.destroy()
    for h in host:
        h.free()
    return out


def bench_moe(tier_amd, hip, stream):
    """Config 5: 64 experts, top-8 of softmax(router logits ~N(0,1)), hidden 2048, expert ffn
    1408; 4096 tokens sorted by expert; gate/up q4_K, down q5_0 (K = 1408 is not a whole
    number of 256-element super-blocks); grouped GEMMs + per-token weighted combine.  Each
    expert's gate and up rows are stored stacked (one 2816-row weight, as MoE engines keep
    w1/w3), so one grouped GEMM gives both from one split of the routed rows."""
    T, E, topk, H, F = 4096, 64, 8, 2048, 1408
    rng = np.random.default_rng(18)
    logits = rng.standard_normal((T, E))
    prob = np.exp(logits - logits.max(1, keepdims=True))
    prob /= prob.sum(1, keepdims=True)
    top = np.argsort(-prob, axis=1, kind="stable")[:, :topk]
    pair_exp = top.ravel()
    pair_w = prob[np.arange(T)[:, None], top].ravel().astype(np.float32)
    order = np.argsort(pair_exp, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    offsets = np.concatenate([[0], np.cumsum(np.bincount(pair_exp, minlength=E))]).astype(np.int32).tolist()
    P = T * topk
    # 8 distinct quantized experts per matrix, copied to 64 device buffers
    log("bench: moe weights")
    base = {}
    for name, qt, N, K in (("gate", tier_amd.Q4_K, F, H), ("up", tier_amd.Q4_K, F, H), ("down", tier_amd.Q5_0, H, F)):
        base[name] = [_quantized(tier_amd, qt, N, K, 19 + 31 * j + len(base)) for j in range(8)]
    gu = [np.concatenate([base["gate"][j], base["up"][j]]) for j in range(8)]
    ws_ = {"gate_up": (tier_amd.Q4_K, 2 * F, H, [hip.to_device(gu[e % 8]) for e in range(E)]),
           "down": (tier_amd.Q5_0, H, F, [hip.to_device(base["down"][e % 8]) for e in range(E)])}
    Xs = hip.to_device(rng.standard_normal((P, H), dtype=np.float32))
    A = hip.to_device(rng.standard_normal((P, F), dtype=np.float32))
    GU, D = hip.DeviceBuffer(P * 2 * F * 4), hip.DeviceBuffer(P * H * 4)
    TP, PW, OUT = hip.to_device(inv.reshape(T, topk).astype(np.int32)), hip.to_device(pair_w[order]), \
        hip.DeviceBuffer(T * H * 4)
    wsb = max(tier_amd.qgemm_grouped_ws_bytes([q] * E, offsets, N, K) for q, N, K, _ in ws_.values())
    WS = hip.DeviceBuffer(wsb)

    def step(_i):
        for name, dst, src in (("gate_up", GU, Xs), ("down", D, A)):
            qt, N, K, bufs = ws_[name]
            tier_amd.qgemm_grouped([b.ptr for b in bufs], [qt] * E, [tier_amd.q_row_bytes(qt, K)] * E, src.ptr,
                                   offsets, dst.ptr, N, K, tier_amd.MODE_X3REF, WS.ptr, wsb, stream)
        tier_amd.moe_combine(D.ptr, TP.ptr, PW.ptr, OUT.ptr, T, topk, H, stream)

    log("bench: moe grouped GEMMs")
    km = time_steady(hip, stream, step, 5)
    flop = 2.0 * P * (2 * F * H + H * F)
    tf = flop / (km * 1e-3) / 1e12
    return {"experts": E, "topk": topk, "tokens": T, "us": round(km * 1e3, 1), "TFLOPS": round(tf, 1),
            "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4), "types": "gate/up q4_K, down q5_0",
            "includes": "gate+up as one grouped GEMM of the stacked 2816-row expert weights, down, combine "
                        "(64 experts each); no activation between"}


def _read_floor(hip, stream, lib, nbytes: int) -> float:
    """Milliseconds per launch of one non-temporal read of `nbytes` (probe.hip read_once,
    2048 workgroups), rotated over enough copies to exceed the MALL, as a GemvCase is."""
    nbytes = nbytes // 16 * 16
    copies = max(2, -(-(MALL_BYTES * 5 // 4) // nbytes))
    bufs = [hip.DeviceBuffer(nbytes) for _ in range(copies)]
    for b in bufs:
        b.fill_bytes(1)
    out = hip.DeviceBuffer(1 << 16)

    def read(i):
        if lib.tiermm_probe_read(bufs[i % copies].ptr, nbytes, 2048, 1, out.ptr, stream.handle):
            raise RuntimeError("tiermm_probe_read")
    rd = min(time_launches(hip, stream, read, 200, 20) for _ in range(3))
    for b in bufs:
        b.free()
    return rd


def bench_floors(hip, stream, head: GemvCase, head_ms: float, secondary=None):
    """What the hardware gives the two roofs on this box, from libtiermm_probe.so
    (tier_amd/csrc/probe.hip): one read of the headline's bytes with nothing else to
    do (non-temporal 16-byte loads, 2048 workgroups, over the same number of rotated
    copies as the headline) -- and of the weight bytes of the short decode lines, whose
    time is mostly the fixed cost of a launch --, and a register-only
    v_mfma_f32_32x32x16_f16 loop on random-like operands (1024 workgroups x 4 waves x 8
    independent accumulators)."""
    lib = probe_lib()
    nbytes = head.N * head.rb // 16 * 16
    log("bench: read floor")
    rd = _read_floor(hip, stream, lib, nbytes)
    short = {}
    for name, wbytes in (("q4_K_5120x5120_m1", 5120 * 2880), ("q8_0_4096x4096_m1", 4096 * 4352),
                         ("q4_K_5120x14336_m1", 5120 * 8064)):
        r = _read_floor(hip, stream, lib, wbytes)
        short[name] = {"bytes": wbytes, "us_per_launch": round(r * 1e3, 3),
                       "frac_hbm": round(wbytes / (r * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        line = (secondary or {}).get(name)
        if line:
            short[name]["line_over_read"] = round(line["us_per_step"] / (r * 1e3), 3)
    seed = hip.to_device((np.arange(1024, dtype=np.uint64) * 2654435761 % (1 << 32)).astype(np.uint32))
    mo = hip.DeviceBuffer(1024 * 256 * 4)

    def mfma(_i):
        if lib.tiermm_probe_mfma(seed.ptr, 1024, 4096, mo.ptr, stream.handle):
            raise RuntimeError("tiermm_probe_mfma")
    log("bench: mfma ceiling")
    mm = time_steady(hip, stream, mfma, 5)
    tf = 1024 * 4 * 8 * 4096 * 32768 / (mm * 1e-3) / 1e12
    return {"read_once": {"bytes": nbytes, "us_per_launch": round(rd * 1e3, 3),
                          "GB/s": round(nbytes / (rd * 1e-3) / 1e9, 1),
                          "frac_hbm": round(nbytes / (rd * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                          "headline_over_read": round(head_ms / rd, 3)},
            "read_once_short_lines": short,
            "mfma_f16": {"TFLOPS": round(tf, 1), "frac_dense_peak": round(tf / FP16_PEAK_TFLOPS, 4),
                         "x3_target_over_this": round(0.6 * FP16_PEAK_TFLOPS / tf, 4)}}


def measured_traffic():
    """HBM bytes per headline launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's reading for a copy
    of known size), or (None, None) when no summary is present."""
    path = os.path.join(ROOT, "profiles", "q4k_gemv_13824x5120_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None, None
    return int(d["bytes_per_launch"]), f"profiles/q4k_gemv_13824x5120.md ({d['kernel']})"


def _host_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(case: GemvCase, budget_s: float):
    """The reference q_val GEMV (oracle/_ref, built from quant.h) on every host thread, and on
    one thread; bounded repetitions of each."""
    import oracle
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    W = np.ascontiguousarray(case.blocks)
    if oracle.ref_available():
        kind = "reference"
        runner = lambda n: (lambda: oracle.ref_gemv_threads(W, case.qtype, case.x, case.N, case.K, n))  # noqa: E731
    else:  # the C restatement, single thread (lane order of gemv_q)
        kind, threads = "port", 1
        runner = lambda n: (lambda: oracle.gemv_lanes(W, case.qtype, case.x, case.N, case.K, 64))  # noqa: E731

    def timed(run, budget):
        run()
        reps, t0 = 0, time.perf_counter()
        while True:
            run()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget or reps >= 200:
                return reps, el

    reps, el = timed(runner(threads), budget_s)
    gbs = case.bytes * reps / el / 1e9
    out = {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": kind,
           "sample": f"{reps} full {case.N}x{case.K} q4_K GEMVs ({el:.1f} s wall, {el * threads:.0f} thread-s)",
           "host": _host_model(), "nproc": os.cpu_count()}
    if threads > 1:
        reps1, el1 = timed(runner(1), budget_s / 2)
        out["single_core"] = {"value": round(case.bytes * reps1 / el1 / 1e9, 3), "unit": "GB/s",
                              "sample": f"{reps1} full GEMVs on 1 thread ({el1:.1f} s)"}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host baseline")
    ap.add_argument("--no-secondary", action="store_true", help="headline only")
    ap.add_argument("--secondary", default="", help="comma-separated secondary names to run (default: all)")
    ap.add_argument("--cpu-seconds", type=float, default=3.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    import tier_amd
    from tier_amd import hip

    hip.set_device(0)
    tier_amd.init(0)
    cus = hip.attribute(hip.ATTR_MULTIPROCESSORS)
    clk_mhz = hip.attribute(hip.ATTR_CLOCK_RATE_KHZ) / 1000.0
    stream = hip.Stream()

    # ---------------------------------------------------------------- headline
    log("bench: preparing q4_K 13824x5120 GEMV inputs")
    head = GemvCase(tier_amd, hip, tier_amd.Q4_K, 13824, 5120, seed=3)
    settle(hip, stream, tier_amd, head)
    per = time_gemv(hip, stream, tier_amd, head, args.steps, args.warmup)
    wall = per * args.steps
    value = head.bytes * args.steps / (wall * 1e-3) / 1e9
    achieved = head.bytes / (per * 1e-3) / 1e9
    log(f"bench: q4_K GEMV {per * 1e3:.2f} us/step")

    secondary = {}
    only = {n for n in args.secondary.split(",") if n}
    want = lambda name: not args.no_secondary and (not only or name in only)  # noqa: E731
    if not args.no_secondary:
        reps, warm = max(200, args.steps), 20
        for name, qt, N, K in (("q4_K_5120x5120_m1", tier_amd.Q4_K, 5120, 5120),
                               ("q4_K_14336x5120_m1", tier_amd.Q4_K, 14336, 5120),
                               ("q4_K_5120x14336_m1", tier_amd.Q4_K, 5120, 14336),
                               ("q8_0_4096x4096_m1", tier_amd.Q8_0, 4096, 4096),
                               ("q5_K_5120x14336_m1", tier_amd.Q5_K, 5120, 14336),
                               ("q6_K_5120x14336_m1", tier_amd.Q6_K, 5120, 14336),
                               # long rows (gemv_q has no K bound, tier.cpp:300-306)
                               ("q4_K_8192x28672_m1", tier_amd.Q4_K, 8192, 28672),
                               ("q5_K_8192x28672_m1", tier_amd.Q5_K, 8192, 28672),
                               ("q8_0_4096x28672_m1", tier_amd.Q8_0, 4096, 28672)):
            if not want(name):
                continue
            log(f"bench: {name}")
            c = GemvCase(tier_amd, hip, qt, N, K, seed=N + K)
            settle(hip, stream, tier_amd, c)
            # median of three timed runs: one run of ~1 ms can catch a stall of the host's
            # launch loop (q4_K 5120x5120 read 7.7 us in one full run against 5.9-6.0 us)
            km = float(np.median([time_gemv(hip, stream, tier_amd, c, reps, warm) for _ in range(3)]))
            secondary[name] = {"GB/s": round(c.bytes / (km * 1e-3) / 1e9, 1),
                               "frac_hbm": round(c.bytes / (km * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                               "us_per_step": round(km * 1e3, 2)}
            del c
        # quantized GEMM at M=512 (config 3), x3-ref semantics
        for name, N, K in (("q4_K_5120x5120_m512", 5120, 5120), ("q4_K_14336x5120_m512", 14336, 5120),
                           ("q4_K_5120x14336_m512", 5120, 14336)):
            if not want(name):
                continue
            log(f"bench: {name}")
            M = 512
            rng = np.random.default_rng(N * 7 + K)
            blocks = tier_amd.q_row(tier_amd.Q4_K, rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
            Wd = hip.to_device(blocks)
            X = hip.to_device(rng.standard_normal((M, K), dtype=np.float32))
            Y = hip.DeviceBuffer(M * N * 4)
            wsb = tier_amd.qgemm_ws_bytes(tier_amd.Q4_K, M, N, K)
            WS = hip.DeviceBuffer(wsb)
            rb = tier_amd.q_row_bytes(tier_amd.Q4_K, K)
            f = lambda i: tier_amd.qgemm(Wd.ptr, tier_amd.Q4_K, rb, X.ptr, Y.ptr, M, N, K, N,  # noqa: E731
                                         tier_amd.MODE_X3REF, 0.0, WS.ptr, wsb, stream)
            km = time_steady(hip, stream, f, 20)
            tf = 2.0 * M * N * K / (km * 1e-3) / 1e12
            secondary[name] = {"TFLOPS": round(tf, 2), "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4),
                               "us_per_call": round(km * 1e3, 1)}
            del Wd, X, Y, WS
    # x3-2x2 GEMM, config 2
    if want("x3s_4096x5120x5120"):
        log("bench: x3s_4096x5120x5120")
        M, N, K = 4096, 5120, 5120
        rng = np.random.default_rng(8)
        Wf = hip.to_device(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        Xf = hip.to_device(rng.standard_normal((M, K), dtype=np.float32))
        bufs = [hip.DeviceBuffer(n) for n in (M * K * 2, M * K * 2, M * 4, N * K * 2, N * K * 2, N * 4, M * N * 4)]
        xh, xl, xe, wh, wl, we, Y = bufs
        tier_amd.x3s_split(Wf.ptr, wh.ptr, wl.ptr, we.ptr, N, K, stream)
        f = lambda i: (tier_amd.x3s_split(Xf.ptr, xh.ptr, xl.ptr, xe.ptr, M, K, stream),  # noqa: E731
                       tier_amd.x3s_gemm(xh.ptr, xl.ptr, xe.ptr, wh.ptr, wl.ptr, we.ptr, Y.ptr, M, N, K, N, stream))
        km = time_steady(hip, stream, f, 20)
        tf = 2.0 * M * N * K / (km * 1e-3) / 1e12
        secondary["x3s_4096x5120x5120"] = {"TFLOPS": round(tf, 2), "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4),
                                           "us_per_call": round(km * 1e3, 1), "includes": "X split + GEMM"}
        del bufs, Wf, Xf
    # fp3gemm (tier.cpp:922-943) on the decoder's down-projection weight (fp16 W 5120x14336),
    # 4096 tokens: the forward (OP_T) and the dX product (OP_N, W read in place), equal flops
    for name, opA in (("x3_fwd_4096x5120x14336", tier_amd.OP_T), ("x3_dx_4096x14336x5120", tier_amd.OP_N)):
        if not want(name):
            continue
        log(f"bench: {name}")
        T, Nw, Kw = 4096, 5120, 14336
        rng = np.random.default_rng(22)
        Wh = hip.to_device((rng.standard_normal((Nw, Kw), dtype=np.float32) * np.float32(0.02)).astype(np.float16))
        if opA == tier_amd.OP_T:  # out[T][Nw] = x[T][Kw] W^T
            m, n, k = Nw, T, Kw
        else:  # dX[T][Kw] = dY[T][Nw] W
            m, n, k = Kw, T, Nw
        Bm = hip.to_device(rng.standard_normal((n, k), dtype=np.float32))
        C = hip.DeviceBuffer(n * m * 4)
        C.fill_bytes(0)
        wsb = tier_amd.x3_gemm_ws_bytes(m, n, k)
        WS = hip.DeviceBuffer(wsb)
        beta = 0.0 if opA == tier_amd.OP_T else 1.0
        f = lambda i: tier_amd.fp3gemm(opA, m, n, k, Wh.ptr, Kw, Bm.ptr, beta, C.ptr, m, WS.ptr, wsb,  # noqa: E731
                                       stream)
        km = time_steady(hip, stream, f, 10)
        tf = 2.0 * m * n * k / (km * 1e-3) / 1e12
        secondary[name] = {"TFLOPS": round(tf, 2), "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4),
                           "us_per_call": round(km * 1e3, 1), "beta": beta,
                           "includes": "x split into three fp16 parts + GEMM (dX: W read in place, no transpose)"}
        del Wh, Bm, C, WS
    # the x3-off fallback's fp32 products (sgemm, tier.cpp:1196-1200, 1229-1236) at the
    # decoder's down projection (W 5120x14336): forward and dX, 4096 tokens, beta = 1 for dX
    for name, opA in (("sgemm_fwd_4096x5120x14336", tier_amd.OP_T), ("sgemm_dx_4096x14336x5120", tier_amd.OP_N)):
        if not want(name):
            continue
        log(f"bench: {name}")
        T, Nw, Kw = 4096, 5120, 14336
        rng = np.random.default_rng(21)
        Wf = hip.to_device(rng.standard_normal((Nw, Kw), dtype=np.float32) * np.float32(0.02))
        if opA == tier_amd.OP_T:  # out[T][Nw] = x[T][Kw] W^T
            m, n, k, lda, Bm = Nw, T, Kw, Kw, hip.to_device(rng.standard_normal((T, Kw), dtype=np.float32))
        else:  # dX[T][Kw] = dY[T][Nw] W
            m, n, k, lda, Bm = Kw, T, Nw, Kw, hip.to_device(rng.standard_normal((T, Nw), dtype=np.float32))
        C = hip.DeviceBuffer(n * m * 4)
        C.fill_bytes(0)
        wsb = tier_amd.sgemm_ws_bytes(opA, m, n, k)
        WS = hip.DeviceBuffer(wsb)
        beta = 0.0 if opA == tier_amd.OP_T else 1.0
        f = lambda i: tier_amd.sgemm(opA, m, n, k, Wf.ptr, lda, Bm.ptr, k, beta, C.ptr, m,  # noqa: E731
                                     WS.ptr, wsb, stream)
        km = time_steady(hip, stream, f, 10)
        tf = 2.0 * m * n * k / (km * 1e-3) / 1e12
        secondary[name] = {"TFLOPS": round(tf, 2), "frac_x3_peak": round(tf / X3_PEAK_TFLOPS, 4),
                           "us_per_call": round(km * 1e3, 1), "beta": beta,
                           "includes": "both operands' two-part splits (dX: column maxima + transposed split) + GEMM"}
        del Wf, Bm, C, WS
    if want("decode_layer_m1"):
        log("bench: decode layer M=1")
        secondary["decode_layer_m1"] = bench_decode_layer(tier_amd, hip, stream)
    if want("decoder_layer_t4096"):
        secondary["decoder_layer_t4096"] = bench_decoder_layer(tier_amd, hip, stream)
    if want("decoder_layer_t4096_shared_splits"):
        secondary["decoder_layer_t4096_shared_splits"] = bench_decoder_layer_shared(tier_amd, hip, stream)
    for T in (256, 4096):  # chat prefill: chunks of 256 rows (tier.cpp:2538), and the config's batch
        if want(f"chat_prefill_t{T}"):
            secondary[f"chat_prefill_t{T}"] = bench_decoder_layer(tier_amd, hip, stream, T, tier_amd.MODE_F32)
    if want("moe_t4096"):
        secondary["moe_t4096"] = bench_moe(tier_amd, hip, stream)
    if want("chat_streamed_4_layers"):
        secondary["chat_streamed_4_layers"] = bench_chat_stream(tier_amd, hip, stream)

    if want("floors"):
        secondary["floors"] = bench_floors(hip, stream, head, per, secondary)

    traffic, traffic_src = measured_traffic()
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline")
        try:
            cpu = cpu_baseline(head, args.cpu_seconds)
        except Exception as e:  # the baseline is reported, not required
            log(f"bench: cpu baseline unavailable: {e}")

    out = {
        "metric": "q4_K dequant-matmul GB/s (M=1) & TFLOPS (M=512), % of MI355X roofline",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_K/fp32",
        "data": "synthetic: W ~N(0,0.02) quantized to q4_K by the host quantizer, x ~N(0,1); "
                f"weight rotated over {head.copies} HBM copies",
        "config": {"workload": "q4_K decode GEMV 13824x5120 (M=1), tiermm_qgemv", "N": 13824, "K": 5120, "M": 1,
                   "bytes_per_step": head.bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "us_per_launch": round(per * 1e3, 3)},
        "cpu_baseline": cpu,
        "device": {"cus": cus, "clock_mhz": clk_mhz},
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)
    stream.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())

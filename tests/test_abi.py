"""The C ABI library on the CPU: it loads, exports every declared symbol, and its
host-side code (registry, quantizer, argument checks) behaves like the reference.
No kernel is launched here."""
import os
import re

import numpy as np
import pytest

import oracle
import tier_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "tiermm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tiermm_\w+)\s*\(", text)))


def test_exports_every_declared_symbol():
    names = _declared()
    assert len(names) >= 18
    lib = tier_amd.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(tier_amd.EXPORTS) == names


def test_probe_library_loads():
    """bench.py's measurement kernels (the read floor and the fp16 MFMA ceiling) build and load."""
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(tier_amd.__file__), "libtiermm_probe.so"))
    for n in ("tiermm_probe_read", "tiermm_probe_read_lds", "tiermm_probe_mfma", "tiermm_bench_qgemv"):
        assert hasattr(lib, n), n


def test_registry_matches_oracle_table():
    for t in (0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29, 30, 34, 35, 39, 200, 201):
        assert tier_amd.q_info(t) == oracle.block(t)
        be, _ = oracle.block(t)
        for cols in (0, be, 256 * be, 5120 if 5120 % be == 0 else be * 3):
            assert tier_amd.q_row_bytes(t, cols) == oracle.row_bytes(t, cols)
    with pytest.raises(tier_amd.TiermmUnsupported):
        tier_amd.q_info(99)
    assert not tier_amd.q_cols_ok(tier_amd.Q4_K, 1408)  # F4: 1408 % 256 != 0
    assert tier_amd.q_cols_ok(tier_amd.Q8_0, 1408)


@pytest.mark.parametrize("name", ["q8_0", "q4_K", "q5_K", "q6_K"])
def test_quantizer_bytes_match_reference_golden(golden, name):
    g = golden["quant"]
    t = {"q8_0": tier_amd.Q8_0, "q4_K": tier_amd.Q4_K, "q5_K": tier_amd.Q5_K, "q6_K": tier_amd.Q6_K}[name]
    got = tier_amd.q_row(t, g["x"], nthreads=3)
    assert np.array_equal(got, g[name])


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference checkout)")
@pytest.mark.parametrize("t", [tier_amd.Q8_0, tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K])
def test_quantizer_bytes_match_reference_build(t):
    rng = np.random.default_rng(100 + t)
    x = np.concatenate([rng.standard_normal((24, 2048)) * 0.02,
                        rng.standard_normal((4, 2048)) * 30,       # large values
                        np.zeros((2, 2048)),                       # all-zero rows
                        rng.standard_normal((2, 2048)) * 1e-9]).astype(np.float32)
    x[0, :256] = 0.0
    x[1, 5] = 1e3  # an outlier inside one block
    assert np.array_equal(tier_amd.q_row(t, x), oracle.ref_quantize(x, t))


@pytest.mark.parametrize("t,lim", [(tier_amd.Q8_0, 0.007), (tier_amd.Q6_K, 0.022), (tier_amd.Q5_K, 0.042),
                                   (tier_amd.Q4_K, 0.08)])
def test_quantizer_error_bounds(t, lim):
    """check_quant.py:105-120: rel. Frobenius error of quantize->dequant on N(0,0.02) rows."""
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((32, 4096)) * 0.02).astype(np.float32)
    back = oracle.dequant(tier_amd.q_row(t, x), t, 4096)
    assert oracle.rel_fro(back, x) <= lim


def test_argument_checks_return_before_device_work():
    L = tier_amd.lib()
    # unknown type id
    assert L.tiermm_dequant(16, 99, 66, 256, 0, 1, 16, tier_amd.OUT_F16, None) == tier_amd.UNSUPPORTED
    # rb inconsistent with cols
    assert L.tiermm_dequant(16, tier_amd.Q4_K, 100, 256, 0, 1, 16, tier_amd.OUT_F16, None) == tier_amd.EINVAL
    # misaligned Q4_K rows
    assert L.tiermm_qgemv(18, tier_amd.Q4_K, 144, 16, 16, 1, 256, None) == tier_amd.EINVAL
    # columns not whole blocks (F4: down_proj K=1408 cannot be Q4_K)
    assert L.tiermm_qgemv(16, tier_amd.Q4_K, 792, 16, 16, 1, 1408, None) == tier_amd.UNSUPPORTED
    # x must be 16-byte aligned (any K is taken: gemv_q has no K bound)
    assert L.tiermm_qgemv(16, tier_amd.Q8_0, 34 * 1024, 20, 16, 1, 32768, None) == tier_amd.EINVAL
    # dX layout: lda must cover m (A is m x k column-major); unknown op / mode
    assert L.tiermm_x3_gemm(tier_amd.OP_N, 64, 64, 64, 16, 32, 16, 0.0, 16, 64, None, 0, None) == tier_amd.EINVAL
    assert L.tiermm_x3_gemm(7, 64, 64, 64, 16, 64, 16, 0.0, 16, 64, None, 0, None) == tier_amd.EINVAL
    assert L.tiermm_qgemm(16, tier_amd.Q4_K, 144, 16, 16, 2, 4, 256, 4, 7, 0.0, None, 0, None) == tier_amd.EINVAL
    # dense GEMV: unknown weight type, misaligned rows
    assert L.tiermm_gemv(16, tier_amd.Q4_K, 16, 16, 4, 64, None) == tier_amd.UNSUPPORTED
    assert L.tiermm_gemv(18, tier_amd.F16, 16, 16, 4, 64, None) == tier_amd.EINVAL
    # grouped GEMM: offsets must start at 0 and not decrease
    import ctypes
    I2 = ctypes.c_int * 2
    assert L.tiermm_qgemm_grouped((ctypes.c_void_p * 1)(16), (ctypes.c_int * 1)(tier_amd.Q4_K),
                                  (ctypes.c_size_t * 1)(144), 16, I2(1, 2), 1, 16, 4, 256, 0, None, 0,
                                  None) == tier_amd.EINVAL
    assert L.tiermm_qgemm_grouped((ctypes.c_void_p * 1)(16), (ctypes.c_int * 1)(tier_amd.Q4_K),
                                  (ctypes.c_size_t * 1)(144), 16, I2(0, -1), 1, 16, 4, 256, 0, None, 0,
                                  None) == tier_amd.EINVAL
    # K not a multiple of the 32-element K step
    assert L.tiermm_x3s_gemm(16, 16, 16, 16, 16, 16, 16, 4, 4, 48, 4, None) == tier_amd.UNSUPPORTED
    assert L.tiermm_split3_f16(16, 16, 10, 5, 0, None) == tier_amd.EINVAL
    assert "part_stride" in tier_amd.last_error()
    # pre-split x: K in whole 32-steps, aligned planes at least M*K apart
    assert L.tiermm_qgemm_x3parts(16, tier_amd.F16, 96, 16, 96, 0, 16, 2, 4, 48, 4, 0.0, None, 0,
                                  None) == tier_amd.UNSUPPORTED
    assert L.tiermm_qgemm_x3parts(16, tier_amd.Q4_K, 144, 16, 511, 0, 16, 2, 4, 256, 4, 0.0, None, 0,
                                  None) == tier_amd.EINVAL
    assert L.tiermm_qgemm_x3parts(16, tier_amd.Q4_K, 144, 18, 512, 1, 16, 2, 4, 256, 4, 0.0, None, 0,
                                  None) == tier_amd.EINVAL
    assert L.tiermm_qgemm_x3parts(16, tier_amd.Q4_K, 144, 16, 512, 2, 16, 2, 4, 256, 4, 0.0, None, 0,
                                  None) == tier_amd.EINVAL  # unknown layout
    assert L.tiermm_split3_f16_ktiled(16, 16, 2, 48, 96, None) == tier_amd.UNSUPPORTED
    # chat_fp3 mirrors: an unsupported shape -> False, not an exception (the allocation-free
    # variant keeps K a multiple of 32: it has no workspace to pad into)
    assert tier_amd.chat_fp3_noalloc(16, 16, 16, 4, 48, 4, 4) is False
    # legacy 32-blocks and dense rows are GPU types now; dense rows of any length, written
    # element by element to an output of their natural alignment
    assert L.tiermm_dequant(16, tier_amd.Q4_1, 19, 32, 0, 1, 16, tier_amd.OUT_F16, None) == tier_amd.EINVAL
    assert L.tiermm_dequant(16, tier_amd.F16, 24, 12, 0, 1, 17, tier_amd.OUT_F16, None) == tier_amd.EINVAL
    assert "2-byte aligned" in tier_amd.last_error()
    assert L.tiermm_qgemv(18, tier_amd.F16, 128, 16, 16, 1, 64, None) == tier_amd.EINVAL  # dense rows 16-aligned
    # batched GEMV: batch size, negative rows, a misaligned weight of a live matrix, a null
    # output of a live matrix, misaligned x; matrices without rows are not read
    VP4, I4 = ctypes.c_void_p * 5, ctypes.c_int * 5
    bq = lambda w, y, n, cnt, x=16: L.tiermm_qgemv_batch(VP4(*w), tier_amd.Q4_K, 144, x, VP4(*y), I4(*n), cnt, 256,
                                                          None)
    assert bq([16] * 5, [16] * 5, [16] * 5, 5) == tier_amd.EINVAL
    assert bq([16] * 5, [16] * 5, [16] * 5, 0) == tier_amd.EINVAL
    assert bq([16, 16, 0, 0, 0], [16, 16, 0, 0, 0], [16, -1, 0, 0, 0], 2) == tier_amd.EINVAL
    assert bq([16, 18, 0, 0, 0], [16, 16, 0, 0, 0], [16, 16, 0, 0, 0], 2) == tier_amd.EINVAL
    assert bq([16, 16, 0, 0, 0], [16, 0, 0, 0, 0], [16, 16, 0, 0, 0], 2) == tier_amd.EINVAL
    assert bq([16, 16, 0, 0, 0], [16, 16, 0, 0, 0], [16, 16, 0, 0, 0], 2, x=20) == tier_amd.EINVAL
    assert bq([0, 0, 0, 0, 0], [0, 0, 0, 0, 0], [0, 0, 0, 0, 0], 3) == tier_amd.OK  # no rows: nothing to do
    # chat set: slot count, null handles, registration checks (no HIP call on these paths)
    out = ctypes.c_void_p()
    assert L.tiermm_chat_create(1, None, ctypes.byref(out)) == tier_amd.EINVAL and not out.value
    assert L.tiermm_chat_create(9, None, ctypes.byref(out)) == tier_amd.EINVAL
    assert L.tiermm_chat_create(2, None, None) == tier_amd.EINVAL
    i = ctypes.c_int()
    assert L.tiermm_chat_add(None, tier_amd.Q4_K, 144, 1, 256, 16, None, ctypes.byref(i)) == tier_amd.EINVAL
    assert L.tiermm_chat_place(None, 0, 0, None, None) == tier_amd.EINVAL
    assert L.tiermm_chat_lin(None, 0, 16, 16, 1, 0) == tier_amd.EINVAL
    assert L.tiermm_chat_restart(None, 0) == tier_amd.EINVAL
    assert L.tiermm_chat_info(None, 0, None, None, None, None) == tier_amd.EINVAL
    L.tiermm_chat_destroy(None)
    assert L.tiermm_host_free(None) == tier_amd.OK
    assert L.tiermm_host_alloc(16, None) == tier_amd.EINVAL


def test_workspace_sizes():
    # three planes of B, plus the transposed weight for TIERMM_OP_N
    assert tier_amd.x3_gemm_ws_bytes(5120, 4096, 5120) == 3 * 4096 * 5120 * 2 + 5120 * 5120 * 2
    assert tier_amd.x3_rows_ws_bytes(256, 5120, 14336) == 3 * 256 * 5120 * 2
    # the fused types decode W inside the GEMM at every M: the three fp16 planes of x, then
    # split-K partial sums (2 splits at this shape on 256 CUs)
    for t in (tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K, tier_amd.Q8_0):
        assert tier_amd.qgemm_ws_bytes(t, 512, 5120, 5120) == 3 * 512 * 5120 * 2 + 2 * 512 * 5120 * 4
        assert tier_amd.qgemm_ws_bytes(t, 4096, 5120, 5120) == 3 * 4096 * 5120 * 2
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q4_K, 512, 14336, 5120) == 3 * 512 * 5120 * 2
    # K = 14336 at M = 4096: four K splits with partial sums (up to 1 GiB of them); at
    # M = 16384 those would not fit, and four K chunks are added into Y in turn instead
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q5_K, 4096, 5120, 14336) == \
        3 * 4096 * 14336 * 2 + 4 * 4096 * 5120 * 4
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q5_K, 16384, 5120, 14336) == 3 * 16384 * 14336 * 2
    # other types stage fp16 W in the workspace as well
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q4_0, 512, 5120, 5120) == 5120 * 5120 * 2 + 3 * 512 * 5120 * 2
    # the fp32 semantics: the fused types keep no copy of W (x's hi and lo planes, the
    # row exponents of x and W, and at K = 14336 four K splits of partial sums); the others expand
    # W in chunks of rows within 256 MiB (1600 rows of K = 20480: 1638 rounded down to
    # whole 320-row tiles)
    F32 = tier_amd.MODE_F32
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q4_K, 256, 14336, 5120, F32) == 2 * 256 * 5120 * 2 + 1024 + 14336 * 4
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q6_K, 256, 5120, 14336, F32) == \
        2 * 256 * 14336 * 2 + 1024 + 5120 * 4 + 4 * 256 * 5120 * 4
    K = 20480
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q4_0, 256, 14336, K, F32) == \
        1600 * K * 4 + 2 * 1600 * K * 2 + 1600 * 4 + 2 * 256 * K * 2 + 1024
    # at M = 4096 the chunk grows to the 3840 rows that give the big-tile kernel its
    # 192 tiles (16 x 12), where the weight has them
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q4_0, 4096, 14336, K, F32) == \
        3840 * K * 4 + 2 * 3840 * K * 2 + 3840 * 4 + 2 * 4096 * K * 2 + 4096 * 4
    assert tier_amd.qgemm_ws_bytes(tier_amd.Q4_0, 4096, 3000, K, F32) == \
        1600 * K * 4 + 2 * 1600 * K * 2 + 1600 * 4 + 2 * 4096 * K * 2 + 4096 * 4
    # routed experts: 256-row tiles that fill the chip stage the fp16 weights of
    # up to 64 experts (1 GiB at most); few or mostly empty tiles keep one expert's
    E, N, K = 64, 1408, 2048
    full = [512 * e for e in range(E + 1)]
    planes = 3 * full[-1] * K * 2
    assert tier_amd.qgemm_grouped_ws_bytes([tier_amd.Q4_0] * E, full, N, K) == planes + 64 * N * K * 2
    assert tier_amd.qgemm_grouped_ws_bytes([tier_amd.Q4_0] * E, full, 14336, 5120) == \
        planes // K * 5120 + (1 << 30) // (14336 * 5120 * 2) * 14336 * 5120 * 2
    # every routed type decoded inside the GEMM: the planes only
    assert tier_amd.qgemm_grouped_ws_bytes([tier_amd.Q5_0] * E, full, N, K) == planes
    assert tier_amd.qgemm_grouped_ws_bytes([tier_amd.Q4_K, tier_amd.Q6_K] * (E // 2), full, N, K) == planes
    sparse = [100 * e for e in range(E + 1)]  # 100 rows per 256-row tile
    assert tier_amd.qgemm_grouped_ws_bytes([tier_amd.Q4_0] * E, sparse, N, K) == \
        3 * sparse[-1] * K * 2 + N * K * 2
    for t in (tier_amd.Q4_K, tier_amd.Q5_0):  # decoded inside the grouped GEMM
        assert tier_amd.qgemm_grouped_ws_bytes([t] * E, sparse, N, K) == 3 * sparse[-1] * K * 2


def _mats(n_layers, no_v=()):
    keys = tier_amd.SLOTS
    return [(l, k, 0, 0) for l in range(n_layers) for k in keys if not (k == "self_attn.v_proj" and l in no_v)]


def test_recipe_types_hand_checked():
    """tier.cpp:2701-2713 / tierlm.py:1858-1874 on stacks worked out by hand: with 8 layers the
    "more" layers are 0 (first eighth), 7 (last eighth), 3 and 6 (every third after the first eighth)."""
    def of(rec, mats, key):
        return [t for (l, k, *_), t in zip(mats, tier_amd.recipe_types(rec, mats)) if k == key]
    m8 = _mats(8)
    assert of("Q4_K_M", m8, "self_attn.v_proj") == ["q6_K", "q4_K", "q4_K", "q6_K", "q4_K", "q4_K", "q6_K", "q6_K"]
    assert of("Q4_K_M", m8, "mlp.down_proj") == ["q6_K", "q4_K", "q4_K", "q6_K", "q4_K", "q4_K", "q6_K", "q6_K"]
    assert of("Q4_K_M", m8, "self_attn.q_proj") == ["q4_K"] * 8
    assert of("Q4_K_S", m8, "self_attn.v_proj") == ["q5_K"] * 4 + ["q4_K"] * 4
    assert of("Q4_K_S", m8, "mlp.down_proj") == ["q5_K"] + ["q4_K"] * 7
    assert of("Q5_K_S", m8, "self_attn.v_proj") == ["q5_K"] * 8
    assert of("Q5_K_M", m8, "mlp.down_proj") == ["q6_K", "q5_K", "q5_K", "q6_K", "q5_K", "q5_K", "q6_K", "q6_K"]
    assert set(tier_amd.recipe_types("Q6_K", m8)) == {"q6_K"}
    assert set(tier_amd.recipe_types("Q8_0", m8)) == {"q8_0"}
    # 48 layers: first and last six, and 8, 11, ..., 41
    raised = set(range(6)) | set(range(42, 48)) | set(range(8, 42, 3))
    downs = of("Q4_K_M", _mats(48), "mlp.down_proj")
    assert [i for i, t in enumerate(downs) if t == "q6_K"] == sorted(raised)
    # v_proj ranks count only the layers that have one: without v in layers 2 and 5, the
    # six v_proj have ranks 0..5 and the raised ranks are 2 and 5 (layers 3 and 7)
    mv = _mats(8, no_v=(2, 5))
    assert of("Q4_K_M", mv, "self_attn.v_proj") == ["q4_K", "q4_K", "q6_K", "q4_K", "q4_K", "q6_K"]
    with pytest.raises(tier_amd.TiermmError):
        tier_amd.recipe_types("Q3_K", m8)


def test_qgemm_plan_query(monkeypatch):
    """The fused GEMM's plan query (no device needed): types it does not decode have none, a
    valid TIERMM_QGEMM_TILE is the plan run, an invalid one falls back to the cost model."""
    monkeypatch.delenv("TIERMM_QGEMM_TILE", raising=False)
    assert tier_amd.qgemm_plan(tier_amd.Q4_0, 300, 1000, 8192) is None
    model = tier_amd.qgemm_plan(tier_amd.Q4_K, 300, 1000, 8192)
    bn, ks, kc = model
    assert ks * kc >= 2  # K = 8192 needs at least two accumulators (K chunks of at most 6144)
    monkeypatch.setenv("TIERMM_QGEMM_TILE", "128,1,2")
    assert tier_amd.qgemm_plan(tier_amd.Q4_K, 300, 1000, 8192) == (128, 1, 2)
    monkeypatch.setenv("TIERMM_QGEMM_TILE", "100,1,2")  # no such tile width
    assert tier_amd.qgemm_plan(tier_amd.Q4_K, 300, 1000, 8192) == model

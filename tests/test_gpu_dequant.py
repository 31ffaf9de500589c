"""GPU parity of tiermm_dequant (dq_k<T>, tier.cpp:293-298): bit-exact with the oracle."""
import numpy as np
import pytest

import oracle
import tier_amd
from helpers import quantized_weight
from tier_amd import hip

pytestmark = pytest.mark.gpu

TYPES = {"q8_0": tier_amd.Q8_0, "q5_0": tier_amd.Q5_0, "q4_K": tier_amd.Q4_K, "q5_K": tier_amd.Q5_K,
         "q6_K": tier_amd.Q6_K}
OUTS = {"f32": (tier_amd.OUT_F32, np.uint32), "f16": (tier_amd.OUT_F16, np.uint16),
        "bf16": (tier_amd.OUT_BF16, np.uint16)}


def _expect(blocks, t, cols, out, r0=0, nrows=None):
    f = oracle.dequant(blocks, t, cols, oracle.OUT_F32, r0, nrows)
    if out == tier_amd.OUT_F32:
        return f.view(np.uint32).ravel()
    if out == tier_amd.OUT_F16:
        return oracle.f2h(f)
    return oracle.f2bf(f)


def _run(gpu, blocks, t, cols, out, r0=0, nrows=None):
    rb = tier_amd.q_row_bytes(t, cols)
    rows = blocks.size // rb
    nrows = rows - r0 if nrows is None else nrows
    esz = 4 if out == tier_amd.OUT_F32 else 2
    W = hip.to_device(blocks)
    O = hip.DeviceBuffer(max(nrows * cols * esz, 16))
    tier_amd.dq_launch(W.ptr, t, rb, cols, r0, nrows, O.ptr, out)
    hip.synchronize()
    return O.download(np.uint32 if esz == 4 else np.uint16, nrows * cols)


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("outname", list(OUTS))
def test_dequant_golden_blocks(gpu, golden, name, outname):
    """Random blocks of every type (check_quant.py's construction) against the reference's own values."""
    t = TYPES[name]
    out = OUTS[outname][0]
    if name == "q5_0":
        rng = np.random.default_rng(9)
        blocks = oracle.random_blocks(rng, t, 512 // 32 * 8)
    else:
        blocks = golden["dequant"][f"{name}_blocks"]
    cols = 512
    got = _run(gpu, blocks, t, cols, out)
    want = _expect(blocks, t, cols, out)
    if name != "q5_0" and out == tier_amd.OUT_F32:
        assert np.array_equal(want, golden["dequant"][f"{name}_f32bits"].ravel())
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name", list(TYPES))
def test_dequant_quantized_weights_rows_subset(gpu, name):
    """N(0,0.02) weights quantized by the host quantizer; rows r0..r0+nrows only (chat prefill chunks)."""
    t = TYPES[name]
    N, K = 40, 5120
    blocks = quantized_weight(t, N, K, seed=30 + t)
    for out in (tier_amd.OUT_F16, tier_amd.OUT_F32):
        got = _run(gpu, blocks, t, K, out, r0=7, nrows=29)
        assert np.array_equal(got, _expect(blocks, t, K, out, 7, 29))


def test_dequant_special_blocks(gpu):
    """fp16 subnormal and zero scales, extreme 6-bit scales, all nibble values (bit-exact incl. fp16 subnormal outputs)."""
    rng = np.random.default_rng(77)
    cases = []
    for d in (0.0, 2.0 ** -24, 3 * 2.0 ** -24, 6.1e-5, 1.0, -2.0, 65504.0 / 1024):
        b = rng.integers(0, 256, size=(4, 144), dtype=np.uint8)
        b[:, 0:2] = np.array([d], np.float16).view(np.uint8)
        b[:, 2:4] = np.array([abs(d) / 3], np.float16).view(np.uint8)
        b[1, 4:16] = 0xff
        b[2, 4:16] = 0
        cases.append(b)
    blocks = np.concatenate(cases)
    for out in OUTS.values():
        got = _run(gpu, blocks, tier_amd.Q4_K, 256, out[0])
        assert np.array_equal(got, _expect(blocks, tier_amd.Q4_K, 256, out[0]))
    q6 = rng.integers(0, 256, size=(6, 210), dtype=np.uint8)
    q6[0, 192:208] = 0x80  # int8 scales -128
    q6[1, 192:208] = 0x7f
    q6[:, 208:210] = np.array([2.0 ** -20], np.float16).view(np.uint8)
    got = _run(gpu, q6, tier_amd.Q6_K, 256, tier_amd.OUT_F16)
    assert np.array_equal(got, _expect(q6, tier_amd.Q6_K, 256, tier_amd.OUT_F16))


def test_dequant_full_layer_shape(gpu):
    """A whole 14336x5120 Q4_K matrix to fp16 (the training path's dq_launch, tier.cpp:515), checked by hash of rows."""
    t, N, K = tier_amd.Q4_K, 14336, 5120
    blocks = quantized_weight(t, N, K, seed=41)
    got = _run(gpu, blocks, t, K, tier_amd.OUT_F16).reshape(N, K)
    rows = np.random.default_rng(0).choice(N, 300, replace=False)
    rows = np.concatenate([rows, [0, N - 1]])
    for r in rows:
        assert np.array_equal(got[r], _expect(blocks[r:r + 1], t, K, tier_amd.OUT_F16)), r


MORE = {"q4_0": tier_amd.Q4_0, "q4_1": tier_amd.Q4_1, "q5_1": tier_amd.Q5_1}


@pytest.mark.parametrize("name", list(MORE))
@pytest.mark.parametrize("outname", list(OUTS))
def test_dequant_golden_blocks_legacy_types(gpu, golden, name, outname):
    """Q4_0 / Q4_1 / Q5_1 (quant.h:64-67) against the reference's own values and the oracle."""
    t, out = MORE[name], OUTS[outname][0]
    blocks = golden["dequant"][f"{name}_blocks"]
    got = _run(gpu, blocks, t, 512, out)
    want = _expect(blocks, t, 512, out)
    if out == tier_amd.OUT_F32:
        assert np.array_equal(want, golden["dequant"][f"{name}_f32bits"].ravel())
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name", list(MORE))
def test_dequant_legacy_types_random_rows(gpu, name):
    """Random blocks (fp16 scales and minimums ~N(0,0.02)), a row window, every output type."""
    t = MORE[name]
    rng = np.random.default_rng(50 + t)
    K = 1024
    blocks = oracle.random_blocks(rng, t, 37 * K // 32)
    for out in OUTS.values():
        got = _run(gpu, blocks, t, K, out[0], r0=5, nrows=31)
        assert np.array_equal(got, _expect(blocks, t, K, out[0], 5, 31))


@pytest.mark.parametrize("t", [tier_amd.F32, tier_amd.F16, tier_amd.BF16])
def test_dequant_dense_rows(gpu, t):
    """q_val's F32 / F16 / BF16 cases (quant.h:61-63): conversions of stored rows, incl. fp16 subnormals."""
    rng = np.random.default_rng(60 + t)
    K, N = 264, 9
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    w[0, :8] = [0.0, -0.0, 2.0 ** -24, -(2.0 ** -20), 65504.0, -65504.0, 1e-30, 1.5e4]
    if t == tier_amd.F32:
        blocks = w.view(np.uint8)
    elif t == tier_amd.F16:
        blocks = w.astype(np.float16).view(np.uint8)
    else:
        blocks = oracle.f2bf(w).view(np.uint8)
    blocks = np.ascontiguousarray(blocks).reshape(N, -1)
    for out in OUTS.values():
        got = _run(gpu, blocks, t, K, out[0])
        assert np.array_equal(got, _expect(blocks, t, K, out[0]))


TABLED = {"q2_K": tier_amd.Q2_K, "q3_K": tier_amd.Q3_K, "iq4_nl": tier_amd.IQ4_NL, "iq4_xs": tier_amd.IQ4_XS,
          "tq1_0": tier_amd.TQ1_0, "tq2_0": tier_amd.TQ2_0, "mxfp4": tier_amd.MXFP4, "nf4": tier_amd.NF4,
          "fp4": tier_amd.FP4}


@pytest.mark.parametrize("name", list(TABLED))
@pytest.mark.parametrize("outname", list(OUTS))
def test_dequant_more_types_bit_exact(gpu, name, outname):
    """q_val's other closed-form and 16-level types (quant.h:69-73, 76-80, 92-94, 116-119), every byte
    value in the payload, against the oracle (itself pinned to the reference build)."""
    t, out = TABLED[name], OUTS[outname][0]
    be, bb = oracle.block(t)
    rng = np.random.default_rng(90 + t)
    blocks = oracle.random_blocks(rng, t, 512)
    if t == tier_amd.MXFP4:
        blocks[:4, 0] = [0, 1, 2, 254]  # subnormal, smallest normal and near-overflow scales
    cols = be * 64
    got = _run(gpu, blocks.reshape(512 * bb // tier_amd.q_row_bytes(t, cols), -1), t, cols, out)
    want = _expect(blocks, t, cols, out)
    assert np.array_equal(got, want)


LATTICE = {"iq2_xxs": tier_amd.IQ2_XXS, "iq2_xs": tier_amd.IQ2_XS, "iq2_s": tier_amd.IQ2_S,
           "iq3_xxs": tier_amd.IQ3_XXS, "iq3_s": tier_amd.IQ3_S, "iq1_s": tier_amd.IQ1_S, "iq1_m": tier_amd.IQ1_M}


@pytest.mark.parametrize("name", list(LATTICE))
@pytest.mark.parametrize("outname", list(OUTS))
def test_dequant_lattice_types_bit_exact(gpu, golden, name, outname):
    """The lattice-grid types (quant.h:95-115): the golden blocks against the reference's own values,
    and 3000 random blocks -- enough that every grid point is read (test_oracle checks that on the
    same construction) -- against the oracle, which is pinned to the reference build."""
    t, out = LATTICE[name], OUTS[outname][0]
    blocks = golden["dequant"][f"{name}_blocks"]
    got = _run(gpu, blocks, t, 512, out)
    want = _expect(blocks, t, 512, out)
    if out == tier_amd.OUT_F32:
        assert np.array_equal(want, golden["dequant"][f"{name}_f32bits"].ravel())
    assert np.array_equal(got, want)
    rng = np.random.default_rng(300 + t)
    blocks = oracle.random_blocks(rng, t, 3000).reshape(300, -1)
    assert np.array_equal(_run(gpu, blocks, t, 2560, out), _expect(blocks, t, 2560, out))

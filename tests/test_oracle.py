"""The oracle pinned against the reference's golden vectors and the mathematics (CPU only).

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong shift or byte offset, a swapped scale/min) fails it.
"""
import os

import numpy as np
import pytest

import oracle

NAMES = {"q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1, "q5_0": oracle.Q5_0, "q5_1": oracle.Q5_1,
         "q8_0": oracle.Q8_0, "q4_K": oracle.Q4_K, "q5_K": oracle.Q5_K, "q6_K": oracle.Q6_K,
         "iq2_xxs": oracle.IQ2_XXS, "iq2_xs": oracle.IQ2_XS, "iq2_s": oracle.IQ2_S, "iq3_xxs": oracle.IQ3_XXS,
         "iq3_s": oracle.IQ3_S, "iq1_s": oracle.IQ1_S, "iq1_m": oracle.IQ1_M}


# ------------------------------------------------------------------ golden vectors
@pytest.mark.parametrize("name", list(NAMES))
def test_dequant_matches_reference_golden(golden, name):
    g = golden["dequant"]
    cols = int(g["cols"])
    blocks = g[f"{name}_blocks"]
    got = oracle.dequant(blocks, NAMES[name], cols)
    want = g[f"{name}_f32bits"]
    assert np.array_equal(got.view(np.uint32), want), name


def test_f2h_matches_reference_golden(golden):
    g = golden["f16"]
    assert np.array_equal(oracle.f2h(g["f32"]), g["f2h"])


# types without golden vectors in the reference's tests: pinned against the reference build
MORE = {"q2_K": oracle.Q2_K, "q3_K": oracle.Q3_K, "iq4_nl": oracle.IQ4_NL, "iq4_xs": oracle.IQ4_XS,
        "tq1_0": oracle.TQ1_0, "tq2_0": oracle.TQ2_0, "mxfp4": oracle.MXFP4, "nf4": oracle.NF4, "fp4": oracle.FP4}


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference checkout)")
@pytest.mark.parametrize("name", list(NAMES) + list(MORE))
def test_dequant_matches_reference_build(name):
    t = NAMES[name] if name in NAMES else MORE[name]
    rng = np.random.default_rng(1000 + t)
    be, bb = oracle.block(t)
    cols = 2048
    blocks = oracle.random_blocks(rng, t, cols // be * 16)
    got = oracle.dequant(blocks, t, cols)
    want = oracle.ref_dequant(blocks, t, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference checkout)")
def test_row_bytes_and_h2f_match_reference_build():
    R = oracle.ref()
    for t in (0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29, 30, 34, 35, 39, 200, 201, 99):
        for cols in (0, 256, 512, 1408, 5120):
            assert oracle.row_bytes(t, cols) == R.ref_q_row_bytes(t, cols), (t, cols)
    for h in range(0, 65536, 7):
        a = np.float32(oracle.lib().orc_h2f(h))
        b = np.float32(R.ref_q_h2f(h))
        if np.isnan(a):
            assert np.isnan(b)
        else:
            assert a.view(np.uint32) == b.view(np.uint32), h


# ------------------------------------------------------------- fp16 / bf16 conversion
def test_h2f_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.h2f(h)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin]) == np.isnan(want[~fin]))


def test_f2h_roundtrip_all_fp16():
    """Every finite fp16 value converts back to itself (cpu_gpu_sim.py:113-118)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    fin = ((h >> 10) & 31) != 31
    assert np.array_equal(oracle.f2h(oracle.h2f(h[fin])), h[fin])
    nan = h[((h >> 10) & 31) == 31]
    nan = nan[(nan & 1023) != 0]
    assert np.all((oracle.f2h(oracle.h2f(nan)) & 0x7fff) == 0x7e00)  # NaN -> sign|0x7e00


def _f2h_sample():
    """fp32 bit patterns: every 61st pattern, plus all patterns within +-4 of each fp16 rounding boundary region."""
    step = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    # values around the fp16 subnormal/normal/overflow boundaries and ties
    edges = []
    for e in range(100, 145):
        base = np.uint32(e << 23)
        for m in (0, 0x1000, 0x2000, 0x3000, 0x7fe000, 0x7ff000, 0x400000, 0x401000):
            for d in range(-4, 5):
                edges.append((int(base) + m + d) & 0xffffffff)
    e = np.array(edges, dtype=np.uint32)
    u = np.concatenate([step, e, e | np.uint32(0x80000000)])
    return u.view(np.float32)


def test_f2h_vs_numpy_rne():
    f = _f2h_sample()
    f = f[np.isfinite(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f2h(f), want)


@pytest.mark.skipif(os.environ.get("TIER_EXHAUSTIVE") != "1", reason="set TIER_EXHAUSTIVE=1 for all 2^32 inputs")
def test_f2h_exhaustive_vs_numpy():
    for c in range(256):
        u = (np.arange(1 << 24, dtype=np.uint64) + (c << 24)).astype(np.uint32)
        f = u.view(np.float32)
        fin = np.isfinite(f)
        with np.errstate(over="ignore"):
            want = f.astype(np.float16).view(np.uint16)
        got = oracle.f2h(f)
        assert np.array_equal(got[fin], want[fin]), c


def test_f2bf_vs_round_to_nearest_even():
    rng = np.random.default_rng(3)
    u = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 1 << 16, size=4096, dtype=np.uint32) << 16) | np.uint32(0x8000)
    u = np.concatenate([u, ties, ties + np.uint32(1), ties - np.uint32(1)])
    f = u.view(np.float32)
    f = f[np.isfinite(f)]
    # exact RNE in float64: bf16 keeps 8 significant bits; compare the decoded value
    got = (oracle.f2bf(f).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    lo = (f.view(np.uint32) & np.uint32(0xffff0000)).view(np.float32).astype(np.float64)
    hi_bits = (f.view(np.uint32) & np.uint32(0xffff0000)) + np.uint32(0x10000)
    hi = hi_bits.view(np.float32).astype(np.float64)
    # past the largest bf16 the next step is 2^128 in unbounded arithmetic, which rounds to inf
    over = np.isinf(hi)
    hi[over] = np.copysign(2.0 ** 128, x[over])
    dlo, dhi = np.abs(x - lo), np.abs(hi - x)
    lo_even = ((f.view(np.uint32) >> 16) & 1) == 0
    want = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo_even, lo, hi)))
    want[np.abs(want) == 2.0 ** 128] *= np.inf
    assert np.array_equal(got, want)


# ------------------------------------------------------------- closed-form block cases
def _q4k_block(d, dmin, scs, mns, nibbles):
    """Build one Q4_K block from scales/mins (6-bit) and 256 nibbles: inverse of quant.h:47-48, 83-84."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    q = np.zeros(12, np.uint8)
    for j in range(8):
        ls, lm = scs[j], mns[j]
        if j < 4:
            q[j] = ls
            q[j + 4] = lm
        else:
            q[j + 4] = (ls & 15) | ((lm & 15) << 4)
            q[j - 4] |= (ls >> 4) << 6
            q[j] |= (lm >> 4) << 6
    b[4:16] = q
    for g in range(4):
        for l in range(32):
            b[16 + 32 * g + l] = nibbles[64 * g + l] | (nibbles[64 * g + 32 + l] << 4)
    return b


def test_q4k_closed_form():
    rng = np.random.default_rng(21)
    for _ in range(20):
        d = float(np.float16(rng.standard_normal() * 0.01))
        dmin = float(np.float16(abs(rng.standard_normal()) * 0.01))
        scs = rng.integers(0, 64, 8)
        mns = rng.integers(0, 64, 8)
        nib = rng.integers(0, 16, 256)
        blk = _q4k_block(d, dmin, scs, mns, nib)
        got = oracle.dequant(blk, oracle.Q4_K, 256)[0]
        s = np.arange(256) // 32
        # exact products, one rounding for the subtraction (done in float32)
        want = (np.float32(d) * scs[s].astype(np.float32) * nib.astype(np.float32)) - \
            (np.float32(dmin) * mns[s].astype(np.float32))
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_q4k_special_cases():
    nib = np.full(256, 15)
    blk = _q4k_block(0.0, 0.0, [63] * 8, [63] * 8, nib)
    assert np.all(oracle.dequant(blk, oracle.Q4_K, 256) == 0)             # d = dmin = 0
    blk = _q4k_block(1.0, 0.0, [63] * 8, [0] * 8, nib)
    assert np.all(oracle.dequant(blk, oracle.Q4_K, 256) == 63 * 15)      # max scale * max nibble
    sub = float(np.float16(2.0 ** -24))                                   # smallest fp16 subnormal d
    blk = _q4k_block(sub, sub, [1] * 8, [1] * 8, np.arange(256) % 16)
    want = (np.float32(sub) * (np.arange(256) % 16)).astype(np.float32) - np.float32(sub)
    assert np.array_equal(oracle.dequant(blk, oracle.Q4_K, 256)[0], want)


def test_q6k_closed_form_and_sign_extremes():
    rng = np.random.default_rng(22)
    for trial in range(10):
        d = float(np.float16(rng.standard_normal() * 0.01))
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        if trial == 0:
            sc[:] = -128
        q = rng.integers(0, 64, 256)  # stored value; element = q - 32
        b = np.zeros(210, np.uint8)
        for i in range(256):
            a, r = i // 128, i % 128
            b[64 * a + r % 64] |= (q[i] & 15) << (4 * (r // 64))
            b[128 + 32 * a + r % 32] |= (q[i] >> 4) << (2 * (r // 32))
        b[192:208] = sc.view(np.uint8)
        b[208:210] = np.array([d], np.float16).view(np.uint8)
        got = oracle.dequant(b, oracle.Q6_K, 256)[0]
        want = np.float32(d) * sc[np.arange(256) // 16].astype(np.float32) * (q - 32).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_q8_0_all_int8_values():
    b = np.zeros((8, 34), np.uint8)
    vals = np.arange(-128, 128, dtype=np.int8).reshape(8, 32)
    b[:, 2:] = vals.view(np.uint8)
    b[:, 0:2] = np.array([0.5], np.float16).view(np.uint8)
    got = oracle.dequant(b.reshape(-1), oracle.Q8_0, 256)[0]
    assert np.array_equal(got, vals.reshape(-1).astype(np.float32) * 0.5)


def test_q5k_fifth_bit():
    """Q5_K element = nibble | qh bit (i/32) of byte i%32 (quant.h:86): set every high bit."""
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[4:8] = 1  # sc = 1 for sub-blocks 0..3
    b[12:16] = 1  # sc low bits for sub-blocks 4..7
    b[16:48] = 0xff
    got = oracle.dequant(b, oracle.Q5_K, 256)[0]
    assert np.all(got == 16.0)
    b[16:48] = 0
    b[16 + 5] = 1 << 3  # element 3*32+5 = 101
    got = oracle.dequant(b, oracle.Q5_K, 256)[0]
    assert got[101] == 16.0 and np.count_nonzero(got) == 1


# ------------------------------------------------------------------- GEMV / split
def test_gemv_lanes_close_to_f64():
    """The reference's lane-strided fp32 gemv_q sits within 1e-6 of fp64 (sets the scale of the GPU bar)."""
    rng = np.random.default_rng(4)
    blocks = oracle.random_blocks(rng, oracle.Q4_K, 64 * 20)
    x = rng.standard_normal(5120).astype(np.float32)
    y64 = oracle.gemv_f64(blocks, oracle.Q4_K, x, 64, 5120)
    y32 = oracle.gemv_lanes(blocks, oracle.Q4_K, x, 64, 5120, 64)
    assert oracle.rel_fro(y32, y64) < 1e-6
    # and the fp64 GEMV is the fp64 dot of the dequantized rows
    W = oracle.dequant(blocks, oracle.Q4_K, 5120).astype(np.float64)
    assert oracle.rel_fro(W @ x.astype(np.float64), y64) < 1e-14


def test_split3_reconstruction():
    """h+m+l reconstructs x: triple_rel < 0.02 * single_rel (cpu_gpu_sim.py:142-153), v-h exact."""
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-60000, 60000, 100000),
                        np.ldexp(rng.uniform(-1, 1, 10000), rng.integers(-40, 10, 10000))]).astype(np.float32)
    n = x.size
    p = oracle.split3(x, order=0)
    h, m, l = (oracle.h2f(p[i * n:(i + 1) * n]).astype(np.float64) for i in range(3))
    xd = x.astype(np.float64)
    single = np.sqrt(((h - xd) ** 2).sum() / (xd ** 2).sum())
    triple = np.sqrt(((h + m + l - xd) ** 2).sum() / (xd ** 2).sum())
    assert triple < 0.02 * single
    # h is the RNE fp16 of x, m the RNE of the exact residual
    assert np.array_equal(p[:n], oracle.f2h(x))
    assert np.array_equal(p[n:2 * n], oracle.f2h((x - h.astype(np.float32)).astype(np.float32)))
    # LMH layout holds the same parts in reverse order
    q = oracle.split3(x, order=1, stride=n + 3)
    assert np.array_equal(q[:n], p[2 * n:]) and np.array_equal(q[2 * (n + 3):], p[:n])


def test_split3_gemv_accuracy():
    """x3 GEMV with fp16 weights: triple error < 0.15 * single-pass error (cpu_gpu_sim.py:155-180)."""
    rng = np.random.default_rng(0x71e2)
    R, K = 19, 67
    w = oracle.h2f(oracle.f2h(rng.uniform(-1, 1, R * K).astype(np.float32))).reshape(R, K)
    x = rng.uniform(-100, 100, K).astype(np.float32)
    p = oracle.split3(x)
    xh, xm, xl = (oracle.h2f(p[i * K:(i + 1) * K]) for i in range(3))
    ref = w.astype(np.float64) @ x.astype(np.float64)
    y1 = (w * oracle.h2f(oracle.f2h(x))).astype(np.float32).sum(1, dtype=np.float32)
    y3 = np.zeros(R, np.float32)
    for part in (xl, xm, xh):  # lo, mid, hi as fp3gemm accumulates
        for k in range(K):
            y3 = (y3 + w[:, k] * part[k]).astype(np.float32)
    assert oracle.rel_fro(y3, ref) < 0.15 * oracle.rel_fro(y1, ref)


def test_x3s_split_properties():
    rng = np.random.default_rng(6)
    v = (rng.standard_normal((8, 512)) * np.array([0.02, 1, 1e-6, 300, 0, 1e4, 2e-5, 5])[:, None]).astype(np.float32)
    hi, lo, ex = oracle.x3s_split(v)
    assert ex[4] == 0 and not (hi[4] & 0x7fff).any() and not (lo[4] & 0x7fff).any()  # all-zero row (+-0)
    amax = np.abs(v).max(1)
    nz = amax > 0
    scaled = amax[nz] * np.exp2(ex[nz].astype(np.float64))
    assert np.all((scaled >= 2.0 ** 14) & (scaled < 2.0 ** 15))
    vs = v.astype(np.float64) * np.exp2(ex[:, None].astype(np.float64))
    h, l = oracle.h2f(hi).reshape(v.shape), oracle.h2f(lo).reshape(v.shape)
    # hi is the RNE of the scaled value, lo the RNE of the exact residual
    assert np.array_equal(hi.ravel(), oracle.f2h(vs.astype(np.float32)))
    res = vs - h
    ulp_lo = np.exp2(np.floor(np.log2(np.maximum(np.abs(res), 2.0 ** -24))) - 10)
    assert np.all(np.abs(res - l) <= ulp_lo / 2 + 2.0 ** -25)


def test_x3s_product_within_bound():
    """The 2x2 split product in exact arithmetic is within 2^-20 of fp64 (the kernel adds fp32 accumulation)."""
    rng = np.random.default_rng(8)
    W = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    X = rng.standard_normal((48, 1024)).astype(np.float32)
    xh, xl, ex = oracle.x3s_split(X)
    wh, wl, ew = oracle.x3s_split(W)
    Y = oracle.x3s_product_f64(xh, xl, ex, wh, wl, ew)
    ref = X.astype(np.float64) @ W.astype(np.float64).T
    assert oracle.rel_fro(Y, ref) < 2.0 ** -21


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference checkout)")
@pytest.mark.parametrize("name", list(MORE))
def test_more_types_every_code_against_reference_build(name):
    """Every byte value in every position class: blocks whose payload bytes run through 0..255."""
    t = MORE[name]
    be, bb = oracle.block(t)
    rng = np.random.default_rng(77)
    blocks = oracle.random_blocks(rng, t, 256)
    scale = {oracle.Q2_K: (80, 84), oracle.Q3_K: (108, 110), oracle.IQ4_NL: (0, 2), oracle.IQ4_XS: (0, 2),
             oracle.TQ1_0: (52, 54), oracle.TQ2_0: (64, 66), oracle.MXFP4: (0, 1), oracle.NF4: (0, 4),
             oracle.FP4: (0, 4)}[t]
    for j in range(bb):
        if not scale[0] <= j < scale[1]:
            blocks[:, j] = np.arange(256, dtype=np.uint8)  # block k holds byte value k everywhere else
    got = oracle.dequant(blocks, t, be * 256 // be * be)
    want = oracle.ref_dequant(blocks, t, be * 256 // be * be)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_mxfp4_levels_are_twice_e2m1():
    """MXFP4 element = 2^(e-127) * E2M1(code): the oracle's doubled levels over the 2^(e-128) scale."""
    e2m1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for e in (1, 100, 127, 128, 150):
        b = np.zeros((1, 17), np.uint8)
        b[0, 0] = e
        b[0, 1:9] = np.array([c | ((c + 8) << 4) for c in range(8)], np.uint8)  # codes c and c+8
        v = oracle.dequant(b, oracle.MXFP4, 32)[0]
        for c in range(8):
            assert v[c] == np.float32(2.0 ** (e - 127) * e2m1[c])
            assert v[16 + c] == np.float32(-(2.0 ** (e - 127)) * e2m1[c])


LATTICE = {"iq2_xxs": (oracle.IQ2_XXS, 256), "iq2_xs": (oracle.IQ2_XS, 512), "iq2_s": (oracle.IQ2_S, 1024),
           "iq3_xxs": (oracle.IQ3_XXS, 256), "iq3_s": (oracle.IQ3_S, 512), "iq1_s": (oracle.IQ1_S, 2048),
           "iq1_m": (oracle.IQ1_M, 2048)}


def _grid_points(t, b):
    """The grid-point indices the blocks b [n][bytes] read (quant.h:95-115's index arithmetic)."""
    b = b.astype(np.int64)
    u16 = lambda o: b[:, o] | (b[:, o + 1] << 8)  # noqa: E731
    if t == oracle.IQ2_XXS:
        return b[:, 2:66].reshape(len(b), 8, 8)[:, :, :4].ravel()
    if t == oracle.IQ2_XS:
        return np.concatenate([u16(2 + 2 * k) & 511 for k in range(32)])
    if t == oracle.IQ2_S:
        return np.concatenate([b[:, 2 + k] + 256 * ((b[:, 66 + k // 4] >> (2 * (k % 4))) & 3) for k in range(32)])
    if t == oracle.IQ3_XXS:
        return b[:, 2:66].ravel()
    if t == oracle.IQ3_S:
        return np.concatenate([b[:, 2 + k] + 256 * ((b[:, 66 + k // 8] >> (k % 8)) & 1) for k in range(64)])
    if t == oracle.IQ1_S:
        return np.concatenate([b[:, 2 + k] + 256 * ((u16(34 + 2 * (k // 4)) >> (3 * (k % 4))) & 7) for k in range(32)])
    return np.concatenate([b[:, k] + 256 * ((b[:, 32 + k // 2] >> (4 * (k % 2))) & 7) for k in range(32)])


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference checkout)")
@pytest.mark.parametrize("name", list(LATTICE))
def test_lattice_types_every_grid_point_against_reference_build(name):
    """The lattice-grid types (quant.h:95-115) on random blocks (finite fp16 scales) that read every
    point of their grid: bit-exact with the reference's own quant.h and quant_tables.h, which pins
    both the decode and the packed grids it reads (iq_grids.h)."""
    t, npts = LATTICE[name]
    be, bb = oracle.block(t)
    blocks = oracle.random_blocks(np.random.default_rng(300 + t), t, 3000)
    assert len(np.unique(_grid_points(t, blocks))) == npts
    got = oracle.dequant(blocks, t, 256)
    want = oracle.ref_dequant(blocks, t, 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(np.isfinite(want))

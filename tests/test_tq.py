"""The .tq container (tier.cpp:273-292 reader, tier.cpp:2716-2744 / quant.py:60-105 writers).

Host-only: no GPU.  The reader is checked on a header written by hand here
(not by either writer), the writers against each other and against the layout
rules (hb formula, 4096-aligned offsets, row bytes), and the reader's refusals.
"""
import os

import numpy as np
import pytest

import tier_amd
from tier_amd import tq


def _file(path, header: str, size: int, payload=()):
    hb = int(header.split()[1])
    raw = header.encode().ljust(hb, b"\0")
    with open(path, "wb") as f:
        f.truncate(size)
        f.write(raw)
        for off, data in payload:
            f.seek(off)
            f.write(data)


def test_reads_a_hand_written_header(tmp_path):
    p = str(tmp_path / "hand.tq")
    a = bytes(range(256)) + bytes(32)          # Q4_K 2 x 256: 2 * 144 = 288 bytes
    b = np.arange(12, dtype=np.float16).tobytes()  # F16 3 x 4: 24 bytes
    _file(p, "TQB1 4096 2\n#from hand\n#mix Q4_K x1\nw.a Q4_K 2 256 4096 288\nw.b F16 3 4 8192 24 0.125000\n",
          12288, [(4096, a), (8192, b)])
    with tq.TqFile(p) as f:
        assert len(f) == 2
        ea, eb = f.entry(f.find("w.a")), f.entry(f.find("w.b"))
        assert (ea["qtype"], ea["rows"], ea["cols"], ea["offset"], ea["bytes"], ea["rb"], ea["err"]) == \
            (tier_amd.Q4_K, 2, 256, 4096, 288, 144, -1.0)
        assert (eb["qtype"], eb["rows"], eb["cols"], eb["offset"], eb["bytes"], eb["rb"], eb["err"]) == \
            (tier_amd.F16, 3, 4, 8192, 24, 8, 0.125)
        assert f.meta() == {"from": "hand", "mix": "Q4_K x1"}
        assert f.find("w.c") == -1
        assert f.read_rows(f.find("w.a")).tobytes() == a
        assert f.read_rows(f.find("w.b"), 1, 2).tobytes() == b[8:]
    got = tq.info(p)
    assert got["мета"] == {"from": "hand", "mix": "Q4_K x1"} and got["матриц"] == 2
    assert got["типы"] == {"Q4_K": 1, "F16": 1} and got["ошибки"] == {"w.b": 0.125} and got["байт"] == 12288


@pytest.mark.parametrize("header,why", [
    ("TQX1 4096 1\nw Q4_K 1 256 4096 144\n", "magic"),
    ("TQB1 32 1\n", "hb below 64"),
    ("TQB1 4096 1\nw Q4_K 1 256 4096 145\n", "byte count"),
    ("TQB1 4096 1\nw Q4_K 1 255 4096 144\n", "columns not whole blocks"),
    ("TQB1 4096 1\nw Q9_Z 1 256 4096 144\n", "unknown type"),
    ("TQB1 4096 0\n#only meta\n", "no matrices"),
])
def test_reader_refuses(tmp_path, header, why):
    p = str(tmp_path / "bad.tq")
    _file(p, header, 8192)
    with pytest.raises(tier_amd.TiermmError):
        tq.TqFile(p)


def _mats(rng):
    out = []
    for name, t, rows, cols in (("model.layers.0.self_attn.q_proj.weight", tier_amd.Q4_K, 16, 512),
                                ("model.layers.0.self_attn.v_proj.weight", tier_amd.Q6_K, 8, 256),
                                ("model.layers.0.mlp.down_proj.weight", tier_amd.Q8_0, 5, 96),
                                ("lm_head.weight", tier_amd.F16, 3, 40)):
        rb = tier_amd.q_row_bytes(t, cols)
        out.append((name, t, rows, cols, rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)))
    return out


def test_writers_agree_and_follow_the_layout(tmp_path):
    rng = np.random.default_rng(4)
    mats = _mats(rng)
    meta = {"from": "tierlm Q4_K_M", "src": "123 456"}
    pc, pp = str(tmp_path / "c.tq"), str(tmp_path / "py.tq")
    tq.write_tq_arrays(pc, mats, meta)
    names = {tier_amd.Q4_K: "Q4_K", tier_amd.Q6_K: "Q6_K", tier_amd.Q8_0: "Q8_0", tier_amd.F16: "F16"}
    tq.write_tq(pp, [(n, names[t], r, c, (lambda a=a: a.tobytes())) for n, t, r, c, a in mats], meta)
    assert open(pc, "rb").read() == open(pp, "rb").read()
    assert not os.path.exists(pc + ".part") and not os.path.exists(pp + ".part")
    hb = (len(mats) * 200 + 4096 + 4095) // 4096 * 4096
    with tq.TqFile(pc) as f:
        assert f.meta() == meta
        off = hb
        for n, t, r, c, a in mats:
            e = f.entry(f.find(n))
            assert e["offset"] == off and e["offset"] % 4096 == 0 and e["bytes"] == a.nbytes
            assert np.array_equal(f.read_rows(f.find(n)), a)
            off += (a.nbytes + 4095) // 4096 * 4096
        assert os.path.getsize(pc) == off


def test_writer_errors_with_six_decimals(tmp_path):
    rng = np.random.default_rng(5)
    mats = _mats(rng)[:2]
    p = str(tmp_path / "e.tq")
    tq.write_tq_arrays(p, mats, {}, errs=[0.0412345678, 0.02])
    head = open(p, "rb").read(4096).split(b"\0", 1)[0].decode().splitlines()
    assert head[1].endswith(" 0.041235") and head[2].endswith(" 0.020000")
    assert tq.info(p)["ошибки"] == {mats[0][0]: 0.041235, mats[1][0]: 0.02}


def test_python_writer_copies_from_a_source_file(tmp_path):
    src = tmp_path / "src.bin"
    blob = np.random.default_rng(6).integers(0, 256, 1000 + 2 * 144, dtype=np.uint8).tobytes()
    src.write_bytes(blob)
    p = str(tmp_path / "s.tq")
    tq.write_tq(p, [("w", "Q4_K", 2, 256, (str(src), 1000, 288))], {"from": "gguf"})
    with tq.TqFile(p) as f:
        assert f.read_rows(0).tobytes() == blob[1000:]
    with pytest.raises(ValueError):
        tq.write_tq(p, [("w", "Q4_K", 2, 256, (str(src), 1000, 280))], {})


@pytest.mark.parametrize("name", ["q4_0", "q4_1", "q5_0", "q5_1", "q8_0", "q4_K", "q5_K", "q6_K", "iq2_xxs", "iq2_xs",
                                  "iq2_s", "iq3_xxs", "iq3_s", "iq1_s", "iq1_m"])
def test_host_dequant_matches_reference_golden(golden, name):
    """tiermm_dequant_host against q_val values written by the reference's quant.h (fixtures)."""
    g = golden["dequant"]
    blocks, want = g[f"{name}_blocks"], g[f"{name}_f32bits"]
    t = int(g[f"{name}_type"])
    cols = int(g["cols"])
    got = tier_amd.dequant_host(blocks.reshape(-1, blocks.shape[-1]), t, cols)
    assert np.array_equal(got.view(np.uint32).ravel(), want.ravel())


def _write_safetensors(path, tensors):
    import json
    import struct
    head, off, blobs = {}, 0, []
    for name, arr in tensors.items():
        b = arr.tobytes()
        head[name] = {"dtype": "BF16", "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    h = json.dumps(head).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def test_tq_check_metrics(tmp_path):
    """tier --tq-check (tier.cpp:2749-2765) on a two-matrix base: q8_0 and q4_K error levels
    (check_quant.py:117 bounds: 0.7 %, 8 %) and correlations near 1; a matrix quantized from
    other weights is caught (correlation near 0, result 2)."""
    from tier_amd import tq
    rng = np.random.default_rng(9)
    w = {n: (rng.standard_normal(s) * 0.02).astype(np.float32) for n, s in (("a.weight", (64, 512)),
                                                                           ("b.weight", (50, 256)))}
    bf = {n: ((v.view(np.uint32) + 0x8000) >> 16).astype(np.uint16) for n, v in w.items()}  # bf16 source
    model = str(tmp_path / "m.safetensors")
    _write_safetensors(model, bf)
    src = {n: (b.astype(np.uint32) << 16).view(np.float32) for n, b in bf.items()}
    base = str(tmp_path / "m.tq")
    tq.write_tq_arrays(base, [("a.weight", tier_amd.Q8_0, 64, 512, tier_amd.q_row(tier_amd.Q8_0, src["a.weight"])),
                              ("b.weight", tier_amd.Q4_K, 50, 256, tier_amd.q_row(tier_amd.Q4_K, src["b.weight"]))])
    lines = []
    assert tq.check(model, base, say=lines.append) == 0
    import re
    errs = {m.group(1): (float(m.group(2)), float(m.group(3)))
            for m in (re.search(r" (\S+) \S+, ошибка ([\d.]+)%, корреляция ([\d.]+)", l) for l in lines[:-1]) if m}
    assert errs["a.weight"][0] < 0.7 and errs["a.weight"][1] > 0.9999
    assert errs["b.weight"][0] < 8.0 and errs["b.weight"][1] > 0.99
    m = re.search(r"ошибка весов ([\d.]+)%, худшая корреляция (-?[\d.]+) \((.*?)\)", lines[-1], re.I)
    assert m and m.group(3) == "b.weight"
    # a base made from other weights
    other = (rng.standard_normal((50, 256)) * 0.02).astype(np.float32)
    base2 = str(tmp_path / "o.tq")
    tq.write_tq_arrays(base2, [("b.weight", tier_amd.Q4_K, 50, 256, tier_amd.q_row(tier_amd.Q4_K, other))])
    lines = []
    assert tq.check(model, base2, say=lines.append) == 2
    assert "обнаружены" in lines[-1]
    # a matrix the model does not have
    base3 = str(tmp_path / "x.tq")
    tq.write_tq_arrays(base3, [("c.weight", tier_amd.Q4_K, 50, 256, tier_amd.q_row(tier_amd.Q4_K, other))])
    assert tq.check(model, base3, say=lambda s: None) == 2


@pytest.mark.parametrize("t", [tier_amd.Q8_0, tier_amd.Q5_0, tier_amd.Q4_K, tier_amd.Q5_K, tier_amd.Q6_K,
                               tier_amd.Q2_K, tier_amd.Q3_K, tier_amd.IQ4_NL, tier_amd.IQ4_XS, tier_amd.TQ1_0,
                               tier_amd.TQ2_0, tier_amd.MXFP4, tier_amd.NF4, tier_amd.FP4, tier_amd.IQ2_XXS,
                               tier_amd.IQ2_XS, tier_amd.IQ2_S, tier_amd.IQ3_XXS, tier_amd.IQ3_S, tier_amd.IQ1_S,
                               tier_amd.IQ1_M])
def test_host_dequant_matches_oracle_on_random_blocks(t):
    import oracle
    rng = np.random.default_rng(100 + t)
    be, _ = oracle.block(t)
    K = 1024
    blocks = oracle.random_blocks(rng, t, 16 * (K // be)).reshape(16, -1)
    got = tier_amd.dequant_host(blocks, t, K)
    want = oracle.dequant(blocks, t, K, oracle.OUT_F32).reshape(16, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))

"""Write the golden vectors under tests/golden/ from the reference's own quant.h.

Run in the container that holds the reference checkout, after
``make -C oracle ref`` has compiled ``oracle/_ref/libtqref.so`` from
<reference>/tier/quant.h (nothing is copied from the reference; only its
outputs are stored here):

    python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  dequant_golden.npz   for each type (the eight k-quant / legacy types, then the seven
                       lattice-grid IQ types): random blocks built as check_quant.py:31-48
                       builds them (seed 7, 8 rows x 512 cols, fp16 scale fields
                       ~N(0,0.02)) and the reference q_val of every element (fp32 bits)
  quant_golden.npz     x ~N(0,0.02) [8][1024] (seed 11) and the bytes the
                       reference q_row writes for Q8_0, Q4_K, Q5_K, Q6_K
  f16_golden.npz       boundary and random fp32 inputs and the reference q_f2h bits
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402

TYPES = {"q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1, "q5_0": oracle.Q5_0, "q5_1": oracle.Q5_1,
         "q8_0": oracle.Q8_0, "q4_K": oracle.Q4_K, "q5_K": oracle.Q5_K, "q6_K": oracle.Q6_K,
         # appended later: the random draws of the types above stay as they were
         "iq2_xxs": oracle.IQ2_XXS, "iq2_xs": oracle.IQ2_XS, "iq2_s": oracle.IQ2_S, "iq3_xxs": oracle.IQ3_XXS,
         "iq3_s": oracle.IQ3_S, "iq1_s": oracle.IQ1_S, "iq1_m": oracle.IQ1_M}
COLS, ROWS = 512, 8


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libtqref.so is missing: run `make -C oracle ref` where the reference is present")
    rng = np.random.default_rng(7)
    out = {}
    for name, t in TYPES.items():
        be, bb = oracle.block(t)
        blocks = oracle.random_blocks(rng, t, COLS // be * ROWS)
        want = oracle.ref_dequant(blocks.reshape(-1), t, COLS)
        out[f"{name}_blocks"] = blocks.reshape(ROWS, -1)
        out[f"{name}_f32bits"] = want.view(np.uint32)
        out[f"{name}_type"] = np.int32(t)
    np.savez_compressed(os.path.join(HERE, "dequant_golden.npz"), cols=np.int32(COLS), **out)

    rng = np.random.default_rng(11)
    x = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    q = {"x": x}
    for name in ("q8_0", "q4_K", "q5_K", "q6_K"):
        q[name] = oracle.ref_quantize(x, TYPES[name])
    np.savez_compressed(os.path.join(HERE, "quant_golden.npz"), **q)

    R = oracle.ref()
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, 6.1035156e-05, 6.097555e-05,
                         5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 8.940697e-08, 1e-10, 0.333333,
                         1.00048828125, 1.000244140625, 1.0007324, 2049.0, 2051.0, -2.9802326e-08],
                        dtype=np.float32)
    r2 = np.random.default_rng(5)
    rnd = (r2.standard_normal(4000) * np.exp2(r2.integers(-30, 18, 4000))).astype(np.float32)
    f = np.concatenate([specials, rnd])
    h = np.array([R.ref_q_f2h(float(v)) for v in f], dtype=np.uint16)
    np.savez_compressed(os.path.join(HERE, "f16_golden.npz"), f32=f, f2h=h)
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()

"""Write iq_grids.h: the lattice grids of the IQ2/IQ3/IQ1 block formats, packed.

The grids are constants of the GGUF formats IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS,
IQ3_S, IQ1_S and IQ1_M (their q_val reads them, quant.h:95-115).  The reference
carries them in quant_tables.h as int8 values, one per element; every grid
uses a small alphabet, so here a grid point is one 16-bit word of codes:

  IQ2 grids  8 values in {8, 25, 43}          -> eight 2-bit codes (value order)
  IQ3_XXS    4 values in {4, 12, ..., 52, 62} -> four 3-bit codes, value 8c + 4 (c < 7), 62 (c = 7)
  IQ3_S      4 values in {1, 3, ..., 15}      -> four 3-bit codes, value 2c + 1
  IQ1_S      8 values in {-1, 0, 1}           -> eight 2-bit codes, value c - 1

element e of a point in bits [2e, 2e+2) or [3e, 3e+3).  The sign table ksigns is
not stored: entry i is i with bit 7 set when i has an odd number of set bits.

Run where the reference checkout is present (it reads the grids from its
quant_tables.h, nothing else), then commit the header; builds use the header:

    python tier_amd/csrc/gen_iq_grids.py [path/to/quant_tables.h]

The decoders that use the header are pinned against the reference's own quant.h
(oracle/_ref) on blocks that visit every grid point (tests/test_oracle.py).
"""
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT = "/root/reference/tier/quant_tables.h"

# name in quant_tables.h -> (our name, values per point, bits per code, value -> code)
GRIDS = {
    "qt_iq2xxs_grid": ("tm_iq2xxs_grid", 8, 2, {8: 0, 25: 1, 43: 2}),
    "qt_iq2xs_grid": ("tm_iq2xs_grid", 8, 2, {8: 0, 25: 1, 43: 2}),
    "qt_iq2s_grid": ("tm_iq2s_grid", 8, 2, {8: 0, 25: 1, 43: 2}),
    "qt_iq3xxs_grid": ("tm_iq3xxs_grid", 4, 3, {4: 0, 12: 1, 20: 2, 28: 3, 36: 4, 44: 5, 52: 6, 62: 7}),
    "qt_iq3s_grid": ("tm_iq3s_grid", 4, 3, {2 * c + 1: c for c in range(8)}),
    "qt_iq1s_grid": ("tm_iq1s_grid", 8, 2, {-1: 0, 0: 1, 1: 2}),
}


def parse(path):
    text = open(path).read()
    tabs = {}
    for m in re.finditer(r"QTAB_DECL\(\s*\w+\s*,\s*(\w+)\s*,\s*(\d+)\s*,\s*\{([^}]*)\}\s*\)", text):
        vals = [int(v) for v in m.group(3).split(",") if v.strip()]
        assert len(vals) == int(m.group(2)), m.group(1)
        tabs[m.group(1)] = vals
    return tabs


def pack(vals, per, bits, code):
    words = []
    for p in range(len(vals) // per):
        w = 0
        for e in range(per):
            w |= code[vals[p * per + e]] << (bits * e)
        words.append(w)
    return words


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else DEFAULT
    tabs = parse(src)
    ks = tabs["qt_ksigns"]
    assert all(ks[i] == i | ((bin(i).count("1") & 1) << 7) for i in range(128)), "ksigns is not the parity rule"
    out = ["// iq_grids.h -- lattice grids of the IQ2 / IQ3 / IQ1 GGUF block formats, packed",
           "// (written by gen_iq_grids.py, which documents the encoding; do not edit).",
           "// One 16-bit word per grid point: element e's code in bits [2e, 2e+2) (IQ2,",
           "// IQ1_S) or [3e, 3e+3) (IQ3).  Values: IQ2 {8, 25, 43}[c]; IQ3_XXS 8c + 4,",
           "// or 62 for c = 7; IQ3_S 2c + 1; IQ1_S c - 1.  C and C++ (host and device).",
           "#ifndef TM_IQ_GRIDS_H", "#define TM_IQ_GRIDS_H", "#include <stdint.h>",
           "#ifdef __cplusplus", "#define TM_GRID constexpr", "#else", "#define TM_GRID static const", "#endif"]
    for name, (ours, per, bits, code) in GRIDS.items():
        words = pack(tabs[name], per, bits, code)
        out.append(f"TM_GRID uint16_t {ours}[{len(words)}] = {{")
        for i in range(0, len(words), 12):
            out.append("    " + ", ".join(f"0x{w:04x}" for w in words[i:i + 12]) + ",")
        out.append("};")
    out += ["#undef TM_GRID", "#endif", ""]
    dst = os.path.join(HERE, "iq_grids.h")
    with open(dst, "w") as f:
        f.write("\n".join(out))
    print("wrote", dst)


if __name__ == "__main__":
    main()

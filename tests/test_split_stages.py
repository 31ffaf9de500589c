"""Stage ranges of the whole-tile q4_K GEMV in split stages (qgemv_q4k_ws.hip, WS_STAGES:
257..384 row tiles above K = 8192, 256 workgroups).  Workgroup b takes the stages
[T b / G, T (b + 1) / G) of T = tiles x stages per tile (stages of 8 super-blocks).  The
kernel keeps partial sums for at most 3 tiles a workgroup (its R), pairs at most two
workgroups on a tile (one pairing slot per boundary), and computes the ranges in 32-bit
arithmetic; this checks all three over every shape that launch takes.  CPU only."""
import numpy as np

G = 256
GS = 8


def _ranges(tiles, ngrp):
    T = tiles * ngrp
    b = np.arange(G + 1, dtype=np.int64)
    return T * b // G


def test_split_stage_ranges_hold_the_kernel_bounds():
    for K in range(8192 + 256, 14336 + 1, 256):
        ngrp = -(-(K // 256) // GS)
        for tiles in range(257, 385):
            assert tiles * ngrp * G < 2**32  # the kernel's unsigned products
            s = _ranges(tiles, ngrp)
            s0, s1 = s[:-1], s[1:]
            assert np.all(s1 - s0 >= ngrp)  # every range at least a tile long
            first, last = s0 // ngrp, (s1 - 1) // ngrp
            assert np.all(last - first + 1 <= 3), (K, tiles)
            # workgroups that hold a stage of each tile
            owners = np.zeros(tiles, np.int64)
            for a, z in zip(first, last):
                owners[a:z + 1] += 1
            assert owners.min() >= 1 and owners.max() <= 2, (K, tiles)
            # a split tile is the upper part of exactly the workgroup after the boundary
            split = (s0[1:] % ngrp) != 0
            assert np.all(last[:-1][split] == first[1:][split])

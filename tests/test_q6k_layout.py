"""CPU walk of the q6_K decode GEMV's LDS stage layout (qgemv_q6k.hip): for each
workgroup, wave, stage and DMA lane it forms the load address the kernel forms
(the window 4((r/4) % 4) bytes below the dword of the row segment, row N-1 from
its 16-byte boundary, the clamp to W's last 16 bytes), and for each reading lane
the LDS offset it reads row n's super-blocks from, and checks that

* every load is dword-aligned and lies inside W (no clamp moves a load of another
  row than N-1),
* every byte a lane reads is the byte of its own row segment,
* a row's reads stay inside its row pitch.

The layout constants (210-byte super-blocks, the pitch, 1 KiB loads of 64 lanes)
are the kernel's; the shapes are taken from its launch table."""
import numpy as np
import pytest

SBB = 210


def walk(N, K, RT, KS, GS, Wbase=4096):
    rb = K // 256 * SBB
    assert (N * rb) % 16 == 0  # qgemv_q6k_fits
    PITCH = (GS * SBB + 14 + 15) // 16 * 16
    SBYTES = 16 * PITCH
    NLD = (SBYTES + 1023) // 1024
    LAST = (SBYTES - (NLD - 1) * 1024) // 16
    nsb_all = K >> 8
    grid = ((N + 15) // 16 + RT - 1) // RT
    wlast = Wbase + N * rb - 16
    lane = np.arange(64)
    for b in range(grid):
        for wave in range(RT * KS):
            rt, kp = wave // KS, wave % KS
            row0 = (b * RT + rt) * 16
            sbk = kp * nsb_all // KS
            nsb = (kp + 1) * nsb_all // KS - sbk
            rbase = min(row0, N - 1)
            rmax = min(15, N - 1 - rbase)
            for grp in range((nsb + GS - 1) // GS):
                img = np.full(SBYTES, -1, np.int64)
                for j in range(NLD):
                    on = lane if (j < NLD - 1 or LAST == 64) else lane[:LAST]
                    f = np.minimum(j * 1024 + on * 16, SBYTES - 16)
                    r = f // PITCH
                    row = rbase + np.minimum(r, rmax)
                    seg = Wbase + row * rb + (sbk + grp * GS) * SBB
                    ph = np.where(row == N - 1, -1, 4 * ((r >> 2) & 3))
                    win = np.where(ph < 0, seg & ~15, (seg & ~3) - ph)
                    addr = np.minimum(win + f % PITCH, wlast)
                    assert np.all(addr % 4 == 0)
                    assert np.all(addr >= Wbase) and np.all(addr + 16 <= Wbase + N * rb)
                    assert np.all((addr == win + f % PITCH) | (row == N - 1))
                    for a, d in zip(addr, j * 1024 + on * 16):
                        img[d:d + 16] = np.arange(a, a + 16)
                for n in range(16):
                    nrow = rbase + min(n, rmax)
                    shift0 = (Wbase + nrow * rb + sbk * SBB) & 15
                    smask, sph = (15, 0) if nrow == N - 1 else (3, 4 * ((n >> 2) & 3))
                    rowoff = n * PITCH + sph + ((shift0 + 2 * GS * grp) & smask)
                    for i in range(GS):
                        sb = GS * grp + i
                        if GS > 1 and sb >= nsb:
                            continue
                        off = rowoff + i * SBB
                        want = Wbase + nrow * rb + (sbk + sb) * SBB
                        assert np.array_equal(img[off:off + SBB], np.arange(want, want + SBB)), (b, wave, grp, n)
                        assert (off & ~3) + 212 <= (n + 1) * PITCH  # the scale read's last dword


@pytest.mark.parametrize("N,K,RT,KS,GS", [
    (40, 5120, 1, 4, 1),     # <= 256 tiles, K in four parts; rows alternate 8 bytes mod 16
    (1000, 2304, 2, 4, 1),   # rows 2 bytes mod 4 apart; a partial last tile
    (100, 14336, 2, 4, 1),   # every row at one offset mod 16
    (34, 5120, 4, 2, 1),     # eight waves, four tiles; tiles past N
    (70, 5120, 4, 2, 2),     # two super-blocks a stage
])
def test_q6k_stage_layout(N, K, RT, KS, GS):
    walk(N, K, RT, KS, GS)

"""Shared input generators for the tests (seeded, documented)."""
import numpy as np

import tier_amd


def quantized_weight(qtype: int, N: int, K: int, seed: int, sigma: float = 0.02):
    """W ~ N(0, sigma) [N][K] quantized by the host quantizer (byte-identical with quant.h)."""
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K), dtype=np.float32) * sigma).astype(np.float32)
    if qtype == tier_amd.Q5_0:
        return random_blocks_q5_0(rng, N, K)
    return tier_amd.q_row(qtype, W)


def random_blocks_q5_0(rng, N, K):
    """Q5_0 has no quantizer in the reference: random bytes with fp16 d ~N(0,0.02) (check_quant.py:31-48)."""
    nb = K // 32
    b = rng.integers(0, 256, size=(N * nb, 22), dtype=np.uint8)
    b[:, 0:2] = (rng.standard_normal(N * nb) * 0.02).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return b.reshape(N, nb * 22)


def activations(M: int, K: int, seed: int):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((M, K), dtype=np.float32)

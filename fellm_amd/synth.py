"""Seeded synthetic inputs for the parity tests and the benchmark.

GGUF Q4_K / Q6_K tables are generated block by block with the byte layouts
of crates/backend-cpu/src/dequant.rs:193-204 (Q4_K: f16 d, f16 dmin, 12
packed 6-bit scale/min bytes, 128 nibble bytes) and :307-313 (Q6_K: ql[128],
qh[64], int8 scales[16], f16 d).  Scale/min packing follows the inverse of
get_scale_min_k4, as the reference's own test builds it (dequant.rs:478-498).
"""
from __future__ import annotations

import numpy as np

Q4K_BLOCK = 144
Q6K_BLOCK = 210
QK_K = 256


def pack_scale_min_k4(ls: np.ndarray, lm: np.ndarray) -> np.ndarray:
    """Pack 8 six-bit scales and mins per block into 12 bytes: ls, lm [..., 8] -> [..., 12]."""
    ls = ls.astype(np.uint8)
    lm = lm.astype(np.uint8)
    out = np.zeros(ls.shape[:-1] + (12,), np.uint8)
    for j in range(8):
        if j < 4:
            out[..., j] |= ls[..., j]
            out[..., j + 4] |= lm[..., j]
        else:
            out[..., j + 4] |= (ls[..., j] & 0x0F) | ((lm[..., j] & 0x0F) << 4)
            out[..., j - 4] |= (ls[..., j] >> 4) << 6
            out[..., j] |= (lm[..., j] >> 4) << 6
    return out


def _abs_normal_f16_bits(rng: np.random.Generator, shape, sigma: float) -> np.ndarray:
    return np.abs(rng.normal(0.0, sigma, size=shape)).astype(np.float16).view(np.uint16)


def q4k_table(rng: np.random.Generator, vocab: int, dim: int) -> np.ndarray:
    """uint8 [vocab, dim/256*144]: d, dmin ~ f16(|N(0, 0.01)|), 6-bit sc/m U[0,63], 4-bit quants uniform."""
    assert dim % QK_K == 0
    nb = dim // QK_K
    blocks = np.empty((vocab, nb, Q4K_BLOCK), np.uint8)
    blocks[..., 0:2] = _abs_normal_f16_bits(rng, (vocab, nb), 0.01).view(np.uint8).reshape(vocab, nb, 2)
    blocks[..., 2:4] = _abs_normal_f16_bits(rng, (vocab, nb), 0.01).view(np.uint8).reshape(vocab, nb, 2)
    ls = rng.integers(0, 64, size=(vocab, nb, 8), dtype=np.uint8)
    lm = rng.integers(0, 64, size=(vocab, nb, 8), dtype=np.uint8)
    blocks[..., 4:16] = pack_scale_min_k4(ls, lm)
    blocks[..., 16:] = rng.integers(0, 256, size=(vocab, nb, 128), dtype=np.uint8)
    return blocks.reshape(vocab, nb * Q4K_BLOCK)


def q6k_table(rng: np.random.Generator, vocab: int, dim: int) -> np.ndarray:
    """uint8 [vocab, dim/256*210]: ql, qh uniform bytes, int8 scales uniform, d ~ f16(|N(0, 0.01)|)."""
    assert dim % QK_K == 0
    nb = dim // QK_K
    blocks = rng.integers(0, 256, size=(vocab, nb, Q6K_BLOCK), dtype=np.uint8)
    blocks[..., 208:210] = _abs_normal_f16_bits(rng, (vocab, nb), 0.01).view(np.uint8).reshape(vocab, nb, 2)
    return blocks.reshape(vocab, nb * Q6K_BLOCK)


def q5k_table(rng: np.random.Generator, vocab: int, dim: int) -> np.ndarray:
    """uint8 [vocab, dim/256*176]: d, dmin ~ f16(|N(0, 0.01)|), 6-bit sc/m U[0,63], qh and qs uniform bytes."""
    assert dim % QK_K == 0
    nb = dim // QK_K
    blocks = np.empty((vocab, nb, 176), np.uint8)
    blocks[..., 0:2] = _abs_normal_f16_bits(rng, (vocab, nb), 0.01).view(np.uint8).reshape(vocab, nb, 2)
    blocks[..., 2:4] = _abs_normal_f16_bits(rng, (vocab, nb), 0.01).view(np.uint8).reshape(vocab, nb, 2)
    ls = rng.integers(0, 64, size=(vocab, nb, 8), dtype=np.uint8)
    lm = rng.integers(0, 64, size=(vocab, nb, 8), dtype=np.uint8)
    blocks[..., 4:16] = pack_scale_min_k4(ls, lm)
    blocks[..., 16:] = rng.integers(0, 256, size=(vocab, nb, 160), dtype=np.uint8)
    return blocks.reshape(vocab, nb * 176)


def q8_0_table(rng: np.random.Generator, vocab: int, dim: int) -> np.ndarray:
    """uint8 [vocab, dim/32*34]: per 32-element block d ~ f16(|N(0, 0.01)|), then 32 uniform int8."""
    assert dim % 32 == 0
    nb = dim // 32
    blocks = np.empty((vocab, nb, 34), np.uint8)
    blocks[..., 0:2] = _abs_normal_f16_bits(rng, (vocab, nb), 0.01).view(np.uint8).reshape(vocab, nb, 2)
    blocks[..., 2:] = rng.integers(0, 256, size=(vocab, nb, 32), dtype=np.uint8)
    return blocks.reshape(vocab, nb * 34)


KQUANT_TABLES = {12: q4k_table, 13: q5k_table, 14: q6k_table}
KQUANT_BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


def zipf_ids(rng: np.random.Generator, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    """Token ids Zipf(s) over [0, vocab) by inverse CDF (rank 1 = id 0)."""
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    u = rng.random(n)
    return np.minimum(np.searchsorted(cdf, u, side="left"), vocab - 1).astype(np.uint32)


def paged_layout(rng: np.random.Generator, batch: int, n_blocks: int, block_size: int, max_pos: int,
                 n_layers: int = 1):
    """Block table for one new token per sequence at a random position.

    Returns (positions u32 [batch], table u32 [batch * n_layers * n_logical], n_logical).
    Each row's current logical block maps to a distinct physical block drawn
    from a random permutation of the arena; other entries map to block 0.
    """
    n_logical = (max_pos + block_size - 1) // block_size
    positions = rng.integers(0, max_pos, size=batch, dtype=np.uint32)
    perm = rng.permutation(n_blocks).astype(np.uint32)
    table = np.zeros((batch, n_layers, n_logical), np.uint32)
    for r in range(batch):
        for layer in range(n_layers):
            table[r, layer, positions[r] // block_size] = perm[(r * n_layers + layer) % n_blocks]
    return positions, table.reshape(-1), n_logical

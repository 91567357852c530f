"""Seeded synthetic inputs shared by the parity tests and the benchmark.

The generator is the reference's LCG (examples/quant_probe.rs:47-55):
``state = state * 6364136223846793005 + 1`` (wrapping u64) and
``u = ((state >> 33) as f32) / 2^31``, vectorised with jump-ahead so that
millions of draws take milliseconds. Normals use Box-Muller on consecutive
pairs of draws (evaluated in f64, rounded to f32).
"""
from __future__ import annotations

import numpy as np

_A = 6364136223846793005
_C = 1
_M = (1 << 64) - 1
_BLOCK = 1 << 16


def _affine_pow(k: int) -> tuple[int, int]:
    """(A^k, C*(A^(k-1) + ... + 1)) mod 2^64: k LCG steps as one affine map."""
    a, c = 1, 0
    base_a, base_c = _A, _C
    while k:
        if k & 1:
            a, c = (a * base_a) & _M, (c * base_a + base_c) & _M
        base_a, base_c = (base_a * base_a) & _M, (base_c * base_a + base_c) & _M
        k >>= 1
    return a, c


def lcg_states(seed: int, n: int) -> np.ndarray:
    """The n states following `seed` (state_1 .. state_n)."""
    n = int(n)
    out = np.empty(n, dtype=np.uint64)
    if n == 0:
        return out
    first = min(n, _BLOCK)
    s = seed & _M
    head = np.empty(first, dtype=np.uint64)
    for i in range(first):
        s = (s * _A + _C) & _M
        head[i] = s
    out[:first] = head
    if n > first:
        a, c = _affine_pow(_BLOCK)
        a64, c64 = np.uint64(a), np.uint64(c)
        prev = head
        with np.errstate(over="ignore"):
            for start in range(_BLOCK, n, _BLOCK):
                nxt = prev * a64 + c64
                m = min(_BLOCK, n - start)
                out[start:start + m] = nxt[:m]
                prev = nxt
    return out


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """f32 draws u in [0, 1] (the reference's u) mapped to lo + (hi - lo)*u."""
    u = (lcg_states(seed, n) >> np.uint64(33)).astype(np.float32) / np.float32(2.0 ** 31)
    if lo == 0.0 and hi == 1.0:
        return u
    return (np.float32(lo) + np.float32(hi - lo) * u).astype(np.float32)


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """f32 N(mean, std) draws by Box-Muller over pairs of LCG draws."""
    m = (int(n) + 1) // 2
    u = uniform(seed, 2 * m).astype(np.float64)
    u1 = np.maximum(1.0 - u[0::2], 2.0 ** -32)
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32)


def config_seed(index: int) -> int:
    """Seed of BASELINE configs[index]: 0x5EED0000 + index."""
    return 0x5EED0000 + int(index)


def unique_voxels(seed: int, count: int, resolution: int) -> np.ndarray:
    """`count` distinct int32 (x, y, z) cells of a resolution^3 grid, drawn by
    a seeded Fisher-Yates shuffle of the cell indices (row-major x, y, z)."""
    cells = resolution ** 3
    if count > cells:
        raise ValueError("more voxels than grid cells")
    idx = np.arange(cells, dtype=np.int64)
    u = uniform(seed, count).astype(np.float64)
    for i in range(count):
        j = i + int(u[i] * (cells - i)) if u[i] < 1.0 else cells - 1
        j = min(j, cells - 1)
        idx[i], idx[j] = idx[j], idx[i]
    pick = idx[:count]
    r2 = resolution * resolution
    return np.stack([pick // r2, (pick // resolution) % resolution, pick % resolution], axis=1).astype(np.int32)


def vggt_positions(frames: int, patch_h: int, patch_w: int, specials: int = 5) -> np.ndarray:
    """[frames, specials + h*w, 2] int32: (0, 0) for the special tokens, then
    (y + 1, x + 1) for the patch grid (vggt.rs:288-291, position_getter in
    attention_math.rs:167-183)."""
    pos = np.zeros((frames, specials + patch_h * patch_w, 2), dtype=np.int32)
    yy, xx = np.meshgrid(np.arange(patch_h), np.arange(patch_w), indexing="ij")
    pos[:, specials:, 0] = (yy.reshape(-1) + 1)
    pos[:, specials:, 1] = (xx.reshape(-1) + 1)
    return pos


def q8_0_blocks(seed: int, nblocks: int, d_lo: float = 1e-4, d_hi: float = 1e-2) -> np.ndarray:
    """nblocks GGML block_q8_0 records (34 bytes: f16 d little-endian, then 32
    int8 qs) with qs ~ U[-127, 127] and d = f16(U[d_lo, d_hi])."""
    d = uniform(seed, nblocks, d_lo, d_hi).astype(np.float16)
    q = np.floor(uniform(seed + 1, nblocks * 32) * np.float32(255.0)).astype(np.int32) - 127
    q = np.clip(q, -127, 127).astype(np.int8).reshape(nblocks, 32)
    out = np.empty((nblocks, 34), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)

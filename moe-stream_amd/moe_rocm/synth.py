"""Seeded synthetic inputs for the configured workloads (numpy, host side).

Counter-based SplitMix64: draw(seed, i) is the i-th output of a SplitMix64
stream started at `seed` (Steele, Lea, Flood, "Fast splittable pseudorandom
number generators", OOPSLA 2014), so any element can be generated on its own.
The integer-only parts (MXFP4 and Q4_K block bytes) are also produced on the
GPU by mr_synth_blocks with the same arithmetic, bit for bit; float tensors
(activations, router, biases) use Box-Muller in f64 and are generated here.

Stream layout (one stream per tensor): stream_seed(BASE_SEED, config, layer,
tensor_id, sub) chains draw() over the ids.
"""
from __future__ import annotations

import numpy as np

BASE_SEED = 20261201
GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

# tensor ids of the stream layout
T_GATE, T_UP, T_DOWN = 0, 1, 2
T_ROUTER_W, T_ROUTER_B = 3, 4
T_GATE_B, T_UP_B, T_DOWN_B = 5, 6, 7
T_X = 8
T_SH_GATE, T_SH_UP, T_SH_DOWN, T_SH_GATE_INP = 9, 10, 11, 12
T_ZIPF, T_EXPERTS_PER_LAYER = 13, 14

MXFP4_BLOCK_BYTES, MXFP4_BLOCK_ELEMS = 17, 32
Q4K_BLOCK_BYTES, Q4K_BLOCK_ELEMS = 144, 256
GGML_Q4_K, GGML_MXFP4 = 12, 39


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def draws(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs start..start+count-1 of the SplitMix64 stream seeded with `seed`."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GAMMA)


def draw1(seed: int, i: int) -> int:
    return int(draws(seed, i, 1)[0])


def stream_seed(*ids: int, base: int = BASE_SEED) -> int:
    s = base & 0xFFFFFFFFFFFFFFFF
    for v in ids:
        s = draw1(s, int(v) & 0xFFFFFFFFFFFFFFFF)
    return s


def mxfp4_blocks(seed: int, n_blocks: int, first_block: int = 0) -> np.ndarray:
    """n_blocks MXFP4 blocks (17 bytes each): e8m0 uniform in [119,127], nibbles
    uniform. Block i uses draws 3i (scale), 3i+1 and 3i+2 (16 code bytes, LE)."""
    d = draws(seed, 3 * first_block, 3 * n_blocks).reshape(n_blocks, 3)
    out = np.empty((n_blocks, 17), dtype=np.uint8)
    hi = (d[:, 0] >> np.uint64(32)) * np.uint64(9)
    out[:, 0] = (np.uint64(119) + (hi >> np.uint64(32))).astype(np.uint8)
    out[:, 1:17] = d[:, 1:3].copy().view(np.uint8).reshape(n_blocks, 16)
    return out.reshape(-1)


def _irwin_hall12(d3: np.ndarray) -> np.ndarray:
    """Sum of 12 uint16 (3 draws) -> approximately N(0,1) as exact float32:
    (S - 6*65536) / 65536."""
    u16 = d3.copy().view(np.uint16).reshape(d3.shape[0], 12).astype(np.int64)
    s = u16.sum(axis=1)
    return ((s.astype(np.float32) - np.float32(393216.0)) * np.float32(1.0 / 65536.0)).astype(np.float32)


def q4k_blocks(seed: int, n_blocks: int, first_block: int = 0) -> np.ndarray:
    """n_blocks Q4_K super-blocks (144 bytes). Block i uses draws 24i..24i+23:
    0-2 -> d = fp16(|z| * 0.01), 3-5 -> dmin = fp16(|z| * 0.005) with z the
    Irwin-Hall(12) normal, 6-23 -> 12 scale bytes then 128 quant bytes."""
    d = draws(seed, 24 * first_block, 24 * n_blocks).reshape(n_blocks, 24)
    out = np.empty((n_blocks, 144), dtype=np.uint8)
    zd = _irwin_hall12(d[:, 0:3])
    zm = _irwin_hall12(d[:, 3:6])
    dd = (np.abs(zd) * np.float32(0.01)).astype(np.float32).astype(np.float16)
    dm = (np.abs(zm) * np.float32(0.005)).astype(np.float32).astype(np.float16)
    out[:, 0:2] = dd.view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:4] = dm.view(np.uint8).reshape(n_blocks, 2)
    raw = d[:, 6:24].copy().view(np.uint8).reshape(n_blocks, 144)
    out[:, 4:144] = raw[:, 0:140]
    return out.reshape(-1)


def blocks(ggml_type: int, seed: int, n_blocks: int, first_block: int = 0) -> np.ndarray:
    if ggml_type == GGML_MXFP4:
        return mxfp4_blocks(seed, n_blocks, first_block)
    if ggml_type == GGML_Q4_K:
        return q4k_blocks(seed, n_blocks, first_block)
    raise ValueError(f"unsupported ggml type {ggml_type}")


def normal(seed: int, n: int, sigma: float = 1.0) -> np.ndarray:
    """float32 N(0, sigma^2) by Box-Muller in f64 (cosine branch), element i
    from draws 2i and 2i+1."""
    d = draws(seed, 0, 2 * n).reshape(n, 2)
    u1 = ((d[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (d[:, 1] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (z * sigma).astype(np.float32)


def uniform_int(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform in [lo, hi] (multiply-shift on the high 32 bits)."""
    d = draws(seed, 0, n)
    span = np.uint64(hi - lo + 1)
    return (np.uint64(lo) + (((d >> np.uint64(32)) * span) >> np.uint64(32))).astype(np.int64)


def matrix_bytes(ggml_type: int, rows: int, cols: int) -> int:
    if ggml_type == GGML_MXFP4:
        return rows * (cols // 32) * 17
    if ggml_type == GGML_Q4_K:
        return rows * (cols // 256) * 144
    raise ValueError(ggml_type)


def block_bytes(ggml_type: int) -> int:
    return MXFP4_BLOCK_BYTES if ggml_type == GGML_MXFP4 else Q4K_BLOCK_BYTES


def block_elems(ggml_type: int) -> int:
    return MXFP4_BLOCK_ELEMS if ggml_type == GGML_MXFP4 else Q4K_BLOCK_ELEMS

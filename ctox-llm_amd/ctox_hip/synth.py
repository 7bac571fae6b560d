"""Seeded synthetic workloads in the crate's packed CTOXQ layout.

Packing follows Q/src/quant.rs:20-29 and :113-119 / :178-184 (reference
tree, Q/ = models/qwen38_27b/): a block is a little-endian binary16 scale
followed by the codes, Q4 low nibble = even element, Q2 crumb i at bits
2*(i%4) of byte i/4. Rows are dense runs of blocks with no padding.

Distributions are the BASELINE configs: codes uniform, block scales
fp16(|N(0, 0.02)|). (The Q2 "mins" of the BASELINE text have no field in
the crate's symmetric Q2_B64 block and are not generated.)
"""
from __future__ import annotations

import numpy as np

BLOCK_LEN = 64


def pack_q4(codes: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """codes uint8 [rows, cols] in 0..15, scales float16 [rows, cols/64] -> uint8 bytes."""
    rows, cols = codes.shape
    nb = cols // BLOCK_LEN
    c = codes.reshape(rows, nb, BLOCK_LEN)
    packed = (c[:, :, 0::2] | (c[:, :, 1::2] << 4)).astype(np.uint8)
    sc = np.ascontiguousarray(scales_f16.astype(np.float16)).view(np.uint8).reshape(rows, nb, 2)
    return np.concatenate([sc, packed], axis=2).reshape(-1)


def pack_q2(codes: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    rows, cols = codes.shape
    nb = cols // BLOCK_LEN
    c = codes.reshape(rows, nb, BLOCK_LEN)
    packed = (c[:, :, 0::4] | (c[:, :, 1::4] << 2) | (c[:, :, 2::4] << 4) | (c[:, :, 3::4] << 6)).astype(np.uint8)
    sc = np.ascontiguousarray(scales_f16.astype(np.float16)).view(np.uint8).reshape(rows, nb, 2)
    return np.concatenate([sc, packed], axis=2).reshape(-1)


def random_matrix(dtype: int, rows: int, cols: int, seed: int, scale_sigma: float = 0.02) -> np.ndarray:
    """dtype 0 = Q2_B64, 1 = Q4_B64. Returns the packed bytes (uint8)."""
    rng = np.random.default_rng(seed)
    nb = cols // BLOCK_LEN
    scales = np.abs(rng.standard_normal((rows, nb), dtype=np.float32) * scale_sigma).astype(np.float16)
    if dtype == 1:
        codes = rng.integers(0, 16, size=(rows, cols), dtype=np.uint8)
        return pack_q4(codes, scales)
    codes = rng.integers(0, 4, size=(rows, cols), dtype=np.uint8)
    return pack_q2(codes, scales)


def unpack_dense(dtype: int, packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Dequantizes to float64 [rows, cols] (value = scale * (2c - off)/off)."""
    nb = cols // BLOCK_LEN
    bb = 34 if dtype == 1 else 18
    blk = packed.reshape(rows, nb, bb)
    scale = blk[:, :, :2].copy().view(np.float16).reshape(rows, nb).astype(np.float64)
    body = blk[:, :, 2:]
    if dtype == 1:
        codes = np.empty((rows, nb, 64), dtype=np.int64)
        codes[:, :, 0::2] = body & 0x0F
        codes[:, :, 1::2] = body >> 4
        w = (2 * codes - 15) / 15.0
    else:
        codes = np.empty((rows, nb, 64), dtype=np.int64)
        for s in range(4):
            codes[:, :, s::4] = (body >> (2 * s)) & 3
        w = (2 * codes - 3) / 3.0
    return (w * scale[:, :, None]).reshape(rows, cols)


def activation(kind: str, n: int, seed: int, batch: int = 1) -> np.ndarray:
    """'normal': N(0,1); 'swiglu': SiLU(N(0,1)) * N(0,1) (the down-projection input)."""
    rng = np.random.default_rng(seed)
    if kind == "normal":
        return rng.standard_normal((batch, n), dtype=np.float32)
    g = rng.standard_normal((batch, n), dtype=np.float32)
    u = rng.standard_normal((batch, n), dtype=np.float32)
    return (g / (1.0 + np.exp(-g)) * u).astype(np.float32)

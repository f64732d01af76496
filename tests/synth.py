"""Seeded synthetic inputs in ggml block formats (numpy only).

Distributions follow the workload definitions: Q8_0 weights with qs uniform
in [-127, 127] and d = fp16(|N(0, 0.02)| / 127); Q4_0 weights with nibbles
uniform in [0, 15] and d = fp16(|N(0, 0.02)| / 8); activations N(0, 1).
"""
import numpy as np


def f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_weights(rng, n, k):
    nb = k // 32
    qs = rng.integers(-127, 128, size=(n, nb, 32), dtype=np.int64).astype(np.int8)
    d = f16_bits(np.abs(rng.normal(0.0, 0.02, size=(n, nb))) / 127.0)
    blk = np.empty((n, nb, 34), dtype=np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    blk[:, :, 2:] = qs.view(np.uint8)
    return blk.reshape(n, nb * 34)


def q4_0_weights(rng, n, k):
    nb = k // 32
    nib = rng.integers(0, 16, size=(n, nb, 32), dtype=np.int64).astype(np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, 0.02, size=(n, nb))) / 8.0)
    blk = np.empty((n, nb, 18), dtype=np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    blk[:, :, 2:] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    return blk.reshape(n, nb * 18)


def q8_0_split(blocks, n, k):
    """(qs int8 [n, k], d float32 [n, k/32]) from ggml Q8_0 bytes."""
    b = np.ascontiguousarray(blocks).reshape(n, k // 32, 34)
    d = b[:, :, 0:2].copy().view(np.uint16).reshape(n, k // 32).view(np.float16).astype(np.float32)
    qs = b[:, :, 2:].copy().view(np.int8).reshape(n, k)
    return qs, d


def xq_to_blocks(qs, d_bits, k):
    """planar activation (qs int8 [k], d fp16 bits [k/32]) -> ggml block_q8_0 bytes"""
    nb = k // 32
    blk = np.empty((nb, 34), dtype=np.uint8)
    blk[:, 0:2] = np.ascontiguousarray(d_bits, dtype=np.uint16).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = np.ascontiguousarray(qs, dtype=np.int8).view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def rel_err(y, ref):
    """max_i |y_i - ref_i| / max(|ref_i|, rms(ref)): relative error with an rms floor so that
    outputs near zero do not dominate."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    floor = np.sqrt(np.mean(ref * ref)) + 1e-30
    return float(np.max(np.abs(y - ref) / np.maximum(np.abs(ref), floor)))

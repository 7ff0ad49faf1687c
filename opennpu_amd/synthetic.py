"""Seeded synthetic inputs with the distributions of the benchmark configurations.

  * weights: 4-bit codes uniform in 0..15 (= v + 8, v uniform in [-8, 7]), packed two per byte
    with the low nibble holding the even k; g128s scales bf16(|N(0, 0.02)| + 1e-4);
    GGUF Q4_0 d = fp16(|N(0, 0.01)|)
  * activations: bf16(N(0, 1)); router logits N(0, 1) fp32
Everything is returned as numpy arrays in the staging layout of include/onpu.h (bf16 / fp16 as
uint16 bit patterns). numpy's default_rng(seed) makes the arrays reproducible anywhere.
"""
import numpy as np

FMT_Q4NX, FMT_Q4S, FMT_G128S, FMT_Q4_0 = 0, 1, 2, 3


def bf16_bits(x):
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_float(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def stage_bytes(fmt, N, K):
    if fmt == FMT_Q4_0:
        return N * (K // 32) * 18
    g = 128 if fmt == FMT_G128S else 32
    return N * K // 2 + N * (K // g) * 2 * (2 if fmt == FMT_Q4NX else 1)


def weights(fmt, N, K, seed, scale_sigma=None, signed=False):
    """One [N][K] matrix in the staging layout (uint8 array of stage_bytes(fmt, N, K)). signed: each
    bf16 scale (and q4nx min) gets a random sign, so that the weights have mean zero (uniform codes
    alone give u - 8 a mean of -1/2)."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, size=N * K // 2, dtype=np.uint8)
    if fmt == FMT_Q4_0:
        sig = 0.01 if scale_sigma is None else scale_sigma
        d = np.abs(rng.normal(0.0, sig, size=N * (K // 32))).astype(np.float16).view(np.uint16)
        blk = np.empty((N * (K // 32), 18), np.uint8)
        blk[:, 0] = (d & 0xFF).astype(np.uint8)
        blk[:, 1] = (d >> 8).astype(np.uint8)
        blk[:, 2:] = codes.reshape(-1, 16)
        return blk.reshape(-1)
    g = 128 if fmt == FMT_G128S else 32
    sig = 0.02 if scale_sigma is None else scale_sigma
    s = bf16_bits(np.abs(rng.normal(0.0, sig, size=N * (K // g))) + 1e-4)
    if signed:
        s |= (rng.integers(0, 2, size=s.size, dtype=np.uint16) << 15).astype(np.uint16)
    parts = [codes, s.view(np.uint8)]
    if fmt == FMT_Q4NX:
        m = bf16_bits(rng.normal(0.0, sig * 4, size=N * (K // g)))
        parts.append(m.view(np.uint8))
    return np.concatenate(parts)


def activations(M, K, seed):
    """bf16 bits [M][K] of N(0, 1)."""
    rng = np.random.default_rng(seed)
    return bf16_bits(rng.standard_normal((M, K), dtype=np.float32))


def logits(T, E, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((T, E), dtype=np.float32)

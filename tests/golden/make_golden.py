"""Writes the golden fixtures in this folder (run: python tests/golden/make_golden.py).

The reference holds no golden vectors for the int4 path, so these are built from the formats'
definitions with numpy alone — no code of this library and none of the oracle's C restatement:
  * codes v in [-8, 7] and scales are drawn, then packed by hand into the staging layout of
    include/onpu.h (low nibble = even k; GGUF block_q4_0: element j in the low nibble of qs[j],
    element j + 16 in its high nibble, w = (q - 8) * d — ggml's Q4_0 definition);
  * the dequantized weights are built from (v, s) directly, not by reading the packed bytes back,
    so a nibble-order or offset mistake in an unpacker fails the fixture;
  * y is numpy float64 matmul of those weights with the bf16 activations; router outputs come from
    numpy softmax + stable argsort; argmax from numpy (first maximum).
Inputs and expected outputs are stored together in golden.npz (about 90 KB).
"""
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_float(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_nibbles(u):
    """codes u [N][K] (0..15) -> bytes [N][K/2], even k in the low nibble"""
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def case(fmt, N, K, M, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    if fmt == 3:                                          # GGUF Q4_0
        d = np.abs(rng.normal(0, 0.01, size=(N, K // 32))).astype(np.float16)
        blocks = np.empty((N, K // 32, 18), np.uint8)
        blocks[:, :, 0:2] = d.view(np.uint8).reshape(N, K // 32, 2)
        ub = u.reshape(N, K // 32, 32)
        blocks[:, :, 2:] = ub[:, :, :16] | (ub[:, :, 16:] << 4)
        st = blocks.reshape(-1)
        w = (u.astype(np.float64) - 8) * np.repeat(d.astype(np.float64), 32, axis=1)
    else:
        g = 128 if fmt == 2 else 32
        s = bf16_bits(np.abs(rng.normal(0, 0.02, size=(N, K // g))) + 1e-4)
        sf = np.repeat(bf16_float(s).astype(np.float64), g, axis=1)
        parts = [pack_nibbles(u).reshape(-1), s.reshape(-1).view(np.uint8)]
        if fmt == 0:                                      # q4nx: w = u * s + m (fp32 product, then sum)
            m = bf16_bits(rng.normal(0, 0.08, size=(N, K // g)))
            mf = np.repeat(bf16_float(m), g, axis=1)
            prod = (u.astype(np.float32) * bf16_float(np.repeat(s, g, axis=1))).astype(np.float32)
            w = (prod + mf).astype(np.float32).astype(np.float64)
            parts.append(m.reshape(-1).view(np.uint8))
        else:
            w = (u.astype(np.float64) - 8) * sf
        st = np.concatenate(parts)
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    y = bf16_float(x).astype(np.float64) @ w.T
    return st, x, u, w.astype(np.float32), y


def route_case(T, E, k, seed):
    rng = np.random.default_rng(seed)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, 3] = lg[0, 5] = lg[0].max() + 0.5                # a tie at the top: the lower id comes first
    p = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(p, ids, axis=1)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return lg, ids, w


def main():
    out = {}
    for fmt, N, K, M, seed in [(0, 16, 256, 3, 10), (1, 16, 256, 3, 11), (2, 24, 384, 3, 12), (3, 20, 256, 5, 13)]:
        st, x, u, w, y = case(fmt, N, K, M, seed)
        out.update({f"f{fmt}_st": st, f"f{fmt}_x": x, f"f{fmt}_u": u, f"f{fmt}_w": w, f"f{fmt}_y": y,
                    f"f{fmt}_shape": np.array([N, K, M], np.int64)})
    lg, ids, w = route_case(6, 128, 8, 20)
    out.update(route_logits=lg, route_ids=ids, route_w=w)
    v = np.random.default_rng(21).standard_normal((4, 1000)).astype(np.float32)
    v[1, 10] = v[1, 700] = v[1].max() + 1.0                # tie: the first index wins
    out.update(argmax_in=v, argmax_out=np.argmax(v, axis=1).astype(np.int32))
    np.savez_compressed(HERE / "golden.npz", **out)
    print("wrote", HERE / "golden.npz")


if __name__ == "__main__":
    main()

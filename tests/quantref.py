"""Shared by tests/test_quant_ref.py, tests/test_npu_layout.py (CPU) and tests/test_codec_gpu.py
(GPU): the reference's bf16 rounding, Mat geometry, search quantizers, packing and output gather
built from llama/ggml-opennpu/opennpu_core.hpp lines 37-254 and 540-561 (oracle/Makefile `ref`,
oracle/ref_core.cpp; outputs in oracle/_ref/), and the weight groups the comparisons run on."""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle.oracle as orc

ROOT = Path(__file__).resolve().parents[1]
REFCORE = Path("/root/reference/llama/ggml-opennpu/opennpu_core.hpp")
REF = ROOT / "oracle" / "_ref"


def load(name):
    path = REF / name
    if not path.exists():
        if not REFCORE.exists():
            pytest.skip("the reference checkout is not on this machine")
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "ref"], check=True)
    L = C.CDLL(str(path))
    P, I64, I = C.c_void_p, C.c_int64, C.c_int
    L.ref_geometry.argtypes = [I64, I64, I, I, P]
    L.ref_quant_sym32_n.argtypes = [P, I64, P, P]
    L.ref_quant_asym32_n.argtypes = [P, I64, P, P, P]
    L.ref_f2bf_n.argtypes = [P, I64, P]
    L.ref_pack_mat.restype, L.ref_pack_mat.argtypes = I64, [P, I64, I64, I, I, P]
    L.ref_gather.argtypes = [I64, I64, I, I, P, P]
    return L


def ref_pack(L, fmt, W, ncols):
    """pack_mat(Mat(N, K, ncols, q4s?), W) by the reference's own code: its nbytes packed bytes"""
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    nbytes = orc.geometry(N, K, ncols, fmt == orc.FMT_Q4S)[7]
    out = np.zeros(nbytes, np.uint8)
    assert L.ref_pack_mat(p(W), N, K, ncols, fmt, p(out)) == nbytes
    return out


def p(a):
    return a.ctypes.data


def ref_sym(L, X):
    """quant_sym32 over X [G][32]: codes [G][32], bf16 d [G]"""
    X = np.ascontiguousarray(X, np.float32)
    G = X.shape[0]
    q = np.empty((G, 32), np.uint8)
    d = np.empty(G, np.uint16)
    L.ref_quant_sym32_n(p(X), G, p(q), p(d))
    return q, d


def ref_asym(L, X):
    """quant_asym32 over X [G][32]: codes [G][32], bf16 s [G], m [G]"""
    X = np.ascontiguousarray(X, np.float32)
    G = X.shape[0]
    q = np.empty((G, 32), np.uint8)
    s = np.empty(G, np.uint16)
    m = np.empty(G, np.uint16)
    L.ref_quant_asym32_n(p(X), G, p(q), p(s), p(m))
    return q, s, m


GPR = 64                                    # groups per matrix row (K = 2048)


def groups(kind, G, seed):
    """G groups of 32 weights of one kind (float32 [G][32])"""
    rng = np.random.default_rng(seed)
    if kind == "normal":
        X = rng.standard_normal((G, 32)) * 0.02
    elif kind == "heavy":                   # Student t, 2 degrees of freedom: outliers in most groups
        X = rng.standard_t(2, (G, 32)) * 0.01
    elif kind == "positive":
        X = np.abs(rng.standard_normal((G, 32))) * rng.choice([1e-3, 0.05, 3.0], (G, 1)) + 1e-4
    elif kind == "tiny":                    # down to the subnormal range (scales flush to zero there)
        X = rng.standard_normal((G, 32)) * 10.0 ** rng.uniform(-44, -30, (G, 1))
    elif kind == "huge":                    # squared errors overflow to inf near the top
        X = rng.standard_normal((G, 32)) * 10.0 ** rng.uniform(25, 37.5, (G, 1))
    elif kind == "scales":                  # one magnitude per group over 1e-8 .. 1e3
        X = rng.standard_normal((G, 32)) * 10.0 ** rng.uniform(-8, 3, (G, 1))
    elif kind == "grid":                    # exact grids v*d (v in -8..7) and half-way points
        v = rng.integers(-8, 8, (G, 32)).astype(np.float64)
        half = rng.random((G, 32)) < 0.25
        d = orc.bf2f(orc.f2bf_np(np.abs(rng.standard_normal(G)) * 0.01 + 1e-4)).astype(np.float64)
        X = (v + 0.5 * half) * d[:, None]
        X[::3] -= X[::3].min(axis=1, keepdims=True)         # shifted grids for q4nx's u*s + m
    elif kind == "ties":                    # planted ties: +-absmax both present, repeated extremes,
        X = rng.standard_normal((G, 32)) * 0.02             # constant, zero and single-spike groups
        a = np.abs(X).max(axis=1)
        i, j = rng.integers(0, 32, G), rng.integers(0, 32, G)
        X[np.arange(G), i] = a
        X[np.arange(G), j] = -a
        X[0::7] = X[0::7, :1]                               # constant groups (range 0)
        X[1::7] = 0.0                                       # all-zero groups
        X[2::7, 1:] = 0.0                                   # one value, the rest zero
        X[3::7, ::2] = X[3::7, :1]                          # half the group at one value
        X[4::7] = np.round(X[4::7] * 50) / 50               # few distinct values, many repeats
    else:
        raise ValueError(kind)
    return X.astype(np.float32)


KINDS = ["normal", "heavy", "positive", "tiny", "huge", "scales", "grid", "ties"]
G_PER_KIND = 128 * GPR                      # 8192 groups per kind and seed
SEEDS = 16                                  # 8 kinds x 16 seeds x 8192 = 1,048,576 groups per format


def stage_sym(q, d, N, K):
    """codes [N][K] + bf16 d [N][K/32] -> q4s staging bytes (low nibble = even k)"""
    q = q.reshape(N, K)
    codes = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return np.concatenate([codes.ravel(), d.ravel().view(np.uint8)])


def ref_staging(L, fmt, X):
    """groups X [G][32] as a matrix of GPR groups per row -> (W, the reference's staging bytes)"""
    W = np.ascontiguousarray(X, np.float32).reshape(-1, 32 * GPR)
    N, K = W.shape
    if fmt == orc.FMT_Q4S:
        q, d = ref_sym(L, X)
        return W, stage_sym(q, d, N, K)
    q, s, m = ref_asym(L, X)
    return W, orc.stage_q4nx(q.reshape(N, K), s.reshape(N, K // 32), m.reshape(N, K // 32))


def staging_source():
    """(fn(fmt, X) -> (W, staging bytes), label): the reference's as-written build where it is on
    this machine (it travels with built libraries), else the oracle, which tests/test_quant_ref.py
    pins to that build byte for byte"""
    path = REF / "libonpu_core_ref.so"
    if path.exists() or REFCORE.exists():
        L = load("libonpu_core_ref.so")
        return (lambda fmt, X: ref_staging(L, fmt, X)), "reference build"

    def orc_staging(fmt, X):
        W = np.ascontiguousarray(X, np.float32).reshape(-1, 32 * GPR)
        return W, orc.quantize(fmt, W)
    return orc_staging, "oracle"

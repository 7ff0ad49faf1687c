"""GPU parity of the weight codecs (onpu_quantize_dev, onpu_transcode_q4k_dev) against the oracle.

The oracle restates the reference's quantizers (opennpu_core.hpp:103-169; ggml's Q4_0 rule) and its
Q4_K -> q4nx transcode (ggml-opennpu.cpp:103-138); tests/test_oracle.py pins them. Here the GPU
quantizes weights already in HBM into a handle, and the handle's dequantized weights must equal the
dequantization of the oracle's staging bytes bit for bit (codes and parameters identical), for
fp32 and bf16 inputs, ragged row counts, banks and strided rows. Integer-and-rounding work: the bar
is bit-exact.
"""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc

pytestmark = pytest.mark.gpu
FMTS = [orc.FMT_Q4NX, orc.FMT_Q4S, orc.FMT_G128S, orc.FMT_Q4_0]


def _weights(rng, N, K):
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[1, 5] = 0.7                                   # an outlier
    W[2] = 0.0                                      # an all-zero row
    W[3, :64] = 0.25                                # constant groups
    return W


def _bf16_round(W):
    return orc.bf2f(orc.f2bf_np(W)).reshape(W.shape)


@pytest.mark.parametrize("wdt", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_dev_equals_oracle(gpu, fmt, wdt):
    import torch
    from opennpu_amd.device import QMatrix
    rng = np.random.default_rng(40 + fmt)
    for N, K in [(37, 512), (16, 256), (5, 1024)]:
        W = _weights(rng, N, K)
        if wdt == "bf16":
            W = _bf16_round(W)
            Wd = torch.from_numpy(orc.f2bf_np(W).view(np.int16)).view(torch.bfloat16).cuda()
        else:
            Wd = torch.from_numpy(W).cuda()
        q = QMatrix(N, K, fmt)
        try:
            print(f"quantize_dev fmt {fmt} {wdt} N={N} K={K}", flush=True)
            q.quantize(Wd)
            torch.cuda.synchronize()
            got = q.dequant()
        finally:
            q.free()
        want = orc.dequant(fmt, orc.quantize(fmt, W), N, K)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (fmt, wdt, N, K)


def test_quantize_dev_strided_rows_and_gemv(gpu):
    """rows ldw > K apart (a column slice of a wider tensor); the quantized matrix's GEMV equals
    that of the same matrix loaded from the oracle's staging bytes, bit for bit"""
    import torch
    from opennpu_amd import synthetic as syn
    from opennpu_amd.device import QMatrix
    rng = np.random.default_rng(50)
    N, K, fmt = 300, 768, orc.FMT_Q4S
    Wide = (rng.standard_normal((N, K + 96)) * 0.02).astype(np.float32)
    W = np.ascontiguousarray(Wide[:, :K])
    q1, q2 = QMatrix(N, K, fmt), QMatrix(N, K, fmt, orc.quantize(fmt, W))
    try:
        q1.quantize(torch.from_numpy(Wide).cuda()[:, :K])
        x = torch.from_numpy(syn.activations(3, K, 51).view(np.int16)).view(torch.bfloat16).cuda().reshape(3, K)
        y1, y2 = q1.mv(x), q2.mv(x)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
    finally:
        q1.free()
        q2.free()


@pytest.mark.parametrize("fmt", [orc.FMT_Q4NX, orc.FMT_G128S])
def test_quantize_dev_bank_experts(gpu, fmt):
    """experts [1, 3) of a 3-expert bank from one [2][N][K] tensor; expert 0 stays as loaded"""
    import torch
    from opennpu_amd.device import QFfn
    rng = np.random.default_rng(60 + fmt)
    E, H, I = 3, 256, 128                           # I a multiple of 128 for g128s's down K
    gu = [(rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32) for _ in range(E)]
    dn = [(rng.standard_normal((H, I)) * 0.02).astype(np.float32) for _ in range(E)]
    f = QFfn(E, H, I, fmt)
    try:
        f.load(orc.quantize(fmt, gu[0]), orc.quantize(fmt, dn[0]), e0=0)
        f.quantize(torch.from_numpy(np.stack(gu[1:])).cuda(), torch.from_numpy(np.stack(dn[1:])).cuda(), e0=1)
        torch.cuda.synchronize()
        L = f.L
        for e in range(E):
            for h, Ws, N, K in ((f.gu, gu, 2 * I, H), (f.dn, dn, H, I)):
                got = np.empty((N, K), np.float32)
                assert L.onpu_dense_dequant(h, e, C.c_void_p(got.ctypes.data), 0) == 0
                want = orc.dequant(fmt, orc.quantize(fmt, Ws[e]), N, K)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (e, N, K)
    finally:
        f.free()


def _q4k_blocks(rng, N, K):
    nb = N * (K // 256)
    b = rng.integers(0, 256, (nb, 144)).astype(np.uint8)
    b[:, 0:2] = rng.uniform(1e-4, 3e-2, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = rng.uniform(0, 1e-2, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[1, 4:16] = 0                                  # zero scales and mins: the tie rule
    return b.reshape(N, K // 256 * 144)


def test_transcode_q4k_dev_equals_oracle(gpu):
    import torch
    from opennpu_amd.device import QMatrix
    rng = np.random.default_rng(70)
    for N, K in [(21, 512), (64, 2048)]:
        blocks = _q4k_blocks(rng, N, K)
        q = QMatrix(N, K, orc.FMT_Q4NX)
        try:
            print(f"transcode_q4k_dev N={N} K={K}", flush=True)
            q.transcode_q4k(torch.from_numpy(blocks).cuda())
            torch.cuda.synchronize()
            got = q.dequant()
        finally:
            q.free()
        u, s, m = orc.transcode_q4k(blocks, N, K)
        want = orc.dequant(orc.FMT_Q4NX, orc.stage_q4nx(u, s, m), N, K)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (N, K)


def test_codec_argument_errors(gpu):
    """host-side checks: a Q4_K transcode into a non-q4nx handle, K not a multiple of 256, a row
    stride below K, an expert range past E: each returns -1 with a message and launches nothing"""
    import torch
    from opennpu_amd.device import QMatrix
    L = gpu
    q1 = QMatrix(16, 256, orc.FMT_Q4S)
    q2 = QMatrix(16, 128 + 32 * 3, orc.FMT_Q4NX)
    try:
        blk = torch.zeros((16, 144), dtype=torch.uint8, device="cuda")
        p = C.c_void_p(blk.data_ptr())
        assert L.onpu_transcode_q4k_dev(q1.h, 0, 1, p, 144, None) == -1
        assert L.onpu_transcode_q4k_dev(q2.h, 0, 1, p, 144, None) == -1
        W = torch.zeros((16, 256), dtype=torch.float32, device="cuda")
        assert L.onpu_quantize_dev(q1.h, 0, 1, C.c_void_p(W.data_ptr()), 128, 0, None) == -1
        assert L.onpu_quantize_dev(q1.h, 1, 1, C.c_void_p(W.data_ptr()), 256, 0, None) == -1
        assert L.onpu_quantize_dev(q1.h, 0, 1, C.c_void_p(W.data_ptr()), 256, 2, None) == -1
        assert b"bad arguments" in L.onpu_last_error()
    finally:
        q1.free()
        q2.free()


@pytest.mark.parametrize("fmt", [orc.FMT_Q4S, orc.FMT_Q4NX])
def test_quantize_dev_equals_reference_build(gpu, fmt):
    """onpu_quantize_dev writes the reference's own q4s / q4nx choices (opennpu_core.hpp:103-169
    compiled as written, oracle/_ref) on 2^20 groups per format: normal, heavy-tailed, all-positive,
    tiny and huge magnitudes, exact grids and planted ties. Compared through the handle's
    dequantized weights, bit for bit (codes, scales and the sign of -0 all show there)."""
    import torch
    from opennpu_amd.device import QMatrix
    from tests.quantref import KINDS, groups, staging_source
    stage, label = staging_source()
    for kind in KINDS:
        X = groups(kind, 1 << 17, 500 + KINDS.index(kind))
        W, want_st = stage(fmt, X)
        N, K = W.shape
        q = QMatrix(N, K, fmt)
        try:
            print(f"quantize_dev vs {label}: fmt {fmt} kind {kind} N={N} K={K}", flush=True)
            q.quantize(torch.from_numpy(W).cuda())
            torch.cuda.synchronize()
            got = q.dequant()
        finally:
            q.free()
        want = orc.dequant(fmt, want_st, N, K)
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"{kind}: {bad.size} weights differ from the {label}, first at {bad[:4]}"

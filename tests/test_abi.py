"""CPU checks of the C ABI: the library loads, exports every symbol include/onpu.h declares, and its
host-only routines (reference geometry, staging sizes, launch plans, packing) behave; no GPU needed."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "onpu.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(onpu_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_header_symbol():
    L = _lib.lib()
    syms = header_symbols()
    assert len(syms) > 40
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert sorted(_lib.EXPORTS) == syms, "ctypes declarations and header differ"


def test_no_gpu_here_means_not_ok():
    import torch
    L = _lib.lib()
    if not torch.cuda.is_available():
        assert L.onpu_ok() == 0
        assert L.onpu_dense_new3(64, 128, 2) is None      # construction refuses without a GPU
        with pytest.raises(RuntimeError):
            _lib.require_gpu()


# values of the reference Mat formula (model.py:151-187) at the benchmark shapes, as listed for
# (N, K, ncols, sym) -> (R, S, tiles, kc, nbytes)
GEOMETRY = [
    ((4096, 4096, 8, 0), (4, 2, 4, 8, 10_485_760)),
    ((6144, 4096, 8, 0), (4, 2, 6, 8, None)),
    ((24576, 4096, 8, 0), (4, 2, 24, 8, None)),
    ((4096, 12288, 8, 0), (1, 8, 16, 6, None)),
    ((1536, 2048, 1, 0), (1, 1, 6, 8, None)),
    ((2048, 768, 1, 0), (1, 1, 8, 3, None)),
    ((151936, 4096, 8, 0), (4, 2, 149, 8, None)),
]


@pytest.mark.parametrize("args,want", GEOMETRY)
def test_reference_geometry(args, want):
    L = _lib.lib()
    out = (C.c_int64 * 8)()
    L.onpu_geometry2(*args, out)
    got = tuple(out)
    assert got == orc.geometry(*args)
    R, S, tiles, kc, nbytes = want
    assert got[:4] == (R, S, tiles, kc)
    if nbytes is not None:
        assert got[7] == nbytes
    # every staging layout fits in the reference's buffer size for the same matrix
    for fmt in (0, 1, 2, 3):
        N, K = args[0], args[1]
        if K % orc.group(fmt) == 0:
            sym_out = (C.c_int64 * 8)()
            L.onpu_geometry2(N, K, args[2], fmt, sym_out)
            assert L.onpu_stage_bytes(fmt, N, K) == orc.stage_bytes(fmt, N, K) <= sym_out[7]


SHAPES = [(16, 128), (72, 512), (300, 1024), (129, 2080), (6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288),
          (1536, 2048), (2048, 768), (151936, 4096), (14336, 4096), (4096, 14336), (40, 32)]


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_launch_plans_are_built_variants(fmt):
    """Every plan the host picks names a kernel variant that exists, fits its launch bounds and
    the 32 KiB reduction buffer, and covers all K blocks."""
    L = _lib.lib()
    out = (C.c_int64 * 10)()
    for N, K in SHAPES:
        if K % orc.group(fmt):
            continue
        KB = -(-K // 128)
        for M in (1, 2, 5, 8, 16, 17, 33, 64):
            for slots, epi in ((1, 0), (8, 0), (8, 1)):
                if epi == 1 and (N % 32):
                    continue
                L.onpu_plan_gemv(fmt, N, K, M, slots, epi, out)
                mb, rt, nb, xl, tw, kw, bpw, gx, built, maxw = tuple(out)
                assert built, (fmt, N, K, M, epi, tuple(out))
                assert tw * kw <= maxw and tw * kw * rt * mb <= 32
                if xl:                             # x rows + column sums + reduction <= 160 KiB
                    gpb = 1 if fmt == orc.FMT_G128S else 4
                    xb = M * (KB * 128 + 8) * 2 + KB * gpb * 64
                    assert mb == 1 and xb + tw * kw * rt * mb * 1024 <= 163840, (fmt, N, K, M, tuple(out))
                assert kw * bpw >= KB and (kw - 1) * bpw < KB
                NT = -(-N // 16)
                groups = NT // 2 if epi == 1 else NT
                assert gx * tw >= groups
                if epi == 1:
                    assert gx * tw == groups
                assert mb * 16 >= min(M, 64)
        for k in (1, 2, 4, 6, 8, 16):              # MoE decode down projection, weighted slot sum
            L.onpu_plan_gemv(fmt, N, K, 1, k, 2, out)
            mb, rt, nb, xl, tw, kw, bpw, gx, built, maxw = tuple(out)
            assert built and kw % k == 0 and kw <= maxw and kw <= 16, (N, K, k, tuple(out))
            assert (kw // k) * bpw >= KB


def test_mv_plans():
    """onpu_plan_mv (what onpu_dense_mv_dev runs) over shapes and row counts: the GEMV only up to 64
    rows; GEMM tiles of the fewest 16-row blocks that hold the rows up to 64 (1 / 2 / 4), 128 rows
    beyond; K ranges that cover every K block, none empty, at least 4 blocks each unless forced, and
    fp32 partials within the 64 MiB split-K workspace; the stream-K kernel only above 128 rows"""
    L = _lib.lib()
    o = (C.c_int64 * 7)()
    seen = set()
    for N in (64, 1000, 4096, 14336, 24576, 57344, 151936):
        for K in (512, 4096, 8192, 14336, 28672):
            KB = -(-K // 128)
            for M in (1, 2, 4, 8, 12, 16, 17, 24, 32, 33, 48, 64, 65, 96, 128, 129, 256, 512, 2048):
                L.onpu_plan_mv(2, N, K, M, o)
                path, mb, ntw, S, kbs, wgs, deep = tuple(o)
                seen.add((path, mb if path == 1 else 0, deep))
                assert deep in (0, 1) and (not deep or (path == 1 and mb <= 2 and S * wgs <= 512)), (N, K, M, tuple(o))
                assert path in (0, 1, 2) and (path != 0 or M <= 64) and (path != 2 or M > 128), (N, K, M, tuple(o))
                if path != 1:
                    continue
                want = 1 if M <= 16 else 2 if M <= 32 else 4 if M <= 64 else 8
                assert mb == want and (ntw == 2 or mb == 8), (N, K, M, tuple(o))
                assert S * kbs >= KB and (S - 1) * kbs < KB, (N, K, M, tuple(o))
                if S > 1:
                    assert kbs >= 4 and S * M * N * 4 <= 256 * 256 * 1024, (N, K, M, tuple(o))
                assert wgs == -(-M // (16 * mb)) * -(-(-(-N // 16)) // (4 * ntw)), (N, K, M, tuple(o))
    assert {(0, 0, 0), (1, 1, 0), (1, 1, 1), (1, 2, 0), (1, 2, 1), (1, 4, 0), (1, 8, 0), (2, 0, 0)} <= seen, seen


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_argmax_epilogue_plans_sum_like_the_store(fmt):
    """the argmax epilogue's GEMV plan (onpu_dense_argmax_dev) and the plain store's (the no-alloc
    entry point, which stores logits and then runs the separate argmax) agree in everything that
    sets the order of the fp32 sums (K parts, blocks per wave, x from LDS or global, row blocks,
    tile groups per workgroup), for every row count up to 64; only the chunk size may differ"""
    L = _lib.lib()
    a, b = (C.c_int64 * 10)(), (C.c_int64 * 10)()
    for N in (64, 300, 3000, 4096, 6144, 20000, 24576, 151936):
        for K in (256, 512, 1024, 4096, 12288):
            if K % orc.group(fmt):
                continue
            for M in range(1, 65):
                L.onpu_plan_gemv(fmt, N, K, M, 1, 0, a)
                L.onpu_plan_gemv(fmt, N, K, M, 1, 3, b)
                keep = (0, 1, 3, 4, 5, 6, 7)                 # mb, rt, xl, tw, kw, bpw, gx
                assert [a[i] for i in keep] == [b[i] for i in keep], (N, K, M, tuple(a), tuple(b))


def test_pack_round_trip_q4s():
    """onpu_pack writes the reference's packing with its q4s search quantizer; its dequantization
    equals onpu_quant_dequant, and its codes and scales equal the oracle's."""
    L = _lib.lib()
    rng = np.random.default_rng(0)
    N, K = 24, 256
    W = rng.standard_normal((N, K)).astype(np.float32) * 0.05
    g = (C.c_int64 * 8)()
    L.onpu_geometry2(N, K, 8, 1, g)
    out = np.zeros(g[7], np.uint8)
    n = L.onpu_pack(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, 8, 1, out.ctypes.data_as(C.POINTER(C.c_uint8)), 2)
    assert n == g[7]
    st = orc.npu_to_stage(1, out, N, K, 8)
    deq = orc.dequant(1, st, N, K)
    qd = np.empty_like(W)
    L.onpu_quant_dequant(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, 1, qd.ctypes.data_as(C.POINTER(C.c_float)), 2)
    assert np.array_equal(deq, qd)
    # 4-bit quantization noise of Gaussian weights: ~10% of their rms (the search may clip)
    assert np.linalg.norm(deq - W) / np.linalg.norm(W) < 0.15
    # codes and scales agree with the oracle's restatement of quant_sym32, group by group
    for r in range(0, N, 7):
        for gi in range(K // 32):
            q, d = orc.quant_sym32(W[r, 32 * gi:32 * gi + 32])
            assert np.array_equal(orc.unpack(1, st, N, K)[r, 32 * gi:32 * gi + 32], q)
            assert st[N * K // 2:].view(np.uint16)[r * (K // 32) + gi] == d


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_pack_equals_oracle_quantize(fmt):
    """onpu_pack (host quantizers of onpu_codec.h) writes exactly the oracle's bytes, for every
    format (the reference's packing for q4nx / q4s, the staging layout zero-padded for the others),
    Gaussian weights with a few outliers and an all-zero row"""
    L = _lib.lib()
    rng = np.random.default_rng(20 + fmt)
    N, K = 19, 512
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[3, 17] = 0.9
    W[5] = 0.0
    g = (C.c_int64 * 8)()
    L.onpu_geometry2(N, K, 8, fmt, g)
    assert g[7] > 0
    out = np.zeros(g[7], np.uint8)
    n = L.onpu_pack(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, 8, fmt, out.ctypes.data_as(C.POINTER(C.c_uint8)), 3)
    assert n == g[7]
    if fmt in (orc.FMT_Q4NX, orc.FMT_Q4S):
        assert np.array_equal(out, orc.npu_pack(fmt, W, 8))
        return
    sb = orc.stage_bytes(fmt, N, K)
    assert np.array_equal(out[:sb], orc.quantize(fmt, W))
    assert not out[sb:].any()


def test_pack_q4k_equals_oracle_transcode():
    """onpu_pack_q4k (GGUF Q4_K -> q4nx staging on the host) writes exactly the oracle's transcode"""
    L = _lib.lib()
    rng = np.random.default_rng(30)
    N, K = 7, 768
    nb = N * (K // 256)
    blocks = rng.integers(0, 256, (nb, 144)).astype(np.uint8)
    d = (rng.uniform(1e-4, 3e-2, nb)).astype(np.float16)
    dmin = (rng.uniform(0, 1e-2, nb)).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    blocks[0, 4:16] = 0                                   # zero scales and mins in one super-block
    out = np.zeros(orc.stage_bytes(orc.FMT_Q4NX, N, K), np.uint8)
    n = L.onpu_pack_q4k(blocks.ctypes.data_as(C.POINTER(C.c_uint8)), N, K, out.ctypes.data_as(C.POINTER(C.c_uint8)), 2)
    assert n == out.size
    q, s, m = orc.transcode_q4k(blocks, N, K)
    assert np.array_equal(out, orc.stage_q4nx(q, s, m))
    assert L.onpu_pack_q4k(blocks.ctypes.data_as(C.POINTER(C.c_uint8)), N, 384, out.ctypes.data_as(C.POINTER(C.c_uint8)), 1) == 0

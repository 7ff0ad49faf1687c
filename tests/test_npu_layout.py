"""The reference's NPU packing (the bytes of *_buf memory for q4nx and q4s handles, and of npu4's
PackCache files) and the fused FFN's gate_up row order, against the reference's own code.

- pack_mat (llama/ggml-opennpu/opennpu_core.hpp:230-254, pack_block_fn :176-215), compiled from the
  reference checkout (oracle/Makefile `ref`): the library's onpu_pack and the oracle's npu_pack
  write its bytes, byte for byte, over shapes with ragged rows and columns, several K slices, row
  blocks past the matrix (all-zero column blocks) and 1..8 columns; the oracle's npu_to_stage reads
  them back to the staging bytes of the same quantizers.
- gather (opennpu_core.hpp:540-561), the reference host's reading of its NPU's output order: a
  one-hot output vector at each position names the row that position belongs to, which is the
  order onpu_ffn_perm gives (onpu_api.cpp:307-322); the oracle's ffn_order must equal it.

CPU tests; they run where the reference checkout is present. tests/test_npu_layout_gpu.py checks
the device conversion of these bytes."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import _lib
from tests.quantref import REF, REFCORE, load, p, ref_pack

SHAPES = [            # N, K, ncols
    (64, 256, 8), (1, 32, 8), (100, 96, 8), (300, 544, 8), (257, 1024, 1), (1000, 2048, 4),
    (70, 3072, 3), (513, 2080, 2), (2048, 4096, 8), (4096, 4096, 8), (1536, 2048, 1), (768, 768, 6),
]


@pytest.fixture(scope="module")
def ref():
    if not REFCORE.exists() and not (REF / "libonpu_core_ref.so").exists():
        pytest.skip("the reference checkout is not on this machine")
    return load("libonpu_core_ref.so")


def lib_pack(fmt, W, ncols):
    L = _lib.lib()
    N, K = W.shape
    nbytes = orc.geometry(N, K, ncols, fmt == orc.FMT_Q4S)[7]
    out = np.full(nbytes, 0xA5, np.uint8)                 # every byte must be written
    n = L.onpu_pack(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, ncols, fmt, out.ctypes.data_as(C.POINTER(C.c_uint8)),
                    4)
    assert n == nbytes
    return out


def weights(N, K, seed):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((N, K)) * 0.02
    W[:, : K // 3] += 0.01                                   # q4nx mins of both signs
    return W.astype(np.float32)


@pytest.mark.parametrize("fmt", [orc.FMT_Q4NX, orc.FMT_Q4S])
def test_pack_equals_reference_pack_mat(ref, fmt):
    """onpu_pack and the oracle's npu_pack equal the reference's pack_mat; npu_to_stage inverts it"""
    for i, (N, K, ncols) in enumerate(SHAPES):
        g = orc.geometry(N, K, ncols, fmt == orc.FMT_Q4S)
        assert g[7], (N, K, ncols)
        W = weights(N, K, 10 * i + fmt)
        want = ref_pack(ref, fmt, W, ncols)
        assert np.array_equal(lib_pack(fmt, W, ncols), want), (N, K, ncols)
        assert np.array_equal(orc.npu_pack(fmt, W, ncols), want), (N, K, ncols)
        assert np.array_equal(orc.npu_to_stage(fmt, want, N, K, ncols), orc.quantize(fmt, W)), (N, K, ncols)


def test_shapes_cover_padding_cases():
    """the sweep holds every padding case of the layout"""
    seen = set()
    for N, K, ncols in SHAPES:
        R, S, tiles, kc, ks, rows_col, cb, nbytes = orc.geometry(N, K, ncols, False)
        seen.add("ragged rows" if N % 64 else "whole tiles")
        seen.add("ragged K" if K % 256 else "whole K steps")
        if R * rows_col - N >= rows_col:
            seen.add("empty row block")
        if S > 1:
            seen.add("several K slices")
        if tiles % 2:
            seen.add("odd tiles")
        if kc % 2:
            seen.add("odd K steps")
    assert seen >= {"ragged rows", "whole tiles", "ragged K", "whole K steps", "empty row block", "several K slices",
                    "odd tiles", "odd K steps"}, seen


def test_pack_padding_bytes(ref):
    """padding as the reference writes it: code 8 (q4s) / 0 (q4nx) and zero parameters past the
    matrix inside a column block, all-zero column blocks past it"""
    N, K, ncols = 100, 96, 8
    for fmt, pad in ((orc.FMT_Q4S, 0x88), (orc.FMT_Q4NX, 0x00)):
        W = weights(N, K, 7)
        got = lib_pack(fmt, W, ncols)
        R, S, tiles, kc, ks, rows_col, cb, nbytes = orc.geometry(N, K, ncols, fmt == orc.FMT_Q4S)
        assert not got[cb:].any()                            # row blocks 1..7 hold no rows
        pk = got[:cb].reshape(tiles * kc, 4, -1)            # packets [tile, K step][core row]
        assert (pk[:, 1:, :8192] == pad).all()               # core rows 1..3: rows 128.. of the block
        assert not pk[:, 1:, 8192:].any()
        assert (pk[:, 0, :8192] != pad).any()


def gather_order(ref, Ng, Kg, sym):
    """for each gate_up row, the NPU output position gather reads it from"""
    R, S, tiles, kc, ks, rows_col, cb, nbytes = orc.geometry(Ng, Kg, 1, sym)
    per_col = (tiles + tiles % 2) * 4 * 64
    out = np.zeros(Ng, np.float32)
    pos = np.full(Ng, -1, np.int64)
    y = np.zeros(per_col, np.uint16)
    for q in range(per_col):
        y[:] = 0
        y[q] = 0x3F80                                        # bf16 1.0
        ref.ref_gather(Ng, Kg, 1, sym, p(y), p(out))
        nz = np.flatnonzero(out)
        assert nz.size <= 1
        if nz.size:
            pos[nz[0]] = q
    return pos


@pytest.mark.parametrize("shape", [(1536, 2048, 2048, 768), (2048, 1024, 1024, 1024), (3072, 512, 512, 1536),
                                   (512, 256, 256, 256)])
def test_ffn_order_equals_reference_gather(ref, shape):
    """fused shapes: row r of the gate_up bank is read from output position ffn_order[r]"""
    Ng, Kg, Nd, Kd = shape
    for sym in (0, 1):
        want = gather_order(ref, Ng, Kg, sym)
        assert sorted(want) == list(range(Ng))
        assert np.array_equal(orc.ffn_order(Ng, Kg, Nd, Kd, sym), want), (shape, sym)


def test_ffn_order_identity_where_the_reference_does_not_fuse():
    """the reference's rule (onpu_api.cpp:310-311): I a multiple of 256, Kd = I, one column, an
    even tile count, Kg <= 2048; any other shape packs gate_up rows in order"""
    for Ng, Kg, Nd, Kd in [(768, 256, 256, 384), (1536, 2048, 2048, 512), (1536, 4096, 4096, 768),
                           (2560, 512, 512, 1024), (1536 + 256, 512, 512, 896)]:
        assert np.array_equal(orc.ffn_order(Ng, Kg, Nd, Kd, 0), np.arange(Ng)), (Ng, Kg, Nd, Kd)
    assert not np.array_equal(orc.ffn_order(1536, 2048, 2048, 768, 0), np.arange(1536))


def test_staging_formats_keep_staging_bytes():
    """onpu_pack of this library's own formats (g128s, Q4_0): the staging bytes, zero-padded"""
    L = _lib.lib()
    N, K = 200, 512
    W = weights(N, K, 3)
    for fmt in (orc.FMT_G128S, orc.FMT_Q4_0):
        nbytes = orc.geometry(N, K, 8, True)[7]
        out = np.full(nbytes, 0xA5, np.uint8)
        assert L.onpu_pack(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, 8, fmt,
                           out.ctypes.data_as(C.POINTER(C.c_uint8)), 2) == nbytes
        sb = orc.stage_bytes(fmt, N, K)
        assert np.array_equal(out[:sb], orc.quantize(fmt, W)) and not out[sb:].any()

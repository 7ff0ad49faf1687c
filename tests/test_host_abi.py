"""The reference loader's contract, checked on the CPU (no GPU calls): the library loads under the
reference's own ctypes declarations (opennpu/native/npu4/model.py:281-335), exports every entry
that loader declares or binds when present, reports the reference's Mat geometry, packs into its
own buffer size, and refuses to construct device objects where no GPU is visible (the loader then
returns None, because onpu_ok() is 0)."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc
from tests import hostabi as ha


@pytest.fixture(scope="module")
def L():
    return ha.bind()


def test_loader_contract(L):
    for name in ha.REQUIRED + ha.OPTIONAL:
        assert hasattr(L, name), name
    # OPENNPU_LIBONPU names the file the reference opens; the default path is the in-tree build
    assert ha.library_path().exists()


@pytest.mark.parametrize("N,K,ncols,sym", [(4096, 4096, 8, 1), (6144, 4096, 8, 0), (4096, 12288, 8, 1),
                                           (1536, 2048, 1, 1), (2048, 768, 1, 0), (151936, 4096, 8, 1),
                                           (24576, 4096, 8, 0), (96, 256, 2, 1)])
def test_geometry_as_check_geometry_compares_it(L, N, K, ncols, sym):
    """model.py:353-360 compares all eight values of onpu_geometry2 with its own Mat"""
    assert ha.geometry(L, N, K, ncols, sym) == orc.geometry(N, K, ncols, sym)
    if sym == 0:
        out = (C.c_int64 * 8)()
        L.onpu_geometry(N, K, ncols, out)
        assert tuple(out) == orc.geometry(N, K, ncols, 0)


def test_no_geometry_is_all_zero(L):
    # K / S > 2048 on one column has no geometry: the reference's Mat raises, the C call gives zeros
    assert ha.geometry(L, 64, 32 * 2048, 1, 1) == (0,) * 8


@pytest.mark.parametrize("sym,fmt", [(1, orc.FMT_Q4S), (0, orc.FMT_Q4NX)])
def test_pack_fills_nbytes_and_quant_dequant_reads_it(L, sym, fmt):
    """onpu_pack writes exactly nbytes (the reference's packing) and onpu_quant_dequant returns what
    those bytes dequantize to (the HIPREC residual pass of model.py:816 uses it)"""
    rng = np.random.default_rng(0)
    N, K = 40, 256
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    nbytes = ha.geometry(L, N, K, 8, sym)[7]
    buf = np.full(nbytes, 0xAB, np.uint8)
    assert ha.pack_into(L, W, 8, sym, buf.ctypes.data_as(ha.U8P)) == nbytes
    assert np.array_equal(buf, orc.npu_pack(fmt, W, 8))
    st = orc.npu_to_stage(fmt, buf, N, K, 8)
    assert np.array_equal(st, orc.quantize(fmt, W))
    qd = np.empty_like(W)
    L.onpu_quant_dequant(ha.fp(W), N, K, sym, ha.fp(qd), 3)
    assert np.array_equal(qd.view(np.uint32), orc.dequant(fmt, st, N, K).view(np.uint32))


def test_pack_rejects_k_off_the_group(L):
    W = np.zeros((8, 48), np.float32)
    buf = np.zeros(1 << 16, np.uint8)
    assert ha.pack_into(L, W, 8, 1, buf.ctypes.data_as(ha.U8P)) == 0


def test_without_a_gpu_the_loader_gets_none(L):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: the GPU tests cover construction")
    assert L.onpu_ok() == 0                      # model.py:332: clib() returns None on this
    assert L.onpu_dense_new2(64, 256, 1) is None
    assert L.onpu_bank_new2(64, 256, 4, 1, 1) is None
    assert L.onpu_ffn_new(512, 256, 256, 256, 8, 1) is None
    assert L.onpu_last_error()

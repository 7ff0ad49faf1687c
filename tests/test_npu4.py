"""Host side of the npu4 operator mirror (opennpu_amd/npu4.py), CPU only: the reference loader's
rules, Mat geometry and packing through the library, and loud failure without a GPU."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import npu4


def test_mat_matches_reference_geometry():
    for N, K, ncols, sym in [(4096, 4096, 8, 1), (6144, 4096, 8, 0), (4096, 12288, 8, 1), (1536, 2048, 1, 1),
                             (2048, 768, 1, 0), (151936, 4096, 8, 1)]:
        m = npu4.Mat(N, K, ncols, bool(sym))
        assert (m.R, m.S, m.tiles, m.kc, m.ks, m.rows_col, m.cb, m.nbytes) == orc.geometry(N, K, ncols, sym)
        npu4.check_geometry(m)


def test_mat_without_geometry_raises_value_error():
    with pytest.raises(ValueError):
        npu4.Mat(64, 32 * 2048, 1)                 # K / S > 2048 on one column: no geometry


def test_expert_cols():
    assert npu4.expert_cols(8, 1536, 2048) == 1
    assert npu4.expert_cols(4, 1536, 2048) == 2
    assert npu4.expert_cols(6) == 1                 # 8 % 6 != 0


def test_pack_writes_the_staging_layout_and_quant_dequant_agrees():
    rng = np.random.default_rng(0)
    W = rng.standard_normal((40, 256)).astype(np.float32) * 0.05
    for sym, fmt in [(True, orc.FMT_Q4S), (False, orc.FMT_Q4NX)]:
        m = npu4.Mat(40, 256, 8, sym)
        blob = m.pack(W)
        assert blob.size == m.nbytes
        sb = orc.stage_bytes(fmt, 40, 256)
        assert not blob[sb:].any()
        # the oracle's reading of the staged bytes is what the library says the device computes with
        assert np.array_equal(orc.dequant(fmt, blob[:sb], 40, 256), npu4.quant_dequant(W, sym))


def test_no_gpu_means_no_device_path():
    """clib() follows the reference (None when onpu_ok() != 1); the modules then raise instead of
    computing elsewhere"""
    npu4._CLIB[:] = [False, None]
    if npu4._lib.lib().onpu_ok() == 1:
        pytest.skip("a GPU is visible: covered by the GPU tests")
    assert npu4.clib() is None
    with pytest.raises(RuntimeError, match="not usable"):
        npu4.NPULinearGroup(["q"], [np.zeros((64, 256), np.float32)])

"""The benchmark's CPU leg times the reference's dequant-matmul pattern: its numpy dequant must be
the oracle's dequant bit for bit, so that the timed work is the work the reference does."""
import numpy as np
import pytest

import bench
import oracle.oracle as orc
from opennpu_amd import synthetic as syn


@pytest.mark.parametrize("fmt,N,K", [(orc.FMT_G128S, 40, 256), (orc.FMT_G128S, 8, 4096),
                                     (orc.FMT_Q4_0, 33, 128), (orc.FMT_Q4_0, 16, 4096)])
def test_cpu_dequant_is_the_oracles(fmt, N, K):
    st = syn.weights(fmt, N, K, 5 + N)
    got = bench.cpu_dequant(orc, fmt, st, N, K)
    assert np.array_equal(got.view(np.uint32), orc.dequant(fmt, st, N, K).view(np.uint32))

"""GPU parity of the int8 GEMV (onpu_gemv_i8_dev) against the oracle's restatement of the
reference's host onpu_gemv_i8 (onpu_cpu.cpp:276-299): fp32 accumulation in another order, so
max|y - r| <= 1e-5 max|r| against the fp64 oracle."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K", [(37, 2048), (11264, 2048), (2048, 5632), (5, 16), (300, 32768)])
def test_gemv_i8_dev(gpu, N, K):
    import torch
    rng = np.random.default_rng(N + K)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    W[0] = -128                                  # extreme codes
    W[-1] = 127
    s = rng.uniform(1e-3, 2e-2, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    x[::7] += 3.0                                # a mean far from zero (the bias term matters)
    Wd, sd, xd = torch.from_numpy(W).cuda(), torch.from_numpy(s).cuda(), torch.from_numpy(x).cuda()
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    P = lambda t: C.c_void_p(t.data_ptr())
    print(f"gemv_i8_dev N={N} K={K}", flush=True)
    assert gpu.onpu_gemv_i8_dev(P(Wd), P(sd), N, K, P(xd), P(y), None) == 0
    torch.cuda.synchronize()
    ref = orc.gemv_i8(W, s, x)
    err = np.abs(y.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 1e-5, err


def test_gemv_i8_dev_argument_errors(gpu):
    import torch
    L = gpu
    W = torch.zeros((4, 48), dtype=torch.int8, device="cuda")
    v = torch.zeros((64,), dtype=torch.float32, device="cuda")
    P = lambda t: C.c_void_p(t.data_ptr())
    assert L.onpu_gemv_i8_dev(P(W), P(v), 4, 40, P(v), P(v), None) == -1           # K % 16
    assert L.onpu_gemv_i8_dev(P(W), P(v), 4, 65536, P(v), P(v), None) == -1        # x past the LDS copy
    assert b"onpu_gemv_i8_dev" in L.onpu_last_error()

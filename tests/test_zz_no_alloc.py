"""onpu_dense_argmax_dev_noalloc (the LM-head argmax for callers that cannot allocate) against
onpu_dense_argmax_dev on the same inputs, through the C ABI: logits bit-identical (the same GEMV
kernel) and the same argmax indices, on two calls in a row, the second with fewer rows; the call
moves no device memory (free bytes unchanged), captures into a HIP graph on its first use inside the
capture and replays it correctly, and refuses sizes past its scratch array with a clear error."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _p(t):
    return C.c_void_p(t.data_ptr())


def _stream(torch):
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(scope="module")
def lm(gpu):
    import torch
    from opennpu_amd.device import QMatrix
    N, K = 20000, 1024
    q = QMatrix(N, K, orc.FMT_Q4_0, syn.weights(orc.FMT_Q4_0, N, K, 21))
    yield q, N, K, torch
    q.free()


def _x(torch, M, K, seed):
    bits = syn.activations(M, K, seed)
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda().reshape(M, K)


def _both(L, q, x, torch):
    M, N = x.shape[0], q.N
    lg_a = torch.full((M, N), float("nan"), device="cuda")
    ix_a = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    lg_b = torch.full((M, N), float("nan"), device="cuda")
    ix_b = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    assert L.onpu_dense_argmax_dev(q.h, _p(x), M, _p(lg_a), _p(ix_a), _stream(torch)) == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc = L.onpu_dense_argmax_dev_noalloc(q.h, _p(x), M, _p(lg_b), _p(ix_b), _stream(torch))
    torch.cuda.synchronize()
    assert rc == 0, L.onpu_last_error().decode()
    assert torch.cuda.mem_get_info()[0] == free0, "the no-allocation entry point moved device memory"
    return lg_a, ix_a, lg_b, ix_b


def test_equals_the_allocating_entry_point(lm):
    q, N, K, torch = lm
    L = q.L
    for M, seed in ((8, 1), (3, 2)):              # the second call with fewer rows
        x = _x(torch, M, K, seed)
        lg_a, ix_a, lg_b, ix_b = _both(L, q, x, torch)
        assert torch.equal(lg_a.view(torch.int32), lg_b.view(torch.int32)), M
        assert torch.equal(ix_a, ix_b), M
        want = orc.argmax(lg_a.cpu().numpy())
        assert np.array_equal(ix_b.cpu().numpy(), want), M


def test_planted_ties_over_repeated_calls(gpu):
    """two identical weight rows a < b whose logits are the row maximum (codes 15, a large scale, x
    positive): both entry points return a, call after call (each call leaves the counters at zero)"""
    import torch
    from opennpu_amd.device import QMatrix
    N, K, M = 9000, 256, 3
    L = gpu
    for rep in range(3):
        st = syn.weights(orc.FMT_Q4_0, N, K, 60 + rep).reshape(N, K // 32, 18).copy()
        a, b = sorted(np.random.default_rng(rep).choice(N, 2, replace=False))
        st[a, :, 0:2] = np.array([0.5], np.float16).view(np.uint8)
        st[a, :, 2:] = 0xFF                                   # every code 15: w = 7 * 0.5
        st[b] = st[a]
        q = QMatrix(N, K, orc.FMT_Q4_0, st.reshape(-1))
        bits = orc.f2bf_np(np.abs(np.random.default_rng(70 + rep).standard_normal((M, K))).astype(np.float32))
        x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda().reshape(M, K)
        lg_a, ix_a, lg_b, ix_b = _both(L, q, x, torch)
        assert (ix_b.cpu().numpy() == a).all() and torch.equal(ix_a, ix_b), (a, b, ix_b)
        q.free()


def test_first_use_inside_graph_capture(lm):
    """a fresh matrix whose first argmax call is made inside capture; the graph replays three times
    with eager work between, each replay equal to the eager result"""
    q0, N, K, torch = lm
    from opennpu_amd.device import QMatrix
    q = QMatrix(3000, 512, orc.FMT_Q4_0, syn.weights(orc.FMT_Q4_0, 3000, 512, 22))
    L = q.L
    M = 2
    x = _x(torch, M, 512, 5)
    lg = torch.empty((M, 3000), device="cuda")
    ix = torch.empty((M,), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = L.onpu_dense_argmax_dev_noalloc(q.h, _p(x), M, _p(lg), _p(ix), C.c_void_p(s.cuda_stream))
    assert rc == 0, L.onpu_last_error().decode()
    lg_e = torch.empty_like(lg)
    ix_e = torch.empty_like(ix)
    for rep in range(3):
        x.copy_(_x(torch, M, 512, 40 + rep))
        lg.zero_()
        ix.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert L.onpu_dense_argmax_dev(q.h, _p(x), M, _p(lg_e), _p(ix_e), _stream(torch)) == 0
        torch.cuda.synchronize()
        assert torch.equal(lg.view(torch.int32), lg_e.view(torch.int32)), rep
        assert torch.equal(ix, ix_e), rep
    q.free()


def test_limits_are_refused(lm):
    q, N, K, torch = lm
    L = q.L
    x = _x(torch, 65, K, 3)
    lg = torch.empty((65, N), device="cuda")
    ix = torch.empty((65,), dtype=torch.int32, device="cuda")
    assert L.onpu_dense_argmax_dev_noalloc(q.h, _p(x), 65, _p(lg), _p(ix), _stream(torch)) == -1
    assert b"64 rows" in L.onpu_last_error()
    # 64 rows of a 129 * 4096-wide vocabulary need 8256 keys > 8064
    from opennpu_amd.device import QMatrix
    big = QMatrix(129 * 4096, 32, orc.FMT_Q4_0, syn.weights(orc.FMT_Q4_0, 129 * 4096, 32, 23))
    x = _x(torch, 64, 32, 4)
    lg = torch.empty((64, big.N), device="cuda")
    ix = torch.empty((64,), dtype=torch.int32, device="cuda")
    assert L.onpu_dense_argmax_dev_noalloc(big.h, _p(x), 64, _p(lg), _p(ix), _stream(torch)) == -1
    assert b"8064" in L.onpu_last_error()
    # 62 rows fit (62 * 129 = 7998 keys) and agree with the allocating entry point
    x = x[:62].contiguous()
    lg_a, ix_a, lg_b, ix_b = _both(L, big, x, torch)
    assert torch.equal(ix_a, ix_b)
    big.free()

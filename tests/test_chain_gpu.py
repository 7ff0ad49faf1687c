"""Chained decode GEMVs (onpu_chain_*, opennpu_amd.device.QChain) on the GPU.

A chain runs its GEMVs in order in one launch with a grid barrier between entries. The tests chain
entries that consume earlier entries' outputs (so a missing or leaky barrier shows up as wrong
values), check every output against the oracle on the inputs the chain actually saw, check that
repeated runs and HIP-graph replays reproduce the same bits, and that no barrier wait timed out.
Tolerance: bf16 outputs, max|y-r|/max|r| <= 1e-2 and per element within the bf16 rounding bound
(conftest.check_bf16_out).
"""
import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import synthetic as syn
from tests.conftest import check_bf16_out, from_torch, to_torch_bf16

pytestmark = pytest.mark.gpu


def _bits(t):
    import torch
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _build(fmt, dims, M, seed):
    """dims: [K0, N0 = K1, N1 = K2, ...]: a chain where entry i reads entry i - 1's output"""
    import torch
    from opennpu_amd.device import QMatrix
    sts, mats = [], []
    for i in range(len(dims) - 1):
        K, N = dims[i], dims[i + 1]
        st = syn.weights(fmt, N, K, seed + i)
        sts.append(st)
        mats.append(QMatrix(N, K, fmt, st))
    x0 = to_torch_bf16(syn.activations(M, dims[0], seed + 99)).reshape(M, dims[0])
    ys = [torch.empty((M, dims[i + 1]), dtype=torch.bfloat16, device="cuda") for i in range(len(dims) - 1)]
    xs = [x0] + ys[:-1]
    return sts, mats, xs, ys


@pytest.mark.parametrize("fmt,M", [(orc.FMT_G128S, 1), (orc.FMT_G128S, 5), (orc.FMT_Q4S, 1), (orc.FMT_Q4_0, 3)])
def test_dependent_chain(gpu, fmt, M):
    import torch
    from opennpu_amd.device import QChain
    dims = [512, 1024, 384, 2048, 256, 640]
    sts, mats, xs, ys = _build(fmt, dims, M, 11 + fmt)
    ch = QChain(mats, xs, ys)
    try:
        ch.run()
        torch.cuda.synchronize()
        assert ch.status() == 0
        outs = [_bits(y) for y in ys]
        ins = [_bits(xs[0])] + outs[:-1]
        for i, st in enumerate(sts):
            K, N = dims[i], dims[i + 1]
            ref = orc.qmm(fmt, st, N, K, ins[i])
            check_bf16_out(orc.bf2f(outs[i]), ref, what=f"chain entry {i} fmt {fmt} M {M}")
        # a second run reproduces every output bit for bit
        for y in ys:
            y.zero_()
        ch.run()
        torch.cuda.synchronize()
        assert ch.status() == 0
        for i, y in enumerate(ys):
            assert np.array_equal(_bits(y), outs[i]), f"entry {i} differs between runs"
    finally:
        ch.free()
        for q in mats:
            q.free()


def test_chain_matches_single_launches_and_graph_replays(gpu):
    """independent entries (the decode benchmark's shape of use) against one launch per GEMV, and
    a captured chain replayed several times with eager work in between"""
    import torch
    from opennpu_amd.device import QChain, QMatrix
    M = 1
    shapes = [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)] * 2
    mats, xs, ys, sts = [], [], [], []
    xin = {K: to_torch_bf16(syn.activations(M, K, K)).reshape(M, K) for K in (4096, 12288)}
    for i, (N, K) in enumerate(shapes):
        st = syn.weights(orc.FMT_G128S, N, K, 300 + i)
        sts.append(st)
        mats.append(QMatrix(N, K, orc.FMT_G128S, st))
        xs.append(xin[K])
        ys.append(torch.empty((M, N), dtype=torch.bfloat16, device="cuda"))
    ch = QChain(mats, xs, ys)
    try:
        ch.run()
        torch.cuda.synchronize()
        assert ch.status() == 0
        want = [_bits(y) for y in ys]
        for i, (N, K) in enumerate(shapes[:4]):              # rows checked against the oracle
            check_bf16_out(orc.bf2f(want[i])[:, :1024], orc.qmm(orc.FMT_G128S, sts[i], N, K, _bits(xs[i]), 0, 1024),
                           what=f"independent entry {i}")
        for i, q in enumerate(mats):                          # the single-launch path agrees closely
            y1 = from_torch(q.mv(xs[i]))
            assert np.abs(y1 - orc.bf2f(want[i])).max() <= 1e-2 * np.abs(y1).max()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ch.run()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ch.run()
        for rep in range(3):
            for y in ys:
                y.fill_(0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert ch.status() == 0
            for i, y in enumerate(ys):
                assert np.array_equal(_bits(y), want[i]), f"replay {rep} entry {i}"
    finally:
        ch.free()
        for q in mats:
            q.free()

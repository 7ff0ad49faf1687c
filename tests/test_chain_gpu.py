"""Chained decode GEMVs (onpu_chain_*, opennpu_amd.device.QChain) on the GPU.

A chain runs its GEMVs in order in one launch; an entry whose x is (part of) an earlier entry's
output waits for that output's link words, not for a grid barrier. The tests chain entries that
consume earlier entries' outputs, whole or as a range at an offset (so a missed or early wait shows
up as wrong values), check every output against the oracle on the inputs the chain actually saw,
check that repeated runs and HIP-graph replays reproduce the same bits (each run carries a fresh
tag), that no wait timed out, and that layouts the chain cannot link are refused.
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


def _qwen_like(M, seed, scale=1):
    """one decode layer's shape of dependencies, scaled down: qkv (N 384) -> o reads qkv[0:256],
    o -> gate_up reads all of o, down reads gate_up[256:768] (a range at an offset), the next
    qkv reads down; twice"""
    import torch
    from opennpu_amd.device import QMatrix
    H, Q, I = 256 * scale, 384 * scale, 512 * scale
    plan = []                   # (N, K, source entry or -1, element offset)
    for layer in range(2):
        plan += [(Q, H, -1 if layer == 0 else len(plan) - 1, 0), (H, H, len(plan), 0), (2 * I, H, len(plan) + 1, 0),
                 (H, I, len(plan) + 2, 256 * scale)]
    sts, mats, ys, xs = [], [], [], []
    x0 = to_torch_bf16(syn.activations(M, H, seed + 99)).reshape(M, H)
    for i, (N, K, src, off) in enumerate(plan):
        st = syn.weights(orc.FMT_G128S, N, K, seed + i, scale_sigma=0.002)
        sts.append(st)
        mats.append(QMatrix(N, K, orc.FMT_G128S, st))
        ys.append(torch.empty((M, N), dtype=torch.bfloat16, device="cuda"))
        xs.append(x0 if src < 0 else ys[src][:, off:off + K])
    return plan, sts, mats, xs, ys


def test_linked_ranges_and_runs(gpu):
    """M = 1 entries that read a range of an earlier output (at offsets 0 and 256), five runs in a
    row and graph replays: every output against the oracle on the input the chain saw, the same bits
    run after run, the run count advancing"""
    import torch
    from opennpu_amd.device import QChain
    plan, sts, mats, xs, ys = _qwen_like(1, 500)
    ch = QChain(mats, xs, ys)
    try:
        runs0 = ch.info()[5]
        ch.run()
        torch.cuda.synchronize()
        assert ch.status() == 0
        outs = [_bits(y) for y in ys]
        for i, (N, K, src, off) in enumerate(plan):
            xin = _bits(xs[0]) if src < 0 else outs[src][:, off:off + K]
            check_bf16_out(orc.bf2f(outs[i]), orc.qmm(orc.FMT_G128S, sts[i], N, K, np.ascontiguousarray(xin)),
                           what=f"linked entry {i}")
        for rep in range(4):
            for y in ys:
                y.fill_(0)
            ch.run()
            torch.cuda.synchronize()
            assert ch.status() == 0
            for i, y in enumerate(ys):
                assert np.array_equal(_bits(y), outs[i]), f"run {rep + 2} entry {i}"
        assert ch.info()[5] == runs0 + 5
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                ch.run()
        torch.cuda.current_stream().wait_stream(s)
        for rep in range(3):
            for y in ys:
                y.fill_(0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert ch.status() == 0
            for i, y in enumerate(ys):
                assert np.array_equal(_bits(y), outs[i]), f"replay {rep} entry {i}"
    finally:
        ch.free()
        for q in mats:
            q.free()


def test_refused_layouts(gpu):
    """layouts the chain cannot link are refused with a reason: overlapping outputs, an x written by a
    later entry, a range of an earlier output at M > 1, a range off an 8-element boundary"""
    import torch
    from opennpu_amd.device import QChain, QMatrix
    a = QMatrix(64, 128, orc.FMT_G128S, syn.weights(orc.FMT_G128S, 64, 128, 1))
    b = QMatrix(64, 128, orc.FMT_G128S, syn.weights(orc.FMT_G128S, 64, 128, 2))
    try:
        buf = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
        x1 = to_torch_bf16(syn.activations(1, 128, 3)).reshape(1, 128)
        cases = [
            ([x1, x1], [buf[0, :64].reshape(1, 64), buf[0, 32:96].reshape(1, 64)], 1, "outputs overlap"),
            ([buf[1, :128].reshape(1, 128), x1], [buf[2, :64].reshape(1, 64), buf[1, 64:128].reshape(1, 64)], 1,
             "later entry writes"),
        ]
        for xs, ys, M, what in cases:
            with pytest.raises(RuntimeError, match="onpu_chain_new"):
                QChain([a, b], xs, ys)
        # a range of an earlier output off an 8-element boundary
        y0 = torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda")
        big = QMatrix(256, 128, orc.FMT_G128S, syn.weights(orc.FMT_G128S, 256, 128, 4))
        y1 = torch.zeros((1, 64), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(RuntimeError, match="cannot link"):
            QChain([big, a], [x1, y0[:, 4:132]], [y0, y1])
        # a range at M = 2 (rows of x would not be rows of the output)
        y2 = torch.zeros((2, 256), dtype=torch.bfloat16, device="cuda")
        x2 = to_torch_bf16(syn.activations(2, 128, 5)).reshape(2, 128)
        with pytest.raises(RuntimeError, match="cannot link"):
            QChain([big, a], [x2, y2.view(-1)[:256].reshape(2, 128)], [y2, torch.zeros((2, 64), dtype=torch.bfloat16,
                                                                                     device="cuda")])
        big.free()
    finally:
        a.free()
        b.free()

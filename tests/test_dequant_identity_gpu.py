"""The hot kernels' own unpack and dequantization, read back exactly through identity inputs.

tests/test_dense_gpu.py::test_dequant_bit_exact reads the weights back through k_dequant, a kernel
of its own. Here the GEMV, the prefill GEMM and the grouped MoE GEMM dequantize them themselves:
- GEMV (M <= 64, the decode kernel), fp32 y: x rows one-hot at k give y[m][n] = w[n][k], exactly
  the reference's fp32 dequant (u - 8) s, or u s + m for q4nx, as onpu_quant_dequant defines it
  (onpu_api.cpp:508-529): every group but the one holding k adds exact zeros, and the symmetric
  formats' (u - 8) s and q4nx's u s are exact products (4 by 8 significant bits);
- prefill GEMM (k_qgemm_sk with its split-K exchange, k_qgemm with the K-tail variant and split
  into K ranges, also at 40 rows): X the identity (or rows of it) gives Y = W^T as the bf16 RNE of
  each dequantized weight, the value the reference device feeds its MAC (gemv_any.cc:65,106-107);
- grouped MoE GEMM (the prompt path, k_moe_gemm gate+up then down): weights designed so that one
  product passes the other's values through unchanged (a gate of 32 makes silu exact, 32 * u and
  u / 32 are exact), so that the routed layer returns the bf16 RNE of every up weight, or of every
  down weight, of each expert.
All four formats, negative scales (the sign of every other scale flipped), q4nx mins far below
128 s, and K tails (K % 128 = 32) where the format's group allows them. Values are compared with ==
(+0 and -0 are equal: an fp32 sum of +0 and -0 is +0 on either device).
"""
import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import synthetic as syn
from tests.conftest import from_torch, gemm_exact, to_torch_bf16

pytestmark = pytest.mark.gpu
FMTS = [orc.FMT_Q4NX, orc.FMT_Q4S, orc.FMT_G128S, orc.FMT_Q4_0]


def f2h_bits(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def stage(fmt, codes, scale, mins=None):
    """codes u8 [N][K] (0..15), scales fp32 [N][K / g] (exact in bf16, fp16 for Q4_0), q4nx mins
    [N][K / 32] -> staging bytes"""
    codes = np.asarray(codes, np.uint8)
    N, K = codes.shape
    if fmt == orc.FMT_Q4_0:
        q = codes.reshape(N, K // 32, 32)
        blk = np.empty((N, K // 32, 18), np.uint8)
        d = f2h_bits(scale).reshape(N, K // 32)
        blk[..., 0] = (d & 0xFF).astype(np.uint8)
        blk[..., 1] = (d >> 8).astype(np.uint8)
        blk[..., 2:] = q[..., :16] | (q[..., 16:] << 4)
        return blk.reshape(-1)
    parts = [(codes[:, 0::2] | (codes[:, 1::2] << 4)).ravel(), orc.f2bf_np(scale).ravel().view(np.uint8)]
    if fmt == orc.FMT_Q4NX:
        parts.append(orc.f2bf_np(mins).ravel().view(np.uint8))
    return np.concatenate(parts).astype(np.uint8)


def random_weights(fmt, N, K, seed):
    """synthetic weights with every other scale negated and, for q4nx, mins of every magnitude
    (tiny, zero and large against 128 s)"""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    g = orc.group(fmt)
    s = np.abs(rng.standard_normal((N, K // g))) * 0.02 + 1e-4
    s[:, 1::2] *= -1
    s = orc.bf2f(orc.f2bf_np(s)).reshape(s.shape) if fmt != orc.FMT_Q4_0 else s.astype(np.float16).astype(np.float32)
    m = None
    if fmt == orc.FMT_Q4NX:
        m = rng.standard_normal((N, K // 32)) * 0.08 * 10.0 ** rng.integers(-6, 1, (N, K // 32))
        m[:, ::7] = 0.0
        m = orc.bf2f(orc.f2bf_np(m)).reshape(m.shape)
    return stage(fmt, codes, s, m)


def shapes(fmt):
    """(N, K): ragged row tiles, and a K tail of 32 where the format's group allows it"""
    return (272, 1152) if fmt == orc.FMT_G128S else (272, 1056)


def one_hot(M, K, cols):
    x = np.zeros((M, K), np.uint16)
    x[np.arange(M), cols] = 0x3F80                      # bf16 1.0
    return x


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_returns_the_dequantized_weights(gpu, fmt):
    import torch
    from opennpu_amd.device import QMatrix
    N, K = shapes(fmt)
    st = random_weights(fmt, N, K, 60 + fmt)
    W = orc.dequant(fmt, st, N, K)
    q = QMatrix(N, K, fmt, st)
    try:
        k0, step = 0, 0
        sizes = [1, 3, 4, 5, 8, 9, 16, 17, 33, 64]        # every row layout of the decode kernel
        while k0 < K:
            M = min(sizes[step % len(sizes)], K - k0)
            cols = np.arange(k0, k0 + M)
            print(f"gemv identity fmt {fmt} N={N} K={K} rows {k0}..{k0 + M}", flush=True)
            x = to_torch_bf16(one_hot(M, K, cols)).reshape(M, K)
            y = from_torch(q.mv(x, f32=True))
            want = W[:, cols].T
            bad = np.argwhere(~(y == want))
            assert bad.size == 0, f"fmt {fmt}: y[{bad[0]}] = {y[tuple(bad[0])]!r}, weight {want[tuple(bad[0])]!r}"
            if step == 4:                                  # bf16 y: the RNE of the same values
                yb = q.mv(x).view(torch.int16).cpu().numpy().view(np.uint16)
                assert np.array_equal(orc.bf2f(yb).reshape(yb.shape), orc.bf2f(orc.f2bf_np(want)).reshape(want.shape))
            k0 += M
            step += 1
        torch.cuda.synchronize()
    finally:
        q.free()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("case", ["split_k", "tail"])
def test_gemm_returns_the_bf16_weights(gpu, fmt, case):
    """X = the identity (M = K rows): Y = bf16 RNE of W^T. "split_k": 128 or more 256 x 256 tiles,
    the split-K kernel with its partial-tile exchange (K 4096, or 4128 with a tail); "tail": the
    128-row-tile kernel on a ragged shape with the K-tail variant."""
    import torch
    from opennpu_amd.device import QMatrix
    if case == "split_k":
        N, K = 2048, (4096 if fmt == orc.FMT_G128S else 4128)
    else:
        N, K = shapes(fmt)
    st = random_weights(fmt, N, K, 70 + fmt)
    Wb = orc.bf2f(orc.dequant_bf16(fmt, st, N, K)).reshape(N, K)
    q = QMatrix(N, K, fmt, st)
    try:
        print(f"gemm identity fmt {fmt} {case} N={N} K={K}", flush=True)
        x = to_torch_bf16(one_hot(K, K, np.arange(K))).reshape(K, K)
        y = from_torch(q.mv(x, f32=True))
        torch.cuda.synchronize()
    finally:
        q.free()
    bad = np.argwhere(~(y == Wb.T))
    assert bad.size == 0, f"fmt {fmt} {case}: Y[{bad[0]}] = {y[tuple(bad[0])]!r}, weight {Wb.T[tuple(bad[0])]!r}"


@pytest.mark.parametrize("fmt", FMTS)
def test_split_gemm_returns_the_bf16_weights(gpu, fmt):
    """the GEMM split along K at few rows on a 7000 x 8192 matrix (16, 24, 40 rows: GEMMs below 65
    rows with tiles of 16, 32, 64 rows; 96: 128-row tiles in 9 K ranges), rows one-hot at columns
    spread over K and across range boundaries: every range but the one holding the column adds exact
    zeros to the partial sum, so Y is the bf16 RNE of those weight columns, or where the tiles take
    the GEMV's arithmetic (16 rows; 32 rows for g128s) the fp32 dequantized weights themselves"""
    import torch
    from opennpu_amd.device import QMatrix
    N, K = 7000, (8192 if fmt == orc.FMT_G128S else 8224)
    st = random_weights(fmt, N, K, 80 + fmt)
    Wb = orc.bf2f(orc.dequant_bf16(fmt, st, N, K)).reshape(N, K)
    W = orc.dequant(fmt, st, N, K)
    q = QMatrix(N, K, fmt, st)
    try:
        for M in (16, 24, 40, 96):
            cols = np.unique(np.linspace(0, K - 1, M).astype(np.int64))
            cols = np.concatenate([cols, np.arange(K - (M - cols.size), K)])[:M]
            print(f"split gemm identity fmt {fmt} N={N} K={K} M={M}", flush=True)
            x = to_torch_bf16(one_hot(M, K, cols)).reshape(M, K)
            y = from_torch(q.mv(x, f32=True))
            torch.cuda.synchronize()
            want = (W if gemm_exact(fmt, M) else Wb)[:, cols].T
            bad = np.argwhere(~(y == want))
            assert bad.size == 0, f"fmt {fmt} M {M}: Y[{bad[0]}] = {y[tuple(bad[0])]!r}, weight {want[tuple(bad[0])]!r}"
    finally:
        q.free()


def designed(fmt, N, K, kind):
    """weights of exact value: "const32" every weight 32; "select" w[i][k] = 1/32 where i == k, else 0"""
    g = orc.group(fmt)
    m = None
    if kind == "const32":
        if fmt == orc.FMT_Q4NX:
            codes, s, m = np.zeros((N, K)), np.ones((N, K // g)), np.full((N, K // 32), 32.0)
        else:
            codes, s = np.full((N, K), 12), np.full((N, K // g), 8.0)           # (12 - 8) * 8
    else:
        eye = np.zeros((N, K))
        i = np.arange(min(N, K))
        eye[i, i] = 1
        if fmt == orc.FMT_Q4NX:
            codes, s, m = eye, np.full((N, K // g), 1 / 32), np.zeros((N, K // 32))
        else:
            codes, s = eye + 8, np.full((N, K // g), 1 / 32)                   # (9 - 8) / 32
    return stage(fmt, codes.astype(np.uint8), s, m)


def moe_shapes(fmt):
    return (512, 256) if fmt == orc.FMT_G128S else (544, 288)       # (H, I): K tails of 32 otherwise


def run_layer(fmt, E, H, I, gu, dn, T, cols, experts):
    """the routed layer on the grouped prompt path: token t is x = one-hot at cols[t], routed to
    experts[t] alone with weight 1; fp32 y [T][H]"""
    import torch
    from opennpu_amd.device import QFfn
    f = QFfn(E, H, I, fmt)
    try:
        f.load(np.concatenate(gu), np.concatenate(dn))
        x = to_torch_bf16(one_hot(T, H, cols)).reshape(T, H)
        ids = torch.from_numpy(np.asarray(experts, np.int32).reshape(T, 1)).cuda()
        w = torch.ones((T, 1), dtype=torch.float32, device="cuda")
        y = from_torch(f.ffn(x, ids, w, f32=True))
        torch.cuda.synchronize()
    finally:
        f.free()
    return y


@pytest.mark.parametrize("fmt", FMTS)
def test_grouped_gate_up_returns_the_bf16_up_weights(gpu, fmt):
    """gate = 32 everywhere (silu(32) = 32 in fp32), down = I / 32: token x = e_k routed to expert e
    gives act = 32 bf16(up_e[:, k]) and y[:I] = bf16(up_e[:, k]), y[I:] = 0, for every k and expert"""
    E = 2
    H, I = moe_shapes(fmt)
    gate = designed(fmt, I, H, "const32")
    ups = [random_weights(fmt, I, H, 80 + 2 * e + fmt) for e in range(E)]
    gu = [np.concatenate([gate[:orc.stage_bytes(fmt, I, H)], u]) if fmt == orc.FMT_Q4_0 else
          stage_rows(fmt, [(gate, I), (u, I)], H) for u in ups]
    dn = [designed(fmt, H, I, "select")] * E
    cols = np.tile(np.arange(H), E)
    experts = np.repeat(np.arange(E), H)
    print(f"grouped gate+up identity fmt {fmt} H={H} I={I} T={E * H}", flush=True)
    y = run_layer(fmt, E, H, I, gu, dn, E * H, cols, experts)
    for e in range(E):
        Ub = orc.bf2f(orc.dequant_bf16(fmt, ups[e], I, H)).reshape(I, H)
        ye = y[e * H:(e + 1) * H]
        bad = np.argwhere(~(ye[:, :I] == Ub.T))
        assert bad.size == 0, f"fmt {fmt} expert {e}: y[{bad[0]}] = {ye[tuple(bad[0])]!r}, weight {Ub.T[tuple(bad[0])]!r}"
        assert not ye[:, I:].any()


@pytest.mark.parametrize("fmt", FMTS)
def test_grouped_down_returns_the_bf16_down_weights(gpu, fmt):
    """gate = 32, up selects column k (w[i][k] = 1/32 at i = k): token x = e_k (k < I) gives act =
    e_k exactly and y = bf16(down_e[:, k]), for every k < I and expert"""
    E = 2
    H, I = moe_shapes(fmt)
    gate = designed(fmt, I, H, "const32")
    sel = designed(fmt, I, H, "select")
    gu = [np.concatenate([gate[:orc.stage_bytes(fmt, I, H)], sel]) if fmt == orc.FMT_Q4_0 else
          stage_rows(fmt, [(gate, I), (sel, I)], H)] * E
    downs = [random_weights(fmt, H, I, 90 + 2 * e + fmt) for e in range(E)]
    cols = np.tile(np.arange(I), E)
    experts = np.repeat(np.arange(E), I)
    print(f"grouped down identity fmt {fmt} H={H} I={I} T={E * I}", flush=True)
    y = run_layer(fmt, E, H, I, gu, downs, E * I, cols, experts)
    for e in range(E):
        Db = orc.bf2f(orc.dequant_bf16(fmt, downs[e], H, I)).reshape(H, I)
        ye = y[e * I:(e + 1) * I]
        bad = np.argwhere(~(ye == Db.T))
        assert bad.size == 0, f"fmt {fmt} expert {e}: y[{bad[0]}] = {ye[tuple(bad[0])]!r}, weight {Db.T[tuple(bad[0])]!r}"


def stage_rows(fmt, parts, K):
    """staging bytes of row blocks stacked (codes, then scales, then q4nx mins, each in row order)"""
    g = orc.group(fmt)
    codes, scales, mins = [], [], []
    for st, n in parts:
        c = n * K // 2
        sb = n * (K // g) * 2
        codes.append(st[:c])
        scales.append(st[c:c + sb])
        if fmt == orc.FMT_Q4NX:
            mins.append(st[c + sb:c + 2 * sb])
    return np.concatenate(codes + scales + mins)

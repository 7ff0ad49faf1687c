"""GPU parity of the dense int4 path (decode GEMV family, prefill GEMM, LM head) against the oracle.

The product is called through libonpu_hip's C ABI (opennpu_amd.device wraps the *_dev entry
points); the oracle is oracle/oracle.c (fp64 dequantize-then-matmul of reference.py:24-28,55).
Tolerances: bf16 outputs max|y-r|/max|r| <= 1e-2 and per element within the bf16 rounding bound
(conftest.check_bf16_out); fp32 logits <= 1e-3 (and <= 1e-4 observed bound).
"""
import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import synthetic as syn
from tests.conftest import check_bf16_out, check_f32_out, from_torch, gemm_exact, to_torch_bf16

pytestmark = pytest.mark.gpu
FMTS = [orc.FMT_Q4NX, orc.FMT_Q4S, orc.FMT_G128S, orc.FMT_Q4_0]


def _mv(fmt, N, K, M, seed, f32=False):
    from opennpu_amd.device import QMatrix
    st = syn.weights(fmt, N, K, seed)
    xb = syn.activations(M, K, seed + 7919)
    q = QMatrix(N, K, fmt, st)
    try:
        y = from_torch(q.mv(to_torch_bf16(xb).reshape(M, K), f32=f32))
    finally:
        q.free()
    return st, xb, y


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bit_exact(gpu, fmt):
    """unpack + dequant in HBM layout == the reference's dequant, bit for bit (fp32 and bf16 RNE),
    with every other scale negative (the quantizers produce those): (u - 8) s is -0 for u = 8 there,
    as the reference's expression gives."""
    from opennpu_amd.device import QMatrix
    for (N, K) in [(48, 256), (37, 384), (16, 2048)] + ([] if fmt == orc.FMT_G128S else [(21, 160)]):
        st = syn.weights(fmt, N, K, 11 + N).copy()
        if fmt == orc.FMT_Q4_0:
            st.reshape(-1, 18)[::2, 1] ^= 0x80                  # sign bit of d (fp16, little endian)
        elif fmt != orc.FMT_Q4NX:
            G = orc.group(fmt)
            st[N * K // 2:N * K // 2 + N * (K // G) * 2].view(np.uint16)[::2] ^= 0x8000
        q = QMatrix(N, K, fmt, st)
        try:
            w = q.dequant()
            wb = q.dequant(bf16=True)
        finally:
            q.free()
        ref = orc.dequant(fmt, st, N, K)
        assert np.array_equal(w.view(np.uint32), ref.view(np.uint32)), (fmt, N, K)
        assert np.array_equal(wb, orc.dequant_bf16(fmt, st, N, K)), (fmt, N, K)


@pytest.mark.parametrize("fmt", FMTS)
def test_golden_fixtures(gpu, fmt):
    """the committed fixtures (tests/golden/golden.npz, built from the format definitions with
    numpy alone): dequant bit-exact, y within the bf16 tolerance, through GEMV and GEMM"""
    import torch
    from pathlib import Path
    from opennpu_amd.device import QMatrix
    G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")
    N, K, M = (int(v) for v in G[f"f{fmt}_shape"])
    q = QMatrix(N, K, fmt, G[f"f{fmt}_st"])
    try:
        assert np.array_equal(q.dequant().view(np.uint32), G[f"f{fmt}_w"].view(np.uint32))
        y = from_torch(q.mv(to_torch_bf16(G[f"f{fmt}_x"]).reshape(M, K)))
        check_bf16_out(y, G[f"f{fmt}_y"], what=f"golden fmt {fmt}")
        # the same rows repeated past the GEMV limit run the MFMA GEMM
        xr = np.tile(G[f"f{fmt}_x"], (80 // M + 1, 1))[:80]
        yr = from_torch(q.mv(to_torch_bf16(xr).reshape(80, K)))
        ref = np.tile(G[f"f{fmt}_y"], (80 // M + 1, 1))[:80]
        assert np.abs(yr - ref).max() <= 1e-2 * np.abs(ref).max()
    finally:
        q.free()
    torch.cuda.synchronize()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [1, 2, 5, 8, 16, 17, 33, 64])
def test_gemv_small(gpu, fmt, M):
    for (N, K) in [(16, 128), (72, 512), (300, 1024)] + ([] if fmt == orc.FMT_G128S else [(129, 2080)]):
        st, xb, y = _mv(fmt, N, K, M, 100 * M + N)
        check_bf16_out(y, orc.qmm(fmt, st, N, K, xb), what=f"fmt {fmt} N {N} K {K} M {M}")


@pytest.mark.parametrize("M", [1, 4, 8])
@pytest.mark.parametrize("name,N,K", [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096),
                                      ("down", 4096, 12288)])
def test_gemv_qwen3_8b(gpu, name, N, K, M):
    """Qwen3-8B decode layer shapes (g128s), every output row against the oracle."""
    st, xb, y = _mv(orc.FMT_G128S, N, K, M, 1 + K + N)
    check_bf16_out(y, orc.qmm(orc.FMT_G128S, st, N, K, xb), what=f"{name} M {M}")


@pytest.mark.parametrize("fmt,N,K,M", [(orc.FMT_Q4NX, 24576, 4096, 8), (orc.FMT_Q4S, 6144, 4096, 1),
                                       (orc.FMT_Q4S, 6144, 4096, 5), (orc.FMT_Q4_0, 4096, 12288, 1),
                                       (orc.FMT_Q4NX, 4096, 4096, 1), (orc.FMT_G128S, 6144, 4096, 2)])
def test_gemv_group_sum_variants(gpu, fmt, N, K, M):
    """Qwen3-8B shapes whose plans take x's group sums from the MFMAs (per-32 formats up to 8 rows,
    g128s waves of at most 4 blocks at 2-8 rows), every output row against the oracle."""
    import ctypes as C
    from opennpu_amd import _lib
    o = (C.c_int64 * 10)()
    _lib.lib().onpu_plan_gemv(fmt, N, K, M, 1, 0, o)
    assert o[3] == 2, tuple(o)                       # the case exercises the MFMA-sum variant
    st, xb, y = _mv(fmt, N, K, M, 7 + K + N + M)
    check_bf16_out(y, orc.qmm(fmt, st, N, K, xb), what=f"fmt {fmt} {N}x{K} M {M}")


# one shape per launch-plan class of plan_gemv (onpu_api.cpp): <= 256 tile groups with K <= 4096,
# K >= 8192, <= 512 tile groups, >= 1024 tile groups (the rule taken at M > 4), vocabulary-sized,
# and the one-row rules for larger models (>= 2048 tile groups; x too long for LDS; one to two
# workgroups per CU), vocabulary-sized with two K parts; ragged N where the class allows it
PLAN_CLASS_SHAPES = [(2048, 2048), (1000, 8192), (6000, 2048), (17000, 1024), (70000, 512), (33600, 1024),
                     (600, 28672), (5120, 5120), (66000, 4224)]


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_plan_classes(gpu, fmt, monkeypatch):
    """every plan class of the decode GEMV at 1-13 rows, all formats, every output row against the
    oracle; the cases take x from global memory, staged with VALU sums and staged with MFMA sums (the
    GEMV forced where the largest shapes would take the GEMM at 13 rows)"""
    import ctypes as C
    from opennpu_amd import _lib
    monkeypatch.setenv("ONPU_FORCE_GEMM", "-1")
    o = (C.c_int64 * 10)()
    seen = set()
    for i, (N, K) in enumerate(PLAN_CLASS_SHAPES):
        for M in (1, 3, 6, 8, 13):
            _lib.lib().onpu_plan_gemv(fmt, N, K, M, 1, 0, o)
            seen.add(o[3])
            st, xb, y = _mv(fmt, N, K, M, 31 * i + M + fmt)
            check_bf16_out(y, orc.qmm(fmt, st, N, K, xb), what=f"fmt {fmt} {N}x{K} M {M} plan {tuple(o)}")
    assert seen == {0, 1, 2}, seen


def test_gemv_config0(gpu):
    """M=1, K=N=4096 g128s, seed 0."""
    st, xb, y = _mv(orc.FMT_G128S, 4096, 4096, 1, 0)
    check_bf16_out(y, orc.qmm(orc.FMT_G128S, st, 4096, 4096, xb), what="config0")


def test_gemv_fp32_out(gpu):
    st, xb, y = _mv(orc.FMT_Q4S, 520, 1024, 3, 5, f32=True)
    check_f32_out(y, orc.qmm(orc.FMT_Q4S, st, 520, 1024, xb))


def check_gemm(y, fmt, st, N, K, xb, n0=0, n1=None, what=""):
    """prefill GEMM: the weights enter MFMA as bf16 RNE of the dequant (the reference device's MAC
    input), so the per-element bound is taken against that oracle; the stated 1e-2 tolerance
    against the exact fp32-dequant oracle."""
    check_bf16_out(y, orc.qmm(fmt, st, N, K, xb, n0, n1, bf16w=True), what=what + " (bf16 weights)")
    err = orc.max_rel_err(y, orc.qmm(fmt, st, N, K, xb, n0, n1))
    assert err <= 1e-2, f"{what} max rel err {err:.3e} vs the exact dequant"


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [65, 130, 256])
def test_gemm_ragged(gpu, fmt, M):
    """prefill GEMM path (M > 64), ragged M and N."""
    N, K = 200, 640 if fmt != orc.FMT_G128S else 768
    st, xb, y = _mv(fmt, N, K, M, 3 * M)
    check_gemm(y, fmt, st, N, K, xb, what=f"gemm fmt {fmt} M {M}")


# (M, N, K) cases of the GEMM split along K (plan_mv: S = min(KB / 4, 2 x CUs / workgroups) ranges of
# K blocks), with the tile rows they take: 96 x 1000 x 8192 (128-row tiles) in 16 ranges of 4 blocks;
# 130 x 998 x 4096, two row tiles and N % 4 != 0 (the sum's per-element path), in 8; GEMMs below 65
# rows (the crossover rule): 40 x 14000 x 4096 (64-row tiles) in 4, 24 x 7000 x 4096 (32-row tiles)
# in 8, 24 x 30000 x 4096 in 2 (g128s: the weights two blocks ahead), 16 x 10000 x 4096 (16-row
# tiles, weights two blocks ahead) in 6 of 6 blocks (the last of 2)
SPLIT_CASES = [(96, 1000, 8192, 8), (130, 998, 4096, 8), (40, 14000, 4096, 4), (24, 7000, 4096, 2),
               (24, 30000, 4096, 2), (16, 10000, 4096, 1)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,mb", SPLIT_CASES)
def test_gemm_split_k(gpu, fmt, M, N, K, mb, monkeypatch):
    """k_qgemm split along K (fp32 partials per range, summed in range order by k_gemm_split_sum)
    with tiles of 16 mb rows: a 384-column slice over all rows and three full rows against the
    oracle (the bf16-weight one, or for the tiles that compute as the GEMV does, the exact one); a second call gives the same bits; the bf16 output is the RNE of the fp32 one; 3 ranges
    (a shorter last one) and no split agree to fp32 summation order"""
    import ctypes as C
    import torch
    from opennpu_amd import _lib
    from opennpu_amd.device import QMatrix
    if fmt != orc.FMT_G128S:
        K -= 32                                       # a K tail inside the last 128-wide block
    o = (C.c_int64 * 7)()
    _lib.lib().onpu_plan_mv(fmt, N, K, M, o)
    assert o[0] == 1 and o[1] == mb and o[3] > 1, tuple(o)     # the split GEMM with these tiles
    st = syn.weights(fmt, N, K, 51 + M)
    xb = syn.activations(M, K, 52 + M)
    q = QMatrix(N, K, fmt, st)
    try:
        x = to_torch_bf16(xb).reshape(M, K)
        y1 = q.mv(x, f32=True)
        y2 = q.mv(x, f32=True)
        yb = q.mv(x)
        monkeypatch.setenv("ONPU_GEMM_SPLIT", "3")
        y3 = q.mv(x, f32=True)
        monkeypatch.setenv("ONPU_GEMM_SPLIT", "1")
        y0 = q.mv(x, f32=True)
        monkeypatch.delenv("ONPU_GEMM_SPLIT")
        assert o[6] == (mb == 1 or (N == 30000 and fmt == orc.FMT_G128S)), tuple(o)
        if o[6]:                       # weights two blocks ahead (the default here) or one: same sums
            monkeypatch.setenv("ONPU_GEMM_DEEP", "0")
            y4 = q.mv(x, f32=True)
            monkeypatch.delenv("ONPU_GEMM_DEEP")
            torch.cuda.synchronize()
            assert torch.equal(y1, y4), "the deeper weight pipeline changed the result"
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), "split-K GEMM is not deterministic"
        assert torch.equal(yb, y1.to(torch.bfloat16)), "bf16 output is not the RNE of the fp32 sums"
        for other, what in ((y0, "no split"), (y3, "3 ranges")):
            d = ((y1 - other).abs().max() / other.abs().max()).item()
            assert d <= 1e-5, f"split-K vs {what} differ by {d:.3e} of max|y|"
        rows = [0, M // 2, M - 1]
        yc = from_torch(yb[:, N - 384:])
        yr = from_torch(yb[rows])
        yf = from_torch(y1[rows])
    finally:
        q.free()
    if gemm_exact(fmt, M):         # tiles that compute as the GEMV does: the exact dequant
        check_bf16_out(yc, orc.qmm(fmt, st, N, K, xb, N - 384, N), what=f"split-K fmt {fmt} {M}x{N}x{K} columns")
        check_bf16_out(yr, orc.qmm(fmt, st, N, K, xb[rows]), what=f"split-K fmt {fmt} {M}x{N}x{K} rows")
        check_f32_out(yf, orc.qmm(fmt, st, N, K, xb[rows]), what=f"split-K fmt {fmt} fp32 rows")
        return
    check_gemm(yc, fmt, st, N, K, xb, N - 384, N, what=f"split-K fmt {fmt} {M}x{N}x{K} column slice")
    check_gemm(yr, fmt, st, N, K, xb[rows], what=f"split-K fmt {fmt} {M}x{N}x{K} rows")
    check_f32_out(yf, orc.qmm(fmt, st, N, K, xb[rows], bf16w=True), what=f"split-K fmt {fmt} fp32 rows")


def test_gemm_split_k_under_capture(gpu):
    """split-K GEMMs recorded in a graph (their partials in the capture's own workspace) at 96, 40
    and 16 rows (128-, 64- and 16-row tiles, the last with the weights two blocks ahead), and the
    long-K matrix that takes the GEMM at one row: replays interleaved with eager GEMMs on the default
    stream each equal the eager results bit for bit"""
    import torch
    from opennpu_amd.device import QMatrix
    shapes = [(96, 4096, 14336), (40, 14336, 4096), (16, 10000, 4096), (1, 4096, 28672)]
    mats = [QMatrix(N, K, orc.FMT_G128S, syn.weights(orc.FMT_G128S, N, K, 70 + M)) for M, N, K in shapes]
    try:
        xs = [to_torch_bf16(syn.activations(M, K, 71 + M)).reshape(M, K) for M, _, K in shapes]
        ref = [q.mv(x) for q, x in zip(mats, xs)]
        torch.cuda.synchronize()
        outs = [torch.empty_like(r) for r in ref]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for q, x, o in zip(mats, xs, outs):
                q.mv(x, out=o)
        for rep in range(3):
            for o in outs:
                o.zero_()
            g.replay()
            torch.cuda.synchronize()
            for o, r in zip(outs, ref):
                assert torch.equal(o, r), f"replay {rep} differs from the eager GEMM"
            ye = mats[0].mv(xs[0])
            torch.cuda.synchronize()
            assert torch.equal(ye, ref[0]), "eager GEMM after a replay differs"
    finally:
        for q in mats:
            q.free()


@pytest.mark.parametrize("N", [20000, 40000])
def test_argmax_at_gemm_rows(gpu, N, monkeypatch):
    """a vocabulary-sized LM head at 16, 24 and 48 rows takes the GEMM (the crossover rule): split
    along K with the argmax launch over its fp32 logits (20000 columns), or unsplit with the argmax
    keys from its epilogue (40000): logits against the bf16-weight oracle on a column slice and two
    rows, argmax equal to the oracle argmax of the returned logits, and to the fused GEMV path's
    argmax (ONPU_FORCE_GEMM=-1) wherever that row's top two logits are apart"""
    import ctypes as C
    import torch
    from opennpu_amd import _lib
    from opennpu_amd.device import QMatrix
    fmt, K = orc.FMT_G128S, 4096
    o = (C.c_int64 * 7)()
    for M in (16, 24, 48):
        _lib.lib().onpu_plan_mv(fmt, N, K, M, o)
        assert o[0] == 1 and (o[3] > 1) == (N == 20000), (N, M, tuple(o))
    st = syn.weights(fmt, N, K, 81)
    q = QMatrix(N, K, fmt, st)
    try:
        for M in (16, 24, 48):
            xb = syn.activations(M, K, 82 + M)
            x = to_torch_bf16(xb).reshape(M, K)
            lg, idx = q.argmax(x)
            monkeypatch.setenv("ONPU_FORCE_GEMM", "-1")
            lgv, idv = q.argmax(x)
            monkeypatch.delenv("ONPU_FORCE_GEMM")
            torch.cuda.synchronize()
            lg, idx, lgv, idv = from_torch(lg), idx.cpu().numpy(), from_torch(lgv), idv.cpu().numpy()
            assert np.array_equal(idx, orc.argmax(lg)) and np.array_equal(idv, orc.argmax(lgv))
            rows = [0, M - 1]
            bw = not gemm_exact(fmt, M)     # exact dequant (GEMV arithmetic) or bf16 RNE weights
            check_f32_out(lg[:, :512], orc.qmm(fmt, st, N, K, xb, 0, 512, bf16w=bw), what=f"M {M} columns")
            check_f32_out(lg[rows], orc.qmm(fmt, st, N, K, xb[rows], bf16w=bw), what=f"M {M} rows")
            top2 = np.sort(lg, axis=1)[:, -2:]
            apart = top2[:, 1] - top2[:, 0] > 1e-2 * np.abs(lg).max()
            assert apart.sum() >= M // 4 and np.array_equal(idx[apart], idv[apart])
    finally:
        q.free()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K", [(2100, 7400, 640), (1000, 14300, 512)])
def test_gemm_stream_k(gpu, fmt, M, N, K, monkeypatch):
    """256-row GEMM with a split of K (k_qgemm_sk) on ragged shapes with more tiles than CUs:
    2100 x 7400 has one round of whole tiles and 5 tiles cut in two; 1000 x 14300 has 224 tiles, each
    cut into a head piece and a tail piece, seven tail pieces per workgroup. A 400-column slice over
    all rows and 32 full rows against the oracle; a second call gives the same bits (the slot words
    need no clearing between launches, and a cut tile's sum does not depend on which piece finished
    first); no wait timed out;
    the plain stream-K split and the 128-row kernel agree to fp32 summation order."""
    import torch
    from opennpu_amd.device import QMatrix
    if fmt != orc.FMT_G128S:
        K -= 32                                       # a K tail inside the last 128-wide block
    st = syn.weights(fmt, N, K, 23)
    xb = syn.activations(M, K, 24)
    q = QMatrix(N, K, fmt, st)
    try:
        x = to_torch_bf16(xb).reshape(M, K)
        y1 = q.mv(x, f32=True)
        y2 = q.mv(x, f32=True)
        monkeypatch.setenv("ONPU_GSK_SCHED", "0")
        ys = q.mv(x, f32=True)
        monkeypatch.setenv("ONPU_GEMM_SK", "0")
        y0 = q.mv(x, f32=True)
        monkeypatch.delenv("ONPU_GEMM_SK")
        monkeypatch.delenv("ONPU_GSK_SCHED")
        yb = q.mv(x)
        torch.cuda.synchronize()
        assert q.L.onpu_gemm_status() == 0, "a split-K wait timed out"
        assert torch.equal(y1, y2), "split-K GEMM is not deterministic"
        for other, what in ((y0, "128-row GEMM"), (ys, "stream-K split")):
            d = ((y1 - other).abs().max() / other.abs().max()).item()
            assert d <= 1e-5, f"two-phase split vs {what} differ by {d:.3e} of max|y|"
        rows = np.random.default_rng(1).choice(M, 32, replace=False)
        yc = from_torch(yb[:, N - 400:])
        yr = from_torch(yb[torch.as_tensor(rows, device=yb.device)])
    finally:
        q.free()
    check_gemm(yc, fmt, st, N, K, xb, N - 400, N, what=f"split-K fmt {fmt} {M}x{N} column slice")
    check_gemm(yr, fmt, st, N, K, xb[rows], what=f"split-K fmt {fmt} {M}x{N} rows")


@pytest.mark.parametrize("name,N,K", [("up", 14336, 4096), ("down", 4096, 14336)])
def test_gemm_llama_ffn(gpu, name, N, K):
    """Llama-3.1-8B FFN prefill at M=2048 (the split-K GEMM: up cuts 192 of its 448 tiles at a K
    block, down cuts all 128 in two): one full row in every 256-row tile and one full column in
    every 256-column tile, so every tile, cut or whole, has a row and a column checked, plus all rows
    of a 128-column slice"""
    import torch
    from opennpu_amd.device import QMatrix
    M = 2048
    st = syn.weights(orc.FMT_G128S, N, K, 17)
    xb = syn.activations(M, K, 18)
    q = QMatrix(N, K, orc.FMT_G128S, st)
    rng = np.random.default_rng(0)
    rows = np.array([256 * t + rng.integers(0, 256) for t in range(M // 256)])
    cols = np.array([256 * t + rng.integers(0, 256) for t in range(N // 256)])
    try:
        y = q.mv(to_torch_bf16(xb).reshape(M, K))
        torch.cuda.synchronize()
        assert q.L.onpu_gemm_status() == 0, "a split-K wait timed out"
        yc = from_torch(y[:, 1000:1128])
        yr = from_torch(y[torch.as_tensor(rows, device=y.device)])
        ycols = from_torch(y[:, torch.as_tensor(cols, device=y.device)])
    finally:
        q.free()
    check_gemm(yc, orc.FMT_G128S, st, N, K, xb, 1000, 1128, what=f"{name} column slice")
    check_gemm(yr, orc.FMT_G128S, st, N, K, xb[rows], what=f"{name} one row per row tile")
    for j, n in enumerate(cols):
        check_gemm(ycols[:, j:j + 1], orc.FMT_G128S, st, N, K, xb, int(n), int(n) + 1,
                   what=f"{name} column {n} (column tile {j})")


@pytest.mark.parametrize("M", [1024, 96])
def test_gemm_two_streams(gpu, M):
    """split-K GEMMs on two streams at once (1024 rows: the stream-K kernel's partial tiles and slot
    words; 96 rows: the 128-row tiles' K-range partials): each stream has its own workspace, so both
    results equal the one-stream results bit for bit"""
    import torch
    from opennpu_amd.device import QMatrix
    N, K = 7168, 4096
    qa = QMatrix(N, K, orc.FMT_G128S, syn.weights(orc.FMT_G128S, N, K, 31))
    qb = QMatrix(N, K, orc.FMT_G128S, syn.weights(orc.FMT_G128S, N, K, 32))
    try:
        xa = to_torch_bf16(syn.activations(M, K, 33)).reshape(M, K)
        xb = to_torch_bf16(syn.activations(M, K, 34)).reshape(M, K)
        ra, rb = qa.mv(xa, f32=True), qb.mv(xb, f32=True)
        torch.cuda.synchronize()
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        outs = []
        for rep in range(3):
            with torch.cuda.stream(sa):
                ya = qa.mv(xa, f32=True)
            with torch.cuda.stream(sb):
                yb = qb.mv(xb, f32=True)
            outs.append((ya, yb))
        torch.cuda.synchronize()
        assert qa.L.onpu_gemm_status() == 0
        for ya, yb in outs:
            assert torch.equal(ya, ra) and torch.equal(yb, rb)
    finally:
        qa.free()
        qb.free()


def test_gemm_first_call_under_capture(gpu):
    """torch.cuda.graph captures on a stream of its own, so the split-K GEMMs it records are that
    stream's first: its workspace is allocated and cleared during the capture (the clearing kernel
    is a node of the graph). Two GEMMs with different cut counts in one graph, replays interleaved
    with eager GEMMs on the default stream, each replay equal to the eager results bit for bit."""
    import torch
    from opennpu_amd.device import QMatrix
    shapes = [(1024, 7168, 4096), (2048, 4096, 14336)]
    mats = [QMatrix(N, K, orc.FMT_G128S, syn.weights(orc.FMT_G128S, N, K, 60 + N)) for _, N, K in shapes]
    try:
        xs = [to_torch_bf16(syn.activations(M, K, 61 + K)).reshape(M, K) for M, _, K in shapes]
        ref = [q.mv(x, f32=True) for q, x in zip(mats, xs)]
        torch.cuda.synchronize()
        outs = [torch.empty_like(r) for r in ref]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for q, x, o in zip(mats, xs, outs):
                q.mv(x, out=o)
        for rep in range(3):
            for o in outs:
                o.zero_()
            g.replay()
            torch.cuda.synchronize()
            for o, r in zip(outs, ref):
                assert torch.equal(o, r), f"replay {rep} differs from the eager GEMM"
            ye = mats[1].mv(xs[1], f32=True)
            torch.cuda.synchronize()
            assert torch.equal(ye, ref[1]), "eager GEMM after a replay differs"
        assert mats[0].L.onpu_gemm_status() == 0
    finally:
        for q in mats:
            q.free()


def test_scratch_over_a_model_of_handles(gpu):
    """36 layers x 4 Qwen3-8B-shaped matrices, an M = 2048 GEMM through each on one stream, then
    host-pointer calls at 2048 rows through several of them: the workspaces do not grow with the
    number of handles (< 1 GiB of device memory beyond weights, inputs and outputs)"""
    import ctypes as C
    import torch
    from opennpu_amd.device import QMatrix
    shapes = [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)]
    st = {s: syn.weights(orc.FMT_G128S, s[0], s[1], 40 + i) for i, s in enumerate(shapes)}
    mats = [QMatrix(N, K, orc.FMT_G128S, st[(N, K)]) for _ in range(36) for N, K in shapes]
    M = 2048
    xs = {K: to_torch_bf16(syn.activations(M, K, K)).reshape(M, K) for K in (4096, 12288)}
    ys = {N: torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for N in (4096, 6144, 24576)}
    xh = np.random.default_rng(5).standard_normal((M, 4096)).astype(np.float32)
    yh = np.empty((M, 24576), np.float32)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    try:
        for q in mats:
            q.mv(xs[q.K], out=ys[q.N])
        torch.cuda.synchronize()
        assert mats[0].L.onpu_gemm_status() == 0
        fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
        for q in mats[:8]:
            if q.K == 4096:
                mats[0].L.onpu_dense_mv(C.c_void_p(q.h), fp(xh), M, fp(yh))
        used = free0 - torch.cuda.mem_get_info()[0]
        assert used < (1 << 30), f"{used / 2**20:.0f} MiB of workspace for 144 handles"
    finally:
        for q in mats:
            q.free()
        mats[0].L.onpu_release_scratch()


@pytest.mark.parametrize("M", [1, 5, 8])
def test_lm_head_q4_0(gpu, M):
    """151936 x 4096 GGUF Q4_0 LM head: fp32 logits and argmax (first maximum). M = 5 and 8 run the
    MFMA group-sum variant (at 8 its workgroups fit twice per CU only without the staged sums)."""
    from opennpu_amd.device import QMatrix
    N, K = 151936, 4096
    st = syn.weights(orc.FMT_Q4_0, N, K, 4)
    xb = syn.activations(M, K, 5 + M)
    q = QMatrix(N, K, orc.FMT_Q4_0, st)
    try:
        lg, idx = q.argmax(to_torch_bf16(xb).reshape(M, K))
        lg, idx = from_torch(lg), idx.cpu().numpy()
    finally:
        q.free()
    ref = orc.qmm(orc.FMT_Q4_0, st, N, K, xb)
    check_f32_out(lg, ref, what="lm head")
    assert np.array_equal(idx, orc.argmax(lg)), "argmax of the returned logits"
    top2 = np.sort(ref, axis=1)[:, -2:]
    for m in range(M):
        if top2[m, 1] - top2[m, 0] > 1e-3 * np.abs(ref).max():
            assert idx[m] == int(np.argmax(ref[m])), f"row {m}"


@pytest.mark.parametrize("fmt,N,K,M", [(orc.FMT_Q4_0, 9000, 1024, 1), (orc.FMT_Q4_0, 9000, 1024, 8),
                                       (orc.FMT_G128S, 4100, 2048, 3)])
def test_argmax_ties_and_replays(gpu, fmt, N, K, M):
    """LM-head argmax: equal to the oracle argmax of the returned logits, with a planted tie at the
    top of row 0 (the last weight row repeats the row holding the maximum: the first column must
    win); repeated calls and graph replays give the same result."""
    import torch
    from opennpu_amd.device import QMatrix
    st = syn.weights(fmt, N, K, 31).copy()
    xb = syn.activations(M, K, 32)
    if fmt == orc.FMT_Q4_0:
        # GGUF rows are contiguous in the staging bytes: the last row repeats the row holding row 0's
        # maximum, so that row 0 has a tie at its top and the first column must win
        rb = st.size // N
        r0 = int(np.argmax(orc.qmm(fmt, st, N, K, xb[:1])[0]))
        assert r0 < N - 1
        st[(N - 1) * rb:] = st[r0 * rb:(r0 + 1) * rb]
    q = QMatrix(N, K, fmt, st)
    try:
        x = to_torch_bf16(xb).reshape(M, K)
        lg1, i1 = q.argmax(x)
        lg2, i2 = q.argmax(x)
        lgg = torch.empty_like(lg1)
        ig = torch.empty_like(i1)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            q.argmax(x, lgg, ig)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            q.argmax(x, lgg, ig)
        for _ in range(3):
            ig.fill_(-1)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(ig, i1), "graph replay argmax differs"
            q.argmax(x)
        torch.cuda.synchronize()
        assert torch.equal(lg1, lg2) and torch.equal(i1, i2)
        lg, idx = from_torch(lg1), i1.cpu().numpy()
    finally:
        q.free()
    assert np.array_equal(idx, orc.argmax(lg)), "argmax of the returned logits"
    if fmt == orc.FMT_Q4_0:
        assert lg[0, r0] == lg[0, N - 1] and idx[0] == r0, "tie at the top of row 0: the first column"
    check_f32_out(lg, orc.qmm(fmt, st, N, K, xb), what="LM-head logits")


@pytest.mark.parametrize("fmt,N,K,M", [(orc.FMT_Q4_0, 151936, 4096, 5), (orc.FMT_G128S, 4100, 2048, 17),
                                       (orc.FMT_Q4S, 3000, 1024, 40), (orc.FMT_Q4NX, 2000, 512, 64),
                                       (orc.FMT_G128S, 40000, 4096, 24), (orc.FMT_Q4_0, 40000, 4096, 64)])
def test_argmax_fused_equals_separate(gpu, fmt, N, K, M, monkeypatch):
    """the argmax from the per-workgroup keys of the GEMV's epilogue (or, at 24 and 64 rows of a
    40000 x 4096 head, of the unsplit small-tile GEMM's) gives the same logits bits and indices as
    the same product followed by the argmax launch over the logits (ONPU_ARGMAX_FUSED=0), also on
    a second call and for a row of NaNs (index 0)"""
    import torch
    from opennpu_amd.device import QMatrix
    st = syn.weights(fmt, N, K, 41)
    xb = syn.activations(M, K, 42)
    q = QMatrix(N, K, fmt, st)
    try:
        x = to_torch_bf16(xb).reshape(M, K)
        x[M - 1] = float("nan")
        monkeypatch.setenv("ONPU_ARGMAX_FUSED", "0")
        lg0, i0 = q.argmax(x)
        monkeypatch.setenv("ONPU_ARGMAX_FUSED", "1")
        lg1, i1 = q.argmax(x)
        lg2, i2 = q.argmax(x)
        torch.cuda.synchronize()
        assert torch.equal(lg0.view(torch.int32), lg1.view(torch.int32)), "logits differ"
        assert torch.equal(i0, i1) and torch.equal(i1, i2), "argmax differs"
        assert int(i1[M - 1]) == 0, "a row of NaNs gives index 0"
        lg, idx = from_torch(lg1), i1.cpu().numpy()
    finally:
        q.free()
    assert np.array_equal(idx[:M - 1], orc.argmax(lg[:M - 1])), "argmax of the returned logits"


def _plant_nan_scale(fmt, st, N, K, row):
    """the first scale (Q4_0: the fp16 d of the first block) of weight row `row` set to NaN, so
    that every row's logit `row` is NaN"""
    st = st.copy()
    if fmt == orc.FMT_Q4_0:
        st[row * (K // 32 * 18):][:2] = np.frombuffer(np.uint16(0x7e00).tobytes(), np.uint8)
    else:
        off = N * K // 2 + row * (K // orc.group(fmt)) * 2
        st[off:off + 2] = np.frombuffer(np.uint16(0x7fc0).tobytes(), np.uint8)
    return st


@pytest.mark.parametrize("fmt,N,K,M", [(orc.FMT_Q4_0, 151936, 4096, 5), (orc.FMT_G128S, 4100, 2048, 17),
                                       (orc.FMT_Q4NX, 2000, 512, 70), (orc.FMT_G128S, 40000, 4096, 16)])
def test_argmax_first_nan_wins(gpu, fmt, N, K, M, monkeypatch):
    """numpy's and torch's argmax, which the reference takes over the logits (npu4/engine.py:358,
    runtime.py:348), return the first NaN of a row that holds one. Rows with NaN logits at two
    columns (NaN scales planted in weight rows N/3 and N/5) give N/5, by the fused keys (<= 64
    rows) and by the argmax launch over the logits (ONPU_ARGMAX_FUSED=0, and 70 rows) alike; the
    oracle agrees with numpy."""
    import torch
    from opennpu_amd.device import QMatrix
    st = syn.weights(fmt, N, K, 43)
    for row in (N // 5, N // 3):
        st = _plant_nan_scale(fmt, st, N, K, row)
    xb = syn.activations(M, K, 44)
    q = QMatrix(N, K, fmt, st)
    try:
        x = to_torch_bf16(xb).reshape(M, K)
        outs = []
        for fused in ("1", "0"):
            monkeypatch.setenv("ONPU_ARGMAX_FUSED", fused)
            lg, idx = q.argmax(x)
            torch.cuda.synchronize()
            outs.append((from_torch(lg), idx.cpu().numpy()))
    finally:
        q.free()
    for lg, idx in outs:
        assert np.isnan(lg[:, N // 5]).all() and np.isnan(lg[:, N // 3]).all()
        assert (idx == N // 5).all(), idx
        assert np.array_equal(idx, np.argmax(lg, axis=1)) and np.array_equal(idx, orc.argmax(lg))


def test_argmax_workspace_survives_growth_under_a_graph(gpu):
    """A graph captured at M = 1 keeps the argmax workspace pointers of that capture. Eager calls at
    larger M (the fused keys up to 64 rows, and 70 rows through the argmax launch over the logits)
    must not free or move what the graph holds: replays after them give the eager results, bit for
    bit."""
    import torch
    from opennpu_amd.device import QMatrix
    fmt, N, K = orc.FMT_Q4_0, 30000, 1024
    st = syn.weights(fmt, N, K, 45)
    q = QMatrix(N, K, fmt, st)
    try:
        x1 = to_torch_bf16(syn.activations(1, K, 46)).reshape(1, K)
        lg_e, i_e = q.argmax(x1)
        lgg = torch.empty_like(lg_e)
        ig = torch.empty_like(i_e)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            q.argmax(x1, lgg, ig)
        for M in (5, 64, 70, 3):
            xm = to_torch_bf16(syn.activations(M, K, 47 + M)).reshape(M, K)
            lg, idx = q.argmax(xm)
            ig.fill_(-1)
            lgg.fill_(0)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(ig, i_e) and torch.equal(lgg.view(torch.int32), lg_e.view(torch.int32)), M
            assert np.array_equal(idx.cpu().numpy(), orc.argmax(from_torch(lg))), M
    finally:
        q.free()


def test_rows_zero_and_reuse(gpu):
    """M = 0 is a no-op; one handle serves several calls with different M."""
    import torch
    from opennpu_amd.device import QMatrix
    N, K = 64, 256
    st = syn.weights(orc.FMT_G128S, N, K, 9)
    q = QMatrix(N, K, orc.FMT_G128S, st)
    try:
        out = torch.zeros((1, N), dtype=torch.bfloat16, device="cuda")
        q.mv(torch.zeros((0, K), dtype=torch.bfloat16, device="cuda"), out=out[:0])
        for M in (3, 1, 9):
            xb = syn.activations(M, K, M)
            y = from_torch(q.mv(to_torch_bf16(xb).reshape(M, K)))
            check_bf16_out(y, orc.qmm(orc.FMT_G128S, st, N, K, xb), what=f"M {M}")
    finally:
        q.free()

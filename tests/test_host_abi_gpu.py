"""The host-pointer call sequences of the reference's npu4 engine (opennpu/native/npu4/model.py),
made as plain ctypes calls (tests/hostabi.py) against libonpu_hip on the GPU:

  dense   onpu_dense_new2 -> onpu_pack into onpu_dense_buf -> onpu_dense_sync -> onpu_dense_mv
          (model.py:801-836: stacked siblings, residual rows, rows from 1 to prompts)
  banks   onpu_bank_new2 -> E x onpu_pack into onpu_bank_buf -> onpu_bank_sync -> onpu_bank_run
          (model.py:926-1068: x per token or per slot)
  FFN     onpu_moe_ffn with SiLU or gpt-oss act and biases; onpu_ffn_new / _fused / _perm / _gu /
          _dn, then onpu_ffn_run (one token) and onpu_ffn_run_many (model.py:926-1020)
  helpers onpu_moe_act, onpu_moe_sum (onpu_cpu.cpp:233-274)

Expected values come from the oracle alone: the packed bytes hold the oracle's quantization of the
fp32 weights (the library's pack equals the oracle's byte for byte, tests/test_host_abi.py),
dequantized by the reference formula and multiplied in fp64 with the bf16-rounded input (the device's input
conversion). Tolerances: fp32 outputs of the GEMV path max|y-r|/max|r| <= 1e-4 (fp32
accumulation); rows > 64 take the MFMA GEMM, whose weights enter as bf16 RNE of the dequant
(<= 1e-4 against that, <= 1e-2 against the exact weights); expert FFNs (bf16 activation between the
two products) <= 1e-2 max and <= 1e-3 mean.
"""
import numpy as np
import pytest

import oracle.oracle as orc
from tests import hostabi as ha

pytestmark = pytest.mark.gpu
FMT = {1: orc.FMT_Q4S, 0: orc.FMT_Q4NX}


@pytest.fixture(scope="module")
def L(gpu):
    L = ha.bind()
    assert L.onpu_ok() == 1                          # the reference loader's last check
    return L


def xbits(x):
    return orc.f2bf_np(np.ascontiguousarray(x, np.float32))


def qdq(W, sym):
    """the oracle's dequantization of the oracle's quantization of W"""
    N, K = W.shape
    return orc.dequant(FMT[sym], orc.quantize(FMT[sym], W), N, K)


def ref_mm(x, Wq):
    return orc.bf2f(xbits(x)).astype(np.float64) @ Wq.astype(np.float64).T


def rel(y, r):
    return np.abs(np.asarray(y, np.float64) - r).max() / max(np.abs(r).max(), 1e-30)


@pytest.mark.parametrize("sym", [1, 0])
def test_dense_rows(L, sym):
    rng = np.random.default_rng(10 + sym)
    N, K = 384, 512
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    h = ha.dense(L, W, sym)
    Wq = qdq(W, sym)
    for rows in (1, 3, 8, 9, 33, 64):
        x = rng.standard_normal((rows, K)).astype(np.float32)
        y = ha.dense_mv(L, h, x, N)
        assert rel(y, ref_mm(x, Wq)) <= 1e-4, (sym, rows, rel(y, ref_mm(x, Wq)))
    # the same handle again with fewer rows: nothing of the larger call leaks into y
    x = rng.standard_normal((2, K)).astype(np.float32)
    assert rel(ha.dense_mv(L, h, x, N), ref_mm(x, Wq)) <= 1e-4
    L.onpu_dense_free(h)


def test_dense_prompt_rows_take_the_gemm(L):
    rng = np.random.default_rng(7)
    N, K = 320, 512
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    h = ha.dense(L, W, 1)
    Wq = qdq(W, 1)
    x = rng.standard_normal((70, K)).astype(np.float32)
    y = ha.dense_mv(L, h, x, N)
    assert rel(y, ref_mm(x, orc.bf2f(orc.f2bf_np(Wq)))) <= 1e-4
    assert rel(y, ref_mm(x, Wq)) <= 1e-2
    L.onpu_dense_free(h)


def test_stacked_siblings_are_the_concatenation(L):
    """q, k and v stacked into one matrix (model.py:1322-1334): one call, each slice equal to its own
    product, and to a handle of that sibling alone"""
    rng = np.random.default_rng(2)
    K, sizes = 512, [256, 64, 64]
    Ws = [(rng.standard_normal((n, K)) * 0.05).astype(np.float32) for n in sizes]
    h = ha.dense(L, np.concatenate(Ws), 1)
    alone = [ha.dense(L, W, 1) for W in Ws]
    for rows in (1, 5):
        x = rng.standard_normal((rows, K)).astype(np.float32)
        y = ha.dense_mv(L, h, x, sum(sizes))
        o = 0
        for W, ha_ in zip(Ws, alone):
            part = y[:, o:o + W.shape[0]]
            assert rel(part, ref_mm(x, qdq(W, 1))) <= 1e-4
            assert rel(part, ha.dense_mv(L, ha_, x, W.shape[0])) <= 1e-5
            o += W.shape[0]
    for p in [h, *alone]:
        L.onpu_dense_free(p)


def test_residual_rows(L):
    """rows [W; W - quant_dequant(W)] in one matrix (model.py:816): the halves added give two
    4-bit passes, closer to W than one"""
    rng = np.random.default_rng(3)
    N, K = 96, 256
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    w1 = np.empty_like(W)
    L.onpu_quant_dequant(ha.fp(W), N, K, 1, ha.fp(w1), 4)
    R = np.concatenate([W, W - w1])
    h = ha.dense(L, R, 1)
    x = rng.standard_normal((2, K)).astype(np.float32)
    yy = ha.dense_mv(L, h, x, 2 * N)
    y = yy[:, :N] + yy[:, N:]
    w2 = qdq(W - w1, 1)
    r = ref_mm(x, w1.astype(np.float64) + w2)
    assert rel(y, r) <= 1e-4
    exact = x.astype(np.float64) @ W.astype(np.float64).T
    assert rel(y, exact) < rel(ref_mm(x, w1), exact)
    L.onpu_dense_free(h)


def _experts(rng, E, H, I):
    gu = [(rng.standard_normal((2 * I, H)) * 0.05).astype(np.float32) for _ in range(E)]
    dn = [(rng.standard_normal((H, I)) * 0.05).astype(np.float32) for _ in range(E)]
    return gu, dn


def _routes(rng, T, E, k):
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    return ids, (w / w.sum(1, keepdims=True)).astype(np.float32)


def _layer_ref(x, gu, dn, ids, w, act, gb=None, db=None, alpha=0.0, limit=0.0):
    """the expert layer with the device's rounding points: gate_up fp64 -> fp32 (+ bias), act in
    fp32, act -> bf16, down in fp64 (+ bias), weighted sum"""
    T, k = ids.shape
    y = np.zeros((T, dn[0].shape[0]))
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            hh = ref_mm(x[t:t + 1], qdq(gu[e], 1)).astype(np.float32)
            if gb is not None:
                hh = hh + gb[e]
            a = orc.silu_mul(hh) if act == 0 else orc.gptoss_act(hh, alpha, limit)
            d = ref_mm(a, qdq(dn[e], 1))[0]
            if db is not None:
                d = d + db[e]
            y[t] += float(w[t, j]) * d
    return y


@pytest.mark.parametrize("ncols", [1, 2])
def test_bank_run(L, ncols):
    """x per token (gate_up of every slot) and x per slot (the down input), y [T][k][N]"""
    rng = np.random.default_rng(20 + ncols)
    E, H, I, T, k = 6, 256, 128, 3, 4
    gu, _ = _experts(rng, E, H, I)
    h = ha.bank(L, gu, ncols, 1)
    ids, _ = _routes(rng, T, E, k)
    x = rng.standard_normal((T, H)).astype(np.float32)
    y = np.full((T, k, 2 * I), np.nan, np.float32)
    L.onpu_bank_run(h, ha.fp(x), 0, T, ha.ip(ids), k, ha.fp(y))
    xs = rng.standard_normal((T * k, H)).astype(np.float32)
    ys = np.full((T, k, 2 * I), np.nan, np.float32)
    L.onpu_bank_run(h, ha.fp(xs), 1, T, ha.ip(ids), k, ha.fp(ys))
    for t in range(T):
        for j in range(k):
            Wq = qdq(gu[ids[t, j]], 1)
            assert rel(y[t, j], ref_mm(x[t:t + 1], Wq)[0]) <= 1e-4
            assert rel(ys[t, j], ref_mm(xs[t * k + j:t * k + j + 1], Wq)[0]) <= 1e-4
    L.onpu_bank_free(h)


@pytest.mark.parametrize("case", ["silu", "silu_bias", "gptoss_bias"])
def test_moe_ffn(L, case):
    rng = np.random.default_rng(hash(case) % 997)
    E, H, I, T, k = 8, 256, 128, 5, 8
    gu, dn = _experts(rng, E, H, I)
    hg, hd = ha.bank(L, gu, 1, 1), ha.bank(L, dn, 1, 1)
    gb = db = None
    act, alpha, limit = 0, 0.0, 0.0
    if case != "silu":
        gb = (rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32)
        db = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    if case == "gptoss_bias":
        act, alpha, limit = 1, 1.702, 7.0
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, w = _routes(rng, T, E, k)
    y = np.full((T, H), np.nan, np.float32)
    L.onpu_moe_ffn(hg, hd, ha.fp(x), T, ha.ip(ids), k, ha.fp(w), act, alpha, limit, ha.fp(gb), ha.fp(db), ha.fp(y))
    r = _layer_ref(x, gu, dn, ids, w, act, gb, db, alpha, limit)
    err = np.abs(y - r)
    assert err.max() / np.abs(r).max() <= 1e-2 and err.mean() / np.abs(r).max() <= 1e-3, case
    L.onpu_bank_free(hg)
    L.onpu_bank_free(hd)


def test_fused_ffn(L):
    """onpu_ffn_new -> fused? -> perm (gate_up rows packed as gu[e][perm]) -> both banks packed and
    synced -> onpu_ffn_run per token, onpu_ffn_run_many over a prompt"""
    rng = np.random.default_rng(31)
    E, H, I, k = 8, 256, 128, 8
    gu, dn = _experts(rng, E, H, I)
    f = L.onpu_ffn_new(2 * I, H, H, I, E, 1)
    assert f and L.onpu_ffn_fused(f) == 1
    perm = np.full(2 * I, -1, np.int32)
    L.onpu_ffn_perm(f, ha.ip(perm))
    assert sorted(perm) == list(range(2 * I))
    ha.bank(L, [g[perm] for g in gu], 1, 1, h=L.onpu_ffn_gu(f))
    ha.bank(L, dn, 1, 1, h=L.onpu_ffn_dn(f))
    x = rng.standard_normal((1, H)).astype(np.float32)
    ids, w = _routes(rng, 1, E, k)
    y = np.full((1, H), np.nan, np.float32)
    assert L.onpu_ffn_run(f, ha.fp(x), ha.ip(ids), k, ha.fp(w), ha.fp(y)) == 1
    r = _layer_ref(x, gu, dn, ids, w, 0)
    assert rel(y, r) <= 1e-2 and np.abs(y - r).mean() / np.abs(r).max() <= 1e-3
    T = 6
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, w = _routes(rng, T, E, k)
    y = np.full((T, H), np.nan, np.float32)
    assert L.onpu_ffn_run_many(f, ha.fp(x), T, ha.ip(ids), k, ha.fp(w), ha.fp(y)) == 1
    r = _layer_ref(x, gu, dn, ids, w, 0)
    assert rel(y, r) <= 1e-2 and np.abs(y - r).mean() / np.abs(r).max() <= 1e-3
    L.onpu_ffn_free(f)


def test_unfusable_ffn_declines(L):
    """a down K that is not half the gate_up N cannot be fused: onpu_ffn_fused is 0 and
    onpu_ffn_run returns 0 so the caller takes its bank path"""
    f = L.onpu_ffn_new(256, 256, 256, 64, 4, 1)
    assert f and L.onpu_ffn_fused(f) == 0
    x = np.zeros((1, 256), np.float32)
    ids = np.arange(4, dtype=np.int32)
    w = np.full(4, 0.25, np.float32)
    y = np.zeros((1, 256), np.float32)
    assert L.onpu_ffn_run(f, ha.fp(x), ha.ip(ids), 4, ha.fp(w), ha.fp(y)) == 0
    L.onpu_ffn_free(f)


def test_moe_act_and_sum(L):
    rng = np.random.default_rng(9)
    rows, Ng, E, T, k, N = 12, 64, 5, 4, 3, 48
    h = (rng.standard_normal((rows, Ng)) * 3).astype(np.float32)
    ids = rng.integers(0, E, rows).astype(np.int32)
    bias = rng.standard_normal((E, Ng)).astype(np.float32)
    for act, alpha, limit in [(0, 0.0, 0.0), (1, 1.702, 7.0)]:
        for b in (None, bias):
            a = np.full((rows, Ng // 2), np.nan, np.float32)
            L.onpu_moe_act(ha.fp(h), rows, Ng, ha.ip(ids), ha.fp(b), act, alpha, limit, ha.fp(a))
            hb = h if b is None else h + b[ids]
            want = orc.silu_mul(hb) if act == 0 else orc.gptoss_act(hb, alpha, limit)
            assert np.allclose(a, want, rtol=1e-5, atol=1e-6), (act, b is None)
    o = rng.standard_normal((T, k, N)).astype(np.float32)
    sids = rng.integers(0, E, (T, k)).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    sb = rng.standard_normal((E, N)).astype(np.float32)
    for b in (None, sb):
        y = np.full((T, N), np.nan, np.float32)
        L.onpu_moe_sum(ha.fp(o), T, k, N, ha.ip(sids), ha.fp(w), ha.fp(b), ha.fp(y))
        assert np.allclose(y, orc.moe_sum(o, sids, w, b), rtol=1e-5, atol=1e-5)


def test_dense_mv_reports_a_timed_out_wait(L, monkeypatch):
    """More than 64 rows run the split-K GEMM, whose partial-tile exchange waits are bounded. A wait
    that gives up leaves Y invalid, and onpu_dense_mv must say so rather than return stale rows (the
    reference aborts on a device failure: ONPU_ASSERT, opennpu_core.hpp:30-32). The time-out is
    forced from the host: ONPU_SPIN_LIMIT=0 makes every bounded wait give up without polling, and
    every kernel still ends normally. With ONPU_WAIT_TIMEOUT=error the call returns y all NaN and
    onpu_last_error names the wait (the default is the reference's abort). The next call, at the
    default limit, is right again: the workspace's flags and tags survive the forced time-out."""
    rng = np.random.default_rng(77)
    N, K, M = 16384, 1024, 512        # 2 x 64 tiles of 256 x 256 on 256 CUs: every tile cut in half
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    h = ha.dense(L, W, 1)
    x = rng.standard_normal((M, K)).astype(np.float32)
    try:
        monkeypatch.setenv("ONPU_SPIN_LIMIT", "0")
        monkeypatch.setenv("ONPU_WAIT_TIMEOUT", "error")
        y = ha.dense_mv(L, h, x, N)
        assert np.isnan(y).all(), "a timed-out split-K wait returned numbers"
        assert b"split-K partial-tile wait gave up" in L.onpu_last_error()
        monkeypatch.delenv("ONPU_SPIN_LIMIT")
        y = ha.dense_mv(L, h, x, N)
        r = ref_mm(x[::16], qdq(W, 1))
        assert rel(y[::16], r) <= 1e-2, "the call after the forced time-out"
    finally:
        L.onpu_dense_free(h)


def test_ffn_run_reports_a_timed_out_wait(L, monkeypatch):
    """The one-launch MoE decode (ONPU_MOE_FUSED=1) waits, bounded, for the act rows the other
    workgroups publish. Forced to give up (ONPU_SPIN_LIMIT=0), onpu_ffn_run returns 0, "not done",
    which sends the reference's caller to its bank path, with y NaN and the reason in
    onpu_last_error (ONPU_WAIT_TIMEOUT=error). The next call is right: the kernel's counters come
    back to zero even when its consumers gave up before every producer arrived."""
    rng = np.random.default_rng(78)
    E, H, I, k = 8, 256, 128, 8
    gu, dn = _experts(rng, E, H, I)
    f = L.onpu_ffn_new(2 * I, H, H, I, E, 1)
    assert f and L.onpu_ffn_fused(f) == 1
    try:
        ha.bank(L, gu, 1, 1, h=L.onpu_ffn_gu(f))
        ha.bank(L, dn, 1, 1, h=L.onpu_ffn_dn(f))
        x = rng.standard_normal((1, H)).astype(np.float32)
        ids, w = _routes(rng, 1, E, k)
        r = _layer_ref(x, gu, dn, ids, w, 0)
        monkeypatch.setenv("ONPU_MOE_FUSED", "1")
        monkeypatch.setenv("ONPU_WAIT_TIMEOUT", "error")
        for limit in ("0", None, "0", None):
            if limit is None:
                monkeypatch.delenv("ONPU_SPIN_LIMIT", raising=False)
            else:
                monkeypatch.setenv("ONPU_SPIN_LIMIT", limit)
            y = np.full((1, H), 7.0, np.float32)
            done = L.onpu_ffn_run(f, ha.fp(x), ha.ip(ids), k, ha.fp(w), ha.fp(y))
            if limit is None:
                assert done == 1 and rel(y, r) <= 1e-2, "the call after a forced time-out"
            else:
                assert done == 0 and np.isnan(y).all(), "a timed-out MoE decode wait"
                assert b"MoE decode's wait for its act rows gave up" in L.onpu_last_error()
    finally:
        L.onpu_ffn_free(f)

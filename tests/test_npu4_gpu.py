"""The reference's own call pattern over libonpu_hip on the GPU: npu4.NPULinearGroup / NPULinear /
NPUExperts (opennpu_amd/npu4.py, mirroring opennpu/native/npu4/model.py) pack fp32 weights with
onpu_pack, upload through *_buf + *_sync and run the host-pointer entry points (onpu_dense_mv,
onpu_ffn_run, onpu_moe_ffn, onpu_bank_run, onpu_moe_act, onpu_moe_sum) exactly as the reference
module does.

Expected values come from the oracle alone: the weights are quantized with the oracle's restatement
of the reference quantizers (orc.quant_sym32 / quant_asym32), dequantized by the reference formula,
and multiplied in fp64 with the bf16-rounded inputs. Tolerances: fp32 outputs of the GEMV path
max|y-r|/max|r| <= 1e-4 (fp32 accumulation); the prefill GEMM and the expert FFN (bf16 weights in
MFMA, bf16 activation between the two products) <= 1e-2, with the mean error <= 1e-3.
"""
import numpy as np
import pytest

import oracle.oracle as orc

pytestmark = pytest.mark.gpu


def oracle_qdq(W, sym):
    """W quantized per 32 weights by the oracle's quantizers, dequantized as onpu_api.cpp:518"""
    N, K = W.shape
    out = np.empty_like(W, dtype=np.float32)
    for n in range(N):
        for g in range(K // 32):
            x = np.ascontiguousarray(W[n, 32 * g:32 * g + 32], np.float32)
            if sym:
                q, d = orc.quant_sym32(x)
                df = orc.bf2f(np.array([d], np.uint16))[0]
                out[n, 32 * g:32 * g + 32] = (q.astype(np.float32) - 8) * df
            else:
                q, s, m = orc.quant_asym32(x)
                sf, mf = orc.bf2f(np.array([s, m], np.uint16))
                out[n, 32 * g:32 * g + 32] = (q.astype(np.float32) * sf).astype(np.float32) + mf
    return out


def xbf(x):
    return orc.bf2f(orc.f2bf_np(np.ascontiguousarray(x, np.float32))).astype(np.float64)


def rel(y, r):
    return np.abs(np.asarray(y, np.float64) - r).max() / max(np.abs(r).max(), 1e-30)


@pytest.fixture(scope="module")
def npu4(gpu):
    from opennpu_amd import npu4 as m
    m._CLIB[:] = [False, None]
    assert m.clib() is not None
    return m


@pytest.mark.parametrize("sym", [True, False])
def test_linear_group_siblings(npu4, sym):
    """q, k, v siblings stacked into one matrix; each sibling's slice against its own product"""
    import torch
    rng = np.random.default_rng(1 + sym)
    K, sizes = 512, [256, 64, 64]
    Ws = [(rng.standard_normal((n, K)) * 0.05).astype(np.float32) for n in sizes]
    g = npu4.NPULinearGroup(["q", "k", "v"], Ws, sym=sym)
    assert g.m.N == 384 and g.m.nbytes == orc.geometry(384, K, 8, int(sym))[7]
    for rows in (1, 3, 9):
        x = torch.from_numpy(rng.standard_normal((rows, K)).astype(np.float32))
        for i, W in enumerate(Ws):
            y = g.compute(x, i)
            r = xbf(x.numpy()) @ oracle_qdq(W, sym).astype(np.float64).T
            assert rel(y, r) <= 1e-4, (sym, rows, i, rel(y, r))
    # the first sibling's call computed all of them: the same object gives the same buffer
    x = torch.from_numpy(rng.standard_normal((2, K)).astype(np.float32))
    a = g.compute(x, 0)
    assert g.compute(x, 2).base is a.base


def test_linear_group_prefill_rows(npu4):
    """more than 64 rows run the MFMA GEMM (weights enter as bf16 RNE of the dequant)"""
    import torch
    rng = np.random.default_rng(7)
    K, N = 512, 320
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    g = npu4.NPULinearGroup(["up"], [W], sym=True)
    x = torch.from_numpy(rng.standard_normal((70, K)).astype(np.float32))
    y = g.full(x)
    wd = oracle_qdq(W, True)
    r = xbf(x.numpy()) @ wd.astype(np.float64).T
    rb = xbf(x.numpy()) @ orc.bf2f(orc.f2bf_np(wd)).astype(np.float64).T
    assert rel(y, rb) <= 1e-4
    assert rel(y, r) <= 1e-2


def test_linear_group_residual(npu4):
    """residual rows [W; W - quant_dequant(W)]: the two 4-bit passes added"""
    import torch
    rng = np.random.default_rng(3)
    K, N = 256, 96
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    g = npu4.NPULinearGroup(["o"], [W], sym=True, residual=True)
    x = torch.from_numpy(rng.standard_normal((2, K)).astype(np.float32))
    y = g.full(x)
    w1 = oracle_qdq(W, True)
    w2 = oracle_qdq(W - w1, True)
    r = xbf(x.numpy()) @ (w1.astype(np.float64) + w2.astype(np.float64)).T
    assert y.shape == (2, N)
    assert rel(y, r) <= 1e-4
    # and the residual pass is closer to W than one pass
    exact = x.numpy().astype(np.float64) @ W.astype(np.float64).T
    assert rel(y, exact) < rel(xbf(x.numpy()) @ w1.astype(np.float64).T, exact)


def test_npu_linear_module(npu4):
    import torch
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((128, 256)) * 0.05).astype(np.float32)
    b = torch.from_numpy(rng.standard_normal(128).astype(np.float32))
    g = npu4.NPULinearGroup(["proj"], [W], sym=True)
    lin = npu4.NPULinear(g, 0, 256, 128, b)
    x = torch.from_numpy(rng.standard_normal((2, 3, 256)).astype(np.float32))
    y = lin(x)
    assert y.shape == (2, 3, 128) and y.dtype == torch.float32
    r = xbf(x.numpy().reshape(6, 256)) @ oracle_qdq(W, True).astype(np.float64).T + b.numpy()
    assert rel(y.numpy().reshape(6, 128), r) <= 1e-4


class _Orig:
    def __init__(self, act_fn=None, gptoss=None):
        self.act_fn = act_fn
        if gptoss:
            self.alpha, self.limit = gptoss
            self._apply_gate = lambda t: t      # present: marks the gpt-oss activation


def _experts_ref(x, gu, dn, ids, w, act, gu_bias=None, dn_bias=None, alpha=0.0, limit=0.0, sym=True):
    T, k = ids.shape
    xb = xbf(x)
    gq = {e: oracle_qdq(gu[e], sym).astype(np.float64) for e in np.unique(ids)}
    dq = {e: oracle_qdq(dn[e], sym).astype(np.float64) for e in np.unique(ids)}
    y = np.zeros((T, dn[0].shape[0]))
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            h = (xb[t] @ gq[e].T).astype(np.float32)
            if gu_bias is not None:
                h = h + gu_bias[e]
            a = orc.silu_mul(h[None]) if act == 0 else orc.gptoss_act(h[None], alpha, limit)
            d = xbf(a)[0] @ dq[e].T
            if dn_bias is not None:
                d = d + dn_bias[e]
            y[t] += float(w[t, j]) * d
    return y


def _route(rng, T, E, k):
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    return ids, w / w.sum(1, keepdims=True)


@pytest.mark.parametrize("case", ["fused_decode", "moe_ffn_silu", "bias_silu", "gptoss", "torch_act"])
def test_experts(npu4, case):
    import torch
    rng = np.random.default_rng(hash(case) % 1000)
    E, H, I, k = 8, 256, 128, 8
    gu = [(rng.standard_normal((2 * I, H)) * 0.05).astype(np.float32) for _ in range(E)]
    dn = [(rng.standard_normal((H, I)) * 0.05).astype(np.float32) for _ in range(E)]
    gb = db = None
    alpha = limit = 0.0
    act = 0
    if case in ("fused_decode", "moe_ffn_silu"):
        orig = _Orig(torch.nn.functional.silu)
    elif case == "bias_silu":
        orig = _Orig(torch.nn.functional.silu)
        gb = (rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32)
        db = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    elif case == "gptoss":
        alpha, limit, act = 1.702, 7.0, 1
        orig = _Orig(gptoss=(alpha, limit))
    else:
        orig = _Orig(torch.nn.functional.gelu)       # no library activation: bank_run + torch act
    ex = npu4.NPUExperts(orig, gu, dn, k, gu_bias=gb, dn_bias=db, sym=True)
    assert (ex.cffn is not None) == (case in ("fused_decode", "moe_ffn_silu"))
    T = 1 if case == "fused_decode" else 5
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, w = _route(rng, T, E, k)
    y = ex(torch.from_numpy(x), torch.from_numpy(ids.astype(np.int64)), torch.from_numpy(w)).numpy()
    if case == "torch_act":
        # the reference applies act_fn(gate) * up in torch on the fp32 gate_up output
        gq = [oracle_qdq(gu[e], True).astype(np.float64) for e in range(E)]
        dq = [oracle_qdq(dn[e], True).astype(np.float64) for e in range(E)]
        r = np.zeros((T, H))
        for t in range(T):
            for j in range(k):
                e = ids[t, j]
                h = torch.from_numpy((xbf(x[t:t + 1]) @ gq[e].T).astype(np.float32))
                a = (torch.nn.functional.gelu(h[:, :I]) * h[:, I:]).numpy()
                r[t] += float(w[t, j]) * (xbf(a)[0] @ dq[e].T)
    else:
        r = _experts_ref(x, gu, dn, ids, w, act, gb, db, alpha, limit)
    err = np.abs(y - r)
    scale = np.abs(r).max()
    assert err.max() / scale <= 1e-2, (case, err.max() / scale)
    assert err.mean() / scale <= 1e-3, (case, err.mean() / scale)


def test_moe_act_and_sum_helpers(npu4):
    """onpu_moe_act / onpu_moe_sum (the CPU helpers of onpu_cpu.cpp:233-274) against the oracle"""
    import ctypes as C
    lib = npu4.clib()
    rng = np.random.default_rng(9)
    rows, Ng, E, T, k, N = 12, 64, 5, 4, 3, 48
    h = (rng.standard_normal((rows, Ng)) * 3).astype(np.float32)
    ids = rng.integers(0, E, rows).astype(np.int32)
    bias = rng.standard_normal((E, Ng)).astype(np.float32)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    ip = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))
    for act, alpha, limit in [(0, 0.0, 0.0), (1, 1.702, 7.0)]:
        for b in (None, bias):
            a = np.empty((rows, Ng // 2), np.float32)
            lib.onpu_moe_act(fp(h), rows, Ng, ip(ids), None if b is None else fp(b), act, alpha, limit, fp(a))
            hb = h if b is None else h + b[ids]
            want = orc.silu_mul(hb) if act == 0 else orc.gptoss_act(hb, alpha, limit)
            assert np.allclose(a, want, rtol=1e-5, atol=1e-6), (act, b is None)
    o = rng.standard_normal((T, k, N)).astype(np.float32)
    sids = rng.integers(0, E, (T, k)).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    sb = rng.standard_normal((E, N)).astype(np.float32)
    for b in (None, sb):
        y = np.empty((T, N), np.float32)
        lib.onpu_moe_sum(fp(o), T, k, N, ip(sids), fp(w), None if b is None else fp(b), fp(y))
        assert np.allclose(y, orc.moe_sum(o, sids, w, b), rtol=1e-5, atol=1e-5)

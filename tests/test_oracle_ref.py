"""The oracle's restatements of the reference's CPU helpers against the reference itself: the
reference's llama/ggml-opennpu/onpu_cpu.cpp compiled from its own source with its own flags
(oracle/Makefile `ref`, output in oracle/_ref/, never committed). Functions pinned here:
orc_silu_mul / orc_gptoss_act (onpu_moe_act, onpu_cpu.cpp:233-256), orc_moe_sum (onpu_moe_sum,
:259-274), orc_attn_step (onpu_attn_step / _bf16, :180-229) and orc_gemv_i8 (onpu_gemv_i8,
:276-299).

The reference build contracts multiply-adds and vectorises its reductions (-O3 -march=native
-fopenmp-simd), the oracle rounds every operation as written, so the comparison is to a tolerance
of a few fp32 ulps of the result's scale; a dropped term, a wrong sign or a transposed index is
off by orders of magnitude more. Runs where the reference checkout is present (this is a CPU
test: the reference never reaches the GPU box)."""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle.oracle as orc

ROOT = Path(__file__).resolve().parents[1]
REFSRC = Path("/root/reference/llama/ggml-opennpu/onpu_cpu.cpp")
REFLIB = ROOT / "oracle" / "_ref" / "libonpu_cpu_ref.so"


@pytest.fixture(scope="module")
def ref():
    if not REFLIB.exists():
        if not REFSRC.exists():
            pytest.skip("the reference checkout is not on this machine")
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "ref"], check=True)
    L = C.CDLL(str(REFLIB))
    P, I64, I, F = C.c_void_p, C.c_int64, C.c_int, C.c_float
    L.onpu_moe_act.argtypes = [P, I64, I64, P, P, I, F, F, P]
    L.onpu_moe_sum.argtypes = [P, I64, I, I64, P, P, P, P]
    L.onpu_gemv_i8.argtypes = [P, P, I64, I64, P, P]
    L.onpu_attn_step.argtypes = [P, I, I, P, P, I, I64, I64, I64, P, P, F, P]
    L.onpu_attn_step_bf16.argtypes = L.onpu_attn_step.argtypes
    return L


def p(a):
    return None if a is None else a.ctypes.data


def close(got, want, rtol):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
    assert err <= rtol, err
    return err


@pytest.mark.parametrize("act,alpha,limit", [(0, 0.0, 0.0), (1, 1.702, 7.0), (1, 1.0, 2.5)])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_act(ref, act, alpha, limit, bias):
    rng = np.random.default_rng(40 + act + 2 * bias)
    rows, Ng, E = 37, 96, 5
    h = (rng.standard_normal((rows, Ng)) * 4).astype(np.float32)
    ids = rng.integers(0, E, rows).astype(np.int32)
    b = (rng.standard_normal((E, Ng)) * 2).astype(np.float32) if bias else None
    want = np.empty((rows, Ng // 2), np.float32)
    ref.onpu_moe_act(p(h), rows, Ng, p(ids), p(b), act, alpha, limit, p(want))
    hb = h if b is None else h + b[ids]
    got = orc.silu_mul(hb) if act == 0 else orc.gptoss_act(hb, alpha, limit)
    close(got, want, 1e-6)


@pytest.mark.parametrize("bias", [False, True])
def test_moe_sum(ref, bias):
    rng = np.random.default_rng(50 + bias)
    T, k, N, E = 9, 8, 200, 16
    o = rng.standard_normal((T, k, N)).astype(np.float32)
    ids = rng.integers(0, E, (T, k)).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    b = rng.standard_normal((E, N)).astype(np.float32) if bias else None
    want = np.empty((T, N), np.float32)
    ref.onpu_moe_sum(p(o), T, k, N, p(ids), p(w), p(b), p(want))
    close(orc.moe_sum(o, ids, w, b), want, 1e-6)


@pytest.mark.parametrize("N,K", [(64, 96), (300, 2048), (7, 40)])
def test_gemv_i8(ref, N, K):
    rng = np.random.default_rng(N + K)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = (rng.random(N) * 0.01).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    want = np.empty(N, np.float32)
    ref.onpu_gemv_i8(p(W), p(s), N, K, p(x), p(want))
    # the oracle sums in fp64; the reference in fp32 over 32-wide lanes: ~K * 2^-24 of the scale
    close(orc.gemv_i8(W, s, x), want, 2e-6 * np.sqrt(K))


@pytest.mark.parametrize("Hq,Hkv,D,S", [(8, 2, 64, 50), (32, 8, 128, 300), (4, 4, 32, 7)])
@pytest.mark.parametrize("kv", ["f32", "bf16"])
@pytest.mark.parametrize("extras", [False, True])
def test_attn_step(ref, Hq, Hkv, D, S, kv, extras):
    rng = np.random.default_rng(Hq * 7 + S + (kv == "bf16") + 3 * extras)
    q = rng.standard_normal((Hq, D)).astype(np.float32)
    Kf = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    Vf = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    if kv == "bf16":
        K, V = orc.f2bf_np(Kf).reshape(Kf.shape), orc.f2bf_np(Vf).reshape(Vf.shape)
    else:
        K, V = Kf, Vf
    mask = sinks = None
    if extras:
        mask = np.where(rng.random(S) < 0.3, -np.inf, rng.standard_normal(S)).astype(np.float32)
        mask[0] = 0.0
        sinks = rng.standard_normal(Hq).astype(np.float32)
    scale = D ** -0.5
    want = np.empty((Hq, D), np.float32)
    fn = ref.onpu_attn_step_bf16 if kv == "bf16" else ref.onpu_attn_step
    fn(p(q), Hq, D, p(K), p(V), Hkv, S, S * D, D, p(mask), p(sinks), scale, p(want))
    close(orc.attn_step(q, K, V, mask, sinks, scale), want, 2e-6)

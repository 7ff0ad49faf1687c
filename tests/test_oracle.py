"""Pins the oracle (oracle/oracle.c, oracle/oracle.py) before it is trusted as the checker.

Each oracle routine is checked against something other than its own formula: a library routine
(torch / numpy conversions, softmax, top-k, silu, float64 matmul), the committed golden fixtures
(tests/golden/golden.npz, built from the format definitions with numpy alone), closed forms on
hand-built inputs, invariants, or brute force on tiny inputs. The cases are chosen so that a
plausible mistake fails one of them: a swapped nibble order, a missing -8 offset, a min added
before the product, a dropped scale, a transposed operand, a tie broken the wrong way.
CPU only.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from opennpu_amd import synthetic as syn
from oracle import oracle as orc

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")
FMTS = (orc.FMT_Q4NX, orc.FMT_Q4S, orc.FMT_G128S, orc.FMT_Q4_0)


def torch_bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ bf16 / fp16 conversions
def test_f2bf_matches_torch_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32),
        # exact ties between two bf16 values (low 16 bits = 0x8000), both parities of the kept bit
        (rng.integers(0, 1 << 15, 4000, dtype=np.uint32) << 17 | 0x8000).view(np.float32),
        (rng.integers(0, 1 << 15, 4000, dtype=np.uint32) << 17 | 0x18000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4028235e38, 1.1754942e-38], np.float32),
    ]).astype(np.float32)
    x = x[~np.isnan(x)]                  # NaN payloads differ between conversions; checked below
    want = torch_bf16_bits(x)
    got_c = np.array([orc.lib().orc_f2bf(float(v)) for v in x[:3000]], np.uint16)
    assert np.array_equal(got_c, want[:3000])
    assert np.array_equal(orc.f2bf(x), want)
    assert np.array_equal(orc.f2bf_np(x), want)
    # NaN stays NaN
    nb = orc.f2bf(np.array([np.nan], np.float32))[0]
    assert (nb & 0x7F80) == 0x7F80 and (nb & 0x7F) != 0


def test_bf2f_is_exact_widening():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = orc.bf2f(h)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.isnan(got[np.isnan(want)]).all()


def test_h2f_matches_numpy_float16():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_h2f(int(v)) for v in h], np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.isnan(got[~fin]).all()


# ------------------------------------------------------------------ unpack / dequant
@pytest.mark.parametrize("fmt", FMTS)
def test_golden_unpack_and_dequant(fmt):
    N, K, _ = GOLD[f"f{fmt}_shape"]
    st = GOLD[f"f{fmt}_st"]
    assert st.size == orc.stage_bytes(fmt, N, K)
    assert np.array_equal(orc.unpack(fmt, st, N, K), GOLD[f"f{fmt}_u"])
    assert np.array_equal(orc.dequant(fmt, st, N, K).view(np.uint32), GOLD[f"f{fmt}_w"].view(np.uint32))
    # bf16 of the dequantized weight = torch's rounding of the fp32 weight
    assert np.array_equal(orc.dequant_bf16(fmt, st, N, K), torch_bf16_bits(GOLD[f"f{fmt}_w"]))


def test_unpack_exhaustive_bytes():
    """every byte value at every position of a row: even k <- low nibble, odd k <- high nibble"""
    N, K = 2, 512
    codes = np.concatenate([np.arange(256, dtype=np.uint8), np.arange(256, dtype=np.uint8)[::-1]])
    scales = orc.f2bf(np.full(N * K // 32, 1.0, np.float32))
    st = np.concatenate([codes, scales.view(np.uint8)])
    u = orc.unpack(orc.FMT_Q4S, st, N, K).reshape(-1)
    assert np.array_equal(u[0::2], codes & 15) and np.array_equal(u[1::2], codes >> 4)
    # unit scale: w = u - 8 exactly, spanning -8 .. 7
    w = orc.dequant(orc.FMT_Q4S, st, N, K).reshape(-1)
    assert np.array_equal(w, u.astype(np.float32) - 8)
    assert w.min() == -8 and w.max() == 7


def test_q4_0_hand_built_block():
    """GGUF block_q4_0: fp16 d, then qs[16]; element j <- qs[j] & 15, element j + 16 <- qs[j] >> 4"""
    d = np.float16(0.25)
    qs = np.array([0x10 * ((j + 3) % 16) + j for j in range(16)], np.uint8)
    blk = np.concatenate([np.frombuffer(d.tobytes(), np.uint8), qs])
    w = orc.dequant(orc.FMT_Q4_0, blk, 1, 32)[0]
    want = [(j - 8) * 0.25 for j in range(16)] + [(((j + 3) % 16) - 8) * 0.25 for j in range(16)]
    assert w.tolist() == want


def test_q4nx_min_is_added_after_the_rounded_product():
    """w = fp32(u * s) + m, with s and m bf16: a case where a fused or reordered sum differs"""
    s, m = np.float32(1.0 + 2 ** -7), np.float32(-(2 ** 4))        # both exact in bf16
    u = np.arange(16, dtype=np.uint8)
    st = np.concatenate([(u[0::2] | (u[1::2] << 4)).astype(np.uint8), np.zeros(8, np.uint8),
                         orc.f2bf(np.array([s], np.float32)).view(np.uint8),
                         orc.f2bf(np.array([m], np.float32)).view(np.uint8)])
    u32 = np.concatenate([u, np.zeros(16, np.uint8)])
    w = orc.dequant(orc.FMT_Q4NX, st, 1, 32)[0]
    want = (u32.astype(np.float32) * s).astype(np.float32) + m
    assert np.array_equal(w, want)
    assert w[0] == -16.0 and w[15] == np.float32(15 * s) + m


# ------------------------------------------------------------------ matmul
@pytest.mark.parametrize("fmt", FMTS)
def test_golden_qmm(fmt):
    N, K, M = GOLD[f"f{fmt}_shape"]
    y = orc.qmm(fmt, GOLD[f"f{fmt}_st"], N, K, GOLD[f"f{fmt}_x"])
    ref = GOLD[f"f{fmt}_y"]
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
    # row slices agree with the whole
    assert np.array_equal(orc.qmm(fmt, GOLD[f"f{fmt}_st"], N, K, GOLD[f"f{fmt}_x"], 3, N - 2), y[:, 3:N - 2])


def test_qmm_bf16w_equals_numpy_on_rounded_weights():
    fmt = orc.FMT_G128S
    N, K, M = GOLD[f"f{fmt}_shape"]
    wb = orc.bf2f(torch_bf16_bits(GOLD[f"f{fmt}_w"])).astype(np.float64)
    ref = orc.bf2f(GOLD[f"f{fmt}_x"]).astype(np.float64) @ wb.T
    y = orc.qmm(fmt, GOLD[f"f{fmt}_st"], N, K, GOLD[f"f{fmt}_x"], bf16w=True)
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())


def test_matmul_f64_brute_force_and_orientation():
    rng = np.random.default_rng(3)
    W = rng.standard_normal((7, 5)).astype(np.float32)
    x = rng.standard_normal((3, 5))
    y = orc.matmul_f64(W, x)
    for m in range(3):
        for n in range(7):
            assert abs(y[m, n] - sum(float(x[m, k]) * float(W[n, k]) for k in range(5))) < 1e-12
    # linearity in x
    x2 = rng.standard_normal((3, 5))
    assert np.allclose(orc.matmul_f64(W, 2 * x + x2), 2 * y + orc.matmul_f64(W, x2), atol=1e-12)


def test_qmm_f32_torch_pattern():
    fmt = orc.FMT_G128S
    N, K, M = GOLD[f"f{fmt}_shape"]
    y = orc.qmm_f32_torch(fmt, GOLD[f"f{fmt}_st"], N, K, GOLD[f"f{fmt}_x"])
    ref = GOLD[f"f{fmt}_y"]
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


# ------------------------------------------------------------------ MoE pieces
def test_route_golden_and_torch():
    lg = GOLD["route_logits"]
    ids, w = orc.route(lg, 8)
    assert np.array_equal(ids, GOLD["route_ids"])
    assert np.allclose(w, GOLD["route_w"], rtol=1e-6, atol=0)
    assert ids[0, 0] == 3 and ids[0, 1] == 5                     # the tie goes to the lower id
    # torch softmax + topk on distinct logits; renormalised weights sum to 1
    t = torch.from_numpy(lg[1:]).double()
    p = torch.softmax(t, dim=1)
    tw, ti = torch.topk(p, 8, dim=1)
    assert np.array_equal(ids[1:], ti.numpy())
    assert np.allclose(w[1:], (tw / tw.sum(1, keepdim=True)).numpy(), rtol=1e-6)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)
    # no renorm: the raw probabilities
    _, w0 = orc.route(lg[1:], 8, renorm=False)
    assert np.allclose(w0, tw.numpy(), rtol=1e-6)


def test_silu_mul_matches_torch():
    rng = np.random.default_rng(4)
    h = (rng.standard_normal((5, 64)) * 4).astype(np.float32)
    a = orc.silu_mul(h)
    t = torch.from_numpy(h)
    want = (torch.nn.functional.silu(t[:, :32]) * t[:, 32:]).numpy()
    assert np.allclose(a, want, rtol=2e-6, atol=1e-6)


def test_gptoss_act_clamps_and_interleaves():
    alpha, limit = 1.702, 7.0
    h = np.array([[1.0, 2.0, 9.0, -9.0, -3.0, 8.0]], np.float32)     # pairs (gate, up), interleaved
    a = orc.gptoss_act(h, alpha, limit)[0]
    g = torch.tensor([1.0, 7.0, -3.0], dtype=torch.float64)           # gate clamped above only
    u = torch.tensor([2.0, -7.0, 7.0], dtype=torch.float64)           # up clamped both ways
    want = ((u + 1) * g * torch.sigmoid(alpha * g)).numpy()
    assert np.allclose(a, want, rtol=1e-6)


def test_moe_sum_matches_numpy():
    rng = np.random.default_rng(5)
    T, k, N, E = 3, 4, 16, 6
    o = rng.standard_normal((T, k, N)).astype(np.float32)
    ids = rng.integers(0, E, (T, k)).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    b = rng.standard_normal((E, N)).astype(np.float32)
    want = np.einsum("tk,tkn->tn", w.astype(np.float64), o.astype(np.float64) + b[ids].astype(np.float64))
    assert np.allclose(orc.moe_sum(o, ids, w, b), want, rtol=1e-5, atol=1e-5)
    want0 = np.einsum("tk,tkn->tn", w.astype(np.float64), o.astype(np.float64))
    assert np.allclose(orc.moe_sum(o, ids, w), want0, rtol=1e-5, atol=1e-5)


def test_argmax_golden_first_maximum():
    assert np.array_equal(orc.argmax(GOLD["argmax_in"]), GOLD["argmax_out"])
    assert orc.argmax(GOLD["argmax_in"])[1] == 10


def test_moe_layer_against_dense_composition():
    """the routed layer = sum over slots of w * down(bf16(silu(gate) * up)) with dense numpy products"""
    rng = np.random.default_rng(6)
    E, H, I, T, k = 4, 128, 128, 3, 2
    gu = [syn.weights(orc.FMT_G128S, 2 * I, H, 50 + e) for e in range(E)]
    dn = [syn.weights(orc.FMT_G128S, H, I, 60 + e) for e in range(E)]
    x = orc.f2bf(rng.standard_normal((T, H)).astype(np.float32))
    ids, w = orc.route(rng.standard_normal((T, E)).astype(np.float32), k)
    y = orc.moe_layer(orc.FMT_G128S, gu, dn, E, H, I, x, ids, w)
    xf = orc.bf2f(x).astype(np.float64)
    want = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            h = (xf[t] @ orc.dequant(orc.FMT_G128S, gu[e], 2 * I, H).astype(np.float64).T).astype(np.float32)
            g, u = torch.from_numpy(h[:I]), torch.from_numpy(h[I:])
            a = orc.bf2f(torch_bf16_bits((torch.nn.functional.silu(g) * u).numpy())).astype(np.float64)
            want[t] += float(w[t, j]) * (a @ orc.dequant(orc.FMT_G128S, dn[e], H, I).astype(np.float64).T)
    assert np.abs(y - want).max() <= 1e-3 * np.abs(want).max()


# ------------------------------------------------------------------ geometry
@pytest.mark.parametrize("N,K,ncols,want", [
    (4096, 4096, 8, (4, 2, 4, 8, None, None, None, 10485760)),
    (6144, 4096, 8, (4, 2, 6, None, None, None, None, None)),
    (24576, 4096, 8, (4, 2, 24, None, None, None, None, None)),
    (151936, 4096, 8, (4, 2, 149, 8, None, None, None, None)),
    (4096, 12288, 8, (1, 8, 16, 6, None, None, None, None)),
    (1536, 2048, 1, (1, 1, 6, 8, None, None, None, None)),
    (2048, 768, 1, (1, 1, 8, 3, None, None, None, None)),
])
def test_geometry_known_values(N, K, ncols, want):
    """the values the reference's Mat formula gives at the benchmark shapes (worked by hand from
    model.py:151-187 for the survey of the reference)"""
    got = orc.geometry(N, K, ncols, 0)
    for g, w in zip(got, want):
        if w is not None:
            assert g == w, (got, want)


# ------------------------------------------------------------------ search quantizers (invariants only)
def test_quant_sym32_exact_grid_round_trip():
    """groups that are exactly v * d (d a power of two, v spanning -8..7) come back exactly;
    the exact scale choice on general inputs stays parity unpinned"""
    rng = np.random.default_rng(7)
    for t in range(50):
        d = np.float32(2.0 ** rng.integers(-12, 2))
        v = rng.integers(-8, 8, 32)
        v[rng.integers(0, 32)] = -8
        q, db = orc.quant_sym32((v * d).astype(np.float32))
        assert orc.bf2f(np.array([db], np.uint16))[0] == d
        assert np.array_equal(q.astype(int), v + 8)
    q, db = orc.quant_sym32(np.zeros(32, np.float32))
    assert (q == 8).all()


def test_quant_asym32_exact_grid_round_trip():
    rng = np.random.default_rng(8)
    for t in range(50):
        s = np.float32(2.0 ** rng.integers(-10, 0))
        m = np.float32(-(2.0 ** rng.integers(-4, 3)))
        u = rng.integers(0, 16, 32)
        u[0], u[1] = 0, 15
        q, sb, mb = orc.quant_asym32((u * s + m).astype(np.float32))
        sf, mf = orc.bf2f(np.array([sb, mb], np.uint16))
        assert np.array_equal((q * sf + mf).astype(np.float32), (u * s + m).astype(np.float32))


def test_oracle_rejects_shapes_outside_the_format():
    with pytest.raises(ValueError):
        orc.dequant(orc.FMT_G128S, np.zeros(64 * 32, np.uint8), 64, 64)      # K not a multiple of 128
    with pytest.raises(ValueError):
        orc.qmm(orc.FMT_Q4S, np.zeros(10, np.uint8), 4, 64, np.zeros((1, 64), np.uint16))   # short buffer

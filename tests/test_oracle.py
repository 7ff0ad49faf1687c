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


# ------------------------------------------------------------------ search quantizers
def test_quant_sym32_exact_grid_round_trip():
    """groups that are exactly v * d (d a power of two, v spanning -8..7) come back exactly (the
    exact scale choice on general inputs is pinned against the reference's own build in
    tests/test_quant_ref.py)"""
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


def _groups(rng, n, g):
    """groups of g weights with the shapes a quantizer meets: Gaussian, heavy-tailed, one outlier,
    repeated magnitudes of both signs (ties for the largest |x|), a few exact zeros"""
    out = []
    for t in range(n):
        kind = t % 5
        if kind == 0:
            x = rng.standard_normal(g) * 0.02
        elif kind == 1:
            x = rng.standard_t(2, g) * 0.01
        elif kind == 2:
            x = rng.standard_normal(g) * 0.01
            x[rng.integers(0, g)] = rng.choice([-1, 1]) * 0.3
        elif kind == 3:
            x = rng.choice([-3, -1, 0, 2, 3], g) * 0.004
        else:
            x = rng.standard_normal(g) * 0.05
            x[rng.integers(0, g, 3)] = 0.0
        out.append(x.astype(np.float32))
    return out


def _bf_times(b, j):
    """bf16 bits of 2^j times the bf16 value b (exact away from under- and overflow)"""
    return int(orc.f2bf(np.array([orc.bf2f(np.array([b], np.uint16))[0] * np.float32(2.0 ** j)], np.float32))[0])


@pytest.mark.parametrize("g", [32, 128])
def test_quant_sym_sign_symmetry(g):
    """q4s / g128s: quantizing -x gives the same codes and the negated scale, bit for bit (every
    step of the search is odd in x: the signed absmax, x / d, the refit sum(v x) / sum(v v) and bf16
    rounding; the squared errors are even). A quantizer that took |max|, clamped asymmetrically in
    the wrong direction or biased a refit would break it."""
    rng = np.random.default_rng(60 + g)
    fn = orc.quant_sym32 if g == 32 else orc.quant_sym
    for x in _groups(rng, 400, g):
        q, d = fn(x)
        qn, dn = fn(-x)
        assert np.array_equal(q, qn) and dn == d ^ 0x8000, (x, q, qn, hex(d), hex(dn))


@pytest.mark.parametrize("g", [32, 128])
@pytest.mark.parametrize("j", [-5, -1, 1, 3])
def test_quant_sym_power_of_two_equivariance(g, j):
    """q4s / g128s: quant(2^j x) = (codes, 2^j d) exactly: each step scales exactly by a power of two
    away from under- and overflow, so an absolute epsilon, a constant added to a refit or a scale
    rounded before scaling would break it"""
    rng = np.random.default_rng(70 + g + j)
    fn = orc.quant_sym32 if g == 32 else orc.quant_sym
    for x in _groups(rng, 300, g):
        q, d = fn(x)
        q2, d2 = fn((x * np.float32(2.0 ** j)).astype(np.float32))
        assert np.array_equal(q, q2) and d2 == _bf_times(d, j), (j, hex(d), hex(d2))


@pytest.mark.parametrize("j", [-4, -1, 2, 5])
def test_quant_asym32_power_of_two_equivariance(j):
    """q4nx: quant(2^j x) = (codes, 2^j s, 2^j m) exactly (the stretched grids divide by the range,
    the least-squares refit is homogeneous of degree one in x)"""
    rng = np.random.default_rng(80 + j)
    for x in _groups(rng, 300, 32):
        q, s, m = orc.quant_asym32(x)
        q2, s2, m2 = orc.quant_asym32((x * np.float32(2.0 ** j)).astype(np.float32))
        assert np.array_equal(q, q2), j
        assert s2 == _bf_times(s, j) and m2 == _bf_times(m, j), (j, hex(s), hex(s2), hex(m), hex(m2))


def test_quant_q4_0_sign_and_scale_symmetry():
    """ggml's Q4_0 rule: -x gives the same codes and -d; 2^j x gives the same codes and 2^j d"""
    rng = np.random.default_rng(90)
    for x in _groups(rng, 300, 32):
        q, d = orc.quant_q4_0(x)
        qn, dn = orc.quant_q4_0(-x)
        assert np.array_equal(q, qn) and dn == d ^ 0x8000
        for j in (-2, 3):
            q2, d2 = orc.quant_q4_0((x * np.float32(2.0 ** j)).astype(np.float32))
            want = np.array([np.array([d], np.uint16).view(np.float16)[0] * np.float16(2.0 ** j)], np.float16)
            assert np.array_equal(q, q2) and d2 == int(want.view(np.uint16)[0])


def test_quant_q4_0_half_way_inputs_truncate():
    """ggml computes a code as (int8_t)(x / d + 8.5) with d = max / -8: a truncation, so an input
    exactly half-way between two grid points rounds up (x / d = k + 1/2 -> k + 9), where a
    round-to-nearest-even quantizer gives k + 8 for even k. With max = -8 (d = 1) the products are
    exact: x = 0.5 -> 9, 2.5 -> 11, -1.5 -> 7, -7.5 -> 1, 6.5 -> 15 (rint: 8, 10, 6, 0, 14)"""
    x = np.zeros(32, np.float32)
    x[0] = -8.0
    halves = [0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -7.5, 6.5, 4.5]
    x[1:1 + len(halves)] = halves
    q, dh = orc.quant_q4_0(x)
    assert np.array([dh], np.uint16).view(np.float16)[0] == 1.0
    want = [min(15, int(np.floor(h + 8.5))) for h in halves]
    assert list(q[1:1 + len(halves)]) == want
    assert (q[1], q[3], q[6], q[8], q[9]) == (9, 11, 7, 1, 15)     # round-half-even: 8, 10, 6, 0, 14
    assert q[0] == 0 and (q[1 + len(halves):] == 8).all()


def test_oracle_rejects_shapes_outside_the_format():
    with pytest.raises(ValueError):
        orc.dequant(orc.FMT_G128S, np.zeros(64 * 32, np.uint8), 64, 64)      # K not a multiple of 128
    with pytest.raises(ValueError):
        orc.qmm(orc.FMT_Q4S, np.zeros(10, np.uint8), 4, 64, np.zeros((1, 64), np.uint16))   # short buffer


# ------------------------------------------------------------------ GGUF codecs and the g128s quantizer
def test_f2h_matches_numpy_float16():
    """fp32 -> fp16 RNE against numpy's own conversion, over normal, subnormal, tie and overflow
    values"""
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 5, 4000),
                        np.float32(2.0) ** np.arange(-26, 17),
                        [65504, 65519.99, 65520, -65520, 0.0, -0.0, 2.0 ** -25, 3 * 2.0 ** -25,
                         1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f2h(x), want)


def test_quant_sym_128_exact_grid_round_trip():
    """the g128s quantizer (quant_sym over 128): exact grids v * d come back exactly"""
    rng = np.random.default_rng(12)
    for t in range(30):
        d = np.float32(2.0 ** rng.integers(-12, 2))
        v = rng.integers(-8, 8, 128)
        v[rng.integers(0, 128)] = -8
        q, db = orc.quant_sym((v * d).astype(np.float32))
        assert orc.bf2f(np.array([db], np.uint16))[0] == d
        assert np.array_equal(q.astype(int), v + 8)


def test_quant_q4_0_closed_form():
    """ggml's Q4_0 rule: with the largest magnitude -8 d (d a power of two) the codes are v + 8 and
    d comes back exactly; with it +8 d the scale flips sign and (u - 8) d' still reproduces x; all
    zeros give d = -0 and codes 8"""
    rng = np.random.default_rng(13)
    for t in range(40):
        d = np.float32(2.0 ** rng.integers(-14, 3))
        v = rng.integers(-7, 8, 32)
        i = rng.integers(0, 32)
        v[i] = -8 if t % 2 == 0 else 8
        x = (v * d).astype(np.float32)
        q, dh = orc.quant_q4_0(x)
        dd = np.float32(np.array([dh], np.uint16).view(np.float16)[0])
        assert abs(dd) == d
        assert np.array_equal(((q.astype(np.float32) - 8) * dd).astype(np.float32), x)
        if t % 2 == 0:
            assert np.array_equal(q.astype(int), v + 8)
    q, dh = orc.quant_q4_0(np.zeros(32, np.float32))
    assert dh == 0x8000 and (q == 8).all()            # d = 0 / -8 = -0


def _q4k_block(rng, d, dmin, sv, mv, nib):
    """one GGUF Q4_K super-block (ggml's block_q4_K): fp16 d, dmin, 6-bit (scale, min) pairs of the
    8 sub-blocks packed into 12 bytes as ggml's quantize_row_q4_K packs them, codes [8][32]"""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    sc = np.zeros(12, np.uint8)
    for j in range(4):
        sc[j] = sv[j] | ((sv[j + 4] >> 4) << 6)
        sc[j + 4] = mv[j] | ((mv[j + 4] >> 4) << 6)
        sc[j + 8] = (sv[j + 4] & 0xF) | ((mv[j + 4] & 0xF) << 4)
    b[4:16] = sc
    for c in range(4):                          # sub-blocks 2c (low nibbles) and 2c + 1 (high)
        b[16 + 32 * c:48 + 32 * c] = nib[2 * c] | (nib[2 * c + 1] << 4)
    return b


def test_transcode_q4k_exact_blocks():
    """d = 1, dmin = 1/2 and integer 6-bit scales: every sub-block's scale d sc and min -dmin mn
    are exact in bf16, so the transcode keeps them, the codes are the sub-block's nibbles and the
    q4nx weights equal the Q4_K weights d sc u - dmin mn exactly"""
    rng = np.random.default_rng(14)
    N, K = 3, 512
    blocks, want_u, want_w = [], np.zeros((N, K), np.uint8), np.zeros((N, K), np.float64)
    for r in range(N):
        for sb in range(K // 256):
            sv, mv = rng.integers(1, 64, 8), rng.integers(1, 64, 8)
            nib = rng.integers(0, 16, (8, 32)).astype(np.uint8)
            blocks.append(_q4k_block(rng, 1.0, 0.5, sv, mv, nib))
            for sub in range(8):
                k0 = 256 * sb + 32 * sub
                want_u[r, k0:k0 + 32] = nib[sub]
                want_w[r, k0:k0 + 32] = 1.0 * sv[sub] * nib[sub] - 0.5 * mv[sub]
    q, s, m = orc.transcode_q4k(np.concatenate(blocks), N, K)
    assert np.array_equal(q, want_u)
    w = q.astype(np.float64) * np.repeat(orc.bf2f(s), 32, axis=1) + np.repeat(orc.bf2f(m), 32, axis=1)
    assert np.array_equal(w, want_w)


def test_transcode_q4k_zero_scale_takes_the_first_tie():
    """a zero scale (sc = 0) or min (mn = 0): the neighbours +-2^-133 of bf16 zero reproduce the
    weights equally well in fp32 (u * 2^-133 is absorbed), and the search keeps the first minimum
    in its order (step -1 first), so the stored value is -2^-133 (0x8001); the weights it gives
    equal the exact ones in fp32, but for an all-zero sub-block, which keeps subnormal residues"""
    rng = np.random.default_rng(17)
    sv = np.array([0, 9, 0, 3, 7, 0, 5, 2])
    mv = np.array([4, 0, 0, 6, 0, 8, 1, 3])
    nib = rng.integers(0, 16, (8, 32)).astype(np.uint8)
    nib[:, 0] = 1                                   # not all codes zero
    q, s, m = orc.transcode_q4k(_q4k_block(rng, 1.0, 0.5, sv, mv, nib), 1, 256)
    for sub in range(8):
        if sv[sub] == 0:
            assert s[0, sub] == 0x8001
        if mv[sub] == 0:
            assert m[0, sub] == 0x8001
        u = q[0, 32 * sub:32 * sub + 32].astype(np.float32)
        w = (u * orc.bf2f(s[0, sub:sub + 1])[0]).astype(np.float32) + orc.bf2f(m[0, sub:sub + 1])[0]
        want = (u * np.float32(sv[sub])).astype(np.float32) + np.float32(-0.5 * mv[sub])
        if sv[sub] == 0 and mv[sub] == 0:               # all weights zero: a subnormal residue remains
            assert np.abs(w).max() < 2.0 ** -120
        else:
            assert np.array_equal(w[u > 0], want[u > 0])


def test_transcode_q4k_picks_the_best_neighbour():
    """general fp16 d, dmin: the chosen (s, m) is one of the 3 x 3 bf16 neighbours of the rounded
    exact scale and min, and no neighbour reproduces the exact weights better (fp64 error, with
    fp32-accumulation slack)"""
    rng = np.random.default_rng(15)
    N, K = 4, 256
    blocks, exact = [], []
    for r in range(N):
        sv, mv = rng.integers(1, 64, 8), rng.integers(0, 64, 8)
        nib = rng.integers(0, 16, (8, 32)).astype(np.uint8)
        d, dmin = np.float16(rng.uniform(1e-4, 2e-2)), np.float16(rng.uniform(0, 1e-2))
        blocks.append(_q4k_block(rng, d, dmin, sv, mv, nib))
        exact.append((np.float32(d) * sv.astype(np.float32), -np.float32(dmin) * mv.astype(np.float32), nib))
    q, s, m = orc.transcode_q4k(np.concatenate(blocks), N, K)

    def step(h, dirn):
        f = orc.bf2f(np.array([h], np.uint16))[0]
        if f == 0:
            return 0x0001 if dirn > 0 else 0x8001
        return h + 1 if (f > 0) == (dirn > 0) else h - 1

    for r in range(N):
        S, M, nib = exact[r]
        for sub in range(8):
            u = nib[sub].astype(np.float64)
            s0, m0 = int(orc.f2bf(np.array([S[sub]]))[0]), int(orc.f2bf(np.array([M[sub]]))[0])
            cands = [(step(s0, a) if a else s0, step(m0, b) if b else m0) for a in (-1, 0, 1) for b in (-1, 0, 1)]
            err = lambda c: float(np.sum((u * orc.bf2f(np.array([c[0]], np.uint16))[0]
                                          + orc.bf2f(np.array([c[1]], np.uint16))[0]
                                          - (u * np.float64(S[sub]) + np.float64(M[sub]))) ** 2))
            got = (int(s[r, sub]), int(m[r, sub]))
            assert got in cands
            best = min(err(c) for c in cands)
            assert err(got) <= best * (1 + 1e-4) + 1e-30
            assert np.array_equal(q[r, 32 * sub:32 * sub + 32], nib[sub])


def test_quantize_staging_layout():
    """orc.quantize lays the per-group quantizers' outputs out as the staging layout: codes two per
    byte (low nibble = even k), then scales (then mins); Q4_0 as GGUF blocks"""
    rng = np.random.default_rng(16)
    N, K = 5, 256
    W = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    for fmt in (orc.FMT_Q4NX, orc.FMT_Q4S, orc.FMT_G128S, orc.FMT_Q4_0):
        st = orc.quantize(fmt, W)
        u = orc.unpack(fmt, st, N, K)
        G = orc.group(fmt)
        for r in range(N):
            for g in range(K // G):
                x = W[r, G * g:G * g + G]
                if fmt == orc.FMT_Q4NX:
                    q, sb, mb = orc.quant_asym32(x)
                elif fmt == orc.FMT_Q4_0:
                    q, sb = orc.quant_q4_0(x)
                else:
                    q, sb = orc.quant_sym(x)
                assert np.array_equal(u[r, G * g:G * g + G], q), (fmt, r, g)
                if fmt == orc.FMT_Q4_0:
                    assert st[(r * (K // 32) + g) * 18:][:2].view(np.uint16)[0] == sb
                else:
                    assert st[N * K // 2:].view(np.uint16)[r * (K // G) + g] == sb
                    if fmt == orc.FMT_Q4NX:
                        assert st[N * K // 2 + N * (K // G) * 2:].view(np.uint16)[r * (K // G) + g] == mb


# ------------------------------------------------------------------ decode attention
@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_attn_step_against_torch_float64(kv):
    """GQA decode attention with an additive mask (some -inf) and per-head sinks, against a float64
    torch softmax with the sink as an extra logit without a value"""
    import torch
    rng = np.random.default_rng(90)
    Hq, Hkv, S, D = 8, 2, 300, 64
    q = rng.standard_normal((Hq, D)).astype(np.float32)
    Kf = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    Vf = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    mask = np.where(rng.random(S) < 0.1, -np.inf, rng.standard_normal(S) * 0.1).astype(np.float32)
    sinks = rng.standard_normal(Hq).astype(np.float32)
    if kv == "bf16":
        K, V = orc.f2bf_np(Kf), orc.f2bf_np(Vf)
        Kf, Vf = orc.bf2f(K).reshape(Kf.shape), orc.bf2f(V).reshape(Vf.shape)
    else:
        K, V = Kf, Vf
    for sk in (None, sinks):
        out = orc.attn_step(q, K, V, mask, sk)
        qt = torch.from_numpy(q).double().reshape(Hkv, Hq // Hkv, D)
        s = torch.einsum("grd,gsd->grs", qt, torch.from_numpy(Kf).double()) * D ** -0.5 + torch.from_numpy(mask).double()
        if sk is not None:
            s = torch.cat([s, torch.from_numpy(sk).double().reshape(Hkv, Hq // Hkv, 1)], -1)
        p = torch.softmax(s, -1)[..., :S]
        ref = torch.einsum("grs,gsd->grd", p, torch.from_numpy(Vf).double()).reshape(Hq, D).numpy()
        assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


def test_gemv_i8_against_numpy():
    rng = np.random.default_rng(95)
    W = rng.integers(-128, 128, (37, 300)).astype(np.int8)
    s = rng.uniform(1e-3, 2e-2, 37).astype(np.float32)
    x = rng.standard_normal(300).astype(np.float32)
    want = (W.astype(np.float64) @ x.astype(np.float64)) * s.astype(np.float64)
    assert np.allclose(orc.gemv_i8(W, s, x), want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ Gated DeltaNet decode step
def _gdn_inputs(rng, Hk=2, Hv=4, Dk=16, Dv=8, H=24, Kc=4, L=3):
    C = 2 * Hk * Dk + Hv * Dv
    return dict(x=rng.standard_normal(H), qkv=rng.standard_normal(C), z=rng.standard_normal(Hv * Dv),
                Wb=rng.standard_normal((Hv, H)) * 0.1, Wa=rng.standard_normal((Hv, H)) * 0.1,
                conv_w=rng.standard_normal((C, Kc)) * 0.5, conv_state=rng.standard_normal((C, L)),
                A_log=rng.standard_normal(Hv) * 0.5, dt_bias=rng.standard_normal(Hv) * 0.5,
                norm_w=rng.uniform(0.5, 1.5, Dv), eps=1e-6, S=rng.standard_normal((Hv, Dk, Dv)) * 0.1,
                Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv)


def _silu(v):
    return v / (1 + np.exp(-v))


def test_gdn_conv_state_shifts_and_delta_kernel():
    """the conv state shifts by one and takes qkv; with a unit last tap and zero others, the conv
    output is silu(qkv), which the delta-rule checks below rely on"""
    rng = np.random.default_rng(100)
    a = _gdn_inputs(rng)
    out, cs, S = orc.gdn_step(**a)
    assert np.array_equal(cs[:, :-1], a["conv_state"][:, 1:].astype(np.float32))
    assert np.array_equal(cs[:, -1], a["qkv"].astype(np.float32))


def _unit_conv(a):
    w = np.zeros_like(a["conv_w"])
    w[:, -1] = 1.0
    a["conv_w"] = w


def test_gdn_delta_rule_stores_v_for_k():
    """decay 1 (A_log -> -inf) and beta 1 (Wb x = +60): the delta rule S' = S + k (v - S^T k)^T with
    a unit-norm k leaves S'^T k = v for every value head, whatever S was"""
    rng = np.random.default_rng(101)
    a = _gdn_inputs(rng)
    _unit_conv(a)
    a["A_log"][:] = -1e30
    a["Wb"] = np.outer(np.full(a["Hv"], 1.0), a["x"]) * (60.0 / np.dot(a["x"], a["x"]))
    out, cs, S = orc.gdn_step(**a)
    Hk, Hv, Dk, Dv = a["Hk"], a["Hv"], a["Dk"], a["Dv"]
    co = _silu(a["qkv"].astype(np.float64))
    for h in range(Hv):
        kh = h // (Hv // Hk)
        k = co[Hk * Dk + kh * Dk:Hk * Dk + (kh + 1) * Dk]
        k = k / np.sqrt(np.dot(k, k) + 1e-6)
        v = co[2 * Hk * Dk + h * Dv:2 * Hk * Dk + (h + 1) * Dv]
        assert np.allclose(S[h].astype(np.float64).T @ k, v, rtol=1e-4, atol=1e-5)


def test_gdn_zero_state_output_is_normalised_v():
    """zero state, decay 1, beta 1 and q = k: S' = k v^T, o = (q . k) v with q . k = |k|^2 / (|k|^2 +
    1e-6) / sqrt(Dk), so the gated RMSNorm output is norm_w * o / sqrt(mean(o^2) + eps) * silu(z)"""
    rng = np.random.default_rng(102)
    a = _gdn_inputs(rng)
    _unit_conv(a)
    Hk, Hv, Dk, Dv = a["Hk"], a["Hv"], a["Dk"], a["Dv"]
    a["qkv"][:Hk * Dk] = a["qkv"][Hk * Dk:2 * Hk * Dk]          # q = k
    a["S"][:] = 0
    a["A_log"][:] = -1e30
    a["Wb"] = np.outer(np.full(Hv, 1.0), a["x"]) * (60.0 / np.dot(a["x"], a["x"]))
    out, cs, S = orc.gdn_step(**a)
    co = _silu(a["qkv"].astype(np.float64))
    for h in range(Hv):
        kh = h // (Hv // Hk)
        k = co[Hk * Dk + kh * Dk:Hk * Dk + (kh + 1) * Dk]
        c = np.dot(k, k) / (np.dot(k, k) + 1e-6) / np.sqrt(Dk)
        o = c * co[2 * Hk * Dk + h * Dv:2 * Hk * Dk + (h + 1) * Dv]
        want = a["norm_w"] * o / np.sqrt(np.mean(o * o) + a["eps"]) * _silu(a["z"][h * Dv:(h + 1) * Dv])
        assert np.allclose(out[h * Dv:(h + 1) * Dv], want, rtol=1e-4, atol=1e-5)


def test_gdn_beta_zero_is_pure_decay():
    """beta 0 (Wb x = -60): S' = decay S with decay = exp(-exp(A_log) softplus(Wa x + dt_bias))"""
    rng = np.random.default_rng(103)
    a = _gdn_inputs(rng)
    a["Wb"] = -np.outer(np.full(a["Hv"], 1.0), a["x"]) * (60.0 / np.dot(a["x"], a["x"]))
    out, cs, S = orc.gdn_step(**a)
    ad = a["Wa"] @ a["x"] + a["dt_bias"]
    decay = np.exp(-np.exp(a["A_log"]) * np.log1p(np.exp(ad)))
    assert np.allclose(S, a["S"] * decay[:, None, None], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("fmt", [orc.FMT_G128S, orc.FMT_Q4_0])
@pytest.mark.parametrize("isa", [2, 1, 0])
def test_cpu_baseline_kernel_against_the_oracle(fmt, isa):
    """the benchmark's fused int4 CPU kernel (oracle/cpu_int4.c) against the fp64 oracle product,
    each instruction-set path (AVX-512 where this CPU has it), M from 1 to 8, ragged N"""
    N, K = 131, 1024
    st = syn.weights(fmt, N, K, 3 + fmt)
    for M in (1, 3, 8):
        xb = syn.activations(M, K, 4 + M)
        y, used = orc.cpu_mv(fmt, st, N, K, orc.bf2f(xb).reshape(M, K), threads=2, isa_max=isa)
        assert used <= isa
        assert orc.max_rel_err(y, orc.qmm(fmt, st, N, K, xb)) <= 1e-5, (fmt, isa, M)


def test_argmax_nan_rows_like_numpy():
    """orc_argmax follows numpy's argmax, which the reference calls on the logits
    (npu4/engine.py:358): the first NaN of a row that has one, else the first maximum; ties and
    infinities included"""
    rng = np.random.default_rng(12)
    v = rng.standard_normal((64, 300)).astype(np.float32)
    v[1, 17] = v[1, 200] = np.nan
    v[2, :] = np.nan
    v[3, 299] = np.nan
    v[4, 5] = v[4, 9] = np.inf
    v[5, 0] = np.nan
    v[6, 40] = v[6, 41] = 10.0
    v[7, 3] = -np.inf
    v[7, 250] = np.nan
    v[8:20, rng.integers(0, 300, 12)] = np.nan
    got = orc.argmax(v)
    assert np.array_equal(got, np.argmax(v, axis=1))
    assert list(got[1:8]) == [17, 0, 299, 5, 0, 40, 250]

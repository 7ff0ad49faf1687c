"""GPU parity of the MoE path (router, permutation + grouped products, fused decode FFN) against
the oracle's restatement of reference.py:71-84 (softmax -> top-k -> renorm, dequantized experts,
silu(gate) * up, weighted sum), with the device path's rounding point (act -> bf16)."""
import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import synthetic as syn
from tests.conftest import check_bf16_out, from_torch, to_torch_bf16

pytestmark = pytest.mark.gpu


def check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped, what):
    """Decode (T <= 4) multiplies exact dequantized weights and sums the slots in fp32. The grouped
    prompt path feeds MFMA the bf16 RNE of each weight and returns each expert's rows in bf16, as the
    reference device does, before the fp32 weighted sum. The per-element bound is taken against the
    oracle with the same rounding points; all stay within the stated 1e-2 of the exact oracle."""
    ref = orc.moe_layer(fmt, gu, dn, E, H, I, xb, rid, rw)
    if grouped:
        # an expert row within fp32 rounding of a bf16 rounding boundary may round the other way than
        # the oracle's (one bf16 ulp of that row), so the bound adds 2^-8 sum_j |w_j d_j|
        r, m = orc.moe_layer(fmt, gu, dn, E, H, I, xb, rid, rw, bf16w=True, bf16o=True, mag=True)
        what_g = what + " (bf16 weights, bf16 expert rows)"
        y = np.asarray(y, np.float64)
        scale = np.abs(r).max()
        bad = np.abs(y - r) > 2.0 ** -8 * (np.abs(r) + m) + 2e-4 * scale
        assert not bad.any(), f"{what_g}: {bad.sum()} elements outside the bound; first at {np.argwhere(bad)[0]}"
        assert orc.max_rel_err(y, r) <= 1e-2, what_g
        assert orc.max_rel_err(y, ref) <= 1e-2, what
    else:
        check_bf16_out(y, ref, what=what, floor=2e-4)


def _experts(fmt, E, H, I, seed):
    gu = [syn.weights(fmt, 2 * I, H, seed + 2 * e) for e in range(E)]
    dn = [syn.weights(fmt, H, I, seed + 2 * e + 1) for e in range(E)]
    return gu, dn


def _ffn(fmt, E, H, I, gu, dn):
    from opennpu_amd.device import QFfn
    f = QFfn(E, H, I, fmt)
    f.load(np.concatenate(gu), np.concatenate(dn))
    return f


@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (7, 64, 4), (512, 128, 8), (33, 16, 2)])
def test_route(gpu, T, E, k):
    import torch
    from opennpu_amd.device import QFfn
    lg = syn.logits(T, E, T + E)
    f = QFfn(2, 128, 128, orc.FMT_G128S)          # any handle: routing needs no weights
    try:
        ids, w = f.route(torch.from_numpy(lg).cuda(), k)
        ids, w = ids.cpu().numpy(), w.cpu().numpy()
    finally:
        f.free()
    rid, rw = orc.route(lg, k)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


def test_route_golden(gpu):
    """the committed router fixture (numpy softmax + stable sort), including a tie at the top that
    goes to the lower expert id"""
    import torch
    from pathlib import Path
    from opennpu_amd.device import QFfn
    G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")
    f = QFfn(2, 128, 128, orc.FMT_G128S)
    try:
        ids, w = f.route(torch.from_numpy(G["route_logits"]).cuda(), 8)
        ids, w = ids.cpu().numpy(), w.cpu().numpy()
    finally:
        f.free()
    assert np.array_equal(ids, G["route_ids"])
    np.testing.assert_allclose(w, G["route_w"], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("fmt", [orc.FMT_G128S, orc.FMT_Q4S, orc.FMT_Q4NX])
@pytest.mark.parametrize("T", [1, 3, 8, 40])
def test_moe_ffn_small(gpu, fmt, T):
    """decode (T <= 4: fused gate_up/act + down/slot sum) and grouped (T > 4) paths."""
    import torch
    E, H, I, k = 16, 256, 128, 4
    gu, dn = _experts(fmt, E, H, I, 1000 + T)
    xb = syn.activations(T, H, T)
    rid, rw = orc.route(syn.logits(T, E, 5 + T), k)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        y = f.ffn(to_torch_bf16(xb).reshape(T, H), torch.from_numpy(rid).cuda(), torch.from_numpy(rw).cuda())
        y = from_torch(y)
    finally:
        f.free()
    check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped=T > 4, what=f"moe fmt {fmt} T {T}")


@pytest.mark.parametrize("fmt", [orc.FMT_G128S, orc.FMT_Q4S])
def test_moe_grouped_item_sizes(gpu, fmt):
    """one expert per token with per-expert row counts on both sides of every 16-row block boundary
    and past the 64-row work item (65 = 64 + 1, 130 = 64 + 64 + 2): the grouped GEMM runs 1 to 4 A
    blocks per item and splits an expert's rows into several items."""
    import torch
    counts = [1, 16, 17, 32, 33, 48, 49, 64, 65, 130]
    E, H, I, k = len(counts), 256, 128, 1
    T = sum(counts)
    rng = np.random.default_rng(5)
    rid = rng.permutation(np.repeat(np.arange(E, dtype=np.int32), counts)).reshape(T, k)
    rw = rng.uniform(0.5, 1.0, (T, k)).astype(np.float32)
    gu, dn = _experts(fmt, E, H, I, 4000)
    xb = syn.activations(T, H, 6)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        y = f.ffn(to_torch_bf16(xb).reshape(T, H), torch.from_numpy(rid).cuda(), torch.from_numpy(rw).cuda())
        y = from_torch(y)
    finally:
        f.free()
    check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped=True, what=f"moe item sizes fmt {fmt}")


@pytest.mark.parametrize("fmt", [orc.FMT_Q4S, orc.FMT_Q4NX])
def test_moe_grouped_k_tail(gpu, fmt):
    """grouped products whose K is not a multiple of 128 (H = 288 for gate+up, I = 160 for down):
    the last K block of each reads zeros past K (the grouped GEMM's tail variant)."""
    import torch
    E, H, I, k, T = 8, 288, 160, 2, 40
    gu, dn = _experts(fmt, E, H, I, 5000)
    xb = syn.activations(T, H, 7)
    rid, rw = orc.route(syn.logits(T, E, 8), k)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        y = f.ffn(to_torch_bf16(xb).reshape(T, H), torch.from_numpy(rid).cuda(), torch.from_numpy(rw).cuda())
        y = from_torch(y)
    finally:
        f.free()
    check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped=True, what=f"moe K tail fmt {fmt}")


@pytest.mark.parametrize("T,check_tokens", [(1, 1), (512, 512)])
def test_moe_qwen3_30b_a3b(gpu, T, check_tokens):
    """128 experts, H=2048, I=768, top-8 (router on device), g128s; every token checked."""
    import torch
    E, H, I, k = 128, 2048, 768, 8
    fmt = orc.FMT_G128S
    gu, dn = _experts(fmt, E, H, I, 77)
    xb = syn.activations(T, H, 78)
    lg = syn.logits(T, E, 79)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        ids, w = f.route(torch.from_numpy(lg).cuda(), k)
        y = from_torch(f.ffn(to_torch_bf16(xb).reshape(T, H), ids, w))
        ids, w = ids.cpu().numpy(), w.cpu().numpy()
    finally:
        f.free()
    rid, rw = orc.route(lg, k)
    assert np.array_equal(ids, rid)
    tok = np.random.default_rng(1).choice(T, check_tokens, replace=False)
    check_moe(y[tok], fmt, gu, dn, E, H, I, xb[tok], rid[tok], rw[tok], grouped=T > 4, what=f"qwen3-30b-a3b T {T}")


@pytest.mark.parametrize("fmt,E,H,I,k,T", [(orc.FMT_G128S, 128, 2048, 768, 8, 1), (orc.FMT_Q4S, 64, 512, 256, 4, 3),
                                             (orc.FMT_Q4NX, 24, 384, 160, 6, 4), (orc.FMT_G128S, 16, 256, 128, 16, 2),
                                             (orc.FMT_Q4S, 256, 256, 128, 8, 2)])
def test_moe_decode_routed_gate_up(gpu, fmt, E, H, I, k, T, monkeypatch):
    """decode from logits at T <= 4 (the default path): the gate+up launch routes each workgroup's
    token and writes ids / w, equal to the oracle router; y within the bf16 bound of the oracle layer
    and bit-equal to the router kernel followed by the FFN launches on the same ids / w; graph replays
    give the same bits."""
    import torch
    monkeypatch.delenv("ONPU_MOE_FUSED", raising=False)
    gu, dn = _experts(fmt, E, H, I, 700 + E + T)
    xb = syn.activations(T, H, 701 + T)
    lg = syn.logits(T, E, 702 + k)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        x = to_torch_bf16(xb).reshape(T, H)
        lgd = torch.from_numpy(lg).cuda()
        y, ids, w = f.decode(lgd, x, k)
        i2, w2 = f.route(lgd, k)
        y2 = f.ffn(x, i2, w2)
        torch.cuda.synchronize()
        assert torch.equal(ids, i2) and torch.equal(w, w2), "ids / w differ from the router kernel's"
        assert torch.equal(y, y2), "routed decode differs from router kernel + FFN"
        yg, ig, wg = torch.empty_like(y), torch.empty_like(ids), torch.empty_like(w)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            f.decode(lgd, x, k, out=yg, ids=ig, w=wg)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            f.decode(lgd, x, k, out=yg, ids=ig, w=wg)
        for _ in range(3):
            yg.zero_()
            ig.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(yg, y) and torch.equal(ig, ids) and torch.equal(wg, w), "graph replay differs"
            ye, _, _ = f.decode(lgd, x, k)
            torch.cuda.synchronize()
            assert torch.equal(ye, y), "eager decode after a replay differs"
        ids, w, y = ids.cpu().numpy(), w.cpu().numpy(), from_torch(y)
    finally:
        f.free()
    rid, rw = orc.route(lg, k)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=2e-6, atol=1e-7)
    check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped=False, what=f"routed decode fmt {fmt} E {E} T {T}")


@pytest.mark.parametrize("fmt,T", [(orc.FMT_G128S, 8), (orc.FMT_Q4S, 40)])
def test_moe_decode_prompt_path(gpu, fmt, T, monkeypatch):
    """decode from logits past the decode path's 4 tokens: the router kernel, then the grouped
    products; ids / w equal the oracle router, y the oracle layer (grouped bounds) and, bit for bit,
    an explicit route + FFN"""
    import torch
    monkeypatch.delenv("ONPU_MOE_FUSED", raising=False)
    E, H, I, k = 32, 256, 128, 4
    gu, dn = _experts(fmt, E, H, I, 800 + T)
    xb = syn.activations(T, H, 801 + T)
    lg = syn.logits(T, E, 802 + T)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        x = to_torch_bf16(xb).reshape(T, H)
        lgd = torch.from_numpy(lg).cuda()
        y, ids, w = f.decode(lgd, x, k)
        i2, w2 = f.route(lgd, k)
        y2 = f.ffn(x, i2, w2)
        torch.cuda.synchronize()
        assert torch.equal(ids, i2) and torch.equal(w, w2) and torch.equal(y, y2)
        ids, w, y = ids.cpu().numpy(), w.cpu().numpy(), from_torch(y)
    finally:
        f.free()
    rid, rw = orc.route(lg, k)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=2e-6, atol=1e-7)
    check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped=True, what=f"decode prompt path fmt {fmt} T {T}")


# g128s needs whole 128-wide groups along the down projection's K = I: no I = 160 case for it
_ONE_LAUNCH = [(fmt, *shape) for fmt in (orc.FMT_G128S, orc.FMT_Q4S, orc.FMT_Q4NX)
               for shape in ((128, 2048, 768, 8, 1), (128, 2048, 768, 8, 4), (16, 512, 256, 4, 3), (24, 384, 160, 6, 2))
               if not (fmt == orc.FMT_G128S and shape[2] % 128)]


@pytest.mark.parametrize("fmt,E,H,I,k,T", _ONE_LAUNCH)
def test_moe_decode_one_launch(gpu, fmt, E, H, I, k, T, monkeypatch):
    """router + gate_up / SiLU * up + down / weighted sum in one launch (k_moe_decode): ids and w
    equal the oracle router, y within the bf16 bound of the oracle layer; the multi-launch path (the
    router kernel, then the two GEMV launches) agrees; repeated calls and graph replays give the same
    bits (the act counters are left at zero), and no wait timed out."""
    import torch
    gu, dn = _experts(fmt, E, H, I, 300 + E + T)
    xb = syn.activations(T, H, 301 + T)
    lg = syn.logits(T, E, 302 + k)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        x = to_torch_bf16(xb).reshape(T, H)
        lgd = torch.from_numpy(lg).cuda()
        monkeypatch.setenv("ONPU_MOE_FUSED", "1")
        y1, ids, w = f.decode(lgd, x, k)
        y2, _, _ = f.decode(lgd, x, k)
        monkeypatch.setenv("ONPU_MOE_FUSED", "0")
        y0, ids0, w0 = f.decode(lgd, x, k)
        monkeypatch.setenv("ONPU_MOE_FUSED", "1")
        # graph replays interleaved with eager work on the same handle
        yg = torch.empty_like(y1)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            f.decode(lgd, x, k, out=yg)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            f.decode(lgd, x, k, out=yg)
        for _ in range(3):
            yg.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(yg, y1), "graph replay differs from the eager one-launch decode"
            ye, _, _ = f.decode(lgd, x, k)
            torch.cuda.synchronize()
            assert torch.equal(ye, y1), "eager decode after a replay differs"
        assert f.status() == 0, "a one-launch decode gave up waiting for its act tiles"
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), "one-launch decode is not deterministic"
        assert torch.equal(ids, ids0) and torch.equal(w, w0)
        d = ((y1.float() - y0.float()).abs().max() / y0.float().abs().max()).item()
        assert d <= 4e-3, f"one-launch vs multi-launch decode differ by {d:.3e} of max|y|"
        ids, w, y = ids.cpu().numpy(), w.cpu().numpy(), from_torch(y1)
    finally:
        f.free()
    rid, rw = orc.route(lg, k)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=2e-6, atol=1e-7)
    check_moe(y, fmt, gu, dn, E, H, I, xb, rid, rw, grouped=False, what=f"one-launch moe fmt {fmt} E {E} T {T}")


@pytest.mark.parametrize("fused", ["0", "1"])
def test_moe_decode_workspace_survives_growth_under_a_graph(gpu, fused, monkeypatch):
    """A graph captured around a T = 1 decode keeps the FFN workspace pointers of that capture;
    eager calls at T = 4 and at a prompt's T = 40 (grouped path: permutation, items, act rows) must
    not free or move what the graph holds. Replays after them give the eager T = 1 bits, for the
    two-launch decode and the one-launch kernel (ONPU_MOE_FUSED=1)."""
    import torch
    monkeypatch.setenv("ONPU_MOE_FUSED", fused)
    E, H, I, k = 16, 512, 256, 8
    fmt = orc.FMT_G128S
    gu, dn = _experts(fmt, E, H, I, 900)
    f = _ffn(fmt, E, H, I, gu, dn)
    try:
        x1 = to_torch_bf16(syn.activations(1, H, 901)).reshape(1, H)
        lg1 = torch.from_numpy(syn.logits(1, E, 902)).cuda()
        y1, i1, w1 = f.decode(lg1, x1, k)
        yg, ig, wg = torch.empty_like(y1), torch.empty_like(i1), torch.empty_like(w1)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            f.decode(lg1, x1, k, out=yg, ids=ig, w=wg)
        for T in (4, 40, 2):
            xT = to_torch_bf16(syn.activations(T, H, 903 + T)).reshape(T, H)
            lgT = torch.from_numpy(syn.logits(T, E, 904 + T)).cuda()
            f.decode(lgT, xT, k)
            yg.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(yg, y1) and torch.equal(ig, i1) and torch.equal(wg, w1), T
        assert f.status() == 0
    finally:
        f.free()


_SPLIT = [(orc.FMT_G128S, 128, 2048, 768, 2048, 8, 1), (orc.FMT_G128S, 128, 2048, 768, 2048, 8, 4),
          (orc.FMT_Q4S, 24, 544, 160, 200, 16, 4), (orc.FMT_Q4NX, 16, 512, 96, 130, 6, 3),
          (orc.FMT_Q4_0, 8, 256, 64, 256, 8, 2), (orc.FMT_G128S, 12, 4096, 256, 4000, 4, 2)]


@pytest.mark.parametrize("sv", ["16", "32"])
@pytest.mark.parametrize("fmt,E,H,I,Nd,k,T", _SPLIT)
def test_moe_decode_split_along_I(gpu, fmt, E, H, I, Nd, k, T, sv, monkeypatch):
    """The default decode path at T <= 4 (k_moe_dsplit, then k_moe_dsum): each workgroup takes 16
    or 32 values of I (ONPU_DS_SV; the library picks 16 while every workgroup gets a CU of its own) of
    one slot's expert through gate / up, SiLU * up and down from the down bank's step-major copy (a
    16-value slice is half a 32-wide K step), no workgroup waiting for another. From logits and from given ids / w, y agrees
    with the oracle layer (bf16 bound) and with the two-launch path (an FFN built with
    ONPU_MOE_DSPLIT=0, so without the copy) to fp32 summation order; ids / w equal the router's.
    Ragged down rows (Nd not a multiple of 64), K tails, k up to 16, H = 4096 (the generic variant);
    T up to 4 (the library takes the split path for T = 1 by default; the test raises the limit)."""
    import torch
    from opennpu_amd.device import QFfn
    monkeypatch.delenv("ONPU_MOE_FUSED", raising=False)
    monkeypatch.setenv("ONPU_MOE_DSPLIT_MAX_T", "4")
    monkeypatch.setenv("ONPU_DS_SV", sv)
    gu = [syn.weights(fmt, 2 * I, H, 1100 + 2 * e) for e in range(E)]
    dn = [syn.weights(fmt, Nd, I, 1101 + 2 * e) for e in range(E)]
    xb = syn.activations(T, H, 1102 + T)
    lg = syn.logits(T, E, 1103 + k)
    outs = {}
    for split in ("1", "0"):
        monkeypatch.setenv("ONPU_MOE_DSPLIT", split)
        f = QFfn(E, H, I, fmt, Nd=Nd)
        try:
            f.load(np.concatenate(gu), np.concatenate(dn))
            x = to_torch_bf16(xb).reshape(T, H)
            lgd = torch.from_numpy(lg).cuda()
            print(f"moe decode split={split} sv={sv} fmt {fmt} E {E} H {H} I {I} Nd {Nd} k {k} T {T}", flush=True)
            y, ids, w = f.decode(lgd, x, k, f32=True)
            y2 = f.ffn(x, ids, w, f32=True)
            torch.cuda.synchronize()
            assert torch.equal(y, y2), "decode from logits and from ids / w differ"
            outs[split] = (from_torch(y), ids.cpu().numpy(), w.cpu().numpy())
        finally:
            f.free()
    (y1, i1, w1), (y0, i0, w0) = outs["1"], outs["0"]
    rid, rw = orc.route(lg, k)
    assert np.array_equal(i1, rid) and np.array_equal(i0, rid)
    assert np.array_equal(w1, w0)
    ref = orc.moe_layer(fmt, gu, dn, E, H, I, xb, rid, rw, Nd=Nd)
    err = orc.max_rel_err(y1, ref)
    assert err <= 4e-3, f"split decode vs oracle: {err:.3e}"
    d = np.abs(y1 - y0).max() / np.abs(y0).max()
    assert d <= 4e-3, f"split decode vs two launches: {d:.3e}"


def test_moe_decode_split_follows_weight_reloads(gpu, monkeypatch):
    """Loading new weights into some experts (from staging bytes, and by GPU quantization) updates
    the down bank's step-major copy with them: the split decode then equals a fresh FFN holding the
    new weights, bit for bit."""
    import torch
    from opennpu_amd.device import QFfn
    monkeypatch.delenv("ONPU_MOE_FUSED", raising=False)
    monkeypatch.delenv("ONPU_MOE_DSPLIT", raising=False)
    monkeypatch.setenv("ONPU_MOE_DSPLIT_MAX_T", "4")
    fmt, E, H, I, k = orc.FMT_Q4S, 8, 256, 128, 8
    gu = [syn.weights(fmt, 2 * I, H, 1200 + e) for e in range(E)]
    dn = [syn.weights(fmt, H, I, 1300 + e) for e in range(E)]
    dn_new = [syn.weights(fmt, H, I, 1400 + e) for e in range(E)]
    x = to_torch_bf16(syn.activations(2, H, 1201)).reshape(2, H)
    lgd = torch.from_numpy(syn.logits(2, E, 1202)).cuda()
    rng = np.random.default_rng(5)
    Wq = torch.from_numpy((rng.standard_normal((2, H, I)) * 0.02).astype(np.float32)).cuda()
    gq = torch.from_numpy((rng.standard_normal((2, 2 * I, H)) * 0.02).astype(np.float32)).cuda()
    f = QFfn(E, H, I, fmt)
    g = QFfn(E, H, I, fmt)
    try:
        f.load(np.concatenate(gu), np.concatenate(dn))
        f.decode(lgd, x, k)
        f.load(np.concatenate(gu[2:5]), np.concatenate(dn_new[2:5]), e0=2)     # experts 2..4 reloaded
        f.quantize(gq, Wq, e0=6)                                                # experts 6, 7 quantized
        y, _, _ = f.decode(lgd, x, k, f32=True)
        ref_dn = dn[:2] + dn_new[2:5] + dn[5:6]
        g.load(np.concatenate(gu[:6]), np.concatenate(ref_dn), e0=0)
        g.quantize(gq, Wq, e0=6)
        y2, _, _ = g.decode(lgd, x, k, f32=True)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
    finally:
        f.free()
        g.free()

"""GPU parity of decode attention (onpu_attn_step_dev) against the oracle's restatement of the
reference's host step (onpu_cpu.cpp:180-229; oracle pinned against a float64 torch softmax in
tests/test_oracle.py). fp32 arithmetic in a different summation order (chunks of the sequence,
rescaled partials): max|out - ref| <= 1e-5 max|ref|.
"""
import numpy as np
import pytest

import oracle.oracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _case(rng, Hq, Hkv, D, S, Smax, kv, masked, sinks):
    q = rng.standard_normal((Hq, D)).astype(np.float32)
    Kf = rng.standard_normal((Hkv, Smax, D)).astype(np.float32)
    Vf = rng.standard_normal((Hkv, Smax, D)).astype(np.float32)
    mask = None
    if masked:
        mask = np.where(rng.random(S) < 0.15, -np.inf, rng.standard_normal(S) * 0.2).astype(np.float32)
        if S > 2100:
            mask[100:2100] = -np.inf                     # whole chunks masked
    sk = rng.standard_normal(Hq).astype(np.float32) if sinks else None
    if kv == "bf16":
        K, V = orc.f2bf_np(Kf), orc.f2bf_np(Vf)
    else:
        K, V = Kf, Vf
    return q, K, V, mask, sk


@pytest.mark.parametrize("kv", ["bf16", "f32"])
@pytest.mark.parametrize("Hq,Hkv,D,S,Smax,masked,sinks", [
    (32, 8, 128, 1000, 1000, False, False),      # Qwen3-8B heads
    (32, 8, 128, 4100, 4352, True, False),       # cache slice: rows of a longer cache, masked chunks
    (64, 8, 64, 3000, 3000, True, True),         # gpt-oss heads with sinks
    (8, 8, 64, 17, 17, False, False),            # one query head per kv head, a short sequence
    (12, 2, 96, 777, 800, True, True),           # 6 query heads per kv head, D = 96
    (16, 1, 256, 2500, 2500, False, True),       # 16 query heads on one kv head, D = 256
])
def test_attn_step_dev(gpu, kv, Hq, Hkv, D, S, Smax, masked, sinks):
    import torch
    from opennpu_amd.device import attn_step
    rng = np.random.default_rng(Hq * 1000 + S)
    q, K, V, mask, sk = _case(rng, Hq, Hkv, D, S, Smax, kv, masked, sinks)
    ref = orc.attn_step(q, np.ascontiguousarray(K[:, :S]), np.ascontiguousarray(V[:, :S]), mask, sk)
    tdt = torch.bfloat16 if kv == "bf16" else torch.float32
    to = (lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()) if kv == "bf16" else \
        (lambda a: torch.from_numpy(a).cuda())
    Kd, Vd = to(K)[:, :S], to(V)[:, :S]
    assert Kd.dtype == tdt and Kd.stride(1) == D and Kd.stride(0) == Smax * D
    qd = torch.from_numpy(q).cuda()
    md = None if mask is None else torch.from_numpy(mask).cuda()
    sd = None if sk is None else torch.from_numpy(sk).cuda()
    print(f"attn_step_dev {kv} Hq={Hq} Hkv={Hkv} D={D} S={S}", flush=True)
    out = attn_step(qd, Kd, Vd, md, sd)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= TOL, err
    # repeated calls and a graph replay give the same bits
    ws = torch.empty((gpu.onpu_attn_ws_bytes(Hq, D, Hkv, S),), dtype=torch.uint8, device="cuda")
    o2 = attn_step(qd, Kd, Vd, md, sd, ws=ws)
    og = torch.empty_like(out)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        attn_step(qd, Kd, Vd, md, sd, out=og, ws=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attn_step(qd, Kd, Vd, md, sd, out=og, ws=ws)
    for _ in range(2):
        og.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(og, out)
    assert torch.equal(o2, out)


def test_attn_step_dev_argument_errors(gpu):
    """rejected on the host, nothing launched: Hq not a multiple of Hkv, D not a multiple of 8,
    more than 16 query heads per kv head, a short workspace"""
    import torch
    import ctypes as C
    L = gpu
    q = torch.zeros((64,), dtype=torch.float32, device="cuda")
    kv = torch.zeros((4096,), dtype=torch.float32, device="cuda")
    ws = torch.zeros((1 << 16,), dtype=torch.uint8, device="cuda")
    P = lambda t: C.c_void_p(t.data_ptr())
    assert L.onpu_attn_step_dev(P(q), 6, 8, P(kv), P(kv), 0, 4, 16, 128, 8, None, None, 1.0, P(q), P(ws), ws.numel(), None) == -1
    assert L.onpu_attn_step_dev(P(q), 4, 12, P(kv), P(kv), 0, 2, 16, 192, 12, None, None, 1.0, P(q), P(ws), ws.numel(), None) == -1
    assert L.onpu_attn_step_dev(P(q), 32, 8, P(kv), P(kv), 0, 1, 16, 128, 8, None, None, 1.0, P(q), P(ws), ws.numel(), None) == -1
    assert L.onpu_attn_step_dev(P(q), 4, 8, P(kv), P(kv), 0, 2, 16, 128, 8, None, None, 1.0, P(q), P(ws), 4, None) == -1
    assert b"onpu_attn_step_dev" in L.onpu_last_error()

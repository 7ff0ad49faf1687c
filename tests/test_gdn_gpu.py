"""GPU parity of the Gated DeltaNet decode step (onpu_gdn_step_dev) against the oracle's restatement
of the reference's host onpu_gdn_step (onpu_cpu.cpp:107-171; the oracle is pinned by delta-rule
invariants in tests/test_oracle.py). The conv state update is a copy (bit-exact); S and out are fp32
sums in another order: max|y - r| <= 1e-5 max|r| (2e-5 for out, after the RMS normalisation)."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("Hk,Hv,Dk,Dv,H,Kc,L", [(16, 32, 128, 128, 2048, 4, 3), (2, 6, 48, 32, 100, 4, 5),
                                                (4, 4, 64, 64, 512, 2, 1)])
def test_gdn_step_dev(gpu, Hk, Hv, Dk, Dv, H, Kc, L):
    import torch
    rng = np.random.default_rng(Hv * 100 + Dk)
    Cc = 2 * Hk * Dk + Hv * Dv
    a = dict(x=rng.standard_normal(H), qkv=rng.standard_normal(Cc), z=rng.standard_normal(Hv * Dv),
             Wb=rng.standard_normal((Hv, H)) / np.sqrt(H), Wa=rng.standard_normal((Hv, H)) / np.sqrt(H),
             conv_w=rng.standard_normal((Cc, Kc)) * 0.5, conv_state=rng.standard_normal((Cc, L)),
             A_log=rng.standard_normal(Hv) * 0.5, dt_bias=rng.standard_normal(Hv) * 0.5,
             norm_w=rng.uniform(0.5, 1.5, Dv), eps=1e-6, S=rng.standard_normal((Hv, Dk, Dv)) * 0.1)
    f32 = {k: np.ascontiguousarray(v, np.float32) for k, v in a.items() if k != "eps"}
    out_r, cs_r, S_r = orc.gdn_step(**a, Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv)
    d = {k: torch.from_numpy(v).cuda() for k, v in f32.items()}
    out = torch.empty(Hv * Dv, dtype=torch.float32, device="cuda")
    ws = torch.empty((gpu.onpu_gdn_ws_bytes(Hk, Hv, Dk, Dv),), dtype=torch.uint8, device="cuda")
    P = lambda t: C.c_void_p(t.data_ptr())
    print(f"gdn_step_dev Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}", flush=True)
    rc = gpu.onpu_gdn_step_dev(P(d["x"]), H, P(d["qkv"]), P(d["z"]), P(d["Wb"]), P(d["Wa"]), P(d["conv_w"]), Kc,
                               P(d["conv_state"]), L, P(d["A_log"]), P(d["dt_bias"]), P(d["norm_w"]), 1e-6, P(d["S"]),
                               Hk, Hv, Dk, Dv, P(out), P(ws), ws.numel(), None)
    assert rc == 0, gpu.onpu_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(d["conv_state"].cpu().numpy(), cs_r)
    S = d["S"].cpu().numpy()
    assert np.abs(S - S_r).max() <= 1e-5 * np.abs(S_r).max()
    o = out.cpu().numpy()
    assert np.abs(o - out_r).max() <= 2e-5 * np.abs(out_r).max()


def test_gdn_step_dev_argument_errors(gpu):
    import torch
    L = gpu
    v = torch.zeros((1 << 16,), dtype=torch.float32, device="cuda")
    P = C.c_void_p(v.data_ptr())
    args = lambda Hk, Hv, Dk, Dv, wsb: (P, 64, P, P, P, P, P, 4, P, 3, P, P, P, 1e-6, P, Hk, Hv, Dk, Dv, P, P, wsb, None)
    assert L.onpu_gdn_step_dev(*args(3, 8, 64, 64, 1 << 18)) == -1          # Hv not a multiple of Hk
    assert L.onpu_gdn_step_dev(*args(2, 4, 64, 48, 1 << 18)) == -1          # Dv does not divide 256
    assert L.onpu_gdn_step_dev(*args(2, 4, 256, 256, 1 << 18)) == -1        # Dk * Dv past the LDS copy
    assert L.onpu_gdn_step_dev(*args(2, 4, 64, 64, 16)) == -1               # short workspace
    assert b"onpu_gdn_step_dev" in L.onpu_last_error()

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) and the built libonpu_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """torch on a visible GPU plus the built library on gfx950; fails (never skips) otherwise."""
    import torch
    from opennpu_amd import require_gpu
    assert torch.cuda.is_available(), "no GPU visible to torch"
    return require_gpu()


def to_torch_bf16(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).cuda()


def from_torch(t):
    return t.float().cpu().numpy()


def gemm_exact(fmt, M):
    """whether the GEMM computes the exact dequant at M <= 64 rows (its 16-row tiles, and g128s
    32-row tiles, take the decode GEMV's arithmetic) rather than bf16 RNE weights"""
    import oracle.oracle as orc
    return M <= 16 or (M <= 32 and fmt == orc.FMT_G128S)


def check_bf16_out(y, ref, tol=1e-2, what="", floor=2e-5):
    """bf16 outputs against the fp64 oracle: the stated tolerance max|y-r|/max|r| <= tol, and per
    element within half a bf16 ulp of the exact result plus an fp32-accumulation floor."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(y - ref).max() / scale
    assert err <= tol, f"{what} max rel err {err:.3e} > {tol}"
    bound = 2.0 ** -8 * np.abs(ref) + floor * scale
    bad = np.abs(y - ref) > bound
    assert not bad.any(), f"{what} {bad.sum()} elements outside the bf16 rounding bound; first at {np.argwhere(bad)[0]}"
    return err


def check_f32_out(y, ref, tol=1e-3, what=""):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(y - ref).max() / scale
    assert err <= tol, f"{what} max rel err {err:.3e} > {tol}"
    assert err <= 1e-4, f"{what} fp32 outputs off by {err:.3e} of max|r| (fp32 accumulation should be ~1e-6)"
    return err

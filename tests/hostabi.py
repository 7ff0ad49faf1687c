"""Plain ctypes calls of libonpu_hip's host-pointer entry points, for the boundary tests.

The reference's Python reaches the int4 path through ctypes (opennpu/native/npu4/model.py:281-335)
with fp32 host arrays: a matrix's bytes go into the library's own buffer (onpu_dense_buf /
onpu_bank_buf, filled by onpu_pack), onpu_*_sync hands them to the device, and onpu_dense_mv,
onpu_bank_run, onpu_moe_ffn, onpu_ffn_run and onpu_ffn_run_many compute with them. `bind` opens the
library a second time and declares only the argument types that loader declares, so the tests call
the entry points with the reference's own declarations; each helper below is one C call or one
such sequence, written out so that a test reads as the call order it checks.
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
P, I64, I32, F = C.c_void_p, C.c_int64, C.c_int, C.POINTER(C.c_float)
I32P, U8P = C.POINTER(C.c_int32), C.POINTER(C.c_uint8)

# the entry points model.py:281-335 declares unconditionally, and those it binds when present
REQUIRED = ["onpu_ok", "onpu_geometry", "onpu_dense_new", "onpu_dense_new2", "onpu_geometry2", "onpu_bank_new2",
            "onpu_dense_buf", "onpu_dense_sync", "onpu_dense_free", "onpu_dense_mv", "onpu_bank_new", "onpu_bank_buf",
            "onpu_bank_sync", "onpu_bank_free", "onpu_bank_run"]
OPTIONAL = ["onpu_quant_dequant", "onpu_pack", "onpu_ffn_new", "onpu_ffn_gu", "onpu_ffn_dn", "onpu_ffn_fused",
            "onpu_ffn_free", "onpu_ffn_perm", "onpu_ffn_run", "onpu_ffn_run_many", "onpu_moe_ffn"]


def library_path():
    return Path(os.environ.get("OPENNPU_LIBONPU", ROOT / "opennpu_amd" / "libonpu_hip.so"))


def bind(path=None):
    """A fresh ctypes handle on the library with the reference loader's declarations."""
    import torch  # noqa: F401  - the library and torch share one HIP runtime
    L = C.CDLL(str(path or library_path()))
    L.onpu_ok.restype = C.c_int
    L.onpu_geometry.argtypes = [I64, I64, C.c_int, C.POINTER(I64)]
    L.onpu_geometry2.argtypes = [I64, I64, C.c_int, C.c_int, C.POINTER(I64)]
    L.onpu_dense_new.restype, L.onpu_dense_new.argtypes = P, [I64, I64]
    L.onpu_dense_new2.restype, L.onpu_dense_new2.argtypes = P, [I64, I64, C.c_int]
    L.onpu_bank_new.restype, L.onpu_bank_new.argtypes = P, [I64, I64, I64, C.c_int]
    L.onpu_bank_new2.restype, L.onpu_bank_new2.argtypes = P, [I64, I64, I64, C.c_int, C.c_int]
    L.onpu_dense_buf.restype, L.onpu_dense_buf.argtypes = U8P, [P]
    L.onpu_bank_buf.restype, L.onpu_bank_buf.argtypes = U8P, [P]
    for n in ("onpu_dense_sync", "onpu_dense_free", "onpu_bank_sync", "onpu_bank_free", "onpu_ffn_fused",
              "onpu_ffn_free"):
        getattr(L, n).argtypes = [P]
    L.onpu_dense_mv.argtypes = [P, F, I64, F]
    L.onpu_bank_run.argtypes = [P, F, C.c_int, I64, I32P, C.c_int, F]
    L.onpu_quant_dequant.argtypes = [F, I64, I64, C.c_int, F, C.c_int]
    L.onpu_pack.restype = I64
    L.onpu_pack.argtypes = [F, I64, I64, C.c_int, C.c_int, U8P, C.c_int]
    L.onpu_ffn_new.restype, L.onpu_ffn_new.argtypes = P, [I64, I64, I64, I64, I64, C.c_int]
    for n in ("onpu_ffn_gu", "onpu_ffn_dn"):
        getattr(L, n).restype, getattr(L, n).argtypes = P, [P]
    L.onpu_ffn_perm.argtypes = [P, I32P]
    L.onpu_ffn_run.argtypes = [P, F, I32P, C.c_int, F, F]
    L.onpu_ffn_run_many.argtypes = [P, F, I64, I32P, C.c_int, F, F]
    L.onpu_moe_ffn.argtypes = [P, P, F, I64, I32P, C.c_int, F, C.c_int, C.c_float, C.c_float, F, F, F]
    L.onpu_moe_act.argtypes = [F, I64, I64, I32P, F, C.c_int, C.c_float, C.c_float, F]
    L.onpu_moe_sum.argtypes = [F, I64, C.c_int, I64, I32P, F, F, F]
    L.onpu_last_error.restype = C.c_char_p
    return L


def fp(a):
    return None if a is None else a.ctypes.data_as(F)


def ip(a):
    return a.ctypes.data_as(I32P)


def f32(a):
    return None if a is None else np.ascontiguousarray(a, np.float32)


def geometry(L, N, K, ncols, sym):
    out = (C.c_int64 * 8)()
    L.onpu_geometry2(N, K, ncols, sym, out)
    return tuple(out)


def pack_into(L, W, ncols, sym, dst, threads=4):
    """onpu_pack straight into library memory at dst (a ctypes uint8 pointer); returns bytes written."""
    W = f32(W)
    return L.onpu_pack(fp(W), W.shape[0], W.shape[1], ncols, sym, dst, threads)


def dense(L, W, sym):
    """onpu_dense_new2 -> onpu_pack into onpu_dense_buf -> onpu_dense_sync."""
    N, K = W.shape
    h = L.onpu_dense_new2(N, K, sym)
    assert h, L.onpu_last_error().decode()
    nbytes = geometry(L, N, K, 8, sym)[7]
    assert pack_into(L, W, 8, sym, L.onpu_dense_buf(h)) == nbytes
    L.onpu_dense_sync(h)
    return h


def dense_mv(L, h, x, N):
    x = f32(x)
    y = np.full((x.shape[0], N), np.nan, np.float32)       # overwritten by the call
    L.onpu_dense_mv(h, fp(x), x.shape[0], fp(y))
    return y


def bank(L, Ws, ncols, sym, h=None):
    """onpu_bank_new2 (or a handle of a fused FFN) -> each expert packed at e * nbytes of
    onpu_bank_buf -> onpu_bank_sync."""
    E = len(Ws)
    N, K = Ws[0].shape
    if h is None:
        h = L.onpu_bank_new2(N, K, E, ncols, sym)
        assert h, L.onpu_last_error().decode()
    nbytes = geometry(L, N, K, ncols, sym)[7]
    base = C.cast(L.onpu_bank_buf(h), C.c_void_p).value
    for e, W in enumerate(Ws):
        assert pack_into(L, W, ncols, sym, C.cast(base + e * nbytes, U8P)) == nbytes
    L.onpu_bank_sync(h)
    return h

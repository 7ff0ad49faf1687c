"""Loads libonpu_hip.so (built in-tree by opennpu_amd/build.py) and declares its C ABI.

The argument types follow the reference's own ctypes binding, clib() in
opennpu/native/npu4/model.py:281-335, plus this library's device-pointer extensions
(include/onpu.h). torch is imported first when it is installed so that the library and torch
share one HIP runtime in the process (both name it libamdhip64.so.7).
"""
import ctypes as C
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("OPENNPU_LIBONPU", HERE / "libonpu_hip.so"))

FMT_Q4NX, FMT_Q4S, FMT_G128S, FMT_Q4_0 = 0, 1, 2, 3
FMT_NAMES = {"q4nx": FMT_Q4NX, "q4s": FMT_Q4S, "g128s": FMT_G128S, "q4_0": FMT_Q4_0}

_LIB = None


class LibraryMissing(RuntimeError):
    """libonpu_hip.so is not built (run opennpu_amd/build.py) or cannot be loaded."""


def _declare(lib):
    P, I64, I32, F = C.c_void_p, C.c_int64, C.c_int, C.POINTER(C.c_float)
    I32P, U8P, I64P = C.POINTER(C.c_int32), C.POINTER(C.c_uint8), C.POINTER(C.c_int64)
    sig = {
        # reference entries (llama/ggml-opennpu/onpu_api.cpp, onpu_cpu.cpp)
        "onpu_ok": (I32, []),
        "onpu_batched_ok": (I32, []),
        "onpu_geometry2": (None, [I64, I64, I32, I32, I64P]),
        "onpu_geometry": (None, [I64, I64, I32, I64P]),
        "onpu_stats": (None, [I64P, C.POINTER(C.c_double)]),
        "onpu_has_shape": (I32, [I32, I32, I32]),
        "onpu_dense_new2": (P, [I64, I64, I32]),
        "onpu_dense_new": (P, [I64, I64]),
        "onpu_dense_buf": (U8P, [P]),
        "onpu_dense_bytes": (I64, [P]),
        "onpu_dense_sync": (None, [P]),
        "onpu_dense_free": (None, [P]),
        "onpu_dense_mv": (None, [P, F, I64, F]),
        "onpu_bank_new2": (P, [I64, I64, I64, I32, I32]),
        "onpu_bank_new": (P, [I64, I64, I64, I32]),
        "onpu_bank_buf": (U8P, [P]),
        "onpu_bank_expert_bytes": (I64, [P]),
        "onpu_bank_sync": (None, [P]),
        "onpu_bank_free": (None, [P]),
        "onpu_bank_run": (None, [P, F, I32, I64, I32P, I32, F]),
        "onpu_moe_ffn": (None, [P, P, F, I64, I32P, I32, F, I32, C.c_float, C.c_float, F, F, F]),
        "onpu_moe_act": (None, [F, I64, I64, I32P, F, I32, C.c_float, C.c_float, F]),
        "onpu_moe_sum": (None, [F, I64, I32, I64, I32P, F, F, F]),
        "onpu_ffn_new": (P, [I64, I64, I64, I64, I64, I32]),
        "onpu_ffn_gu": (P, [P]),
        "onpu_ffn_dn": (P, [P]),
        "onpu_ffn_fused": (I32, [P]),
        "onpu_ffn_perm": (None, [P, I32P]),
        "onpu_ffn_run": (I32, [P, F, I32P, I32, F, F]),
        "onpu_ffn_run_many": (I32, [P, F, I64, I32P, I32, F, F]),
        "onpu_ffn_free": (None, [P]),
        "onpu_pack": (I64, [F, I64, I64, I32, I32, U8P, I32]),
        "onpu_quant_dequant": (None, [F, I64, I64, I32, F, I32]),
        # MI355X-native extensions
        "onpu_last_error": (C.c_char_p, []),
        "onpu_stage_bytes": (I64, [I32, I64, I64]),
        "onpu_dense_new3": (P, [I64, I64, I32]),
        "onpu_bank_new3": (P, [I64, I64, I64, I32]),
        "onpu_ffn_new3": (P, [I64, I64, I64, I64, I64, I32]),
        "onpu_dense_load": (I32, [P, P]),
        "onpu_bank_load": (I32, [P, I64, I64, P]),
        "onpu_dense_info": (None, [P, I64P]),
        "onpu_plan_gemv": (None, [I32, I64, I64, I32, I64, I32, I64P]),
        "onpu_plan_mv": (None, [I32, I64, I64, I64, I64P]),
        "onpu_dense_dequant": (I32, [P, I64, P, I32]),
        "onpu_dense_mv_dev": (I32, [P, P, I64, P, I32, P]),
        "onpu_dense_argmax_dev": (I32, [P, P, I64, P, P, P]),
        "onpu_dense_argmax_dev_noalloc": (I32, [P, P, I64, P, P, P]),
        "onpu_gemm_status": (I32, []),
        "onpu_release_scratch": (None, []),
        "onpu_moe_route_dev": (I32, [P, I64, I32, I32, I32, P, P, P]),
        "onpu_moe_ffn_dev": (I32, [P, P, I64, P, I32, P, P, I32, P]),
        "onpu_moe_decode_dev": (I32, [P, P, P, I64, I32, I32, I32, P, P, P, I32, P]),
        "onpu_moe_status": (I32, [P]),
        "onpu_quantize_dev": (I32, [P, I64, I64, P, I64, I32, P]),
        "onpu_transcode_q4k_dev": (I32, [P, I64, I64, P, I64, P]),
        "onpu_pack_q4k": (I64, [U8P, I64, I64, U8P, I32]),
        "onpu_gemv_i8_dev": (I32, [P, P, I64, I64, P, P, P]),
        "onpu_gdn_ws_bytes": (I64, [I32, I32, I32, I32]),
        "onpu_gdn_step_dev": (I32, [P, I32, P, P, P, P, P, I32, P, I32, P, P, P, C.c_float, P, I32, I32, I32, I32, P,
                                    P, I64, P]),
        "onpu_attn_ws_bytes": (I64, [I32, I32, I32, I64]),
        "onpu_attn_step_dev": (I32, [P, I32, I32, P, P, I32, I32, I64, I64, I64, P, P, C.c_float, P, P, I64, P]),
        "onpu_chain_new": (P, [C.POINTER(P), C.POINTER(P), C.POINTER(P), I32, I64, I32]),
        "onpu_chain_run": (I32, [P, P]),
        "onpu_chain_status": (I32, [P]),
        "onpu_chain_info": (None, [P, I64P]),
        "onpu_chain_free": (None, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return sorted(sig)


EXPORTS = None


def lib():
    """The loaded library (raises LibraryMissing: there is no fallback path)."""
    global _LIB, EXPORTS
    if _LIB is None:
        if not LIB_PATH.exists():
            raise LibraryMissing(f"{LIB_PATH} is not built: run `python -m opennpu_amd.build`")
        try:
            import torch  # noqa: F401  - one HIP runtime for torch and the library
        except ImportError:
            pass
        try:
            L = C.CDLL(str(LIB_PATH))
        except OSError as e:
            raise LibraryMissing(f"cannot load {LIB_PATH}: {e}") from e
        EXPORTS = _declare(L)
        _LIB = L
    return _LIB


def check(rc, what="libonpu_hip"):
    """Raise on a negative return code of an int-returning entry point."""
    if rc < 0:
        raise RuntimeError(f"{what}: {lib().onpu_last_error().decode()}")
    return rc


def require_gpu():
    """The library on a usable gfx950 GPU, or RuntimeError (never a CPU fallback)."""
    L = lib()
    if L.onpu_ok() != 1:
        raise RuntimeError("libonpu_hip: no usable gfx950 GPU")
    return L

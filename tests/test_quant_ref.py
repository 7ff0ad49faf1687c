"""The reference's own bf16 rounding, Mat geometry and per-32 search quantizers, compiled here, against
the oracle's restatements (orc_f2bf, orc_geometry, orc_quant_sym32, orc_quant_asym32) and the
library's host codecs (onpu_geometry2, onpu_pack for q4s and q4nx).

The reference code is lines 37-254 of llama/ggml-opennpu/opennpu_core.hpp (namespace onpu:
f2bf / bf2f :50-62, Mat :65-97, quant_asym32 :103-138, quant_sym32 :142-169, pack_mat :174-254),
copied unedited from the reference checkout at build time and compiled through
oracle/ref_core.cpp (oracle/Makefile `ref`; outputs in oracle/_ref/, never committed). Those lines
need only standard headers; the XRT includes of the header serve the device code after them.

Two builds:
- as written (-ffp-contract=off): the oracle and the library must equal it byte for byte, on more
  than 10^6 groups per format (normal, heavy-tailed, all-positive, tiny and huge magnitudes,
  exact grids, planted ties);
- with the reference's own flags (llama/build.sh:74, -O3 -march=native): GCC fuses multiply-adds
  there, the least-squares refits round differently, and the search keeps another candidate in a
  fraction of the groups (test_native_build_rates measures it per kind); the library writes the
  as-written bytes.

CPU tests: they run where the reference checkout is present (the reference never reaches the GPU
box; the GPU codecs are compared with the as-written build in tests/test_codec_gpu.py)."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import _lib
from tests.quantref import (GPR, KINDS, G_PER_KIND, SEEDS, REFCORE, REF, groups, load, p, ref_asym, ref_pack,
                            ref_staging, ref_sym)


@pytest.fixture(scope="module")
def ref():
    if not REFCORE.exists() and not (REF / "libonpu_core_ref.so").exists():
        pytest.skip("the reference checkout is not on this machine")
    return load("libonpu_core_ref.so")


@pytest.fixture(scope="module")
def ref_native():
    if not REFCORE.exists():
        pytest.skip("the reference checkout is not on this machine")
    return load("libonpu_core_ref_native.so")


def pack(fmt, W):
    """the library's onpu_pack (host codecs) for 8 columns: the reference's packed bytes"""
    L = _lib.lib()
    N, K = W.shape
    g = (C.c_int64 * 8)()
    L.onpu_geometry2(N, K, 8, fmt, g)
    out = np.zeros(g[7], np.uint8)
    n = L.onpu_pack(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, 8, fmt, out.ctypes.data_as(C.POINTER(C.c_uint8)), 8)
    assert n == g[7]
    return out


@pytest.mark.parametrize("kind", KINDS)
def test_quant_sym32_equals_reference(ref, kind):
    """q4s: the oracle's orc_quant_sym32 writes the reference's codes and bf16 scales, and the
    library's onpu_pack the bytes of the reference's pack_mat, byte for byte"""
    for seed in range(SEEDS):
        X = groups(kind, G_PER_KIND, 1000 * KINDS.index(kind) + seed)
        W, want = ref_staging(ref, orc.FMT_Q4S, X)
        got = orc.quantize(orc.FMT_Q4S, W)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{kind} seed {seed}: oracle differs at {bad.size} bytes, first {bad[:4]}"
        assert np.array_equal(pack(orc.FMT_Q4S, W), ref_pack(ref, orc.FMT_Q4S, W, 8)), f"{kind} seed {seed}: onpu_pack"


@pytest.mark.parametrize("kind", KINDS)
def test_quant_asym32_equals_reference(ref, kind):
    """q4nx: the oracle's orc_quant_asym32 writes the reference's codes and bf16 (scale, min) pairs,
    and the library's onpu_pack the bytes of the reference's pack_mat, byte for byte"""
    for seed in range(SEEDS):
        X = groups(kind, G_PER_KIND, 2000 * KINDS.index(kind) + seed)
        W, want = ref_staging(ref, orc.FMT_Q4NX, X)
        got = orc.quantize(orc.FMT_Q4NX, W)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{kind} seed {seed}: oracle differs at {bad.size} bytes, first {bad[:4]}"
        assert np.array_equal(pack(orc.FMT_Q4NX, W), ref_pack(ref, orc.FMT_Q4NX, W, 8)), f"{kind} seed {seed}: onpu_pack"


def test_single_group_wrappers_equal_reference(ref):
    """the per-group entry points the other tests use (orc.quant_sym32 / quant_asym32)"""
    X = groups("ties", 7 * 40, 5)
    q, d = ref_sym(ref, X)
    qa, s, m = ref_asym(ref, X)
    for g in range(X.shape[0]):
        gq, gd = orc.quant_sym32(X[g])
        assert np.array_equal(gq, q[g]) and gd == d[g], g
        gq, gs, gm = orc.quant_asym32(X[g])
        assert np.array_equal(gq, qa[g]) and (gs, gm) == (s[g], m[g]), g


def test_f2bf_equals_reference(ref):
    """the oracle's f2bf (and so every bf16 staging the tests build) against the reference's f2bf:
    all 2^16 exponent/sign/top-mantissa patterns with the rounding tail at its edges, NaNs,
    infinities, subnormals and random patterns"""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    tails = np.array([0, 1, 0x7fff, 0x8000, 0x8001, 0xffff], np.uint32)
    bits = (hi[:, None] | tails[None, :]).ravel()
    bits = np.concatenate([bits, np.random.default_rng(3).integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    x = bits.view(np.float32)
    want = np.empty(x.size, np.uint16)
    ref.ref_f2bf_n(p(x), x.size, p(want))
    assert np.array_equal(orc.f2bf_np(x).ravel(), want)


NS = [1, 63, 64, 255, 256, 257, 1000, 1024, 2048, 4096, 6144, 12288, 14336, 24576, 151936, 200003]
KS = [32, 256, 512, 2048, 2049, 3072, 4096, 12288, 14336, 16384, 16385, 20000, 32768]


@pytest.mark.parametrize("sym", [0, 1])
def test_geometry_equals_reference_mat(ref, sym):
    """Mat(N, K, ncols, sym): the oracle's orc_geometry and the library's onpu_geometry2 give the
    reference's eight values (zeros where Mat has no geometry) over an (N, K, ncols) sweep"""
    L = _lib.lib()
    out = np.zeros(8, np.int64)
    lib_out = (C.c_int64 * 8)()
    n_none = 0
    for N in NS:
        for K in KS:
            for ncols in (1, 2, 3, 4, 6, 8):
                ref.ref_geometry(N, K, ncols, sym, p(out))
                want = tuple(int(v) for v in out)
                n_none += want == (0,) * 8
                assert orc.geometry(N, K, ncols, sym) == want, (N, K, ncols, sym)
                L.onpu_geometry2(N, K, ncols, sym, lib_out)
                assert tuple(lib_out) == want, (N, K, ncols, sym)
                if sym == 0:
                    L.onpu_geometry(N, K, ncols, lib_out)
                    assert tuple(lib_out) == want, (N, K, ncols)
    assert 0 < n_none < len(NS) * len(KS) * 6          # both outcomes occur in the sweep


def test_native_build_rates(ref, ref_native):
    """The reference built with its own flags (llama/build.sh:74, -O3 -march=native) against the
    source as written. GCC fuses multiply-adds there; the least-squares refits then round
    differently in their last bits, a bf16-rounded (s, m) or d can land on its neighbour, and the
    search keeps another candidate. Measured with this image's GCC 11 on 2^17 groups per kind:
    q4s differs in 0-2 groups per kind; q4nx in ~2e-5 of Gaussian groups, more in groups of
    repeated values or exact grids (about 7 % of the planted-tie kind), where an exact fit found
    as written can be missed. The library writes the as-written bytes: the source's own arithmetic,
    the same with every compiler and CPU (the deployed bytes depend on both)."""
    rates = {}
    for kind in KINDS:
        X = groups(kind, 1 << 17, 99 + KINDS.index(kind))
        q0, d0 = ref_sym(ref, X)
        q1, d1 = ref_sym(ref_native, X)
        a0, a1 = ref_asym(ref, X), ref_asym(ref_native, X)
        sym = int(np.count_nonzero((q0 != q1).any(axis=1) | (d0 != d1)))
        asym = int(np.count_nonzero((a0[0] != a1[0]).any(axis=1) | (a0[1] != a1[1]) | (a0[2] != a1[2])))
        rates[kind] = (sym / X.shape[0], asym / X.shape[0])
    print("native build vs as written, groups differing (q4s, q4nx):",
          {k: (f"{a:.1e}", f"{b:.1e}") for k, (a, b) in rates.items()})
    assert all(a <= 1e-4 for a, _ in rates.values())
    assert all(rates[k][1] <= 2e-4 for k in ("normal", "heavy", "tiny", "huge", "scales"))
    assert rates["ties"][1] > 0           # the flags do change the bytes: the choice is real

"""GPU: handles of the reference's constructors read the reference's NPU packing.

onpu_dense_new2, onpu_bank_new2 and onpu_ffn_new (q4nx, q4s) take the reference's packed bytes in
their *_buf memory (pack_mat, opennpu_core.hpp:174-254; tests/test_npu_layout.py pins onpu_pack and
the oracle's npu_pack to the reference's own code); *_sync turns them into the staging layout on
the device (k_npu_stage) and then into the tiled layout. The weights a handle then holds must
equal the oracle's dequantization of the oracle's quantization, bit for bit, over ragged shapes,
several K slices, empty column blocks and 1..8 columns, for bytes written by onpu_pack and by the
oracle's packer alike; a fused FFN's gate_up bank packed in the reference's row order
(onpu_ffn_perm) reads back in logical order. A PackCache-style file (model.py:712-759: the packed
bytes of a buffer, read back into a fresh handle's buffer) round-trips."""
import ctypes as C

import numpy as np
import pytest

import oracle.oracle as orc
from opennpu_amd import _lib
from tests import hostabi as ha

pytestmark = pytest.mark.gpu
FMT = {1: orc.FMT_Q4S, 0: orc.FMT_Q4NX}


@pytest.fixture(scope="module")
def L(gpu):
    L = ha.bind()
    assert L.onpu_ok() == 1
    return L


def weights(rng, N, K):
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[:, : K // 3] += 0.01
    W[min(1, N - 1), : min(K, 64)] = 0.0
    return W


def held(h, e, N, K):
    """the fp32 weights expert e of handle h holds on the device"""
    out = np.empty((N, K), np.float32)
    assert _lib.lib().onpu_dense_dequant(C.c_void_p(h), e, C.c_void_p(out.ctypes.data), 0) == 0
    return out


def qdq(fmt, W):
    N, K = W.shape
    return orc.dequant(fmt, orc.quantize(fmt, W), N, K)


def same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("sym", [0, 1])
def test_dense_reads_reference_packing(L, sym):
    """onpu_dense_new2 (8 columns) -> onpu_pack into its buffer -> sync: the held weights"""
    rng = np.random.default_rng(70 + sym)
    for N, K in [(1, 32), (100, 96), (300, 544), (513, 2080), (2048, 4096), (4096, 4096)]:
        W = weights(rng, N, K)
        h = ha.dense(L, W, sym)
        try:
            assert same(held(h, 0, N, K), qdq(FMT[sym], W)), (N, K)
        finally:
            L.onpu_dense_free(h)


@pytest.mark.parametrize("sym", [0, 1])
def test_bank_reads_oracle_packer_bytes(L, sym):
    """onpu_bank_new2 over 1..8 columns, each expert's bytes from the oracle's packer (the bytes the
    reference's own pack_mat writes): the held weights of every expert"""
    rng = np.random.default_rng(80 + sym)
    for N, K, ncols, E in [(257, 1024, 1, 3), (1000, 2048, 4, 2), (70, 3072, 3, 2), (768, 768, 6, 3)]:
        Ws = [weights(rng, N, K) for _ in range(E)]
        h = L.onpu_bank_new2(N, K, E, ncols, sym)
        assert h, L.onpu_last_error().decode()
        try:
            nbytes = ha.geometry(L, N, K, ncols, sym)[7]
            assert _lib.lib().onpu_bank_expert_bytes(C.c_void_p(h)) == nbytes
            buf = np.ctypeslib.as_array(L.onpu_bank_buf(h), shape=(E * nbytes,))
            for e, W in enumerate(Ws):
                buf[e * nbytes:(e + 1) * nbytes] = orc.npu_pack(FMT[sym], W, ncols)
            L.onpu_bank_sync(h)
            for e, W in enumerate(Ws):
                assert same(held(h, e, N, K), qdq(FMT[sym], W)), (N, K, ncols, e)
        finally:
            L.onpu_bank_free(h)


@pytest.mark.parametrize("sym", [0, 1])
def test_pack_cache_file_round_trip(L, sym, tmp_path):
    """a bank's buffer written to a file and read into a fresh handle's buffer (npu4's PackCache
    save / load) holds the same weights; the file equals the reference's packing"""
    rng = np.random.default_rng(90 + sym)
    N, K, E, ncols = 512, 2048, 3, 2
    Ws = [weights(rng, N, K) for _ in range(E)]
    h = ha.bank(L, Ws, ncols, sym)
    nbytes = ha.geometry(L, N, K, ncols, sym)[7]
    path = tmp_path / "bank.bin"
    with open(path, "wb") as f:
        f.write(memoryview(np.ctypeslib.as_array(L.onpu_bank_buf(h), shape=(E * nbytes,))))
    L.onpu_bank_free(h)
    data = np.fromfile(path, np.uint8)
    for e, W in enumerate(Ws):
        assert np.array_equal(data[e * nbytes:(e + 1) * nbytes], orc.npu_pack(FMT[sym], W, ncols)), e
    h2 = L.onpu_bank_new2(N, K, E, ncols, sym)
    assert h2
    try:
        with open(path, "rb") as f:
            f.readinto(memoryview(np.ctypeslib.as_array(L.onpu_bank_buf(h2), shape=(E * nbytes,))))
        L.onpu_bank_sync(h2)
        for e, W in enumerate(Ws):
            assert same(held(h2, e, N, K), qdq(FMT[sym], W)), e
    finally:
        L.onpu_bank_free(h2)


@pytest.mark.parametrize("sym", [0, 1])
def test_fused_ffn_reference_row_order(L, sym):
    """onpu_ffn_new at a shape the reference fuses with a non-trivial gate_up order (Qwen3-30B-A3B's
    experts: gate_up 1536 x 2048, down 2048 x 768): onpu_ffn_perm gives the reference's order, the
    bank packed as gu[e][perm] holds gu[e] in logical order, and onpu_ffn_run computes the layer"""
    from tests.test_host_abi_gpu import _layer_ref, _routes, rel
    rng = np.random.default_rng(100 + sym)
    E, H, I, k = 4, 2048, 768, 2
    gu = [weights(rng, 2 * I, H) for _ in range(E)]
    dn = [weights(rng, H, I) for _ in range(E)]
    f = L.onpu_ffn_new(2 * I, H, H, I, E, sym)
    assert f and L.onpu_ffn_fused(f) == 1
    try:
        perm = np.full(2 * I, -1, np.int32)
        L.onpu_ffn_perm(f, ha.ip(perm))
        want = orc.ffn_order(2 * I, H, H, I, sym)
        assert np.array_equal(perm, want) and not np.array_equal(perm, np.arange(2 * I))
        ha.bank(L, [g[perm] for g in gu], 1, sym, h=L.onpu_ffn_gu(f))
        ha.bank(L, dn, 1, sym, h=L.onpu_ffn_dn(f))
        for e in range(E):
            assert same(held(L.onpu_ffn_gu(f), e, 2 * I, H), qdq(FMT[sym], gu[e])), e
            assert same(held(L.onpu_ffn_dn(f), e, H, I), qdq(FMT[sym], dn[e])), e
        if sym == 1:                                   # _layer_ref dequantizes as q4s
            x = (rng.standard_normal((1, H)) * 0.5).astype(np.float32)
            ids, w = _routes(rng, 1, E, k)
            y = np.full((1, H), np.nan, np.float32)
            assert L.onpu_ffn_run(f, ha.fp(x), ha.ip(ids), k, ha.fp(w), ha.fp(y)) == 1
            r = _layer_ref(x, gu, dn, ids, w, 0)
            assert rel(y, r) <= 1e-2 and np.abs(y - r).mean() / np.abs(r).max() <= 1e-3
    finally:
        L.onpu_ffn_free(f)

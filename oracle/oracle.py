"""ORACLE — test infrastructure only.

Python access to the C restatement in oracle/oracle.c (built by oracle/Makefile into
oracle/_build/liboracle.so) plus numpy restatements used beside it. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker: nothing in the product path calls it.

Each function cites the reference file:line it restates; tests/test_oracle.py pins each one
against library routines, closed forms, invariants or brute force (see oracle.c's header).
"""
import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

FMT_Q4NX, FMT_Q4S, FMT_G128S, FMT_Q4_0 = 0, 1, 2, 3
_lib = None


def build():
    """Compile oracle.c (gcc) into oracle/_build/liboracle.so."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P, I64, I32 = C.c_void_p, C.c_int64, C.c_int
        L.orc_f2bf.restype, L.orc_f2bf.argtypes = C.c_uint16, [C.c_float]
        L.orc_bf2f.restype, L.orc_bf2f.argtypes = C.c_float, [C.c_uint16]
        L.orc_h2f.restype, L.orc_h2f.argtypes = C.c_float, [C.c_uint16]
        L.orc_group.restype, L.orc_group.argtypes = I64, [I32]
        L.orc_stage_bytes.restype, L.orc_stage_bytes.argtypes = I64, [I32, I64, I64]
        L.orc_unpack.argtypes = [I32, P, I64, I64, P]
        L.orc_dequant.argtypes = [I32, P, I64, I64, P]
        L.orc_dequant_bf16.argtypes = [I32, P, I64, I64, P]
        L.orc_qmm_rows.argtypes = [I32, P, I64, I64, P, I64, I64, I64, P, I32]
        L.orc_matmul_f64.argtypes = [P, I64, I64, P, I64, P]
        L.orc_route.argtypes = [P, I64, I32, I32, I32, P, P]
        L.orc_silu_mul.argtypes = [P, I64, I64, P]
        L.orc_gptoss_act.argtypes = [P, I64, I64, C.c_float, C.c_float, P]
        L.orc_moe_sum.argtypes = [P, I64, I32, I64, P, P, P, P]
        L.orc_argmax.argtypes = [P, I64, I64, P]
        L.orc_geometry.argtypes = [I64, I64, I32, I32, P]
        L.orc_quant_sym32.argtypes = [P, P, P]
        L.orc_quant_sym.argtypes = [P, I32, P, P]
        L.orc_quant_asym32.argtypes = [P, P, P, P]
        L.orc_f2h.restype, L.orc_f2h.argtypes = C.c_uint16, [C.c_float]
        L.orc_quant_q4_0.argtypes = [P, P, P]
        L.orc_transcode_q4k.argtypes = [P, I64, I64, I64, P, P, P]
        L.orc_quantize.argtypes = [I32, P, I64, I64, P]
        L.orc_gemv_i8.argtypes = [P, P, I64, I64, P, P]
        L.orc_gdn_step.argtypes = [P, I32, P, P, P, P, P, I32, P, I32, P, P, P, C.c_float, P, I32, I32, I32, I32, P]
        L.orc_attn_step.argtypes = [P, I32, I32, P, P, I32, I32, I64, I64, I64, P, P, C.c_float, P]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------ scalars
def f2bf(x):
    """float32 array -> bf16 bit patterns (uint16), RNE (opennpu_core.hpp:50-56)."""
    x = np.ascontiguousarray(x, np.float32)
    return np.fromiter((lib().orc_f2bf(float(v)) for v in x.ravel()), np.uint16, x.size).reshape(x.shape)


def f2bf_np(x):
    """The same RNE rounding vectorised in numpy (used for large arrays)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 64).astype(np.uint16), r)


def bf2f(h):
    """bf16 bits -> float32 (opennpu_core.hpp:57-62)."""
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ formats
def group(fmt):
    return 128 if fmt == FMT_G128S else 32


def stage_bytes(fmt, N, K):
    return int(lib().orc_stage_bytes(fmt, N, K))


def _check(fmt, st, N, K):
    if K % group(fmt) != 0:
        raise ValueError(f"K = {K} is not a multiple of the format's group ({group(fmt)})")
    if np.asarray(st).size < stage_bytes(fmt, N, K):
        raise ValueError("staging buffer smaller than the format's size")


def unpack(fmt, st, N, K):
    """Stored codes u [N][K] (uint8 0..15)."""
    _check(fmt, st, N, K)
    out = np.empty((N, K), np.uint8)
    lib().orc_unpack(fmt, _p(np.ascontiguousarray(st)), N, K, _p(out))
    return out


def dequant(fmt, st, N, K):
    """fp32 dequantized weights [N][K] (onpu_api.cpp:508-529 semantics)."""
    _check(fmt, st, N, K)
    out = np.empty((N, K), np.float32)
    lib().orc_dequant(fmt, _p(np.ascontiguousarray(st)), N, K, _p(out))
    return out


def dequant_bf16(fmt, st, N, K):
    """bf16 (RNE) of the dequantized weights, as bit patterns [N][K] (gemv_any.cc:65,106-107)."""
    _check(fmt, st, N, K)
    out = np.empty((N, K), np.uint16)
    lib().orc_dequant_bf16(fmt, _p(np.ascontiguousarray(st)), N, K, _p(out))
    return out


def qmm(fmt, st, N, K, xb, n0=0, n1=None, bf16w=False):
    """fp64 y[M][n1-n0] = x . dequant(W)^T for rows [n0, n1) (reference.py:24-28,55 pattern,
    accumulated in fp64). xb: bf16 bits [M][K]. bf16w: with the weights rounded to bf16 (RNE) as the
    reference device's MAC sees them (gemv_any.cc:65,106-107)."""
    _check(fmt, st, N, K)
    n1 = N if n1 is None else n1
    xb = np.ascontiguousarray(xb, np.uint16).reshape(-1, K)
    M = xb.shape[0]
    y = np.empty((M, n1 - n0), np.float64)
    lib().orc_qmm_rows(fmt, _p(np.ascontiguousarray(st)), N, K, _p(xb), M, n0, n1, _p(y), int(bf16w))
    return y


def matmul_f64(W, x):
    """fp64 brute force y[M][N] = x[M][K] . W[N][K]^T (W float32, x float64)."""
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float64)
    N, K = W.shape
    M = x.shape[0]
    y = np.empty((M, N), np.float64)
    lib().orc_matmul_f64(_p(W), N, K, _p(x), M, _p(y))
    return y


def qmm_f32_torch(fmt, st, N, K, xb):
    """The reference's own CPU pattern: dequantize W to fp32, then x @ W.T in torch fp32
    (opennpu/native/reference.py:24-28,55). Used as the cpu_baseline workload."""
    import torch
    W = torch.from_numpy(dequant(fmt, st, N, K))
    x = torch.from_numpy(bf2f(xb).reshape(-1, K))
    return (x @ W.T).numpy()


# ------------------------------------------------------------------ MoE pieces
def route(logits, k, renorm=True):
    """softmax -> top-k -> renorm (moe_runtime.py:333-341, reference.py:72-76); ties to the lower id."""
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    lib().orc_route(_p(logits), T, E, k, int(renorm), _p(ids), _p(w))
    return ids, w


def silu_mul(h):
    """act 0: silu(h[:, :I]) * h[:, I:] in fp32 (onpu_cpu.cpp:253)."""
    h = np.ascontiguousarray(h, np.float32)
    rows, Ng = h.shape
    a = np.empty((rows, Ng // 2), np.float32)
    lib().orc_silu_mul(_p(h), rows, Ng, _p(a))
    return a


def gptoss_act(h, alpha, limit):
    """act 1 (onpu_cpu.cpp:245-250)."""
    h = np.ascontiguousarray(h, np.float32)
    rows, Ng = h.shape
    a = np.empty((rows, Ng // 2), np.float32)
    lib().orc_gptoss_act(_p(h), rows, Ng, alpha, limit, _p(a))
    return a


def moe_sum(o, ids, w, bias=None):
    """y[t] = sum_j w[t,j] (o[t,j] + bias[ids[t,j]]) (onpu_cpu.cpp:259-274). o: [T][k][N]."""
    o = np.ascontiguousarray(o, np.float32)
    T, k, N = o.shape
    y = np.empty((T, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_moe_sum(_p(o), T, k, N, _p(np.ascontiguousarray(ids, np.int32)),
                      _p(np.ascontiguousarray(w, np.float32)), None if b is None else _p(b), _p(y))
    return y


def argmax(v):
    """numpy argmax per row (engine.py:358): the first NaN if the row has one, else the first maximum."""
    v = np.ascontiguousarray(v, np.float32)
    rows, N = v.shape
    out = np.empty(rows, np.int32)
    lib().orc_argmax(_p(v), rows, N, _p(out))
    return out


def moe_layer(fmt, gu_st, dn_st, E, H, I, x_bf, ids, w, bf16w=False, bf16o=False, mag=False, Nd=None):
    """A routed-expert FFN layer as reference.py:71-84 computes it (dequantized experts, fp32 act),
    with the two rounding points of the device path: gate_up in fp64 -> fp32, act -> bf16 RNE as the
    down input (the device input conversion, opennpu_core.hpp:418-424), down in fp64, weighted sum.
    gu_st / dn_st: E staging blobs; returns y [T][H] float64. bf16w: the expert weights rounded to
    bf16 (RNE) as the reference device's MAC sees them (gemv_any.cc:65,106-107). bf16o: each expert's
    down output rounded to bf16 before the weighted sum, as the reference device returns it
    (gemv_any.cc:120-130) to the host's fp32 sum (onpu_cpu.cpp:259-274). mag: also return
    sum_j |w_j d_j| per output (the scale of a one-ulp difference in any rounded expert row). Nd: the
    down projection's rows (default H)."""
    T, k = ids.shape
    Nd = H if Nd is None else Nd
    y = np.zeros((T, Nd), np.float64)
    m = np.zeros((T, Nd), np.float64)
    xb = np.asarray(x_bf, np.uint16).reshape(T, H)
    for e in np.unique(ids):
        rows, slots = np.nonzero(ids == e)
        g = qmm(fmt, gu_st[e], 2 * I, H, xb[rows], bf16w=bf16w).astype(np.float32)
        a = f2bf_np(silu_mul(g))
        d = qmm(fmt, dn_st[e], Nd, I, a, bf16w=bf16w)
        if bf16o:
            d = bf2f(f2bf_np(d.astype(np.float32))).astype(np.float64)
        y[rows] += w[rows, slots][:, None].astype(np.float64) * d
        m[rows] += np.abs(w[rows, slots][:, None].astype(np.float64) * d)
    return (y, m) if mag else y


# ------------------------------------------------------------------ geometry / quantizers
def geometry(N, K, ncols, sym):
    """Reference Mat geometry (model.py:151-187): R, S, tiles, kc, ks, rows_col, cb, nbytes."""
    out = np.zeros(8, np.int64)
    lib().orc_geometry(N, K, ncols, int(sym), _p(out))
    return tuple(int(v) for v in out)


def quant_sym32(x):
    """q4s search quantizer for 32 weights (opennpu_core.hpp:142-169): (codes, bf16 d bits)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(32, np.uint8)
    d = np.zeros(1, np.uint16)
    lib().orc_quant_sym32(_p(x), _p(q), _p(d))
    return q, int(d[0])


def quant_asym32(x):
    """q4nx search quantizer for 32 weights (opennpu_core.hpp:103-138): (codes, s bits, m bits)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(32, np.uint8)
    s = np.zeros(1, np.uint16)
    m = np.zeros(1, np.uint16)
    lib().orc_quant_asym32(_p(x), _p(q), _p(s), _p(m))
    return q, int(s[0]), int(m[0])


def quant_sym(x):
    """q4s search quantizer over len(x) weights (32: q4s, 128: g128s; opennpu_core.hpp:142-169):
    (codes, bf16 d bits)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.size, np.uint8)
    d = np.zeros(1, np.uint16)
    lib().orc_quant_sym(_p(x), x.size, _p(q), _p(d))
    return q, int(d[0])


def f2h(x):
    """float32 -> fp16 bits, RNE (ggml's GGML_FP32_TO_FP16)."""
    return np.array([lib().orc_f2h(float(v)) for v in np.ravel(x)], np.uint16).reshape(np.shape(x))


def quant_q4_0(x):
    """ggml's quantize_row_q4_0 rule on 32 weights: (codes in element order, fp16 d bits)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(32, np.uint8)
    d = np.zeros(1, np.uint16)
    lib().orc_quant_q4_0(_p(x), _p(q), _p(d))
    return q, int(d[0])


def transcode_q4k(blocks, N, K, ld=None):
    """GGUF Q4_K rows -> q4nx (ggml-opennpu.cpp:114-138): codes [N][K], bf16 s and m [N][K/32]."""
    if K % 256:
        raise ValueError("Q4_K rows hold whole 256-weight super-blocks")
    ld = K // 256 * 144 if ld is None else ld
    b = np.ascontiguousarray(blocks, np.uint8)
    if b.size < (N - 1) * ld + K // 256 * 144:
        raise ValueError("Q4_K buffer too small")
    q = np.empty((N, K), np.uint8)
    s = np.empty((N, K // 32), np.uint16)
    m = np.empty((N, K // 32), np.uint16)
    lib().orc_transcode_q4k(_p(b), N, K, ld, _p(q), _p(s), _p(m))
    return q, s, m


def quantize(fmt, W):
    """W [N][K] fp32 -> staging bytes of fmt by the quantizers above (what onpu_pack writes)."""
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    if K % group(fmt):
        raise ValueError(f"K = {K} is not a multiple of the format's group ({group(fmt)})")
    out = np.zeros(stage_bytes(fmt, N, K), np.uint8)
    lib().orc_quantize(fmt, _p(W), N, K, _p(out))
    return out


def _params(fmt, st, N, K):
    """bf16 scales [N][K/32] and (q4nx) mins of q4nx / q4s staging bytes"""
    v = np.asarray(st, np.uint8)[N * K // 2:].view(np.uint16)
    G = K // 32
    return v[:N * G].reshape(N, G), (v[N * G:2 * N * G].reshape(N, G) if fmt == FMT_Q4NX else None)


def npu_pack(fmt, W, ncols):
    """W [N][K] fp32 -> the reference's packed bytes for Mat(N, K, ncols, q4s?) (pack_mat,
    opennpu_core.hpp:230-254, with pack_block_fn :176-215), quantized by quantize(). Column block
    c = r S + s at c * cb; empty blocks zero. Inside a block, rows_col x ks codes (code 8 for q4s, 0
    for q4nx, past the matrix) and zero-padded parameters, streamed as packets [tile][K step][core
    row], each: nibbles [8 row octets][32 column octets][8 columns][4 row pairs] (even row in the low
    nibble), then bf16 scales [8 groups][64 rows], then (q4nx) mins likewise."""
    if fmt not in (FMT_Q4NX, FMT_Q4S):
        raise ValueError("the NPU packing holds q4nx or q4s")
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    sym = fmt == FMT_Q4S
    R, S, tiles, kc, ks, rows_col, cb, nbytes = geometry(N, K, ncols, sym)
    if nbytes == 0:
        raise ValueError(f"[{N}, {K}] has no geometry on {ncols} columns")
    st = quantize(fmt, W)
    q = unpack(fmt, st, N, K)
    sc, mn = _params(fmt, st, N, K)
    out = np.zeros(nbytes, np.uint8)
    for r in range(R):
        for s in range(S):
            r0, r1, k0, k1 = r * rows_col, min(N, (r + 1) * rows_col), s * ks, min(K, (s + 1) * ks)
            if r1 <= r0 or k1 <= k0:
                continue
            qb = np.full((rows_col, ks), 8 if sym else 0, np.uint8)
            qb[:r1 - r0, :k1 - k0] = q[r0:r1, k0:k1]
            # [core row, tile, packet row (8 octets x 8), K step, packet column (32 octets x 8)]
            qv = qb.reshape(4, tiles, 8, 8, kc, 32, 8).transpose(1, 4, 0, 2, 5, 6, 3)
            nib = (qv[..., 0::2] | (qv[..., 1::2] << 4)).reshape(tiles, kc, 4, 8192)
            parts = [nib]
            for a in ([sc] if sym else [sc, mn]):
                pb = np.zeros((rows_col, ks // 32), np.uint16)
                pb[:r1 - r0, :(k1 - k0) // 32] = a[r0:r1, k0 // 32:k1 // 32]
                pv = pb.reshape(4, tiles, 64, kc, 8).transpose(1, 3, 0, 4, 2)
                parts.append(np.ascontiguousarray(pv).view(np.uint8).reshape(tiles, kc, 4, 1024))
            c = r * S + s
            out[c * cb:(c + 1) * cb] = np.concatenate(parts, axis=3).ravel()
    return out


def npu_to_stage(fmt, buf, N, K, ncols, rowmap=None):
    """The inverse of npu_pack's layout: packed bytes of Mat(N, K, ncols) -> staging bytes of fmt;
    packed row r becomes staging row rowmap[r] (r without a map)."""
    sym = fmt == FMT_Q4S
    R, S, tiles, kc, ks, rows_col, cb, nbytes = geometry(N, K, ncols, sym)
    buf = np.asarray(buf, np.uint8)[:nbytes]
    q = np.zeros((N, K), np.uint8)
    pars = [np.zeros((N, K // 32), np.uint16) for _ in range(1 if sym else 2)]
    npar = len(pars)
    for r in range(R):
        for s in range(S):
            r0, r1, k0, k1 = r * rows_col, min(N, (r + 1) * rows_col), s * ks, min(K, (s + 1) * ks)
            if r1 <= r0 or k1 <= k0:
                continue
            c = r * S + s
            blk = buf[c * cb:(c + 1) * cb].reshape(tiles, kc, 4, 8192 + npar * 1024)
            nib = blk[..., :8192].reshape(tiles, kc, 4, 8, 32, 8, 4)
            qv = np.empty(nib.shape[:-1] + (8,), np.uint8)
            qv[..., 0::2], qv[..., 1::2] = nib & 15, nib >> 4
            qb = qv.transpose(2, 0, 3, 6, 1, 4, 5).reshape(rows_col, ks)
            q[r0:r1, k0:k1] = qb[:r1 - r0, :k1 - k0]
            for i, a in enumerate(pars):
                pv = np.ascontiguousarray(blk[..., 8192 + 1024 * i:8192 + 1024 * (i + 1)]).view(np.uint16)
                pb = pv.reshape(tiles, kc, 4, 8, 64).transpose(2, 0, 4, 1, 3).reshape(rows_col, ks // 32)
                a[r0:r1, k0 // 32:k1 // 32] = pb[:r1 - r0, :(k1 - k0) // 32]
    if rowmap is not None:
        order = np.empty(N, np.int64)
        order[np.asarray(rowmap)] = np.arange(N)
        q, pars = q[order], [a[order] for a in pars]
    codes = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return np.concatenate([codes.ravel()] + [a.ravel().view(np.uint8) for a in pars])


def ffn_order(Ng, Kg, Nd, Kd, sym):
    """The gate_up row packed at each row of a fused FFN's bank (onpu_ffn_perm, onpu_api.cpp:307-322):
    when the reference fuses the shape (one row block and one K slice per matrix, I = Ng / 2 = Kd a
    multiple of 256, all Ng rows in one column, Kg <= 2048, an even tile count), its NPU writes a
    column's outputs as [tile pair][core row][128 rows], and row r of the bank holds the gate_up row
    that lands at r's output position; else the identity."""
    perm = np.arange(Ng, dtype=np.int32)
    gg, gd = geometry(Ng, Kg, 1, sym), geometry(Nd, Kd, 1, sym)
    I = Ng // 2
    if not (gg[7] and gd[7] and gg[0] == gg[1] == gd[0] == gd[1] == 1 and Ng % 2 == 0 and Kd == I
            and I % 256 == 0 and gg[5] == Ng and Kg <= 2048 and gg[2] % 2 == 0):
        return perm
    tiles = gg[2]
    for t2 in range(tiles // 2):
        for cr in range(4):
            r = cr * tiles * 64 + t2 * 128
            perm[r:r + 128] = (t2 * 4 + cr) * 128 + np.arange(128)
    return perm


def stage_q4nx(q, s, m):
    """codes [N][K] + bf16 s, m [N][K/32] -> q4nx staging bytes (low nibble = even k)."""
    q = np.asarray(q, np.uint8)
    codes = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return np.concatenate([codes.ravel(), np.asarray(s, np.uint16).ravel().view(np.uint8),
                           np.asarray(m, np.uint16).ravel().view(np.uint8)])


def gemv_i8(W, s, x):
    """y[n] = s[n] * sum_k W[n][k] x[k] (onpu_cpu.cpp:276-299), fp64."""
    W = np.ascontiguousarray(W, np.int8)
    N, K = W.shape
    y = np.empty(N, np.float64)
    lib().orc_gemv_i8(_p(W), _p(np.ascontiguousarray(s, np.float32)), N, K, _p(np.ascontiguousarray(x, np.float32)),
                      _p(y))
    return y


def gdn_step(x, qkv, z, Wb, Wa, conv_w, conv_state, A_log, dt_bias, norm_w, eps, S, Hk, Hv, Dk, Dv):
    """One Gated DeltaNet decode token (onpu_cpu.cpp:107-171). conv_state [C][L] and S [Hv][Dk][Dv]
    are updated copies (returned with out [Hv*Dv])."""
    f = lambda a: np.ascontiguousarray(a, np.float32)
    x, qkv, z, Wb, Wa, conv_w = f(x), f(qkv), f(z), f(Wb), f(Wa), f(conv_w)
    A_log, dt_bias, norm_w = f(A_log), f(dt_bias), f(norm_w)
    cs, S = f(conv_state).copy(), f(S).copy()
    C_, L = cs.shape
    out = np.empty(Hv * Dv, np.float32)
    lib().orc_gdn_step(_p(x), x.size, _p(qkv), _p(z), _p(Wb), _p(Wa), _p(conv_w), conv_w.shape[1], _p(cs), L,
                       _p(A_log), _p(dt_bias), _p(norm_w), float(eps), _p(S), Hk, Hv, Dk, Dv, _p(out))
    return out, cs, S


def attn_step(q, K, V, mask=None, sinks=None, scale=None):
    """One decode token of GQA attention (onpu_cpu.cpp:180-229). q [Hq][D] fp32; K, V [Hkv][S][D]
    fp32 or bf16 bits (uint16); mask [S]; sinks [Hq]. Returns out [Hq][D] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    Hq, D = q.shape
    K = np.ascontiguousarray(K)
    V = np.ascontiguousarray(V)
    Hkv, S, _ = K.shape
    bf = int(K.dtype == np.uint16)
    out = np.empty((Hq, D), np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, np.float32)
    sk = None if sinks is None else np.ascontiguousarray(sinks, np.float32)
    lib().orc_attn_step(_p(q), Hq, D, _p(K), _p(V), bf, Hkv, S, S * D, D, None if m is None else _p(m),
                        None if sk is None else _p(sk), float(D ** -0.5 if scale is None else scale), _p(out))
    return out


# ------------------------------------------------------------------ CPU baseline kernels
_cpu = None


def cpu_lib():
    """oracle/_build/libcpuint4.so: the fused int4 CPU GEMV of the benchmark's CPU baseline
    (oracle/cpu_int4.c)."""
    global _cpu
    if _cpu is None:
        p = HERE / "_build" / "libcpuint4.so"
        if not p.exists():
            build()
        L = C.CDLL(str(p))
        P, I64, I32 = C.c_void_p, C.c_int64, C.c_int
        for n in ("cpu_g128s_mv", "cpu_q4_0_mv"):
            getattr(L, n).restype = I32
            getattr(L, n).argtypes = [P, I64, I64, P, I32, P, I32, I32]
        _cpu = L
    return _cpu


def cpu_mv(fmt, st, N, K, x, threads=1, isa_max=2):
    """y [M][N] fp32 = x [M][K] (fp32) . W^T by the fused CPU kernel (g128s or Q4_0, M <= 8);
    returns (y, instruction set used: 2 AVX-512, 1 AVX2, 0 scalar)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    fn = cpu_lib().cpu_g128s_mv if fmt == FMT_G128S else cpu_lib().cpu_q4_0_mv
    if fmt not in (FMT_G128S, FMT_Q4_0):
        raise ValueError("the CPU baseline kernel covers g128s and Q4_0")
    isa = fn(_p(np.ascontiguousarray(st)), N, K, _p(x), M, _p(y), threads, isa_max)
    if isa < 0:
        raise ValueError("cpu_mv: K off the format's group or M outside 1..8")
    return y, isa


def max_rel_err(y, r):
    """max|y - r| / max|r| (the tolerance BASELINE states; offload.py:313-315 reports rel-L2)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.abs(y - r).max() / max(np.abs(r).max(), 1e-30))


if __name__ == "__main__":
    build()
    print("oracle built:", LIB, os.path.getsize(LIB), "bytes")

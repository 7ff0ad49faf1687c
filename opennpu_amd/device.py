"""Device-resident operators over libonpu_hip's *_dev entry points, for callers holding torch
tensors in HBM (tests, the benchmark, a serving loop). torch supplies device memory and the
stream; every product is computed by the library's HIP kernels.

  QMatrix   one int4 matrix (any format): mv (y = x W^T), argmax (LM head), dequant
  QFfn      routed-expert FFN bank (gate_up + down): route, ffn
  QChain    a fixed sequence of QMatrix GEMVs run in order in one launch (onpu_chain_*)
"""
import ctypes as C

import numpy as np

from ._lib import check, require_gpu


def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _np_ptr(a):
    return C.c_void_p(a.ctypes.data)


class QMatrix:
    """An [N][K] int4 matrix resident in HBM (tiled layout), loaded from staging bytes."""

    def __init__(self, N, K, fmt, stage=None):
        self.L = require_gpu()
        self.N, self.K, self.fmt = int(N), int(K), int(fmt)
        self.h = self.L.onpu_dense_new3(self.N, self.K, self.fmt)
        if not self.h:
            raise ValueError(f"unsupported matrix [{N}, {K}] fmt {fmt}")
        if stage is not None:
            self.load(stage)

    def load(self, stage):
        stage = np.ascontiguousarray(stage, np.uint8)
        assert stage.size == self.L.onpu_stage_bytes(self.fmt, self.N, self.K)
        check(self.L.onpu_dense_load(self.h, _np_ptr(stage)), "onpu_dense_load")

    def quantize(self, W):
        """Quantize W (fp32 or bf16 cuda tensor [N][>=K], rows contiguous) on the GPU into this
        matrix, with the format's quantizer (the codes and parameters onpu_pack writes)."""
        import torch
        assert W.is_cuda and W.dtype in (torch.float32, torch.bfloat16) and W.dim() == 2 and W.stride(1) == 1
        assert W.shape[0] == self.N and W.shape[1] >= self.K
        check(self.L.onpu_quantize_dev(self.h, 0, 1, _ptr(W), W.stride(0), int(W.dtype == torch.bfloat16),
                                       _stream()), "onpu_quantize_dev")

    def transcode_q4k(self, blocks):
        """Load GGUF Q4_K rows (uint8 cuda tensor [N][K / 256 * 144]) into this q4nx matrix."""
        import torch
        assert blocks.is_cuda and blocks.dtype == torch.uint8 and blocks.dim() == 2 and blocks.stride(1) == 1
        assert blocks.shape[0] == self.N and blocks.shape[1] >= self.K // 256 * 144
        check(self.L.onpu_transcode_q4k_dev(self.h, 0, 1, _ptr(blocks), blocks.stride(0), _stream()),
              "onpu_transcode_q4k_dev")

    def mv(self, x, out=None, f32=False):
        """x: bf16 cuda tensor [M][K] -> y [M][N] (bf16, or fp32 when f32)."""
        import torch
        assert x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous() and x.shape[-1] == self.K
        M = x.numel() // self.K
        if out is None:
            out = torch.empty((M, self.N), dtype=torch.float32 if f32 else torch.bfloat16, device=x.device)
        check(self.L.onpu_dense_mv_dev(self.h, _ptr(x), M, _ptr(out), int(out.dtype == torch.float32), _stream()),
              "onpu_dense_mv_dev")
        return out

    def argmax(self, x, logits=None, idx=None):
        """LM head: fp32 logits [M][N] and their argmax [M] (int32)."""
        import torch
        M = x.numel() // self.K
        if logits is None:
            logits = torch.empty((M, self.N), dtype=torch.float32, device=x.device)
        if idx is None:
            idx = torch.empty((M,), dtype=torch.int32, device=x.device)
        check(self.L.onpu_dense_argmax_dev(self.h, _ptr(x), M, _ptr(logits), _ptr(idx), _stream()),
              "onpu_dense_argmax_dev")
        return logits, idx

    def dequant(self, bf16=False):
        """Dequantized weights as the GPU holds them: fp32 [N][K] or bf16 bits (uint16)."""
        out = np.empty((self.N, self.K), np.uint16 if bf16 else np.float32)
        check(self.L.onpu_dense_dequant(self.h, 0, _np_ptr(out), int(bf16)), "onpu_dense_dequant")
        return out

    def info(self):
        out = (C.c_int64 * 8)()
        self.L.onpu_dense_info(self.h, out)
        return tuple(out)

    def free(self):
        if self.h:
            self.L.onpu_dense_free(self.h)
            self.h = None


class QFfn:
    """E routed experts: gate_up [Ng = 2I][Kg] and down [Nd][Kd = I], one HBM pool each."""

    def __init__(self, E, H, I, fmt, Nd=None):
        self.L = require_gpu()
        self.E, self.H, self.I, self.fmt = int(E), int(H), int(I), int(fmt)
        self.Nd = int(Nd if Nd is not None else H)
        self.h = self.L.onpu_ffn_new3(2 * self.I, self.H, self.Nd, self.I, self.E, self.fmt)
        if not self.h:
            raise ValueError("unsupported expert shapes")
        self.gu = self.L.onpu_ffn_gu(self.h)
        self.dn = self.L.onpu_ffn_dn(self.h)

    def load(self, gu_stage, dn_stage, e0=0):
        """gu_stage / dn_stage: n experts' staging bytes, concatenated."""
        gu_stage = np.ascontiguousarray(gu_stage, np.uint8)
        dn_stage = np.ascontiguousarray(dn_stage, np.uint8)
        sg = self.L.onpu_stage_bytes(self.fmt, 2 * self.I, self.H)
        n = gu_stage.size // sg
        check(self.L.onpu_bank_load(self.gu, e0, n, _np_ptr(gu_stage)), "onpu_bank_load")
        check(self.L.onpu_bank_load(self.dn, e0, n, _np_ptr(dn_stage)), "onpu_bank_load")

    def quantize(self, gu_w, dn_w, e0=0):
        """Quantize n experts on the GPU into experts [e0, e0 + n): gu_w [n][2I][H] and dn_w
        [n][Nd][I], fp32 or bf16 contiguous cuda tensors."""
        import torch
        for w, h, N, K in ((gu_w, self.gu, 2 * self.I, self.H), (dn_w, self.dn, self.Nd, self.I)):
            assert w.is_cuda and w.dtype in (torch.float32, torch.bfloat16) and w.is_contiguous()
            assert w.dim() == 3 and tuple(w.shape[1:]) == (N, K)
            check(self.L.onpu_quantize_dev(h, e0, w.shape[0], _ptr(w), K, int(w.dtype == torch.bfloat16),
                                           _stream()), "onpu_quantize_dev")

    def route(self, logits, k, renorm=True):
        """logits fp32 cuda [T][E] -> ids int32 [T][k], w fp32 [T][k]."""
        import torch
        T = logits.shape[0]
        ids = torch.empty((T, k), dtype=torch.int32, device=logits.device)
        w = torch.empty((T, k), dtype=torch.float32, device=logits.device)
        check(self.L.onpu_moe_route_dev(_ptr(logits), T, logits.shape[1], k, int(renorm), _ptr(ids), _ptr(w),
                                        _stream()), "onpu_moe_route_dev")
        return ids, w

    def ffn(self, x, ids, w, out=None, f32=False):
        """x bf16 [T][H], ids/w [T][k] -> y [T][Nd] = sum_j w_j down_e(silu(gate_e x) * up_e x)."""
        import torch
        T, k = ids.shape
        if out is None:
            out = torch.empty((T, self.Nd), dtype=torch.float32 if f32 else torch.bfloat16, device=x.device)
        check(self.L.onpu_moe_ffn_dev(self.h, _ptr(x), T, _ptr(ids), k, _ptr(w), _ptr(out),
                                      int(out.dtype == torch.float32), _stream()), "onpu_moe_ffn_dev")
        return out

    def decode(self, logits, x, k, renorm=True, out=None, f32=False, ids=None, w=None):
        """router + FFN from logits fp32 [T][E] and x bf16 [T][H]: returns (y [T][Nd], ids int32 [T][k],
        w fp32 [T][k]); out, ids and w may be given."""
        import torch
        T, E = logits.shape
        if ids is None:
            ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
        if w is None:
            w = torch.empty((T, k), dtype=torch.float32, device=x.device)
        if out is None:
            out = torch.empty((T, self.Nd), dtype=torch.float32 if f32 else torch.bfloat16, device=x.device)
        check(self.L.onpu_moe_decode_dev(self.h, _ptr(logits), _ptr(x), T, E, k, int(renorm), _ptr(ids), _ptr(w),
                                         _ptr(out), int(out.dtype == torch.float32), _stream()),
              "onpu_moe_decode_dev")
        return out, ids, w

    def status(self):
        """1 if a one-launch decode gave up waiting since the last call (then cleared), else 0"""
        return self.L.onpu_moe_status(self.h)

    def free(self):
        if self.h:
            self.L.onpu_ffn_free(self.h)
            self.h = None


class QChain:
    """GEMVs y_i = x_i . W_i^T over QMatrix handles, executed in order in one launch (x_i may be an
    earlier entry's y: that entry publishes y as tagged link words and entry i waits, bounded, until
    every word it reads carries the run's tag). xs / ys: bf16 (ys fp32 if f32) cuda tensors [M][K_i]
    / [M][N_i], fixed for the life of the chain; keep them alive."""

    def __init__(self, mats, xs, ys, f32=False):
        self.L = require_gpu()
        n = len(mats)
        assert n == len(xs) == len(ys) and n > 0
        M = xs[0].numel() // mats[0].K
        for q, x, y in zip(mats, xs, ys):
            assert x.is_cuda and y.is_cuda and x.numel() == M * q.K and y.numel() == M * q.N
        P = C.c_void_p * n
        self._keep = (list(mats), list(xs), list(ys))
        self.h = self.L.onpu_chain_new(P(*[C.c_void_p(q.h) for q in mats]), P(*[_ptr(x) for x in xs]),
                                       P(*[_ptr(y) for y in ys]), n, M, int(f32))
        if not self.h:
            raise RuntimeError(f"onpu_chain_new: {self.L.onpu_last_error().decode()}")

    def run(self):
        check(self.L.onpu_chain_run(self.h, _stream()), "onpu_chain_run")

    def status(self):
        return self.L.onpu_chain_status(self.h)

    def info(self):
        out = (C.c_int64 * 6)()
        self.L.onpu_chain_info(self.h, out)
        return tuple(out)

    def free(self):
        if self.h:
            self.L.onpu_chain_free(self.h)
            self.h = None


def attn_step(q, K, V, mask=None, sinks=None, scale=None, out=None, ws=None):
    """One decode token of grouped-query attention on the GPU (onpu_attn_step_dev): q fp32 [Hq][D];
    K, V [Hkv][S][D] fp32 or bf16 cuda views with unit stride in D and the same strides (a KV
    cache slice); mask fp32 [S] or None; sinks fp32 [Hq] or None. Returns out fp32 [Hq][D]."""
    import torch
    L = require_gpu()
    Hq, D = q.shape
    Hkv, S, _ = K.shape
    assert q.dtype == torch.float32 and q.is_contiguous() and K.dtype == V.dtype
    assert K.stride() == V.stride() and K.stride(2) == 1 and K.shape == V.shape and K.shape[2] == D
    if out is None:
        out = torch.empty((Hq, D), dtype=torch.float32, device=q.device)
    nb = L.onpu_attn_ws_bytes(Hq, D, Hkv, S)
    if ws is None or ws.numel() < nb:
        ws = torch.empty((max(nb, 4),), dtype=torch.uint8, device=q.device)
    check(L.onpu_attn_step_dev(_ptr(q), Hq, D, _ptr(K), _ptr(V), int(K.dtype == torch.bfloat16), Hkv, S,
                               K.stride(0), K.stride(1), None if mask is None else _ptr(mask),
                               None if sinks is None else _ptr(sinks), float(D ** -0.5 if scale is None else scale),
                               _ptr(out), _ptr(ws), ws.numel(), _stream()), "onpu_attn_step_dev")
    return out

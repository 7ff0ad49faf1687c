"""The reference's npu4 operator surface for the int4 matmul path, over libonpu_hip.

Mirrors the pieces of opennpu/native/npu4/model.py that reach the int4 kernels through libonpu:
clib() (model.py:281-335), Mat (:151-217), quant_dequant (:343-350), check_geometry (:353-360),
CArena (:363-379), NPULinearGroup (:789-862), NPULinear (:865-880), NPUExperts with its
libonpu paths _init_c/_forward_c (:883-1020) and expert_cols (:1174-1184). Names, arguments and
the C calls they make are the reference's, so the reference module itself runs unchanged over
this library (OPENNPU_LIBONPU=<repo>/opennpu_amd/libonpu_hip.so). What differs is where no
XDNA2 device exists: there is no pyxrt fallback — a missing or unusable library raises instead of
silently computing somewhere else — and the on-disk pack cache is out of scope (cache must be None).
"""
import ctypes as C
import os

import numpy as np

from . import _lib

NC = 8                                       # device columns the reference's geometry packs for
FUSE_FFN = os.environ.get("OPENNPU_NPU4_FUSE_FFN", "1") != "0"     # model.py:654
FUSE_T_MAX = 1                                                   # model.py:657
FUSE_MANY = os.environ.get("OPENNPU_NPU4_FUSE_MANY", "0") == "1"  # model.py:658

_CLIB = [False, None]


def clib():
    """libonpu_hip with the reference loader's rules (model.py:281-335): None when
    OPENNPU_NPU4_CLIB=0, when the file is missing or does not load, when it lacks
    onpu_dense_new2, or when onpu_ok() != 1."""
    if _CLIB[0]:
        return _CLIB[1]
    _CLIB[0] = True
    if os.environ.get("OPENNPU_NPU4_CLIB", "1") == "0":
        return None
    try:
        lib = _lib.lib()
    except _lib.LibraryMissing:
        return None
    if not hasattr(lib, "onpu_dense_new2") or lib.onpu_ok() != 1:
        return None
    _CLIB[1] = lib
    return lib


def _need():
    lib = clib()
    if lib is None:
        raise RuntimeError(f"libonpu_hip is not usable ({_lib.LIB_PATH}): this build has no other device path")
    return lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class Mat:
    """Geometry of an [N, K] matrix on `ncols` device columns as the reference computes it
    (model.py:151-187), read from onpu_geometry2 so it is the library's own. The MI355X layout
    lives inside the nbytes buffer (onpu_pack writes it), so only the sizes matter here.
    Geometry, pack and quant_dequant are host code: they need the library, not a GPU."""

    def __init__(self, N, K, ncols, sym=False):
        self.N, self.K, self.ncols, self.sym = N, K, ncols, sym
        out = (C.c_int64 * 8)()
        _lib.lib().onpu_geometry2(N, K, ncols, int(sym), out)
        if out[7] == 0:
            raise ValueError(f"[{N}, {K}] needs more than {ncols} columns of K <= 2048")
        self.R, self.S, self.tiles, self.kc, self.ks, self.rows_col, self.cb, self.nbytes = (int(v) for v in out)

    def shapes(self):
        return {(self.tiles, self.kc)}

    def pack(self, W, threads=1):
        """W [N, K] float -> the library's packed bytes (nbytes), via onpu_pack (model.py:189-200)."""
        W = np.ascontiguousarray(W, np.float32)
        out = np.empty(self.nbytes, np.uint8)
        n = _lib.lib().onpu_pack(_fp(W), self.N, self.K, self.ncols, int(self.sym),
                              out.ctypes.data_as(C.POINTER(C.c_uint8)), threads)
        if n != self.nbytes:
            raise ValueError(f"onpu_pack cannot pack [{self.N}, {self.K}] (K % 32 != 0?)")
        return out


def quant_dequant(W, sym=False):
    """What the device makes of W [N, K] (model.py:343-350)."""
    W = np.ascontiguousarray(W, np.float32)
    out = np.empty_like(W)
    _lib.lib().onpu_quant_dequant(_fp(W), W.shape[0], W.shape[1], int(sym), _fp(out), 8)
    return out


def check_geometry(m):
    """The library must pack exactly like Mat (model.py:353-360)."""
    out = (C.c_int64 * 8)()
    _lib.lib().onpu_geometry2(m.N, m.K, m.ncols, int(m.sym), out)
    want = (m.R, m.S, m.tiles, m.kc, m.ks, m.rows_col, m.cb, m.nbytes)
    if tuple(out) != want:
        raise RuntimeError(f"libonpu geometry {tuple(out)} != {want}")


class CArena:
    """Python packs into a library buffer; sync hands it to the device (model.py:363-379)."""

    def __init__(self, ptr, nbytes, sync):
        self.n = int(nbytes)
        self.view = np.ctypeslib.as_array(ptr, shape=(self.n,))
        self.used = 0
        self._sync = sync

    def put(self, blob):
        o = self.used
        self.view[o:o + blob.size] = blob
        self.used += blob.size
        return o

    def sync(self):
        self._sync()


def expert_cols(topk, N=None, K=None):
    """Columns per expert (model.py:1174-1184)."""
    c = NC // topk if topk <= NC and NC % topk == 0 else 1
    while N is not None and c < NC:
        try:
            Mat(N, K, c)
            break
        except ValueError:
            c *= 2
    return c


class NPULinearGroup:
    """Sibling Linears reading the same input, stacked into one matrix (model.py:789-862): the first
    call computes all of them for that input (one onpu_dense_mv), the others take their slice.
    residual: rows [W; W - quant_dequant(W)] (two 4-bit passes, ~8-bit precision), halves added."""

    def __init__(self, names, weights, sizes=None, K=None, cache=None, key=None, sym=False, residual=False):
        if cache is not None:
            raise NotImplementedError("the on-disk pack cache is not part of this build")
        lib = _need()
        self.names = names
        self.sizes = sizes or [w.shape[0] for w in weights]
        self.residual, self.N1 = residual, sum(self.sizes)
        self.m = Mat(self.N1 * (2 if residual else 1), K if K is not None else weights[0].shape[1], NC, sym)
        check_geometry(self.m)
        self.ch = lib.onpu_dense_new2(self.m.N, self.m.K, int(sym))
        if not self.ch:
            raise RuntimeError(f"onpu_dense_new2 rejected [{self.m.N}, {self.m.K}] sym={int(sym)}: "
                               f"{lib.onpu_last_error().decode()}")
        self.arena = CArena(lib.onpu_dense_buf(self.ch), self.m.nbytes, lambda: lib.onpu_dense_sync(self.ch))
        ws = weights() if callable(weights) else weights
        W = np.ascontiguousarray(np.concatenate(ws) if len(ws) > 1 else ws[0], np.float32)
        if residual:
            W = np.concatenate([W, W - quant_dequant(W, self.m.sym)])
        self.arena.put(self.m.pack(W, threads=8))
        self.arena.sync()
        self._key, self._y = None, None

    def compute(self, x, i):
        """x: the caller's input tensor; siblings pass the same object and share one product."""
        if self._key is None or self._key[0] is not x or self._key[1] != x._version:
            xf = np.ascontiguousarray(x.detach().reshape(-1, x.shape[-1]).float().cpu().numpy())
            self._y = np.empty((len(xf), self.m.N), np.float32)
            _need().onpu_dense_mv(self.ch, _fp(xf), len(xf), _fp(self._y))
            if self.residual:
                self._y = self._y[:, :self.N1] + self._y[:, self.N1:]
            self._key = (x, x._version)
        o = sum(self.sizes[:i])
        return self._y[:, o:o + self.sizes[i]]

    def full(self, x):
        self.compute(x, 0)
        return self._y


def _module_base():
    import torch
    return torch.nn.Module


class NPULinear(_module_base()):
    """One sibling of an NPULinearGroup as an nn.Module (model.py:865-880)."""

    def __init__(self, group, i, in_features, out_features, bias):
        import torch
        super().__init__()
        self.group, self.i = group, i
        self.in_features, self.out_features = in_features, out_features
        self.bias = torch.nn.Parameter(bias, requires_grad=False) if bias is not None else None

    def forward(self, x):
        import torch
        shp = x.shape
        y = torch.from_numpy(np.ascontiguousarray(self.group.compute(x, self.i)))
        if self.bias is not None:
            y = y + self.bias.float()
        return y.to(x.dtype).reshape(*shp[:-1], self.out_features)

    def extra_repr(self):
        return f"{self.in_features} -> {self.out_features}, int4 on the MI355X"


class NPUExperts(_module_base()):
    """A 3-D expert bank (model.py:883-1089): forward(hidden [T, H], indices [T, k], weights [T, k]).
    Paths, in the reference's order: one fused FFN call per token (onpu_ffn_run, T <= FUSE_T_MAX),
    tokens grouped per expert (onpu_ffn_run_many, FUSE_MANY), onpu_moe_ffn (SiLU or gpt-oss act
    done by the library), else two onpu_bank_run calls with the activation in torch."""

    def __init__(self, orig, gu, dn, topk, gu_bias=None, dn_bias=None, pool=None, shapes=None, E=None,
                 cache=None, key=None, sym=False):
        import torch
        super().__init__()
        if cache is not None:
            raise NotImplementedError("the on-disk pack cache is not part of this build")
        gs, ds = shapes if shapes else (gu[0].shape, dn[0].shape)
        self.E = E if E is not None else len(gu)
        self.topk = topk
        self.mgu = Mat(*gs, expert_cols(topk, *gs), sym)
        self.mdn = Mat(*ds, expert_cols(topk, *ds), sym)
        self.gu_bias, self.dn_bias = gu_bias, dn_bias
        self.apply_gate = getattr(orig, "_apply_gate", None)
        self.act_fn = getattr(orig, "act_fn", None)
        self.act_kind, self.alpha, self.limit = None, 0.0, 0.0
        if self.apply_gate is not None and hasattr(orig, "alpha") and hasattr(orig, "limit"):
            self.act_kind, self.alpha, self.limit = 1, float(orig.alpha), float(orig.limit)
        elif self.act_fn is torch.nn.functional.silu or type(self.act_fn).__name__ in ("SiLU", "SiLUActivation"):
            self.act_kind = 0
        self._init_c(_need(), gu, dn, pool)

    def _init_c(self, lib, gu, dn, pool):
        check_geometry(self.mgu)
        check_geometry(self.mdn)
        E, g, d = self.E, self.mgu.nbytes, self.mdn.nbytes
        self.cffn, perm = None, None
        if FUSE_FFN and self.act_kind == 0 and self.gu_bias is None and self.dn_bias is None \
                and self.mgu.ncols == 1 and self.mdn.ncols == 1 and self.topk == NC:
            f = lib.onpu_ffn_new(self.mgu.N, self.mgu.K, self.mdn.N, self.mdn.K, E, int(self.mgu.sym))
            if f and lib.onpu_ffn_fused(f):
                self.cffn, self.cgu, self.cdn = f, lib.onpu_ffn_gu(f), lib.onpu_ffn_dn(f)
                perm = np.empty(self.mgu.N, np.int32)
                lib.onpu_ffn_perm(f, perm.ctypes.data_as(C.POINTER(C.c_int32)))
            elif f:
                lib.onpu_ffn_free(f)
        if self.cffn is None:
            self.cgu = lib.onpu_bank_new2(self.mgu.N, self.mgu.K, E, self.mgu.ncols, int(self.mgu.sym))
            self.cdn = lib.onpu_bank_new2(self.mdn.N, self.mdn.K, E, self.mdn.ncols, int(self.mdn.sym))
        if not (self.cgu and self.cdn):
            raise RuntimeError(f"libonpu_hip rejected the expert shapes: {lib.onpu_last_error().decode()}")
        vg = np.ctypeslib.as_array(lib.onpu_bank_buf(self.cgu), shape=(E, g))
        vd = np.ctypeslib.as_array(lib.onpu_bank_buf(self.cdn), shape=(E, d))
        if callable(gu):
            gu, dn = gu()

        def one(e):
            vg[e] = self.mgu.pack(gu[e] if perm is None else np.asarray(gu[e])[perm])
            vd[e] = self.mdn.pack(dn[e])
        list((pool.map if pool else map)(one, range(E)))
        lib.onpu_bank_sync(self.cgu)
        lib.onpu_bank_sync(self.cdn)

    def _forward_c(self, h, idx, w):
        lib = _need()
        T, k = idx.shape
        ids = np.ascontiguousarray(idx, np.int32)
        ip = ids.ctypes.data_as(C.POINTER(C.c_int32))
        h = np.ascontiguousarray(h, np.float32)
        if T <= FUSE_T_MAX and self.cffn is not None:
            wf = np.ascontiguousarray(w, np.float32)
            y = np.empty((T, self.mdn.N), np.float32)
            if all(lib.onpu_ffn_run(self.cffn, _fp(h[t:t + 1]), ids[t].ctypes.data_as(C.POINTER(C.c_int32)), k,
                                    _fp(wf[t:t + 1]), _fp(y[t:t + 1])) for t in range(T)):
                return y
        if T > 1 and self.cffn is not None and FUSE_MANY:
            wf = np.ascontiguousarray(w, np.float32)
            y = np.empty((T, self.mdn.N), np.float32)
            if lib.onpu_ffn_run_many(self.cffn, _fp(h), T, ip, k, _fp(wf), _fp(y)):
                return y
        if self.act_kind is not None:
            f = (lambda b: None if b is None else np.ascontiguousarray(np.asarray(b), np.float32))
            gb, db = f(self.gu_bias), f(self.dn_bias)
            w = np.ascontiguousarray(w, np.float32)
            y = np.empty((T, self.mdn.N), np.float32)
            lib.onpu_moe_ffn(self.cgu, self.cdn, _fp(h), T, ip, k, _fp(w), self.act_kind, self.alpha, self.limit,
                             None if gb is None else _fp(gb), None if db is None else _fp(db), _fp(y))
            return y
        gu = np.empty((T, k, self.mgu.N), np.float32)
        lib.onpu_bank_run(self.cgu, _fp(h), 0, T, ip, k, _fp(gu))
        if self.gu_bias is not None:
            gu += self.gu_bias[idx]
        act = np.ascontiguousarray(self._act(gu.reshape(T * k, -1)), np.float32)
        dn = np.empty((T, k, self.mdn.N), np.float32)
        lib.onpu_bank_run(self.cdn, _fp(act), 1, T, ip, k, _fp(dn))
        if self.dn_bias is not None:
            dn += self.dn_bias[idx]
        return (dn * w[:, :, None]).sum(1)

    def _act(self, gu):
        import torch
        t = torch.from_numpy(gu)
        if self.apply_gate is not None:
            return self.apply_gate(t).numpy()
        gate, up = t.chunk(2, dim=-1)
        return (self.act_fn(gate) * up).numpy()

    def shapes(self):
        return self.mgu.shapes() | self.mdn.shapes()

    def forward(self, hidden_states, indices, weights):
        import torch
        h = hidden_states.detach().float().cpu().numpy()
        idx = indices.detach().cpu().numpy()
        w = weights.detach().float().cpu().numpy()
        return torch.from_numpy(self._forward_c(h, idx, w)).to(hidden_states.dtype)

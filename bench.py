"""Benchmark of the int4 weight-only matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline workload (one "step"): the int4 weight stream of one Qwen3-8B decode token, i.e. the 36
layers' g128s GEMVs at M=1: fused QKV 6144x4096, o 4096x4096, fused gate+up 24576x4096 and down
4096x12288, each layer with its own HBM copy of the weights (3.58 GB per step, far above the
256 MB Infinity Cache), each GEMV reading the previous one's output. The step runs as per-launch
kernels captured in one HIP graph and as one chained launch (captured too); the faster is the
headline (config.launch says which). value = algorithmic bytes per step (int4 codes + bf16 scales
+ x + y) / time, in GB/s.

Also measured in the same run (the "configs" object): M=4 and M=8 decode steps, a single
4096x4096 GEMV rotated over 64 copies, the Llama-3.1-8B prefill FFN GEMMs (M=2048, TFLOPS), the
same GEMMs at 96 rows and the Q4_0 LM head at 16 rows (the GEMM at few rows), the Qwen3-30B-A3B
MoE layer (decode M=1 and prefill M=512, router included), and the 151936x4096
Q4_0 LM head with argmax (M=1, 5), the load-time weight codecs on one layer (GPU quantization
into each format and the GGUF Q4_K transcode, beside the host quantizer), and the per-token steps
the reference runs on the host (decode attention, the int8 shared-expert GEMV). The roofline object is the dominant kernel: the gate+up GEMV,
timed with HIP events over a graph of back-to-back launches on its stream. The cpu_baseline leg
times the reference's own CPU pattern (dequantize to fp32, then x @ W^T in torch fp32,
opennpu/native/reference.py:24-28,55) on one layer of the same workload.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "int4 GEMV HBM GB/s (% peak) + prefill GEMM TFLOPS at 8B / 30B-A3B shapes"
HBM_PEAK = 8.0e12            # MI355X HBM3E, B/s
BF16_PEAK = 2.5e15           # MI355X dense bf16 MFMA, flop/s
G128S, Q4_0 = 2, 3
LAYERS = 36                  # Qwen3-8B
QWEN3_8B = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096), ("down", 4096, 12288)]
# HBM bytes moved per gate+up launch (M=1), from rocprofv3 FETCH_SIZE and WRITE_SIZE runs of
# `bench.py --profile`, each scaled by what the counter reads for a plain 512 MiB copy
# (profiles/qgemv_g128s_gate_up_24576x4096_pmc.md); a hardware-counter figure, not re-measured here
GATE_UP_TRAFFIC = 52_218_291


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def unit_gain_sigma(K):
    """scale sigma for which a g128s GEMV over K has a gain of ~1: sqrt(K * 21.5) * sigma = 1, with
    21.5 the mean of (u - 8)^2 over uniform codes"""
    return 1.0 / np.sqrt(21.5 * K)


def wbytes(fmt, N, K):
    """algorithmic weight bytes: int4 codes + scales"""
    if fmt == Q4_0:
        return N * (K // 32) * 18
    return N * K // 2 + N * (K // 128) * 2


class GraphStep:
    """A list of launches captured in one HIP graph (falls back to eager launches)."""

    def __init__(self, fn, torch):
        self.torch, self.fn = torch, fn
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()                              # warm: first launches load the code object
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.g = None
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn()
            self.g = g
        except Exception as e:  # noqa: BLE001 - eager launches still measure the kernels
            log(f"graph capture failed ({e}); timing eager launches")
        self.mode = "hip_graph" if self.g is not None else "eager"

    def __call__(self):
        if self.g is not None:
            self.g.replay()
        else:
            self.fn()


def time_it(torch, step, iters, warmup):
    """mean seconds per call of step(), HIP events on the current stream"""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        step()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / iters


# Each timed graph of a config repeats its calls this often, so that the gap between two graph
# launches (several microseconds) is spread over many calls, as inside a longer decode step
GRAPH_REPS = 4


def time_med(torch, step, iters, warmup, windows=5):
    """median over `windows` back-to-back timed windows of `iters` calls each (the first after
    `warmup` calls) of the mean seconds per call: one slow window (a clock change) does not move it"""
    return float(np.median([time_it(torch, step, iters, warmup if w == 0 else 0) for w in range(windows)]))


def bf16_tensor(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


# ------------------------------------------------------------------ workloads
def decode_layers(torch, QMatrix, QChain, syn, Ms, steps, warmup):
    """the headline step at each M; returns {M: result}. At M = 1 the step is one decode token's
    dependent GEMVs: qkv reads the previous layer's down output (layer 0: an input row), o reads the
    first 4096 values of qkv (standing in for the attention output), gate+up reads o, down reads the
    first 12288 values of gate+up (standing in for SiLU(gate) * up). It runs as per-launch kernels in
    one HIP graph and as one chained launch (entries wait for the outputs they read) in a graph; the
    faster is the headline. The step has no normalisation, so the synthetic scales are drawn as
    config 0's |N(0, sigma)| + 1e-4 with sigma = 1 / sqrt(21.5 K) instead of 0.02 and a random sign:
    uniform codes give u - 8 a mean of -1/2, which positive scales turn into a common component that
    grows ~7x per GEMV; with signed scales the weights have mean zero, 21.5 is the mean of (u - 8)^2,
    and each output keeps its input's RMS, so all 144 outputs stay finite (signs and magnitudes do
    not change the bytes or the kernels). Every output of the chained launch is compared with the
    per-launch graph's, starting from cleared outputs. At M = 4, 8 the GEMVs read fixed inputs
    (per-launch graph only)."""
    mats = {}
    for name, N, K in QWEN3_8B:
        st = syn.weights(G128S, N, K, 100 + N + K, scale_sigma=unit_gain_sigma(K), signed=True)
        mats[name] = [QMatrix(N, K, G128S, st) for _ in range(LAYERS)]
        del st
    res = {}
    byts_of = lambda M: LAYERS * sum(wbytes(G128S, N, K) + M * K * 2 + M * N * 2 for _, N, K in QWEN3_8B)
    for M in Ms:
        xs = {K: bf16_tensor(torch, syn.activations(M, K, K + M)).reshape(M, K) for K in (4096, 12288)}
        byts = byts_of(M)
        if M == 1:
            h0 = xs[4096]
            ys = {name: [torch.zeros((1, N), dtype=torch.bfloat16, device="cuda") for _ in range(LAYERS)]
                  for name, N, _ in QWEN3_8B}

            def x_of(name, layer):
                if name == "qkv":
                    return h0 if layer == 0 else ys["down"][layer - 1]
                if name == "o":
                    return ys["qkv"][layer][:, :4096]
                if name == "gate_up":
                    return ys["o"][layer]
                return ys["gate_up"][layer][:, :12288]

            order = [(name, layer) for layer in range(LAYERS) for name, _, _ in QWEN3_8B]

            def step():
                for name, layer in order:
                    mats[name][layer].mv(x_of(name, layer), out=ys[name][layer])
        else:
            ys = {name: torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for name, N, _ in QWEN3_8B}

            def step(M=M, xs=xs, ys=ys):
                for layer in range(LAYERS):
                    for name, N, K in QWEN3_8B:
                        mats[name][layer].mv(xs[K], out=ys[name])

        g = GraphStep(step, torch)
        # the graph's outputs, from cleared outputs, equal eager launches' bit for bit, and are finite
        outs = [ys[name][layer] for name, layer in order] if M == 1 else list(ys.values())
        for y in outs:
            y.zero_()
        g()
        torch.cuda.synchronize()
        y_graph = [y.clone() for y in outs]
        assert all(bool(torch.isfinite(y.float()).all()) for y in y_graph), "a decode output is not finite"
        step()
        torch.cuda.synchronize()
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(y_graph, outs)), \
            "graph replay differs from eager launches"
        t = time_it(torch, g, steps, warmup)
        res[M] = {"ms_per_step": t * 1e3, "GBps": byts / t / 1e9, "hbm_frac": byts / t / HBM_PEAK,
                  "bytes_per_step": byts, "tokens_per_s_equiv": M / t, "launch": g.mode}
        if M == 1:
            ch = QChain([mats[nm][ly] for nm, ly in order], [x_of(nm, ly) for nm, ly in order], outs)
            res[M]["chained"] = chained(torch, ch, outs, y_graph, byts, steps, warmup)
        else:
            res[M]["chained"] = {"skipped": "chained entries link to earlier outputs at M = 1 (this step reads "
                                            "ranges of them)"}
        # per-matrix kernels: a graph of the 36 copies of each matrix, back to back, fixed inputs
        per = {}
        yp = {name: torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for name, N, _ in QWEN3_8B}
        for name, N, K in QWEN3_8B:
            def one(name=name, K=K):
                for layer in range(LAYERS):
                    mats[name][layer].mv(xs[K], out=yp[name])
            gm = GraphStep(one, torch)
            tm = time_med(torch, gm, max(20, steps // 2), 3) / LAYERS
            b1 = wbytes(G128S, N, K) + M * K * 2 + M * N * 2
            per[name] = {"us": tm * 1e6, "GBps": b1 / tm / 1e9, "hbm_frac": b1 / tm / HBM_PEAK, "bytes": b1}
        res[M]["per_matrix"] = per
    for v in mats.values():
        for q in v:
            q.free()
    return res


def chained(torch, ch, outs, ref, byts, steps, warmup):
    """the decode step's GEMVs as one chained launch (each entry waits for the output it reads).
    From cleared outputs, every entry's output is compared with the per-launch graph's: the chain
    splits K differently, so the two differ by fp32 and bf16 rounding, compounding over the 144
    dependent entries (relative L2 ~1e-2 at the end); an entry that read its input before it was
    written would read zeros and differ by ~1."""
    gc = GraphStep(ch.run, torch)
    for y in outs:
        y.zero_()
    gc()
    torch.cuda.synchronize()
    worst = 0.0
    for i, (got, want) in enumerate(zip(outs, ref)):
        d = float((got.float() - want.float()).norm() / want.float().norm())
        assert d <= 0.1, f"chained entry {i} differs from the per-launch result: relative L2 {d:.3e}"
        worst = max(worst, d)
    tc = time_it(torch, gc, steps, warmup)
    if ch.status() != 0:
        raise RuntimeError("chained decode: a wait for an earlier entry's output timed out")
    ch.free()
    return {"ms_per_step": tc * 1e3, "GBps": byts / tc / 1e9, "hbm_frac": byts / tc / HBM_PEAK,
            "launch": "one chained launch per step (" + gc.mode + ")",
            "max_rel_l2_vs_per_launch": worst}


def config0(torch, QMatrix, syn, iters):
    N = K = 4096
    st = syn.weights(G128S, N, K, 0)
    copies = [QMatrix(N, K, G128S, st) for _ in range(64)]     # 555 MB rotation
    x = bf16_tensor(torch, syn.activations(1, K, 1)).reshape(1, K)
    y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")

    def step():
        for q in copies:
            q.mv(x, out=y)
    g = GraphStep(step, torch)
    t = time_med(torch, g, iters, 3) / len(copies)
    b = wbytes(G128S, N, K) + K * 2 + N * 2
    for q in copies:
        q.free()
    return {"us_per_call": t * 1e6, "GBps": b / t / 1e9, "hbm_frac": b / t / HBM_PEAK, "bytes": b}


def prefill(torch, QMatrix, syn, iters):
    out = {}
    M = 2048
    for name, N, K in [("up", 14336, 4096), ("down", 4096, 14336)]:
        q = QMatrix(N, K, G128S, syn.weights(G128S, N, K, 7))
        x = bf16_tensor(torch, syn.activations(M, K, 8)).reshape(M, K)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        def step(q=q, x=x, y=y):
            for _ in range(GRAPH_REPS):
                q.mv(x, out=y)
        g = GraphStep(step, torch)
        t = time_med(torch, g, iters, 3) / GRAPH_REPS
        fl = 2.0 * M * N * K
        out[name] = {"us_per_call": t * 1e6, "TFLOPS": fl / t / 1e12, "mfma_frac": fl / t / BF16_PEAK}
        q.free()
    return out


def few_rows(torch, QMatrix, syn, iters):
    """the GEMM at few rows (speculative verification, a prompt chunk, batched decode): the
    Llama-3.1-8B FFN at 96 rows (128-row tiles split along K), and the Q4_0 LM head with argmax at 16
    rows (16-row tiles); each over >= 600 MB of distinct weight copies, so HBM serves every call"""
    out = {}
    for name, fmt, N, K, M in [("ffn_up_M96", G128S, 14336, 4096, 96), ("ffn_down_M96", G128S, 4096, 14336, 96),
                               ("lm_head_q4_0_M16", Q4_0, 151936, 4096, 16)]:
        st = syn.weights(fmt, N, K, 13)
        copies = [QMatrix(N, K, fmt, st) for _ in range(max(2, -(-600_000_000 // st.nbytes)))]
        x = bf16_tensor(torch, syn.activations(M, K, 14)).reshape(M, K)
        lm = name.startswith("lm_head")
        y = torch.empty((M, N), dtype=torch.float32 if lm else torch.bfloat16, device="cuda")
        idx = torch.empty((M,), dtype=torch.int32, device="cuda")

        def step(x=x, y=y, idx=idx, copies=copies, lm=lm):
            for q in copies:
                if lm:
                    q.argmax(x, y, idx)
                else:
                    q.mv(x, out=y)
        g = GraphStep(step, torch)
        t = time_med(torch, g, iters, 3) / len(copies)
        b = wbytes(fmt, N, K) + M * K * 2 + M * N * (4 if lm else 2)
        fl = 2.0 * M * N * K
        out[name] = {"us_per_call": t * 1e6, "GBps": b / t / 1e9, "hbm_frac": b / t / HBM_PEAK,
                     "TFLOPS": fl / t / 1e12}
        for q in copies:
            q.free()
    return out


MOE_COPIES, MOE_ROUNDS = 8, 4


def moe_layers(QFfn, syn):
    """Qwen3-30B-A3B MoE layer (E 128, H 2048, I 768, g128s): MOE_COPIES copies of the 311 MB expert
    pool in HBM (2.5 GB)"""
    E, H, I = 128, 2048, 768
    gu = np.concatenate([syn.weights(G128S, 2 * I, H, 300 + e) for e in range(E)])
    dn = np.concatenate([syn.weights(G128S, H, I, 600 + e) for e in range(E)])
    ffns = []
    for _ in range(MOE_COPIES):
        f = QFfn(E, H, I, G128S)
        f.load(gu, dn)
        ffns.append(f)
    return ffns


def moe_logits(torch, syn, T, E):
    """router logits N(0, 1), a different draw for every (copy, round): [copy][round] cuda tensors"""
    return [[torch.from_numpy(syn.logits(T, E, 9 + 1000 * c + r)).cuda() for r in range(MOE_ROUNDS)]
            for c in range(MOE_COPIES)]


def moe(torch, QFfn, syn, iters):
    """The MoE layer at T = 1 and 512, router included (at T <= 4 the gate+up launch routes). One
    timed graph runs MOE_ROUNDS rounds over the MOE_COPIES pool copies, each call with its own
    logits: at T = 1 the 32 calls read 32 x 8 experts = 623 MB of distinct weights (an expert
    recurs in one copy 8 calls later at most with probability 8/128 per expert), so the 256 MB
    Infinity Cache does not hold them. Bytes per call: the experts its routing hits."""
    E, H, I, k = 128, 2048, 768, 8
    ffns = moe_layers(QFfn, syn)
    per_expert = wbytes(G128S, 2 * I, H) + wbytes(G128S, H, I)
    out = {}
    for T in (1, 512):
        lgs = moe_logits(torch, syn, T, E)
        x = bf16_tensor(torch, syn.activations(T, H, 10)).reshape(T, H)
        y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        hits = []
        for c in range(MOE_COPIES):
            for r in range(MOE_ROUNDS):
                ids, w = ffns[c].route(lgs[c][r], k)
                hits.append(len(np.unique(ids.cpu().numpy())))
        ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w = torch.empty((T, k), dtype=torch.float32, device="cuda")

        def step(lgs=lgs, x=x, y=y, ids=ids, w=w):
            for r in range(MOE_ROUNDS):
                for c, f in enumerate(ffns):
                    f.decode(lgs[c][r], x, k, out=y, ids=ids, w=w)
        g = GraphStep(step, torch)
        calls = MOE_COPIES * MOE_ROUNDS
        t = time_med(torch, g, iters, 3) / calls
        byts = float(np.mean(hits)) * per_expert + T * H * 2 * 2 + T * E * 4
        fl = 2.0 * T * k * (2 * I * H + H * I)
        out[f"M{T}"] = {"us_per_layer": t * 1e6, "GBps": byts / t / 1e9, "hbm_frac": byts / t / HBM_PEAK,
                        "TFLOPS": fl / t / 1e12, "mfma_frac": fl / t / BF16_PEAK, "experts_hit": float(np.mean(hits)),
                        "tokens_per_s": T / t,
                        "rotation": f"{MOE_COPIES} pool copies x {MOE_ROUNDS} routings per graph, "
                                    f"{sum(hits) * per_expert / 1e6:.0f} MB of expert weights read per graph"}
    for f in ffns:
        f.free()
    return out


def lm_head(torch, QMatrix, syn, iters):
    N, K = 151936, 4096
    st = syn.weights(Q4_0, N, K, 11)
    copies = [QMatrix(N, K, Q4_0, st) for _ in range(2)]      # 700 MB rotation
    out = {}
    for M in (1, 5):
        x = bf16_tensor(torch, syn.activations(M, K, 12)).reshape(M, K)
        lg = torch.empty((M, N), dtype=torch.float32, device="cuda")
        idx = torch.empty((M,), dtype=torch.int32, device="cuda")

        def step(x=x, lg=lg, idx=idx):
            for _ in range(GRAPH_REPS):
                for q in copies:
                    q.argmax(x, lg, idx)
        g = GraphStep(step, torch)
        t = time_med(torch, g, iters, 3) / (len(copies) * GRAPH_REPS)
        b = wbytes(Q4_0, N, K) + M * K * 2 + M * N * 4
        out[f"M{M}"] = {"us_per_call": t * 1e6, "GBps": b / t / 1e9, "hbm_frac": b / t / HBM_PEAK}
    for q in copies:
        q.free()
    return out


def codecs(torch, QMatrix):
    """Load-time weight codecs on one Qwen3-8B layer (4 matrices, 174 M weights): GPU quantization
    of fp32 weights already in HBM into each format (onpu_quantize_dev: the search quantizers, the
    GGUF Q4_0 rule) and the GGUF Q4_K -> q4nx transcode (onpu_transcode_q4k_dev), each call
    synchronous (temporary staging, repack into the tiled layout included); beside it the host
    quantizer (onpu_pack) on all host threads over the layer's o matrix (16.8 M weights)."""
    import ctypes as C
    from opennpu_amd import _lib
    L = _lib.lib()
    g = torch.Generator(device="cuda").manual_seed(5)
    Ws = [torch.randn((N, K), generator=g, device="cuda", dtype=torch.float32) * 0.02 for _, N, K in QWEN3_8B]
    nw = sum(N * K for _, N, K in QWEN3_8B)
    out = {}
    for name, fmt in (("q4s", 1), ("q4nx", 0), ("g128s", G128S), ("q4_0", Q4_0)):
        qs = [QMatrix(N, K, fmt) for _, N, K in QWEN3_8B]
        ts = []
        for rep in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for q, W in zip(qs, Ws):
                q.quantize(W)
            ts.append(time.perf_counter() - t0)
        t = float(np.median(ts))
        out[name] = {"ms_per_layer": t * 1e3, "Mweights_per_s": nw / t / 1e6}
        for q in qs:
            q.free()
    # Q4_K super-blocks with random nibbles and 6-bit scales, fp16 d / dmin of typical magnitude
    blocks = []
    for _, N, K in QWEN3_8B:
        b = torch.randint(0, 256, (N, K // 256, 144), generator=g, device="cuda", dtype=torch.uint8)
        b[..., 0:2] = (torch.rand((N, K // 256, 1), generator=g, device="cuda") * 0.02 + 1e-4).half().view(torch.uint8)
        b[..., 2:4] = (torch.rand((N, K // 256, 1), generator=g, device="cuda") * 0.01).half().view(torch.uint8)
        blocks.append(b.reshape(N, K // 256 * 144))
    qs = [QMatrix(N, K, 0) for _, N, K in QWEN3_8B]
    ts = []
    for rep in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for q, b in zip(qs, blocks):
            q.transcode_q4k(b)
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    out["q4k_to_q4nx"] = {"ms_per_layer": t * 1e3, "Mweights_per_s": nw / t / 1e6}
    for q in qs:
        q.free()
    # the host quantizer over the o matrix
    N, K = 4096, 4096
    W = Ws[1].cpu().numpy()
    cores = len(os.sched_getaffinity(0))
    for name, fmt in (("q4s", 1), ("q4nx", 0), ("g128s", G128S), ("q4_0", Q4_0)):
        geo = (C.c_int64 * 8)()
        L.onpu_geometry2(N, K, 8, fmt, geo)
        buf = np.zeros(geo[7], np.uint8)
        t0 = time.perf_counter()
        L.onpu_pack(W.ctypes.data_as(C.POINTER(C.c_float)), N, K, 8, fmt, buf.ctypes.data_as(C.POINTER(C.c_uint8)),
                    cores)
        t = time.perf_counter() - t0
        out[name]["cpu_Mweights_per_s"] = N * K / t / 1e6
        out[name]["cpu_threads"] = cores
    return out


def decode_glue(torch):
    """The per-token steps the reference runs on the host beside the int4 matmuls, on the GPU:
    decode attention at Qwen3-8B heads (Hq 32, Hkv 8, D 128, bf16 KV) for 4K and 32K positions, and
    the int8 shared-expert GEMV (11264 x 2048 gate+up, 2048 x 5632 down); inputs rotated over
    copies that together exceed the 256 MB Infinity Cache. GB/s = bytes read once (K and V; W)."""
    import ctypes as C
    from opennpu_amd import _lib
    from opennpu_amd.device import attn_step
    L = _lib.lib()
    out = {}
    Hq, Hkv, D = 32, 8, 128
    for S in (4096, 32768):
        nbytes = 2 * Hkv * S * D * 2
        nc = max(2, int(np.ceil(600e6 / nbytes)))
        caches = [(torch.randn((Hkv, S, D), device="cuda").bfloat16(), torch.randn((Hkv, S, D), device="cuda").bfloat16())
                  for _ in range(nc)]
        q = torch.randn((Hq, D), device="cuda")
        ws = torch.empty((L.onpu_attn_ws_bytes(Hq, D, Hkv, S),), dtype=torch.uint8, device="cuda")
        o = torch.empty((Hq, D), device="cuda")

        def step(caches=caches, q=q, ws=ws, o=o):
            for K, V in caches:
                attn_step(q, K, V, out=o, ws=ws)
        g = GraphStep(step, torch)
        t = time_med(torch, g, 10, 3) / nc
        out[f"attention_S{S}"] = {"us_per_call": t * 1e6, "GBps": nbytes / t / 1e9, "hbm_frac": nbytes / t / HBM_PEAK}
        del caches
    for name, N, K in (("gemv_i8_gate_up_11264x2048", 11264, 2048), ("gemv_i8_down_2048x5632", 2048, 5632)):
        nc = max(2, int(np.ceil(600e6 / (N * K))))
        Ws = [torch.randint(-128, 128, (N, K), device="cuda", dtype=torch.int8) for _ in range(nc)]
        sc = torch.rand(N, device="cuda") * 0.01
        x = torch.randn(K, device="cuda")
        y = torch.empty(N, device="cuda")
        P = lambda t: C.c_void_p(t.data_ptr())

        def step(Ws=Ws, sc=sc, x=x, y=y, N=N, K=K):
            for W in Ws:
                L.onpu_gemv_i8_dev(P(W), P(sc), N, K, P(x), P(y), C.c_void_p(torch.cuda.current_stream().cuda_stream))
        g = GraphStep(step, torch)
        t = time_med(torch, g, 10, 3) / nc
        out[name] = {"us_per_call": t * 1e6, "GBps": N * K / t / 1e9, "hbm_frac": N * K / t / HBM_PEAK}
        del Ws
    return out


def ceilings(torch):
    """What this GPU delivers to simple kernels (libonpu_probe.so, csrc/onpu_probe.hip) and to the
    vendor bf16 GEMM, so the int4 kernels can be read against measured ceilings as well as the
    published peaks: a streaming read of 4 GiB (every byte once, 16-byte loads, one contiguous
    range per workgroup), a torch device
    copy of 2 GiB, the LDS read rate (ds_read_b128, conflict-free), the bf16 MFMA issue rate
    (v_mfma_f32_16x16x32_bf16, 8 independent accumulators, 2 waves per SIMD), the effective shader
    clock (s_memtime against the 100 MHz s_memrealtime, in the MFMA and LDS probes), how many VALU
    ops a wave issues beside another wave's MFMAs on the same SIMD, and torch's bf16 GEMM (hipBLASLt)
    at the Llama-3.1-8B prefill shapes. Medians of 5 timed windows; the read
    ceiling is the best of 4 or 16 workgroups per CU and 4 or 16 loads in flight per lane."""
    import ctypes as C
    P = C.CDLL(str(ROOT / "opennpu_amd" / "libonpu_probe.so"))
    for n in ("onpu_probe_read", "onpu_probe_lds", "onpu_probe_mfma", "onpu_probe_coissue"):
        getattr(P, n).restype = C.c_int
    P.onpu_probe_read.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    P.onpu_probe_lds.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    P.onpu_probe_mfma.argtypes = P.onpu_probe_lds.argtypes
    P.onpu_probe_coissue.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    clk = torch.zeros(4, dtype=torch.int64, device="cuda")
    st = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def ok(rc):
        if rc != 0:
            raise RuntimeError(f"probe launch failed: {rc}")

    def clock_hz():
        c = clk.cpu().tolist()
        return (c[2] - c[0]) / max(c[3] - c[1], 1) * 100e6

    out = {"cus": cus}
    nb = 4 << 30
    buf = torch.empty(nb, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    rd = {}
    for wpc in (4, 16):
        for unroll in (4, 16):
            t = time_med(torch, lambda: ok(P.onpu_probe_read(buf.data_ptr(), nb, cus * wpc, unroll, sink.data_ptr(),
                                                             clk.data_ptr(), st())), 5, 2)
            rd[f"{wpc}_wg_per_cu_{unroll}_loads"] = nb / t / 1e9
    out["hbm_read_GBps"] = max(rd.values())
    out["hbm_read_by_grid"] = rd
    del buf
    src = torch.empty(2 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    t = time_med(torch, lambda: dst.copy_(src), 5, 2)
    out["copy_GBps_read_plus_write"] = 2 * src.numel() / t / 1e9
    del src, dst
    iters = 4096
    lds = {}
    for waves in (8, 16):
        t = time_med(torch, lambda: ok(P.onpu_probe_lds(cus, waves, iters, sink.data_ptr(), clk.data_ptr(), st())), 5, 2)
        hz = clock_hz()
        byts = cus * waves * 64 * iters * 8 * 16
        lds[f"{waves}_waves"] = {"TBps": byts / t / 1e12, "bytes_per_clk_per_cu": byts / t / hz / cus,
                                 "clock_GHz": hz / 1e9}
    out["lds_read"] = lds
    iters = 2048
    t = time_med(torch, lambda: ok(P.onpu_probe_mfma(cus * 2, 4, iters, sink.data_ptr(), clk.data_ptr(), st())), 5, 2)
    hz = clock_hz()
    fl = cus * 2 * 4 * iters * 8 * 16384.0
    out["mfma_bf16_TFLOPS"] = fl / t / 1e12
    out["mfma_clock_GHz"] = hz / 1e9
    out["mfma_cycles_per_16x16x32"] = (cus * 4 * hz * t) / (fl / 16384.0)
    # VALU issue beside MFMAs on one SIMD (wave 0 of workgroup 0 runs 48 fma per iteration, wave 4
    # on the same SIMD 8 MFMAs): cycles per iteration of each alone and of both together
    cyc = torch.zeros(2, dtype=torch.int64, device="cuda")
    co = {}
    for mode, name in ((0, "valu_alone"), (1, "mfma_alone"), (2, "both")):
        for _ in range(3):
            ok(P.onpu_probe_coissue(mode, cus, iters, sink.data_ptr(), cyc.data_ptr(), st()))
        torch.cuda.synchronize()
        c = cyc.cpu().tolist()
        co[name] = {"valu_wave_cycles_per_iter": c[0] / iters if mode != 1 else None,
                    "mfma_wave_cycles_per_iter": c[1] / iters if mode != 0 else None}
    va, mf, both = co["valu_alone"]["valu_wave_cycles_per_iter"], co["mfma_alone"]["mfma_wave_cycles_per_iter"], co["both"]
    co["valu_cycles_per_op_alone"] = va / 48
    co["mfma_cycles_per_op_alone"] = mf / 8
    # VALU ops the VALU wave completes while the MFMA wave streams (the rest at its lone rate)
    during = 48 - (both["valu_wave_cycles_per_iter"] - both["mfma_wave_cycles_per_iter"]) / (va / 48)
    co["valu_ops_per_mfma_beside"] = during / 8
    out["valu_mfma_coissue"] = co
    gm = {}
    M = 2048
    for name, N, K in [("up", 14336, 4096), ("down", 4096, 14336)]:
        x = torch.randn(M, K, device="cuda").to(torch.bfloat16)
        W = torch.randn(N, K, device="cuda").to(torch.bfloat16)
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        t = time_med(torch, lambda: torch.matmul(x, W.t(), out=y), 10, 3)
        gm[name] = {"us_per_call": t * 1e6, "TFLOPS": 2.0 * M * N * K / t / 1e12}
        del x, W, y
    try:
        lib = str(torch.backends.cuda.preferred_blas_library())
    except Exception:  # noqa: BLE001 - older torch: the default backend
        lib = "default"
    out["bf16_gemm_torch"] = {**gm, "blas": lib}
    return out


def cpu_dequant(orc, fmt, st, N, K):
    """fp32 [N][K] dequantized with numpy as the reference's CPU path writes it (reference.py:24-28:
    unpack the codes, minus 8, times the group scale); the CPU baseline times this"""
    if fmt == Q4_0:
        blk = st.reshape(N, K // 32, 18)
        d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32)
        q = np.concatenate([blk[:, :, 2:] & 15, blk[:, :, 2:] >> 4], axis=2).astype(np.float32)
        return ((q - 8.0) * d).reshape(N, K)
    b = st[:N * K // 2].reshape(N, K // 2)
    u = np.empty((N, K), np.float32)
    u[:, 0::2] = b & 15
    u[:, 1::2] = b >> 4
    u = u.reshape(N, K // 128, 128)
    s = orc.bf2f(st[N * K // 2:].view(np.uint16)).reshape(N, K // 128, 1)
    return ((u - 8.0) * s).reshape(N, K)


def cpu_baseline(syn):
    """The reference's CPU path for every configuration, timed on this host's cores with the same
    seeded inputs as the GPU runs. Protocol (the reference's `timed`, offload.py:302-309): 3 warm-up
    calls, then the median of 10; threads = the cores this process may run on, for torch and for the
    OpenMP kernels. Three paths:
      deq_in   the reference's dequant-matmul (opennpu/native/reference.py:24-28,55): unpack and
               dequantize W to fp32 with numpy inside the timed region, then x @ W^T in torch fp32
      deq_out  the same with W dequantized beforehand (the matmul alone)
      fused    this build's fused int4 CPU kernel (oracle/cpu_int4.c: AVX-512 FMAs on unpacked
               codes, M <= 8), the honest CPU-bandwidth comparison
    Bounded samples where a full configuration would take minutes: they are named in `sample`."""
    import torch
    import oracle.oracle as orc
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass

    def med(fn, warm=3, reps=10):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def xf(M, K, seed):
        return orc.bf2f(syn.activations(M, K, seed)).reshape(M, K)

    out = {"cores": cores, "cpu_model": cpu, "protocol": "3 warm-up calls, median of 10; torch and OpenMP on all cores"}
    # config 0: one 4096 x 4096 GEMV
    N = K = 4096
    st = syn.weights(G128S, N, K, 0)
    x = xf(1, K, 1)
    xt = torch.from_numpy(x)
    Wt = torch.from_numpy(cpu_dequant(orc, G128S, st, N, K))
    b0 = wbytes(G128S, N, K) + K * 2 + N * 2
    t_in = med(lambda: xt @ torch.from_numpy(cpu_dequant(orc, G128S, st, N, K)).T)
    t_out = med(lambda: xt @ Wt.T)
    t_f = med(lambda: orc.cpu_mv(G128S, st, N, K, x, cores))
    isa = orc.cpu_mv(G128S, st, N, K, x, cores)[1]
    out["gemv_4096"] = {p: {"us_per_call": t * 1e6, "GBps": b0 / t / 1e9} for p, t in
                        (("deq_in", t_in), ("deq_out", t_out), ("fused", t_f))}
    out["fused_isa"] = {2: "avx512", 1: "avx2", 0: "scalar"}[isa]
    del Wt
    # config 1: one Qwen3-8B layer (the four matrices) at M = 1, 4, 8
    lay = []
    for name, N, K in QWEN3_8B:
        st = syn.weights(G128S, N, K, 100 + N + K, scale_sigma=unit_gain_sigma(K), signed=True)
        lay.append((name, N, K, st, torch.from_numpy(cpu_dequant(orc, G128S, st, N, K))))
    dec = {}
    for M in (1, 4, 8):
        xs = {K: xf(M, K, K + M) for K in (4096, 12288)}
        xts = {K: torch.from_numpy(v) for K, v in xs.items()}
        byts = sum(wbytes(G128S, N, K) + M * K * 2 + M * N * 2 for _, N, K, _, _ in lay)
        t_out = med(lambda: [xts[K] @ W.T for _, N, K, _, W in lay])
        t_f = med(lambda: [orc.cpu_mv(G128S, st, N, K, xs[K], cores) for _, N, K, st, _ in lay])
        dec[f"M{M}"] = {"deq_out": {"ms_per_layer": t_out * 1e3, "GBps": byts / t_out / 1e9},
                        "fused": {"ms_per_layer": t_f * 1e3, "GBps": byts / t_f / 1e9,
                                  "tokens_per_s_equiv": M / (t_f * LAYERS)}}
    out["qwen3_8b_decode_layer"] = dec
    del lay
    # config 2: Llama-3.1-8B FFN prefill GEMMs, sampled on 512 of the 2048 rows (TFLOPS scale-free)
    pre = {}
    Ms = 512
    for name, N, K in [("up", 14336, 4096), ("down", 4096, 14336)]:
        st = syn.weights(G128S, N, K, 7)
        xt = torch.from_numpy(xf(2048, K, 8)[:Ms].copy())
        W = torch.from_numpy(cpu_dequant(orc, G128S, st, N, K))
        fl = 2.0 * Ms * N * K
        t_out = med(lambda: xt @ W.T)
        t_in = med(lambda: xt @ torch.from_numpy(cpu_dequant(orc, G128S, st, N, K)).T, warm=1, reps=5)
        pre[name] = {"deq_out": {"TFLOPS": fl / t_out / 1e12, "ms_per_2048_rows": t_out * 2048 / Ms * 1e3},
                     "deq_in": {"TFLOPS": fl / t_in / 1e12}}
        del W
    out["llama31_8b_prefill_ffn"] = {**pre, "sample": f"{Ms} of the 2048 rows; deq_in with 1 warm-up and the "
                                                      "median of 5 (the dequant dominates)"}
    # config 3: Qwen3-30B-A3B MoE layer at T = 1 (8 experts hit), the reference's MoE forward
    # (reference.py:71-84: per routed expert gate_up, silu(gate) * up, down, weighted sum)
    E, H, I, k = 128, 2048, 768, 8
    lg = syn.logits(1, E, 9)
    rid, rw = orc.route(lg, k)
    x = xf(1, H, 10)
    xt = torch.from_numpy(x)
    ex = {}
    for e in rid[0]:
        sg, sd = syn.weights(G128S, 2 * I, H, 300 + e), syn.weights(G128S, H, I, 600 + e)
        ex[int(e)] = (sg, sd, torch.from_numpy(cpu_dequant(orc, G128S, sg, 2 * I, H)), torch.from_numpy(cpu_dequant(orc, G128S, sd, H, I)))

    def moe_torch():
        y = torch.zeros(1, H)
        for j, e in enumerate(rid[0]):
            g = xt @ ex[int(e)][2].T
            a = torch.nn.functional.silu(g[:, :I]) * g[:, I:]
            y += float(rw[0, j]) * (a @ ex[int(e)][3].T)
        return y

    def moe_fused():
        y = np.zeros((1, H), np.float32)
        for j, e in enumerate(rid[0]):
            g = orc.cpu_mv(G128S, ex[int(e)][0], 2 * I, H, x, cores)[0]
            a = orc.silu_mul(g)
            y += rw[0, j] * orc.cpu_mv(G128S, ex[int(e)][1], H, I, a, cores)[0]
        return y

    hit = 8 * (wbytes(G128S, 2 * I, H) + wbytes(G128S, H, I))
    t_out, t_f = med(moe_torch), med(moe_fused)
    out["qwen3_30b_a3b_moe"] = {"M1": {"deq_out": {"us_per_layer": t_out * 1e6, "GBps": hit / t_out / 1e9},
                                       "fused": {"us_per_layer": t_f * 1e6, "GBps": hit / t_f / 1e9}}}
    del ex
    # config 4: the Q4_0 LM head, M = 1 and 5 (fused kernel; the torch matmul on pre-dequantized
    # fp32 weights, 2.5 GB)
    N, K = 151936, 4096
    st = syn.weights(Q4_0, N, K, 11)
    W = torch.from_numpy(cpu_dequant(orc, Q4_0, st, N, K))
    lm = {}
    for M in (1, 5):
        x = xf(M, K, 12)
        xt = torch.from_numpy(x)
        b = wbytes(Q4_0, N, K) + M * K * 2 + M * N * 4
        t_out = med(lambda: torch.argmax(xt @ W.T, dim=1))
        t_f = med(lambda: orc.cpu_mv(Q4_0, st, N, K, x, cores)[0].argmax(1))
        lm[f"M{M}"] = {"deq_out": {"us_per_call": t_out * 1e6, "GBps": b / t_out / 1e9},
                       "fused": {"us_per_call": t_f * 1e6, "GBps": b / t_f / 1e9}}
    out["lm_head_q4_0"] = lm
    del W
    head = dec["M1"]["fused"]
    return {"value": head["GBps"], "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": ("one Qwen3-8B layer (QKV, o, gate+up, down; g128s, 99.5 MB), M = 1, by this build's fused "
                       f"int4 CPU kernel ({out['fused_isa']}, {cores} OpenMP threads), median of 10 after 3 "
                       f"warm-ups: {head['ms_per_layer']:.2f} ms per layer; every configuration and the reference's "
                       "dequant-matmul pattern (dequant inside and outside the timed region) under `configs`"),
            "cpu_model": cpu, "configs": out}


def calibration_copy(torch):
    """one plain 512 MiB device copy (torch copy_): what FETCH_SIZE and WRITE_SIZE report for it per
    dispatch gives their unit"""
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()


def profile_target(torch, QMatrix, syn, names=("gate_up",), reps=3, rows=(1,)):
    """Decode GEMVs alone, for hardware-counter runs: each named Qwen3-8B matrix (g128s) at each row
    count in `rows` over its 36 HBM copies (or, for "lm_head", the Q4_0 LM head with its argmax at
    M = 1 and 5, or at the row counts given when they are not just 1, over 2 copies), `reps` eager
    launches each, in the order given, then one plain
    512 MiB device copy (torch copy_) whose FETCH_SIZE / WRITE_SIZE per dispatch calibrate the
    counters' unit."""
    shapes = {name: (N, K) for name, N, K in QWEN3_8B}
    out = []
    for name in names:
        if name == "lm_head":
            # the Q4_0 151936 x 4096 LM head with its argmax at M = 1 then 5 (or `rows`), on 2 copies
            N, K = 151936, 4096
            st = syn.weights(Q4_0, N, K, 11)
            mats = [QMatrix(N, K, Q4_0, st) for _ in range(2)]
            for M in ((1, 5) if tuple(rows) == (1,) else rows):
                x = bf16_tensor(torch, syn.activations(M, K, 12)).reshape(M, K)
                for _ in range(reps):
                    for q in mats:
                        q.argmax(x)
                torch.cuda.synchronize()
                out.append({"matrix": f"lm_head {N}x{K} Q4_0 M={M} + argmax", "launches": reps * len(mats),
                            "algorithmic_bytes_per_launch": wbytes(Q4_0, N, K) + M * K * 2 + M * N * 4})
            for q in mats:
                q.free()
            continue
        N, K = shapes[name]
        st = syn.weights(G128S, N, K, 100 + N + K, scale_sigma=unit_gain_sigma(K), signed=True)
        mats = [QMatrix(N, K, G128S, st) for _ in range(LAYERS)]
        for M in rows:
            x = bf16_tensor(torch, syn.activations(M, K, K + M)).reshape(M, K)
            y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            for _ in range(reps):
                for q in mats:
                    q.mv(x, out=y)
            torch.cuda.synchronize()
            out.append({"matrix": f"{name} {N}x{K} g128s M={M}", "launches": reps * LAYERS,
                        "algorithmic_bytes_per_launch": wbytes(G128S, N, K) + M * K * 2 + M * N * 2})
        for q in mats:
            q.free()
    calibration_copy(torch)
    print(json.dumps({"profile_target": out, "calibration_copy_bytes": 512 << 20}), flush=True)


def profile_gemm(torch, QMatrix, syn, reps=3):
    """The prefill GEMMs alone (Llama-3.1-8B FFN at M=2048: up 14336x4096, down 4096x14336, g128s),
    `reps` launches each, for hardware-counter runs (MFMA busy cycles)."""
    M = 2048
    for name, N, K in [("up", 14336, 4096), ("down", 4096, 14336)]:
        q = QMatrix(N, K, G128S, syn.weights(G128S, N, K, 7))
        x = bf16_tensor(torch, syn.activations(M, K, 8)).reshape(M, K)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        for _ in range(reps):
            q.mv(x, out=y)
        torch.cuda.synchronize()
        q.free()
    print(json.dumps({"profile_target": "prefill GEMM up 14336x4096 and down 4096x14336, M=2048",
                      "launches_each": reps, "flop_per_launch": 2 * M * 14336 * 4096}), flush=True)


def profile_chain(torch, QMatrix, QChain, syn, reps=5):
    """The chained decode step alone, for rocprofv3 runs: the headline's 144 Qwen3-8B GEMVs at M = 1
    (36 HBM copies of each matrix) as one chained launch, first dependent (each entry reads the
    output before it, as in the headline), then independent (every entry reads a fixed input), `reps`
    launches each, then one plain 512 MiB device copy that calibrates the byte counters. The
    difference between the two launches is what the 144 waits on earlier outputs cost."""
    mats = {}
    for name, N, K in QWEN3_8B:
        st = syn.weights(G128S, N, K, 100 + N + K, scale_sigma=unit_gain_sigma(K), signed=True)
        mats[name] = [QMatrix(N, K, G128S, st) for _ in range(LAYERS)]
    order = [(name, layer) for layer in range(LAYERS) for name, _, _ in QWEN3_8B]
    shape = {name: (N, K) for name, N, K in QWEN3_8B}
    ys = {key: torch.zeros((1, shape[key[0]][0]), dtype=torch.bfloat16, device="cuda") for key in order}
    h0 = bf16_tensor(torch, syn.activations(1, 4096, 4097)).reshape(1, 4096)
    fixed = {K: bf16_tensor(torch, syn.activations(1, K, K + 1)).reshape(1, K) for K in (4096, 12288)}

    def x_dep(name, layer):
        if name == "qkv":
            return h0 if layer == 0 else ys[("down", layer - 1)]
        if name == "o":
            return ys[("qkv", layer)][:, :4096]
        if name == "gate_up":
            return ys[("o", layer)]
        return ys[("gate_up", layer)][:, :12288]
    out = []
    for kind in ("dependent", "independent"):
        xs = [x_dep(nm, ly) if kind == "dependent" else fixed[shape[nm][1]] for nm, ly in order]
        ch = QChain([mats[nm][ly] for nm, ly in order], xs, [ys[key] for key in order])
        for _ in range(reps):
            ch.run()
        torch.cuda.synchronize()
        if ch.status() != 0:
            raise RuntimeError("chained decode: a wait for an earlier entry's output timed out")
        ch.free()
        out.append({"chain": kind, "entries": len(order), "launches": reps})
    for v in mats.values():
        for q in v:
            q.free()
    calibration_copy(torch)
    byts = LAYERS * sum(wbytes(G128S, N, K) + K * 2 + N * 2 for _, N, K in QWEN3_8B)
    print(json.dumps({"profile_target": out, "algorithmic_bytes_per_launch": byts,
                      "calibration_copy_bytes": 512 << 20}), flush=True)


def profile_few_rows(torch, QMatrix, syn, reps=2):
    """The GEMM at few rows alone, for rocprofv3 runs: the Llama-3.1-8B FFN at 96 rows (up 14336x4096,
    down 4096x14336, g128s) and the Q4_0 151936x4096 LM head with argmax at 16 rows, `reps` passes
    over the same >= 600 MB of distinct copies as the bench, then one plain 512 MiB device copy that
    calibrates the byte counters."""
    out = []
    for name, fmt, N, K, M in [("ffn_up", G128S, 14336, 4096, 96), ("ffn_down", G128S, 4096, 14336, 96),
                               ("lm_head_q4_0", Q4_0, 151936, 4096, 16)]:
        st = syn.weights(fmt, N, K, 13)
        copies = [QMatrix(N, K, fmt, st) for _ in range(max(2, -(-600_000_000 // st.nbytes)))]
        x = bf16_tensor(torch, syn.activations(M, K, 14)).reshape(M, K)
        lm = name.startswith("lm_head")
        y = torch.empty((M, N), dtype=torch.float32 if lm else torch.bfloat16, device="cuda")
        for _ in range(reps):
            for q in copies:
                if lm:
                    q.argmax(x, y)
                else:
                    q.mv(x, out=y)
        torch.cuda.synchronize()
        out.append({"matrix": f"{name} {N}x{K} M={M}", "launches": reps * len(copies),
                    "algorithmic_bytes_per_call": wbytes(fmt, N, K) + M * K * 2 + M * N * (4 if lm else 2),
                    "flop_per_call": 2 * M * N * K})
        for q in copies:
            q.free()
    calibration_copy(torch)
    print(json.dumps({"profile_target": out, "calibration_copy_bytes": 512 << 20}), flush=True)


def profile_moe(torch, QFfn, syn, reps=3):
    """The Qwen3-30B-A3B MoE layer alone (E 128, H 2048, I 768, top-8, g128s) at T = 512 and T = 1,
    each over the MOE_COPIES pool copies with MOE_ROUNDS different routings (as the bench's MoE
    leg: the T = 1 calls read 623 MB of distinct expert weights, past the Infinity Cache), `reps`
    times (router, permutation, grouped GEMMs, combine / the routing gate+up and down GEMVs), then
    one plain 512 MiB device copy that calibrates FETCH_SIZE / WRITE_SIZE, for hardware-counter and
    trace runs."""
    E, H, I, k = 128, 2048, 768, 8
    ffns = moe_layers(QFfn, syn)
    for T in (512, 1):
        lgs = moe_logits(torch, syn, T, E)
        x = bf16_tensor(torch, syn.activations(T, H, 10)).reshape(T, H)
        y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        for _ in range(reps):
            for r in range(MOE_ROUNDS):
                for c, f in enumerate(ffns):
                    f.decode(lgs[c][r], x, k, out=y)
        torch.cuda.synchronize()
    for f in ffns:
        f.free()
    calibration_copy(torch)
    per_expert = wbytes(G128S, 2 * I, H) + wbytes(G128S, H, I)
    print(json.dumps({"profile_target": "Qwen3-30B-A3B MoE layer, T = 512 then T = 1",
                      "calls_each": reps * MOE_COPIES * MOE_ROUNDS,
                      "gate_up_bytes_per_expert": wbytes(G128S, 2 * I, H), "down_bytes_per_expert": wbytes(G128S, H, I),
                      "algorithmic_bytes_T512_all_experts": E * per_expert}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline step only (no extra configs, no CPU leg)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile", nargs="?", const="gate_up", default=None,
                    help="only the named decode GEMVs (comma-separated: qkv, o, gate_up, down, lm_head; default "
                         "gate_up) plus a calibration copy, for rocprofv3 --pmc runs")
    ap.add_argument("--profile-rows", default="1",
                    help="row counts of the decode GEMVs under --profile (comma-separated, default 1)")
    ap.add_argument("--profile-gemm", action="store_true",
                    help="only the prefill GEMMs, for rocprofv3 --pmc runs")
    ap.add_argument("--profile-chain", action="store_true",
                    help="only the chained decode step, dependent then independent, for rocprofv3 runs")
    ap.add_argument("--profile-few-rows", action="store_true",
                    help="only the GEMMs at few rows (FFN at 96 rows, LM head at 16), for rocprofv3 runs")
    ap.add_argument("--profile-moe", action="store_true",
                    help="only the MoE layer (T = 512 and T = 1), for rocprofv3 runs")
    ap.add_argument("--ceilings", action="store_true",
                    help="only the measured ceilings (HBM read, copy, LDS, MFMA, clock, vendor bf16 GEMM)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the int4 path runs on a single MI355X; --gpus {args.gpus} is not "
              "supported (across GPUs the decode GEMVs would split N, the MoE layer its experts)", file=sys.stderr)
        sys.exit(2)
    import torch
    from opennpu_amd import require_gpu, synthetic as syn
    from opennpu_amd.device import QChain, QFfn, QMatrix
    require_gpu()
    torch.cuda.set_device(0)
    if args.profile:
        profile_target(torch, QMatrix, syn, tuple(args.profile.split(",")),
                       rows=tuple(int(v) for v in args.profile_rows.split(",")))
        return
    if args.profile_gemm:
        profile_gemm(torch, QMatrix, syn)
        return
    if args.profile_chain:
        profile_chain(torch, QMatrix, QChain, syn)
        return
    if args.profile_few_rows:
        profile_few_rows(torch, QMatrix, syn)
        return
    if args.profile_moe:
        profile_moe(torch, QFfn, syn)
        return
    if args.ceilings:
        print(json.dumps({"ceilings": ceilings(torch)}), flush=True)
        return
    t_all = time.perf_counter()
    log("decode layers ...")
    dec = decode_layers(torch, QMatrix, QChain, syn, (1,) if args.quick else (1, 4, 8), args.steps, args.warmup)
    head = dict(dec[1])
    ch1 = dec[1].get("chained", {})
    if "ms_per_step" in ch1 and ch1["ms_per_step"] < head["ms_per_step"]:
        for k in ("ms_per_step", "GBps", "hbm_frac"):
            head[k] = ch1[k]
        head["tokens_per_s_equiv"] = 1.0 / (ch1["ms_per_step"] / 1e3)
        head["launch"] = ch1["launch"]
    configs = {"qwen3_8b_decode": {f"M{M}": v for M, v in dec.items()}}
    if not args.quick:
        log("config 0 ...")
        configs["gemv_4096"] = config0(torch, QMatrix, syn, 50)
        log("prefill ...")
        configs["llama31_8b_prefill_ffn"] = prefill(torch, QMatrix, syn, 20)
        log("few-row GEMMs ...")
        configs["few_rows_gemm"] = few_rows(torch, QMatrix, syn, 20)
        log("moe ...")
        configs["qwen3_30b_a3b_moe"] = moe(torch, QFfn, syn, 30)
        log("lm head ...")
        configs["lm_head_q4_0"] = lm_head(torch, QMatrix, syn, 30)
        log("weight codecs ...")
        configs["weight_codecs_qwen3_8b_layer"] = codecs(torch, QMatrix)
        log("decode attention, int8 GEMV ...")
        configs["decode_glue"] = decode_glue(torch)
        log("measured ceilings ...")
        configs["ceilings"] = ceilings(torch)
    gu = head["per_matrix"]["gate_up"]
    roof = {"kernel": "k_qgemv<g128s> gate+up 24576x4096, M=1 (768 workgroups x 8 waves, x in LDS)",
            "bound": "hbm", "achieved": gu["GBps"], "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": gu["GBps"] / (HBM_PEAK / 1e9), "traffic": GATE_UP_TRAFFIC, "bytes_per_launch": gu["bytes"],
            "us_per_launch": gu["us"]}
    if "ceilings" in configs:
        # the same kernel against the streaming read this GPU measured in this run
        roof["measured_read_ceiling_GBps"] = configs["ceilings"]["hbm_read_GBps"]
        roof["frac_of_measured_ceiling"] = gu["GBps"] / configs["ceilings"]["hbm_read_GBps"]
    cpu = None
    if not (args.quick or args.no_cpu):
        log("cpu baseline ...")
        cpu = cpu_baseline(syn)
    out = {"metric": METRIC, "value": head["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "Qwen3-8B decode token: 36 layers x int4 g128s GEMVs (QKV 6144x4096, o 4096x4096, "
                                  "gate+up 24576x4096, down 4096x12288), M=1, one HBM copy per layer, each GEMV "
                                  "reading the previous one's output",
                      "bytes_per_step": head["bytes_per_step"], "hbm_frac": head["hbm_frac"],
                      "tokens_per_s_equiv": head["tokens_per_s_equiv"], "launch": head["launch"]},
           "roofline": roof, "cpu_baseline": cpu, "configs": configs,
           "wall_s": time.perf_counter() - t_all}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

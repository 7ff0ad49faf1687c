/*
 * ORACLE — test infrastructure only. A plain-C restatement of the reference's CPU arithmetic for
 * the int4 weight-only matmul path, used by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker. Nothing in the product links or calls this file.
 *
 * Every routine names the reference file:line it restates. Pinning (how each routine is checked
 * against something other than its own formula) lives in tests/test_oracle.py:
 *   - bf16 RNE / fp16 decode: against torch's and numpy's own conversions (library routines);
 *   - unpack + dequant: exhaustive byte/nibble round trip and hand-built blocks (GGUF spec);
 *   - matmul: fp64 brute force here vs numpy float64 matmul, plus linearity in x;
 *   - router: torch softmax/topk + the invariants sum(w) = 1, ids = top-k of the logits;
 *   - silu-mul / weighted sum / argmax: torch.nn.functional.silu, numpy, first-max rule;
 *   - geometry: the values the reference formula gives at the benchmark shapes.
 *   - act / weighted sum / attention step / int8 GEMV: also against the reference's own
 *     onpu_cpu.cpp compiled under oracle/_ref (tests/test_oracle_ref.py).
 *   - f2bf, geometry and the search quantizers (orc_quant_sym32 / orc_quant_asym32): byte for
 *     byte against the reference's own opennpu_core.hpp:37-169 compiled as written under oracle/_ref
 *     (tests/test_quant_ref.py, 2^20 groups per format of eight kinds), besides the invariants of
 *     tests/test_oracle.py (exact grids, sign symmetry, power-of-two equivariance). The GGUF codecs (orc_quant_q4_0, orc_transcode_q4k)
 * are checked on hand-built blocks whose results are exact, by the closed forms of the formats
 * (Q4_0's truncation at exact half-way inputs included), and the transcode's choice by a
 * brute-force neighbourhood.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so no fused multiply-adds change rounding).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* weight formats; the numbering is the library's (include/onpu.h) */
enum { FMT_Q4NX = 0, FMT_Q4S = 1, FMT_G128S = 2, FMT_Q4_0 = 3 };

/* ---------------------------------------------------------------- bf16 / fp16
 * f2bf: round to nearest even, NaN kept quiet (llama/ggml-opennpu/opennpu_core.hpp:50-56). */
uint16_t orc_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 64u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}

/* bf2f: widen (opennpu_core.hpp:57-62) */
float orc_bf2f(uint16_t h) {
    uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* IEEE binary16 -> float, exact (GGUF Q4_0 stores d as fp16; ggml's fp16_to_fp32 is exact). */
float orc_h2f(uint16_t h) {
    const uint32_t s = (uint32_t) (h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = s;
        else {                                   /* subnormal: m * 2^-24 */
            float f = ldexpf((float) m, -24);
            memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ---------------------------------------------------------------- staging layout
 * The canonical host layout a caller writes into a handle's staging buffer (include/onpu.h):
 *   Q4NX : codes u8 [N][K/2] (low nibble = even k), scales bf16 [N][K/32], mins bf16 [N][K/32]
 *   Q4S  : codes u8 [N][K/2], scales bf16 [N][K/32]
 *   G128S: codes u8 [N][K/2], scales bf16 [N][K/128]
 *   Q4_0 : GGUF block_q4_0 rows [N][K/32] x {fp16 d, u8 qs[16]} (18 bytes)
 */
int64_t orc_group(int fmt) { return fmt == FMT_G128S ? 128 : 32; }

int64_t orc_stage_bytes(int fmt, int64_t N, int64_t K) {
    const int64_t g = orc_group(fmt);
    if (fmt == FMT_Q4_0) return N * (K / 32) * 18;
    return N * K / 2 + N * (K / g) * 2 * (fmt == FMT_Q4NX ? 2 : 1);
}

/* the stored 4-bit code u (0..15) of element (n, k) */
static int code_at(int fmt, const uint8_t * st, int64_t K, int64_t n, int64_t k) {
    if (fmt == FMT_Q4_0) {
        /* GGUF block: element j of the block <- low nibble of qs[j], element j+16 <- high nibble */
        const uint8_t * blk = st + (n * (K / 32) + k / 32) * 18;
        const int j = (int) (k % 32);
        return j < 16 ? (blk[2 + j] & 0xf) : (blk[2 + j - 16] >> 4);
    }
    const uint8_t b = st[n * (K / 2) + k / 2];
    return (k & 1) ? (b >> 4) : (b & 0xf);
}

/* Dequantized weight of element (n, k) as the reference defines it in fp32:
 *   q4s / g128s / Q4_0: (u - 8) * s   (llama/ggml-opennpu/onpu_api.cpp:518; exact in fp32)
 *   q4nx              : u * s + m     (onpu_api.cpp:521; one rounding per operation)
 * Q4_0's d is fp16 (ggml block_q4_0); g128s is q4s with 128-wide groups. */
static float wq_at(int fmt, const uint8_t * st, int64_t N, int64_t K, int64_t n, int64_t k) {
    const int u = code_at(fmt, st, K, n, k);
    const int64_t g = orc_group(fmt);
    if (fmt == FMT_Q4_0) {
        const uint8_t * blk = st + (n * (K / 32) + k / 32) * 18;
        const uint16_t d = (uint16_t) (blk[0] | (blk[1] << 8));
        return ((float) u - 8.0f) * orc_h2f(d);
    }
    const uint16_t * sc = (const uint16_t *) (st + N * K / 2);
    const float s = orc_bf2f(sc[n * (K / g) + k / g]);
    if (fmt == FMT_Q4NX) {
        const uint16_t * mn = sc + N * (K / g);
        const float m = orc_bf2f(mn[n * (K / g) + k / g]);
        const float p = (float) u * s;
        return p + m;
    }
    return ((float) u - 8.0f) * s;
}

/* unpacked codes [N][K] */
void orc_unpack(int fmt, const uint8_t * st, int64_t N, int64_t K, uint8_t * out) {
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++) out[n * K + k] = (uint8_t) code_at(fmt, st, K, n, k);
}

/* fp32 dequantized W [N][K] (onpu_api.cpp:508-529 semantics) */
void orc_dequant(int fmt, const uint8_t * st, int64_t N, int64_t K, float * W) {
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++) W[n * K + k] = wq_at(fmt, st, N, K, n, k);
}

/* the bf16 weight tile the device's MAC sees: RNE of the fp32 dequant
 * (opennpu/native/npu4/kernels/gemv_any.cc:65,106-107, conv_even rounding) */
void orc_dequant_bf16(int fmt, const uint8_t * st, int64_t N, int64_t K, uint16_t * Wb) {
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++) Wb[n * K + k] = orc_f2bf(wq_at(fmt, st, N, K, n, k));
}

/* ---------------------------------------------------------------- matmul
 * y[m][n] = sum_k x[m][k] * W[n][k]: the dequantize-then-matmul of opennpu/native/reference.py:24-28,55
 * (there torch fp32; here accumulated in fp64, the exact product of the same dequantized weights).
 * x is bf16 (the device input is bf16 RNE of the fp32 activations, opennpu_core.hpp:418-424).
 * Rows [n0, n1) only, so callers can check a slice of a very large matrix. */
void orc_qmm_rows(int fmt, const uint8_t * st, int64_t N, int64_t K, const uint16_t * xb, int64_t M,
                  int64_t n0, int64_t n1, double * y /* [M][n1-n0] */, int bf16w) {
    /* bf16w: the weights the device's bf16 MAC sees, RNE of the dequant (gemv_any.cc:65,106-107) */
    double * xd = (double *) malloc(sizeof(double) * (size_t) (M * K));
    float * w = (float *) malloc(sizeof(float) * (size_t) K);
    for (int64_t i = 0; i < M * K; i++) xd[i] = (double) orc_bf2f(xb[i]);
    for (int64_t n = n0; n < n1; n++) {
        for (int64_t k = 0; k < K; k++) {
            w[k] = wq_at(fmt, st, N, K, n, k);
            if (bf16w) w[k] = orc_bf2f(orc_f2bf(w[k]));
        }
        for (int64_t m = 0; m < M; m++) {
            const double * xr = xd + m * K;
            double acc = 0.0;
            for (int64_t k = 0; k < K; k++) acc += xr[k] * (double) w[k];
            y[m * (n1 - n0) + (n - n0)] = acc;
        }
    }
    free(w);
    free(xd);
}

/* y[m][n] with the weights given dequantized (fp32 [N][K]) and x in fp64 */
void orc_matmul_f64(const float * W, int64_t N, int64_t K, const double * x, int64_t M, double * y) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; k++) acc += x[m * K + k] * (double) W[n * K + k];
            y[m * N + n] = acc;
        }
}

/* ---------------------------------------------------------------- MoE pieces
 * Router: softmax over E logits -> top-k -> renormalised (w / sum w)
 * (opennpu/native/moe_runtime.py:333-341; opennpu/native/reference.py:72-76).
 * Order: descending probability, ties to the lower expert index. */
void orc_route(const float * logits, int64_t T, int E, int k, int renorm, int32_t * ids, float * w) {
    double * p = (double *) malloc(sizeof(double) * (size_t) E);
    char * used = (char *) malloc((size_t) E);
    for (int64_t t = 0; t < T; t++) {
        const float * l = logits + t * E;
        double mx = l[0], s = 0;
        for (int e = 1; e < E; e++) if (l[e] > mx) mx = l[e];
        for (int e = 0; e < E; e++) { p[e] = exp((double) l[e] - mx); s += p[e]; }
        for (int e = 0; e < E; e++) p[e] /= s;
        memset(used, 0, (size_t) E);
        double ws = 0;
        for (int j = 0; j < k; j++) {
            int best = -1;
            for (int e = 0; e < E; e++)
                if (!used[e] && (best < 0 || p[e] > p[best])) best = e;
            used[best] = 1;
            ids[t * k + j] = best;
            ws += p[best];
        }
        for (int j = 0; j < k; j++) w[t * k + j] = (float) (renorm ? p[ids[t * k + j]] / ws : p[ids[t * k + j]]);
    }
    free(used);
    free(p);
}

/* act 0: a[r][i] = silu(h[r][i]) * h[r][I+i], silu(x) = x / (1 + e^-x), fp32
 * (llama/ggml-opennpu/onpu_cpu.cpp:253, :96) */
void orc_silu_mul(const float * h, int64_t rows, int64_t Ng, float * a) {
    const int64_t I = Ng / 2;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t i = 0; i < I; i++) {
            const float g = h[r * Ng + i], u = h[r * Ng + I + i];
            a[r * I + i] = g / (1.f + expf(-g)) * u;
        }
}

/* act 1 (gpt-oss): interleaved gate/up, clamped, gate * sigmoid(alpha * gate) * (up + 1)
 * (onpu_cpu.cpp:245-250) */
void orc_gptoss_act(const float * h, int64_t rows, int64_t Ng, float alpha, float limit, float * a) {
    const int64_t I = Ng / 2;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t i = 0; i < I; i++) {
            float g = h[r * Ng + 2 * i], u = h[r * Ng + 2 * i + 1];
            g = g < limit ? g : limit;
            u = u < limit ? u : limit;
            u = u > -limit ? u : -limit;
            a[r * I + i] = (u + 1.f) * g / (1.f + expf(-alpha * g));
        }
}

/* y[t][n] = sum_j w[t][j] * (o[t][j][n] (+ bias[ids[t][j]][n])) (onpu_cpu.cpp:259-274) */
void orc_moe_sum(const float * o, int64_t T, int k, int64_t N, const int32_t * ids, const float * w,
                 const float * bias, float * y) {
    for (int64_t t = 0; t < T; t++) {
        float * yt = y + t * N;
        for (int64_t n = 0; n < N; n++) yt[n] = 0.f;
        for (int j = 0; j < k; j++) {
            const int64_t r = t * k + j;
            const float * b = bias ? bias + (int64_t) ids[r] * N : NULL;
            for (int64_t n = 0; n < N; n++) yt[n] += w[r] * (o[r * N + n] + (b ? b[n] : 0.f));
        }
    }
}

/* argmax per row as numpy / torch argmax over the logits does it (opennpu/native/npu4/engine.py:358,
 * opennpu/native/runtime.py:348): the first NaN if the row has one, else the first maximum */
void orc_argmax(const float * v, int64_t rows, int64_t N, int32_t * out) {
    for (int64_t r = 0; r < rows; r++) {
        const float * x = v + r * N;
        int64_t b = 0;
        for (int64_t n = 0; n < N; n++) {
            if (x[n] != x[n]) { b = n; break; }
            if (x[n] > x[b]) b = n;
        }
        out[r] = (int32_t) b;
    }
}

/* ---------------------------------------------------------------- reference geometry
 * Mat(N, K, ncols, sym) of opennpu/native/npu4/model.py:151-187 (C++: opennpu_core.hpp:65-97):
 * R row blocks x S K-slices over ncols columns, (tiles, kc) minimising padded packets.
 * out = R, S, tiles, kc, ks, rows_col, cb, nbytes (zeros if no geometry). */
void orc_geometry(int64_t N, int64_t K, int ncols, int sym, int64_t * out) {
    const int NR = 4, GN = 64, GK = 256, KMAX = 2048;
    const int64_t pkt = GN * GK / 2 + (sym ? 1 : 2) * 2 * (GK / 32) * GN;
    double best = -1;
    int64_t R = 0, S = 0, tiles = 0, kc = 0;
    for (int s = 1; s <= ncols; s++) {
        if (ncols % s) continue;
        int64_t kcs = (K + (int64_t) s * GK - 1) / ((int64_t) s * GK);
        if (kcs > KMAX / GK) continue;
        const int64_t r = ncols / s;
        int64_t tl = (N + r * NR * GN - 1) / (r * NR * GN);
        if ((tl * kcs) % 2) {
            if (kcs + 1 <= KMAX / GK && tl * (kcs + 1) < (tl + 1) * kcs) kcs++;
            else tl++;
        }
        const double cost = (double) r * s * tl * kcs * (1 + 0.03 * (s - 1));
        if (best < 0 || cost < best) { best = cost; R = r; S = s; tiles = tl; kc = kcs; }
    }
    if (best < 0) { for (int i = 0; i < 8; i++) out[i] = 0; return; }
    const int64_t cb = tiles * kc * NR * pkt;
    out[0] = R; out[1] = S; out[2] = tiles; out[3] = kc; out[4] = kc * GK;
    out[5] = (int64_t) NR * tiles * GN; out[6] = cb; out[7] = R * S * cb;
}

/* ---------------------------------------------------------------- search quantizers (load time)
 * clamp as std::min(hi, std::max(lo, v)) evaluates it (opennpu_core.hpp:118,128,136,152,160,167):
 * std::max(a, b) is (a < b) ? b : a and std::min(a, b) is (b < a) ? b : a, so a NaN code (0 * inf
 * when a tiny range's reciprocal overflows) becomes lo. */
static float clamp_std(float v, float lo, float hi) {
    const float u = lo < v ? v : lo;
    return u < hi ? u : hi;
}

/* q4s over n weights (n = 32: q4s, 128: g128s): 16 candidate scales around absmax, least-squares
 * refit, bf16, least SSE wins (opennpu_core.hpp:142-169, written there for n = 32). */
void orc_quant_sym(const float * x, int n, uint8_t * q, uint16_t * d_bf) {
    float mx = 0;
    for (int i = 0; i < n; i++) if (fabsf(x[i]) > fabsf(mx)) mx = x[i];
    if (mx == 0) { *d_bf = orc_f2bf(1.0f); memset(q, 8, (size_t) n); return; }
    float best_e = INFINITY, best_d = mx / -8.0f;
    for (int c = 0; c < 16; c++) {
        const float dv = c < 8 ? -9.0f + 2.5f * c / 7 : 6.5f + 1.5f * (c - 8) / 7;
        const float d0 = mx / dv;
        float sqq = 0, sqx = 0;
        for (int i = 0; i < n; i++) {
            const float v = clamp_std(nearbyintf(x[i] / d0), -8.f, 7.f);
            sqq += v * v;
            sqx += v * x[i];
        }
        float d = sqq > 0 ? sqx / sqq : d0;
        d = orc_bf2f(orc_f2bf(d));
        if (d == 0) continue;
        float e = 0;
        for (int i = 0; i < n; i++) {
            const float v = clamp_std(nearbyintf(x[i] / d), -8.f, 7.f);
            const float r = v * d - x[i];
            e += r * r;
        }
        if (e < best_e) { best_e = e; best_d = d; }
    }
    for (int i = 0; i < n; i++) {
        const float v = clamp_std(nearbyintf(x[i] / best_d), -8.f, 7.f);
        q[i] = (uint8_t) (v + 8);
    }
    *d_bf = orc_f2bf(best_d);
}

void orc_quant_sym32(const float * x, uint8_t * q, uint16_t * d_bf) { orc_quant_sym(x, 32, q, d_bf); }

/* q4nx per 32: 21 stretched grids over [min, max], (s, m) refit by least squares, bf16
 * (opennpu_core.hpp:103-138). */
void orc_quant_asym32(const float * x, uint8_t * q, uint16_t * s_bf, uint16_t * m_bf) {
    float lo = x[0], hi = x[0];
    for (int i = 1; i < 32; i++) { if (x[i] < lo) lo = x[i]; if (x[i] > hi) hi = x[i]; }
    const float range = hi - lo;
    if (!(range > 0)) { *s_bf = orc_f2bf(1.0f); *m_bf = orc_f2bf(lo); memset(q, 0, 32); return; }
    float best_e = INFINITY, best_s = range / 15, best_m = lo;
    for (int st = 0; st <= 20; st++) {
        const float isc = (-1.0f + 0.1f * st + 15.0f) / range;
        float sl = 0, sll = 0, sx = 0, slx = 0;
        for (int i = 0; i < 32; i++) {
            const float l = clamp_std(nearbyintf(isc * (x[i] - lo)), 0.f, 15.f);
            sl += l; sll += l * l; sx += x[i]; slx += l * x[i];
        }
        const float D = 32 * sll - sl * sl;
        float sc = range / 15, mn = lo;
        if (D > 0) { sc = (32 * slx - sl * sx) / D; mn = (sll * sx - sl * slx) / D; }
        sc = orc_bf2f(orc_f2bf(sc));
        mn = orc_bf2f(orc_f2bf(mn));
        if (!(sc > 0)) continue;
        float e = 0;
        for (int i = 0; i < 32; i++) {
            const float l = clamp_std(nearbyintf((x[i] - mn) / sc), 0.f, 15.f);
            const float d = l * sc + mn - x[i];
            e += d * d;
        }
        if (e < best_e) { best_e = e; best_s = sc; best_m = mn; }
    }
    best_s = orc_bf2f(orc_f2bf(best_s));
    best_m = orc_bf2f(orc_f2bf(best_m));
    for (int i = 0; i < 32; i++) {
        const float l = clamp_std(nearbyintf((x[i] - best_m) / best_s), 0.f, 15.f);
        q[i] = (uint8_t) l;
    }
    *s_bf = orc_f2bf(best_s);
    *m_bf = orc_f2bf(best_m);
}

/* ---------------------------------------------------------------- GGUF codecs (load time)
 * fp32 -> IEEE binary16, round to nearest even (what ggml's GGML_FP32_TO_FP16 computes). */
uint16_t orc_f2h(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sgn = (u >> 16) & 0x8000u;
    const float a = fabsf(f);
    if (a != a) return (uint16_t) (sgn | 0x7e00u);
    if (a >= 65520.0f) return (uint16_t) (sgn | 0x7c00u);       /* rounds to infinity */
    if (a < 6.103515625e-05f) {                                  /* fp16 subnormal: multiples of 2^-24 */
        return (uint16_t) (sgn | (uint32_t) nearbyintf(a * 16777216.0f));
    }
    int e;
    const float m = frexpf(a, &e);                               /* a = m 2^e, m in [0.5, 1) */
    uint32_t mant = (uint32_t) nearbyintf(ldexpf(m, 11));        /* 11 significant bits, RNE */
    if (mant == 2048u) { mant = 1024u; e++; }
    return (uint16_t) (sgn | ((uint32_t) (e + 14) << 10) | (mant - 1024u));
}

/* ggml's quantize_row_q4_0 rule (llama.cpp 4413a19, the GGUF Q4_0 the reference reads,
 * ggml-opennpu.cpp:78-98): d = vmax / -8 for the first value of largest magnitude, id = 1/d (0 when
 * d = 0), u = min(15, (int8) (x id + 8.5)); codes in element order, d as fp16. */
void orc_quant_q4_0(const float * x, uint8_t * q, uint16_t * d_h) {
    float amax = 0, vmax = 0;
    for (int j = 0; j < 32; j++)
        if (amax < fabsf(x[j])) { amax = fabsf(x[j]); vmax = x[j]; }
    const float d = vmax / -8.0f, id = d != 0 ? 1.0f / d : 0.0f;
    *d_h = orc_f2h(d);
    for (int j = 0; j < 32; j++) {
        const int u = (int) (int8_t) (x[j] * id + 8.5f);
        q[j] = (uint8_t) (u < 15 ? u : 15);
    }
}

/* neighbouring bf16 value (ggml-opennpu.cpp:108-112) */
static uint16_t orc_bf_step(uint16_t h, int dir) {
    const float f = orc_bf2f(h);
    if (f == 0) return dir > 0 ? (uint16_t) 0x0001 : (uint16_t) 0x8001;
    return (uint16_t) (((f > 0) == (dir > 0)) ? h + 1 : h - 1);
}

/* GGUF Q4_K -> q4nx (ggml-opennpu.cpp:114-138). blocks: rows of K/256 super-blocks (144 bytes:
 * fp16 d, fp16 dmin, 12 bytes of packed 6-bit scales/mins, 128 bytes of nibbles), rows ld bytes
 * apart. Out: codes q [N][K] (u8 0..15), bf16 scale s and min m per 32 [N][K/32]. */
void orc_transcode_q4k(const uint8_t * blocks, int64_t N, int64_t K, int64_t ld, uint8_t * q, uint16_t * s,
                       uint16_t * m) {
    for (int64_t r = 0; r < N; r++)
        for (int64_t g = 0; g < K / 32; g++) {
            const uint8_t * b = blocks + r * ld + (g / 8) * 144;
            const int sub = (int) (g % 8);
            const float d = orc_h2f((uint16_t) (b[0] | (b[1] << 8))), dmin = orc_h2f((uint16_t) (b[2] | (b[3] << 8)));
            const uint8_t * sc = b + 4, * qs = b + 16;
            unsigned sv, mv;
            if (sub < 4) { sv = sc[sub] & 63u; mv = sc[sub + 4] & 63u; }
            else {
                sv = (sc[sub + 4] & 0xFu) | ((unsigned) (sc[sub - 4] >> 6) << 4);
                mv = (unsigned) (sc[sub + 4] >> 4) | ((unsigned) (sc[sub] >> 6) << 4);
            }
            uint8_t * qo = q + r * K + 32 * g;
            for (int l = 0; l < 32; l++) {
                const uint8_t byte = qs[(sub / 2) * 32 + l];
                qo[l] = (sub & 1) ? (uint8_t) (byte >> 4) : (uint8_t) (byte & 0xF);
            }
            const float S = d * (float) sv, M = -dmin * (float) mv;
            const uint16_t s0 = orc_f2bf(S), m0 = orc_f2bf(M);
            float best = INFINITY;
            uint16_t bs = s0, bm = m0;
            for (int ds = -1; ds <= 1; ds++)
                for (int dm = -1; dm <= 1; dm++) {
                    const uint16_t sc_ = ds ? orc_bf_step(s0, ds) : s0, mn_ = dm ? orc_bf_step(m0, dm) : m0;
                    const float sf = orc_bf2f(sc_), mf = orc_bf2f(mn_);
                    float e = 0;
                    for (int l = 0; l < 32; l++) {
                        const float t = qo[l] * sf + mf - (qo[l] * S + M);
                        e += t * t;
                    }
                    if (e < best) { best = e; bs = sc_; bm = mn_; }
                }
            s[r * (K / 32) + g] = bs;
            m[r * (K / 32) + g] = bm;
        }
}

/* W [N][K] fp32 -> the staging layout of fmt (orc_stage_bytes bytes), by the quantizers above:
 * the bytes onpu_pack writes (the staging layout is this library's; see the layout comment above). */
void orc_quantize(int fmt, const float * W, int64_t N, int64_t K, uint8_t * out) {
    const int G = fmt == FMT_G128S ? 128 : 32;
    uint8_t q[128];
    uint16_t * sc = (uint16_t *) (out + N * K / 2);
    uint16_t * mn = sc + N * (K / G);
    for (int64_t r = 0; r < N; r++)
        for (int64_t g = 0; g < K / G; g++) {
            const float * x = W + r * K + (int64_t) G * g;
            if (fmt == FMT_Q4_0) {
                uint16_t dh;
                orc_quant_q4_0(x, q, &dh);
                uint8_t * blk = out + (r * (K / 32) + g) * 18;
                blk[0] = (uint8_t) (dh & 0xff);
                blk[1] = (uint8_t) (dh >> 8);
                for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t) (q[j] | (q[16 + j] << 4));
                continue;
            }
            uint16_t s1 = 0, m1 = 0;
            if (fmt == FMT_Q4NX) orc_quant_asym32(x, q, &s1, &m1);
            else orc_quant_sym(x, G, q, &s1);
            for (int i = 0; i < G; i += 2) out[r * (K / 2) + (G * g + i) / 2] = (uint8_t) (q[i] | (q[i + 1] << 4));
            sc[r * (K / G) + g] = s1;
            if (fmt == FMT_Q4NX) mn[r * (K / G) + g] = m1;
        }
}

/* ---------------------------------------------------------------- decode attention (one token)
 * onpu_attn_step / onpu_attn_step_bf16 (onpu_cpu.cpp:180-229): q [Hq][D]; K, V: Hkv heads of S
 * rows (head stride hs, row stride rs, elements; fp32, or bf16 bits when kv_bf16); mask [S] additive
 * or NULL; sinks [Hq] or NULL; out [Hq][D]. fp32, sequential sums in the reference's order. */
void orc_attn_step(const float * q, int Hq, int D, const void * K, const void * V, int kv_bf16, int Hkv, int64_t S,
                   int64_t hs, int64_t rs, const float * mask, const float * sinks, float scale, float * out) {
    const int rep = Hq / Hkv;
    float * p = (float *) malloc((size_t) S * sizeof(float));
    for (int h = 0; h < Hq; h++) {
        const float * qh = q + (int64_t) h * D;
        const int64_t base = (int64_t) (h / rep) * hs;
        float mx = sinks ? sinks[h] : -INFINITY;
        for (int64_t j = 0; j < S; j++) {
            float s = 0.f;
            for (int d = 0; d < D; d++) {
                const int64_t i = base + j * rs + d;
                const float k = kv_bf16 ? orc_bf2f(((const uint16_t *) K)[i]) : ((const float *) K)[i];
                s += qh[d] * k;
            }
            s = s * scale + (mask ? mask[j] : 0.f);
            p[j] = s;
            if (s > mx) mx = s;
        }
        float sum = sinks ? expf(sinks[h] - mx) : 0.f;
        for (int64_t j = 0; j < S; j++) {
            p[j] = expf(p[j] - mx);
            sum += p[j];
        }
        float * o = out + (int64_t) h * D;
        for (int d = 0; d < D; d++) o[d] = 0.f;
        for (int64_t j = 0; j < S; j++) {
            const float pj = p[j] / sum;
            for (int d = 0; d < D; d++) {
                const int64_t i = base + j * rs + d;
                const float v = kv_bf16 ? orc_bf2f(((const uint16_t *) V)[i]) : ((const float *) V)[i];
                o[d] += pj * v;
            }
        }
    }
    free(p);
}

/* ---------------------------------------------------------------- int8 GEMV
 * onpu_gemv_i8 (onpu_cpu.cpp:276-299): y[n] = s[n] * sum_k W[n][k] x[k], W int8; the sum in fp64
 * here (the reference sums in fp32 lanes; the tests carry a tolerance). */
void orc_gemv_i8(const int8_t * W, const float * s, int64_t N, int64_t K, const float * x, double * y) {
    for (int64_t n = 0; n < N; n++) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; k++) acc += (double) W[n * K + k] * (double) x[k];
        y[n] = acc * (double) s[n];
    }
}

/* ---------------------------------------------------------------- Gated DeltaNet decode step
 * onpu_gdn_step (onpu_cpu.cpp:107-171): one token of a Gated DeltaNet layer. Causal conv over the
 * last Kc inputs + SiLU, then the state shifts by one; per value head: L2-normalised q (also / sqrt
 * Dk) and k of its key head, beta = sigmoid(Wb x), decay = exp(-exp(A_log) softplus(Wa x + dt_bias)),
 * S <- decay S; delta = beta (v - S^T k); S <- S + k delta^T; o = S^T q; out = norm_w * o / rms(o)
 * * silu(z). fp32, sequential sums as written there. */
static float orc_silu(float x) { return x / (1.f + expf(-x)); }
static float orc_dot(const float * a, const float * b, int n) {
    float s = 0.f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

void orc_gdn_step(const float * x, int H, const float * qkv, const float * z, const float * Wb, const float * Wa,
                  const float * conv_w, int Kc, float * conv_state, int L, const float * A_log, const float * dt_bias,
                  const float * norm_w, float eps, float * S, int Hk, int Hv, int Dk, int Dv, float * out) {
    const int key_dim = Hk * Dk, C = 2 * key_dim + Hv * Dv, rep = Hv / Hk;
    float * co = (float *) malloc((size_t) C * sizeof(float));
    for (int c = 0; c < C; c++) {
        float * st = conv_state + (int64_t) c * L;
        const float * w = conv_w + (int64_t) c * Kc;
        float s = w[Kc - 1] * qkv[c];
        for (int j = 0; j < Kc - 1; j++) s += w[j] * st[L - (Kc - 1) + j];
        co[c] = orc_silu(s);
        for (int j = 0; j + 1 < L; j++) st[j] = st[j + 1];
        st[L - 1] = qkv[c];
    }
    float * q = (float *) malloc((size_t) Dk * sizeof(float)), * k = (float *) malloc((size_t) Dk * sizeof(float));
    float * kv = (float *) malloc((size_t) Dv * sizeof(float)), * o = (float *) malloc((size_t) Dv * sizeof(float));
    float * delta = (float *) malloc((size_t) Dv * sizeof(float));
    for (int h = 0; h < Hv; h++) {
        const int kh = h / rep;
        for (int i = 0; i < Dk; i++) { q[i] = co[kh * Dk + i]; k[i] = co[key_dim + kh * Dk + i]; }
        const float * v = co + 2 * key_dim + (int64_t) h * Dv;
        const float qn = 1.f / sqrtf(orc_dot(q, q, Dk) + 1e-6f) / sqrtf((float) Dk);
        const float kn = 1.f / sqrtf(orc_dot(k, k, Dk) + 1e-6f);
        for (int i = 0; i < Dk; i++) { q[i] *= qn; k[i] *= kn; }
        const float b = orc_dot(Wb + (int64_t) h * H, x, H), a = orc_dot(Wa + (int64_t) h * H, x, H);
        const float beta = 1.f / (1.f + expf(-b));
        const float ad = a + dt_bias[h];
        const float sp = ad > 20.f ? ad : log1pf(expf(ad));
        const float decay = expf(-expf(A_log[h]) * sp);
        float * Sh = S + (int64_t) h * Dk * Dv;
        for (int j = 0; j < Dv; j++) { kv[j] = 0.f; o[j] = 0.f; }
        for (int i = 0; i < Dk; i++) {
            float * r = Sh + (int64_t) i * Dv;
            for (int j = 0; j < Dv; j++) { r[j] *= decay; kv[j] += r[j] * k[i]; }
        }
        for (int j = 0; j < Dv; j++) delta[j] = (v[j] - kv[j]) * beta;
        for (int i = 0; i < Dk; i++) {
            float * r = Sh + (int64_t) i * Dv;
            for (int j = 0; j < Dv; j++) { r[j] += k[i] * delta[j]; o[j] += r[j] * q[i]; }
        }
        const float ms = orc_dot(o, o, Dv) / Dv;
        const float rn = 1.f / sqrtf(ms + eps);
        for (int j = 0; j < Dv; j++) out[(int64_t) h * Dv + j] = norm_w[j] * (o[j] * rn) * orc_silu(z[(int64_t) h * Dv + j]);
    }
    free(co); free(q); free(k); free(kv); free(o); free(delta);
}

// Load-time host code of libonpu_hip: the reference geometry (reported for compatibility) and the
// weight quantizers behind onpu_pack / onpu_quant_dequant, writing the staging layout
// (include/onpu.h). Nothing here runs per token.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "onpu_common.h"
#include "onpu_host.h"

namespace onpu {

// The reference's Mat (opennpu/native/npu4/model.py:151-187, opennpu_core.hpp:65-97): R row blocks
// x S K-slices over ncols NPU columns, (tiles, kc) chosen to stream the fewest padded packets.
// The formula is kept identical so check_geometry (model.py:353-360) and buffer sizes agree;
// the GPU layout does not use it.
RefGeom ref_geometry(int64_t N, int64_t K, int ncols, bool sym) {
    const int NR = 4, GN = 64, GK = 256, KMAX = 2048;
    const int64_t pkt = GN * GK / 2 + (sym ? 1 : 2) * 2 * (GK / 32) * GN;
    RefGeom g;
    double best = -1;
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
        if (best < 0 || cost < best) { best = cost; g.R = r; g.S = s; g.tiles = tl; g.kc = kcs; }
    }
    if (best < 0) return g;
    g.ks = g.kc * GK;
    g.rows_col = (int64_t) NR * g.tiles * GN;
    g.cb = g.tiles * g.kc * NR * pkt;
    g.nbytes = g.R * g.S * g.cb;
    g.ok = true;
    return g;
}

static float bfr(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// fp32 -> IEEE binary16, round to nearest even (finite inputs; overflow -> inf)
static uint16_t f32_to_f16(float f) {
    union { float f; uint32_t u; } v;
    v.f = f;
    const uint32_t s = (v.u >> 16) & 0x8000u;
    const uint32_t a = v.u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t) (s | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t) (s | 0x7c00u);               // rounds past 65504
    if (a < 0x38800000u) {                                               // subnormal or zero in fp16
        const float m = std::fabs(f) * 16777216.0f;                      // in units of 2^-24
        return (uint16_t) (s | (uint32_t) std::nearbyint(m));            // exact scaling, RNE rounding
    }
    uint32_t r = a - 0x38000000u;                                        // rebias 127 -> 15 (<< 13)
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t) (s | (r >> 13));
}

// q4s-style search over n weights (the reference's quant_sym32, opennpu_core.hpp:142-169, with the
// group length as a parameter): 16 candidate scales around absmax, each refit by least squares and
// rounded to bf16; the least squared error wins. codes u = clamp(rint(x/d), -8, 7) + 8.
static void quant_sym(const float * x, int n, uint8_t * q, uint16_t & d_bf) {
    float mx = 0;
    for (int i = 0; i < n; i++) if (std::fabs(x[i]) > std::fabs(mx)) mx = x[i];
    if (mx == 0) { d_bf = f32_to_bf16(1.0f); std::memset(q, 8, (size_t) n); return; }
    float best_e = INFINITY, best_d = mx / -8.0f;
    for (int c = 0; c < 16; c++) {
        const float dv = c < 8 ? -9.0f + 2.5f * c / 7 : 6.5f + 1.5f * (c - 8) / 7;
        const float d0 = mx / dv;
        float sqq = 0, sqx = 0;
        for (int i = 0; i < n; i++) {
            const float v = std::min(7.0f, std::max(-8.0f, std::nearbyint(x[i] / d0)));
            sqq += v * v;
            sqx += v * x[i];
        }
        float d = sqq > 0 ? sqx / sqq : d0;
        d = bfr(d);
        if (d == 0) continue;
        float e = 0;
        for (int i = 0; i < n; i++) {
            const float v = std::min(7.0f, std::max(-8.0f, std::nearbyint(x[i] / d)));
            const float r = v * d - x[i];
            e += r * r;
        }
        if (e < best_e) { best_e = e; best_d = d; }
    }
    for (int i = 0; i < n; i++)
        q[i] = (uint8_t) (std::min(7.0f, std::max(-8.0f, std::nearbyint(x[i] / best_d))) + 8);
    d_bf = f32_to_bf16(best_d);
}

// q4nx per 32 (the reference's quant_asym32, opennpu_core.hpp:103-138): 21 stretched grids over
// [min, max], (s, m) refit by least squares, bf16-rounded, least squared error wins
static void quant_asym32(const float * x, uint8_t * q, uint16_t & s_bf, uint16_t & m_bf) {
    float lo = x[0], hi = x[0];
    for (int i = 1; i < 32; i++) { lo = std::min(lo, x[i]); hi = std::max(hi, x[i]); }
    const float range = hi - lo;
    if (!(range > 0)) {
        s_bf = f32_to_bf16(1.0f);
        m_bf = f32_to_bf16(lo);
        std::memset(q, 0, 32);
        return;
    }
    float best_e = INFINITY, best_s = range / 15, best_m = lo;
    for (int st = 0; st <= 20; st++) {
        const float isc = (-1.0f + 0.1f * st + 15.0f) / range;
        float sl = 0, sll = 0, sx = 0, slx = 0;
        for (int i = 0; i < 32; i++) {
            const float l = std::min(15.0f, std::max(0.0f, std::nearbyint(isc * (x[i] - lo))));
            sl += l; sll += l * l; sx += x[i]; slx += l * x[i];
        }
        const float D = 32 * sll - sl * sl;
        float sc = range / 15, mn = lo;
        if (D > 0) { sc = (32 * slx - sl * sx) / D; mn = (sll * sx - sl * slx) / D; }
        sc = bfr(sc);
        mn = bfr(mn);
        if (!(sc > 0)) continue;
        float e = 0;
        for (int i = 0; i < 32; i++) {
            const float l = std::min(15.0f, std::max(0.0f, std::nearbyint((x[i] - mn) / sc)));
            const float d = l * sc + mn - x[i];
            e += d * d;
        }
        if (e < best_e) { best_e = e; best_s = sc; best_m = mn; }
    }
    best_s = bfr(best_s);
    best_m = bfr(best_m);
    for (int i = 0; i < 32; i++)
        q[i] = (uint8_t) std::min(15.0f, std::max(0.0f, std::nearbyint((x[i] - best_m) / best_s)));
    s_bf = f32_to_bf16(best_s);
    m_bf = f32_to_bf16(best_m);
}

// GGUF Q4_0 block quantizer (ggml's published quantize_row_q4_0 rule): d = v / -8 for the value v of
// largest magnitude, u = min(15, trunc(x / d + 8.5)); d stored as fp16
static void quant_q4_0(const float * x, uint8_t * blk) {
    float amax = 0, vmax = 0;
    for (int j = 0; j < 32; j++)
        if (amax < std::fabs(x[j])) { amax = std::fabs(x[j]); vmax = x[j]; }
    const float d = vmax / -8.0f, id = d != 0 ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16(d);
    blk[0] = (uint8_t) (dh & 0xff);
    blk[1] = (uint8_t) (dh >> 8);
    for (int j = 0; j < 16; j++) {
        const int a = std::min(15, (int) (int8_t) (x[j] * id + 8.5f));
        const int b = std::min(15, (int) (int8_t) (x[16 + j] * id + 8.5f));
        blk[2 + j] = (uint8_t) (a | (b << 4));
    }
}

// rows [r0, r1) of W [N][K] -> staging layout of format fmt (out holds the whole matrix)
static void pack_rows(int fmt, const float * W, int64_t N, int64_t K, int64_t r0, int64_t r1, uint8_t * out) {
    const int64_t G = fmt_group(fmt);
    uint8_t q[128];
    if (fmt == ONPU_Q4_0) {
        for (int64_t r = r0; r < r1; r++)
            for (int64_t g = 0; g < K / 32; g++) quant_q4_0(W + r * K + 32 * g, out + (r * (K / 32) + g) * 18);
        return;
    }
    uint8_t * codes = out;
    uint16_t * sc = (uint16_t *) (out + N * K / 2);
    uint16_t * mn = sc + N * (K / G);
    for (int64_t r = r0; r < r1; r++)
        for (int64_t g = 0; g < K / G; g++) {
            const float * x = W + r * K + G * g;
            uint16_t s = 0, m = 0;
            if (fmt == ONPU_Q4NX) quant_asym32(x, q, s, m);
            else quant_sym(x, (int) G, q, s);
            for (int64_t i = 0; i < G; i += 2)
                codes[r * (K / 2) + (G * g + i) / 2] = (uint8_t) (q[i] | (q[i + 1] << 4));
            sc[r * (K / G) + g] = s;
            if (fmt == ONPU_Q4NX) mn[r * (K / G) + g] = m;
        }
}

static void parallel_rows(int64_t N, int threads, const std::function<void(int64_t, int64_t)> & f) {
    const int nt = std::max(1, std::min<int>(threads, (int) (N / 16) + 1));
    if (nt == 1) { f(0, N); return; }
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++) th.emplace_back(f, N * t / nt, N * (t + 1) / nt);
    for (auto & t : th) t.join();
}

bool pack_staging(int fmt, const float * W, int64_t N, int64_t K, uint8_t * out, int threads) {
    if (!fmt_valid(fmt) || K % fmt_group(fmt) != 0 || N <= 0) return false;
    parallel_rows(N, threads, [&](int64_t a, int64_t b) { pack_rows(fmt, W, N, K, a, b, out); });
    return true;
}

// staging bytes -> fp32 dequantized weights (the reference's dequant formulas, onpu_api.cpp:508-529)
void dequant_staging(int fmt, const uint8_t * st, int64_t N, int64_t K, float * out, int threads) {
    const int64_t G = fmt_group(fmt);
    parallel_rows(N, threads, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; r++)
            for (int64_t k = 0; k < K; k++) {
                float v;
                if (fmt == ONPU_Q4_0) {
                    const uint8_t * b = st + (r * (K / 32) + k / 32) * 18;
                    const int j = (int) (k % 32);
                    const int u = j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4);
                    v = ((float) u - 8.0f) * f16_to_f32((uint16_t) (b[0] | (b[1] << 8)));
                } else {
                    const uint8_t byte = st[r * (K / 2) + k / 2];
                    const int u = (k & 1) ? (byte >> 4) : (byte & 15);
                    const uint16_t * sc = (const uint16_t *) (st + N * K / 2);
                    const float s = bf16_to_f32(sc[r * (K / G) + k / G]);
                    if (fmt == ONPU_Q4NX) {
                        const float p = (float) u * s;
                        v = p + bf16_to_f32(sc[N * (K / G) + r * (K / G) + k / G]);
                    } else v = ((float) u - 8.0f) * s;
                }
                out[r * K + k] = v;
            }
    });
}

}  // namespace onpu

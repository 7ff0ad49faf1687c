// Load-time host code of libonpu_hip: the reference geometry, the weight quantizers behind onpu_pack /
// onpu_quant_dequant, writing the staging layout (include/onpu.h) or the reference's NPU packing
// (onpu_common.h). Nothing here runs per token.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "onpu_codec.h"
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

// rows [r0, r1) of W [N][K] -> staging layout of format fmt (out holds the whole matrix), with the
// quantizers of onpu_codec.h
static void pack_rows(int fmt, const float * W, int64_t N, int64_t K, int64_t r0, int64_t r1, uint8_t * out) {
    const int64_t G = fmt_group(fmt);
    float x[128];
    uint8_t q[128];
    auto & x32 = *reinterpret_cast<float (*)[32]>(x);
    auto & q32 = *reinterpret_cast<uint8_t (*)[32]>(q);
    if (fmt == ONPU_Q4_0) {
        for (int64_t r = r0; r < r1; r++)
            for (int64_t g = 0; g < K / 32; g++) {
                std::memcpy(x, W + r * K + 32 * g, 32 * sizeof(float));
                uint16_t dh = 0;
                quant_q4_0(x32, q32, dh);
                uint8_t * blk = out + (r * (K / 32) + g) * 18;
                blk[0] = (uint8_t) (dh & 0xff);
                blk[1] = (uint8_t) (dh >> 8);
                for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t) (q[j] | (q[16 + j] << 4));
            }
        return;
    }
    uint8_t * codes = out;
    uint16_t * sc = (uint16_t *) (out + N * K / 2);
    uint16_t * mn = sc + N * (K / G);
    for (int64_t r = r0; r < r1; r++)
        for (int64_t g = 0; g < K / G; g++) {
            std::memcpy(x, W + r * K + G * g, (size_t) G * sizeof(float));
            uint16_t s = 0, m = 0;
            if (fmt == ONPU_Q4NX) quant_asym32(x32, q32, s, m);
            else if (G == 128) quant_sym<128>(x, q, s);
            else quant_sym<32>(x32, q32, s);
            for (int64_t i = 0; i < G; i += 2)
                codes[r * (K / 2) + (G * g + i) / 2] = (uint8_t) (q[i] | (q[i + 1] << 4));
            sc[r * (K / G) + g] = s;
            if (fmt == ONPU_Q4NX) mn[r * (K / G) + g] = m;
        }
}

// GGUF Q4_K rows [r0, r1) (K / 256 super-blocks per row, ld bytes apart) -> q4nx staging
static void q4k_rows(const uint8_t * blocks, int64_t ld, int64_t N, int64_t K, int64_t r0, int64_t r1, uint8_t * out) {
    uint8_t q[32];
    uint16_t * sc = (uint16_t *) (out + N * K / 2);
    uint16_t * mn = sc + N * (K / 32);
    for (int64_t r = r0; r < r1; r++)
        for (int64_t g = 0; g < K / 32; g++) {
            uint16_t s = 0, m = 0;
            q4k_sub(blocks + r * ld + (g / 8) * Q4K_BLOCK, (int) (g % 8), q, s, m);
            for (int i = 0; i < 32; i += 2) out[r * (K / 2) + (32 * g + i) / 2] = (uint8_t) (q[i] | (q[i + 1] << 4));
            sc[r * (K / 32) + g] = s;
            mn[r * (K / 32) + g] = m;
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

bool pack_q4k_staging(const uint8_t * blocks, int64_t ld, int64_t N, int64_t K, uint8_t * out, int threads) {
    if (N <= 0 || K <= 0 || K % 256 != 0 || ld < K / 256 * Q4K_BLOCK) return false;
    parallel_rows(N, threads, [&](int64_t a, int64_t b) { q4k_rows(blocks, ld, N, K, a, b, out); });
    return true;
}

// W [N][K] -> the reference's NPU packing (onpu_common.h) in Mat geometry rg, rg.nbytes at out, with
// the q4s (sym) or q4nx quantizers of onpu_codec.h. Column blocks are first filled with their padding
// (all zero when the block holds no weight; else code 8 (q4s) or 0 (q4nx) and zero parameters), then
// every group of 32 is quantized and its codes and parameters written at their places. Threads take
// pairs of rows, which share their bytes.
bool pack_npu(int sym, const float * W, int64_t N, int64_t K, const RefGeom & rg, uint8_t * out, int threads) {
    if (!rg.ok || N <= 0 || K <= 0 || K % 32 != 0) return false;
    const NpuGeom g = npu_geom(rg.S, rg.tiles, rg.kc, rg.ks, rg.rows_col, rg.cb, sym);
    const int64_t npk = rg.tiles * rg.kc * 4;                 // packets per column block
    for (int64_t c = 0; c < rg.R * rg.S; c++) {
        uint8_t * blk = out + c * rg.cb;
        const int64_t r = c / rg.S, sl = c % rg.S;
        if (r * rg.rows_col >= N || sl * rg.ks >= K) {
            std::memset(blk, 0, (size_t) rg.cb);
            continue;
        }
        for (int64_t p = 0; p < npk; p++) {
            std::memset(blk + p * g.pkt, sym ? 0x88 : 0x00, 64 * 256 / 2);
            std::memset(blk + p * g.pkt + 64 * 256 / 2, 0, (size_t) (g.pkt - 64 * 256 / 2));
        }
    }
    const int64_t pairs = (N + 1) / 2;
    parallel_rows(pairs, threads, [&](int64_t p0, int64_t p1) {
        float x[32];
        uint8_t q[32];
        for (int64_t n = 2 * p0; n < std::min(N, 2 * p1); n++)
            for (int64_t k0 = 0; k0 < K; k0 += 32) {
                std::memcpy(x, W + n * K + k0, sizeof(x));
                uint16_t sc = 0, mn = 0;
                if (sym) quant_sym<32>(x, q, sc);
                else quant_asym32(x, q, sc, mn);
                for (int i = 0; i < 32; i++) {
                    int sh;
                    const int64_t o = npu_code_byte(g, n, k0 + i, sh);
                    out[o] = (uint8_t) ((out[o] & ~(0xF << sh)) | (q[i] << sh));
                }
                const int64_t so = npu_scale_off(g, n, k0);
                out[so] = (uint8_t) (sc & 0xff);
                out[so + 1] = (uint8_t) (sc >> 8);
                if (!sym) {
                    out[so + 1024] = (uint8_t) (mn & 0xff);
                    out[so + 1025] = (uint8_t) (mn >> 8);
                }
            }
    });
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

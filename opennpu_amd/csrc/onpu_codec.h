// Weight codecs of libonpu_hip, one source for the host quantizers behind onpu_pack /
// onpu_pack_q4k (onpu_quant.cpp) and their GPU versions behind onpu_quantize_dev /
// onpu_transcode_q4k_dev (onpu_codec.hip), so that both write the same staging bytes.
// Every multiply and add is rounded on its own (no contraction into fused multiply-adds), divisions
// are IEEE fp32 and rint rounds half to even, on the host and on the GPU alike.
#pragma once
#include "onpu_common.h"

// fp32 -> IEEE binary16, round to nearest even (finite inputs; overflow -> inf, NaN stays NaN)
ONPU_HD uint16_t f32_to_f16(float f) {
    union { float f; uint32_t u; } v;
    v.f = f;
    const uint32_t s = (v.u >> 16) & 0x8000u;
    const uint32_t a = v.u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t) (s | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t) (s | 0x7c00u);               // rounds past 65504
    if (a < 0x38800000u) {                                               // subnormal or zero in fp16
        const float m = __builtin_fabsf(f) * 16777216.0f;                // in units of 2^-24, exact
        return (uint16_t) (s | (uint32_t) __builtin_rintf(m));
    }
    uint32_t r = a - 0x38000000u;                                        // rebias 127 -> 15 (<< 13)
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t) (s | (r >> 13));
}

ONPU_HD float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// min(hi, max(lo, v)) with std::min / std::max semantics (a NaN v gives lo)
ONPU_HD float clamp_code(float v, float lo, float hi) {
    const float u = lo < v ? v : lo;
    return u < hi ? u : hi;
}

// q4s search quantizer over G weights: the reference's quant_sym32 (opennpu_core.hpp:142-169)
// with the group length as a parameter (G = 32: q4s, 128: g128s). 16 candidate scales around the
// value of largest magnitude, each refit by least squares and rounded to bf16; the least squared
// error wins. Codes u = clamp(rint(x / d), -8, 7) + 8.
template <int G>
ONPU_HD void quant_sym(const float (&x)[G], uint8_t (&q)[G], uint16_t & d_bf) {
#pragma clang fp contract(off)
    float mx = 0;
#pragma unroll
    for (int i = 0; i < G; i++) if (__builtin_fabsf(x[i]) > __builtin_fabsf(mx)) mx = x[i];
    if (mx == 0) {
        d_bf = f32_to_bf16(1.0f);
#pragma unroll
        for (int i = 0; i < G; i++) q[i] = 8;
        return;
    }
    float best_e = __builtin_inff(), best_d = mx / -8.0f;
#pragma nounroll
    for (int c = 0; c < 16; c++) {
        const float dv = c < 8 ? -9.0f + 2.5f * c / 7 : 6.5f + 1.5f * (c - 8) / 7;
        const float d0 = mx / dv;
        float sqq = 0, sqx = 0;
#pragma unroll
        for (int i = 0; i < G; i++) {
            const float v = clamp_code(__builtin_rintf(x[i] / d0), -8.0f, 7.0f);
            sqq += v * v;
            sqx += v * x[i];
        }
        float d = sqq > 0 ? sqx / sqq : d0;
        d = bf16_round(d);
        if (d == 0) continue;
        float e = 0;
#pragma unroll
        for (int i = 0; i < G; i++) {
            const float v = clamp_code(__builtin_rintf(x[i] / d), -8.0f, 7.0f);
            const float r = v * d - x[i];
            e += r * r;
        }
        if (e < best_e) { best_e = e; best_d = d; }
    }
#pragma unroll
    for (int i = 0; i < G; i++) q[i] = (uint8_t) (clamp_code(__builtin_rintf(x[i] / best_d), -8.0f, 7.0f) + 8);
    d_bf = f32_to_bf16(best_d);
}

// q4nx search quantizer over 32 weights: the reference's quant_asym32 (opennpu_core.hpp:103-138).
// 21 stretched grids over [min, max]; (s, m) refit by least squares, rounded to bf16; the least
// squared error wins. Codes u = clamp(rint((x - m) / s), 0, 15).
ONPU_HD void quant_asym32(const float (&x)[32], uint8_t (&q)[32], uint16_t & s_bf, uint16_t & m_bf) {
#pragma clang fp contract(off)
    float lo = x[0], hi = x[0];
#pragma unroll
    for (int i = 1; i < 32; i++) {
        lo = x[i] < lo ? x[i] : lo;                 // std::min(lo, x) / std::max(hi, x)
        hi = hi < x[i] ? x[i] : hi;
    }
    const float range = hi - lo;
    if (!(range > 0)) {
        s_bf = f32_to_bf16(1.0f);
        m_bf = f32_to_bf16(lo);
#pragma unroll
        for (int i = 0; i < 32; i++) q[i] = 0;
        return;
    }
    float best_e = __builtin_inff(), best_s = range / 15, best_m = lo;
#pragma nounroll
    for (int st = 0; st <= 20; st++) {
        const float isc = (-1.0f + 0.1f * st + 15.0f) / range;
        float sl = 0, sll = 0, sx = 0, slx = 0;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float l = clamp_code(__builtin_rintf(isc * (x[i] - lo)), 0.0f, 15.0f);
            sl += l;
            sll += l * l;
            sx += x[i];
            slx += l * x[i];
        }
        const float D = 32 * sll - sl * sl;
        float sc = range / 15, mn = lo;
        if (D > 0) {
            sc = (32 * slx - sl * sx) / D;
            mn = (sll * sx - sl * slx) / D;
        }
        sc = bf16_round(sc);
        mn = bf16_round(mn);
        if (!(sc > 0)) continue;
        float e = 0;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float l = clamp_code(__builtin_rintf((x[i] - mn) / sc), 0.0f, 15.0f);
            const float d = l * sc + mn - x[i];
            e += d * d;
        }
        if (e < best_e) { best_e = e; best_s = sc; best_m = mn; }
    }
    best_s = bf16_round(best_s);
    best_m = bf16_round(best_m);
#pragma unroll
    for (int i = 0; i < 32; i++) q[i] = (uint8_t) clamp_code(__builtin_rintf((x[i] - best_m) / best_s), 0.0f, 15.0f);
    s_bf = f32_to_bf16(best_s);
    m_bf = f32_to_bf16(best_m);
}

// GGUF Q4_0 block quantizer (ggml's quantize_row_q4_0 rule, llama.cpp 4413a19): d = v / -8 for the
// value v of largest magnitude (the first such), u = min(15, trunc(x / d + 8.5)) with 1 / d
// precomputed; d stored as fp16. Codes in element order (the caller packs GGUF's nibble order).
ONPU_HD void quant_q4_0(const float (&x)[32], uint8_t (&q)[32], uint16_t & d_h) {
#pragma clang fp contract(off)
    float amax = 0, vmax = 0;
#pragma unroll
    for (int j = 0; j < 32; j++)
        if (amax < __builtin_fabsf(x[j])) { amax = __builtin_fabsf(x[j]); vmax = x[j]; }
    const float d = vmax / -8.0f, id = d != 0 ? 1.0f / d : 0.0f;
    d_h = f32_to_f16(d);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int u = (int) (int8_t) (x[j] * id + 8.5f);
        q[j] = (uint8_t) (u < 15 ? u : 15);
    }
}

// The neighbouring bf16 value of h in direction dir (+1 up, -1 down); from zero, the smallest
// subnormal of that sign (ggml-opennpu.cpp:108-112)
ONPU_HD uint16_t bf16_step(uint16_t h, int dir) {
    const float f = bf16_to_f32(h);
    if (f == 0) return dir > 0 ? (uint16_t) 0x0001 : (uint16_t) 0x8001;
    return (uint16_t) (((f > 0) == (dir > 0)) ? h + 1 : h - 1);
}

// GGUF Q4_K -> q4nx, one 32-weight sub-block (ggml-opennpu.cpp:114-138). A Q4_K super-block of 256
// weights is 144 bytes: fp16 d, fp16 dmin, 12 bytes of 6-bit (scale, min) pairs for its 8
// sub-blocks, 128 bytes of nibbles (sub-blocks 2c and 2c + 1 share bytes [32c, 32c + 32): low
// nibbles, then high). Weight = d sc u - dmin mn with the sub-block's 4-bit codes u, which q4nx
// keeps exactly; its scale d sc and min -dmin mn become the bf16 pair, among the 3 x 3 neighbours
// of their rounded values, with the least squared error against the exact weights (first minimum
// in the order scale step -1, 0, 1 outer, min step inner).
ONPU_HD void q4k_sub(const uint8_t * b, int sub, uint8_t (&q)[32], uint16_t & s_out, uint16_t & m_out) {
#pragma clang fp contract(off)
    const float d = f16_to_f32((uint16_t) (b[0] | (b[1] << 8))), dmin = f16_to_f32((uint16_t) (b[2] | (b[3] << 8)));
    const uint8_t * sc = b + 4, * qs = b + 16;
    uint32_t sv, mv;
    if (sub < 4) {
        sv = sc[sub] & 63u;
        mv = sc[sub + 4] & 63u;
    } else {
        sv = (sc[sub + 4] & 0xFu) | ((uint32_t) (sc[sub - 4] >> 6) << 4);
        mv = (uint32_t) (sc[sub + 4] >> 4) | ((uint32_t) (sc[sub] >> 6) << 4);
    }
    const uint8_t * qq = qs + (sub / 2) * 32;
#pragma unroll
    for (int l = 0; l < 32; l++) q[l] = (sub & 1) ? (uint8_t) (qq[l] >> 4) : (uint8_t) (qq[l] & 0xF);
    const float S = d * (float) sv, M = -dmin * (float) mv;
    const uint16_t s0 = f32_to_bf16(S), m0 = f32_to_bf16(M);
    float best = __builtin_inff();
    s_out = s0;
    m_out = m0;
    for (int ds = -1; ds <= 1; ds++)
        for (int dm = -1; dm <= 1; dm++) {
            const uint16_t sc_ = ds ? bf16_step(s0, ds) : s0, mn_ = dm ? bf16_step(m0, dm) : m0;
            const float sf = bf16_to_f32(sc_), mf = bf16_to_f32(mn_);
            float e = 0;
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const float t = q[l] * sf + mf - (q[l] * S + M);
                e += t * t;
            }
            if (e < best) { best = e; s_out = sc_; m_out = mn_; }
        }
}

// bytes of one Q4_K super-block (256 weights)
constexpr int Q4K_BLOCK = 144;

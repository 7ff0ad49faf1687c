// Shared definitions of the MI355X (gfx950) int4 weight-only matmul library: weight formats, the
// staging (host) layout, the tiled HBM layout, and small device helpers.
//
// HBM layout ("tiled"). A [N][K] int4 matrix is padded to Npad = 16*NT rows and Kpad = 128*KB
// columns and stored as NT*KB blocks, row tile major (all K blocks of tile t are contiguous):
//
//   block(t, b) at (t*KB + b) * BLK bytes:
//     [0, 1024)     nibbles. Lane l = 16*q + r of a wave reads the 16 bytes at 16*l: row 16t + r,
//                   four dwords D_j (j = 0..3) holding k = 128b + 32j + 8q + e, e = 0..7, with
//                   element e at nibble position (e >> 1) + 4*(e & 1). D_j is exactly the B operand
//                   (8 bf16) of v_mfma_f32_16x16x32_bf16 for K step j after unpack8() below.
//     [1024, BLK)   per-row group parameters, [16 rows][GPB groups] of
//                   u16 scale (G128S: GPB = 1; Q4S, Q4_0: GPB = 4) or {u16 scale, u16 min} (Q4NX).
//
// MFMA step j of block b covers k in [128b + 32j, 128b + 32j + 32): one 32-group, a quarter of a
// 128-group, so group scales apply between MFMA steps.
#pragma once
#include <stdint.h>
#include <stddef.h>

enum OnpuFmt { ONPU_Q4NX = 0, ONPU_Q4S = 1, ONPU_G128S = 2, ONPU_Q4_0 = 3, ONPU_NFMT = 4 };

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define ONPU_HD __host__ __device__ __forceinline__
#else
#define ONPU_HD inline
#endif

ONPU_HD int fmt_group(int fmt) { return fmt == ONPU_G128S ? 128 : 32; }
ONPU_HD int fmt_gpb(int fmt) { return 128 / fmt_group(fmt); }          // groups per 128-wide block
ONPU_HD int fmt_has_min(int fmt) { return fmt == ONPU_Q4NX; }
ONPU_HD int fmt_param_bytes(int fmt) { return 16 * fmt_gpb(fmt) * 2 * (fmt_has_min(fmt) ? 2 : 1); }
ONPU_HD int fmt_blk(int fmt) { return 1024 + fmt_param_bytes(fmt); }  // 1056, 1152, 1280
ONPU_HD int fmt_valid(int fmt) { return fmt >= 0 && fmt < ONPU_NFMT; }

// Staging (canonical host) layout, what *_buf memory and onpu_pack hold:
//   Q4NX : codes u8 [N][K/2] (low nibble = even k), scales bf16 [N][K/32], mins bf16 [N][K/32]
//   Q4S  : codes u8 [N][K/2], scales bf16 [N][K/32]
//   G128S: codes u8 [N][K/2], scales bf16 [N][K/128]
//   Q4_0 : GGUF block_q4_0 rows [N][K/32] x {fp16 d, u8 qs[16]}
ONPU_HD int64_t stage_bytes(int fmt, int64_t N, int64_t K) {
    if (fmt == ONPU_Q4_0) return N * (K / 32) * 18;
    return N * K / 2 + N * (K / fmt_group(fmt)) * 2 * (fmt_has_min(fmt) ? 2 : 1);
}

struct Tiled {                       // geometry of one matrix in the tiled HBM layout
    int fmt;
    int64_t N, K, NT, KB, blk, bytes;
};

ONPU_HD Tiled tiled_geom(int fmt, int64_t N, int64_t K) {
    Tiled g;
    g.fmt = fmt; g.N = N; g.K = K;
    g.NT = (N + 15) / 16;
    g.KB = (K + 127) / 128;
    g.blk = fmt_blk(fmt);
    g.bytes = g.NT * g.KB * g.blk;
    return g;
}

// bf16 round-to-nearest-even with NaN kept quiet (the reference's f2bf); host and device
ONPU_HD uint16_t f32_to_bf16(float f) {
    union { float f; uint32_t u; } v;
    v.f = f;
    uint32_t u = v.u;
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 64u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}

ONPU_HD float bf16_to_f32(uint16_t h) {
    union { float f; uint32_t u; } v;
    v.u = (uint32_t) h << 16;
    return v.f;
}

// IEEE binary16 -> f32, exact (device: one v_cvt_f32_f16; fp16 denormals are kept by default)
ONPU_HD float f16_to_f32(uint16_t h) {
#ifdef __HIP_DEVICE_COMPILE__
    return (float) __builtin_bit_cast(_Float16, h);
#endif
    const uint32_t s = (uint32_t) (h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    union { float f; uint32_t u; } v;
    if (e == 0) {
        v.f = (float) m * (1.0f / 16777216.0f);       // m * 2^-24, exact
        v.u |= s;
    } else if (e == 31) v.u = s | 0x7f800000u | (m << 13);
    else v.u = s | ((e + 112) << 23) | (m << 13);
    return v.f;
}

// nibble position of element e (0..7) inside a dword D_j
ONPU_HD int nib_pos(int e) { return (e >> 1) + 4 * (e & 1); }

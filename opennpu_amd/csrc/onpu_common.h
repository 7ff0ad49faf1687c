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

// The reference's NPU packing (opennpu_core.hpp:174-254, Mat.pack model.py:189-217), the byte layout
// of the *_buf memory of handles the reference calls create (q4nx and q4s), so that packed bytes,
// also those the reference's own library or its numpy packer wrote (npu4's PackCache files,
// model.py:712-759), mean the same thing here. With the Mat geometry (R row blocks of rows_col rows x
// S K-slices of ks = 256 kc columns): column block c = r S + s at c * cb bytes; inside it, packets of
// 64 rows x 256 columns in the order [tile t][K step kk][core row cr], a packet holding the rows
// cr * tiles * 64 + t * 64 + [0, 64) and columns kk * 256 + [0, 256): nibbles
// [8 row octets][32 column octets][8 columns][4 bytes of two rows, the even row in the low nibble],
// then bf16 scales [8 groups of 32][64 rows] and (q4nx) mins likewise. Rows and columns past the
// matrix hold code 8 (q4s) or 0 (q4nx) with zero scales; a column block with no rows or columns of
// the matrix is all zero bytes.
struct NpuGeom {
    int64_t S, tiles, kc, ks, rows_col, cb, pkt;
};

ONPU_HD NpuGeom npu_geom(int64_t S, int64_t tiles, int64_t kc, int64_t ks, int64_t rows_col, int64_t cb, int sym) {
    NpuGeom g;
    g.S = S; g.tiles = tiles; g.kc = kc; g.ks = ks; g.rows_col = rows_col; g.cb = cb;
    g.pkt = 64 * 256 / 2 + (sym ? 1 : 2) * 2 * 8 * 64;
    return g;
}

// byte offset of the packet holding weight (n, k); its row within the packet (0..63) and column
// within the packet's 256 (0..255)
ONPU_HD int64_t npu_packet(const NpuGeom & g, int64_t n, int64_t k, int & prow, int & pcol) {
    const int64_t r = n / g.rows_col, lr = n - r * g.rows_col, s = k / g.ks, lc = k - s * g.ks;
    const int64_t cr = lr / (g.tiles * 64), t = (lr - cr * g.tiles * 64) / 64, kk = lc / 256;
    prow = (int) (lr % 64);
    pcol = (int) (lc % 256);
    return (r * g.S + s) * g.cb + ((t * g.kc + kk) * 4 + cr) * g.pkt;
}

// byte holding the code of weight (n, k) and the nibble's shift in it
ONPU_HD int64_t npu_code_byte(const NpuGeom & g, int64_t n, int64_t k, int & shift) {
    int pr, pc;
    const int64_t p = npu_packet(g, n, k, pr, pc);
    shift = 4 * (pr & 1);
    return p + (pr >> 3) * 1024 + (pc >> 3) * 32 + (pc & 7) * 4 + ((pr & 7) >> 1);
}

// byte offset of the bf16 scale of the 32-group of weight (n, k); the min (q4nx) is 1024 bytes on
ONPU_HD int64_t npu_scale_off(const NpuGeom & g, int64_t n, int64_t k) {
    int pr, pc;
    const int64_t p = npu_packet(g, n, k, pr, pc);
    return p + 64 * 256 / 2 + ((pc >> 5) * 64 + pr) * 2;
}

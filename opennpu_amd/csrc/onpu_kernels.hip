// HIP kernels for gfx950 (MI355X, CDNA4) behind the libonpu C ABI (onpu_api.cpp).
//
//   k_repack     staging layout -> tiled HBM layout (onpu_common.h), once per weight upload
//   k_dequant    tiled -> fp32 or bf16 (RNE) dequantized weights (parity checks)
//   k_qgemv      M <= 64 rows: the decode GEMV family. Integer MFMA on biased codes (128 + u) in
//                bf16, group scales applied in fp32 between MFMA steps, x column sums from an
//                extra MFMA against ones; epilogues: store, SiLU(gate) * up, MoE slot sum
//   k_qgemm      M > 64 (prefill): x tile in LDS, int4 tile dequantized to bf16 RNE((u-8)s) in
//                registers and fed to v_mfma_f32_16x16x32_bf16, fp32 accumulate
//   k_route      softmax -> top-k -> renorm router
//   k_moe_*      token -> expert permutation and grouped products
//   k_argmax     per-row argmax of fp32 logits
#include <hip/hip_runtime.h>
#include "onpu_common.h"
#include "onpu_launch.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define DEV static __device__ __forceinline__

DEV f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// D_j -> 8 bf16 holding 128 + u (bf16 0x43XX = 128 + XX for XX < 128), in B-operand order
DEV u32x4 unpack_biased(uint32_t d, uint32_t mag) {
    const uint32_t M = 0x000F000Fu;
    u32x4 r;
    r.x = and_or(d, M, mag);
    r.y = and_or(d >> 4, M, mag);
    r.z = and_or(d >> 8, M, mag);
    r.w = and_or(d >> 12, M, mag);
    return r;
}

// code u (0..15) of element e of D_j
DEV uint32_t code_of(uint32_t d, int e) { return (d >> (4 * nib_pos(e))) & 0xfu; }

DEV float scale_f32(int fmt, uint32_t bits) {
    return fmt == ONPU_Q4_0 ? f16_to_f32((uint16_t) bits) : bf16_to_f32((uint16_t) bits);
}

// dequantized weight (fp32) as the reference defines it: (u - 8) * s, or u * s + m for q4nx.
// u * s is exact in fp32 (4-bit times 8/11-bit), so fmaf rounds exactly once, like mul-then-add.
DEV float dq_val(int fmt, uint32_t u, float s, float m) {
    return fmt_has_min(fmt) ? fmaf((float) u, s, m) : fmaf((float) u, s, -8.0f * s);
}

// two fp32 -> packed bf16 (round to nearest even: v_cvt_pk_bf16_f32), low half = lo
DEV uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 h;
    h.x = (__bf16) lo;
    h.y = (__bf16) hi;
    return __builtin_bit_cast(uint32_t, h);
}

// ------------------------------------------------------------------ repack
// grid (KB, NT, E), 64 threads. st: staging of E experts (stride sstride bytes); out: tiled
// (stride ostride bytes per expert)
template <int FMT>
__global__ __launch_bounds__(64) void k_repack(const uint8_t * __restrict__ st, int64_t sstride, int64_t N,
                                               int64_t K, int64_t KB, uint8_t * __restrict__ out, int64_t ostride) {
    const int lane = threadIdx.x, q = lane >> 4, r = lane & 15;
    const int64_t b = blockIdx.x, t = blockIdx.y;
    st += (int64_t) blockIdx.z * sstride;
    uint8_t * blk = out + (int64_t) blockIdx.z * ostride + (t * KB + b) * fmt_blk(FMT);
    const int64_t n = 16 * t + r;
    const uint32_t pad = fmt_has_min(FMT) ? 0u : 8u;
    u32x4 dv;
    for (int j = 0; j < 4; j++) {
        const int64_t k0 = 128 * b + 32 * j + 8 * q;
        uint32_t d = 0;
        if (FMT == ONPU_Q4_0) {
            for (int e = 0; e < 8; e++) {
                const int64_t k = k0 + e;
                uint32_t u = pad;
                if (n < N && k < K) {
                    const uint8_t * bq = st + (n * (K / 32) + k / 32) * 18 + 2;
                    const int jj = (int) (k % 32);
                    u = jj < 16 ? (bq[jj] & 0xfu) : (bq[jj - 16] >> 4);
                }
                d |= u << (4 * nib_pos(e));
            }
        } else {
            uint32_t w = 0x88888888u * (pad == 8u);
            if (n < N && k0 < K) w = *(const uint32_t *) (st + n * (K / 2) + k0 / 2);   // 8 codes, k0 % 8 == 0
            for (int e = 0; e < 8; e++) d |= ((w >> (4 * e)) & 0xfu) << (4 * nib_pos(e));
        }
        dv[j] = d;
    }
    *(u32x4 *) (blk + 16 * lane) = dv;
    // group parameters [16 rows][GPB] (+ min)
    constexpr int G = FMT == ONPU_G128S ? 128 : 32, GPB = 128 / G;
    if (lane < 16 * GPB) {
        const int rr = lane / GPB, g = lane % GPB;
        const int64_t nn = 16 * t + rr, gi = b * GPB + g;          // group index along K
        uint16_t s = 0, mn = 0;
        if (nn < N && gi * G < K) {
            if (FMT == ONPU_Q4_0) {
                const uint8_t * bb = st + (nn * (K / 32) + gi) * 18;
                s = (uint16_t) (bb[0] | (bb[1] << 8));
            } else {
                const uint16_t * sc = (const uint16_t *) (st + N * K / 2);
                s = sc[nn * (K / G) + gi];
                if (fmt_has_min(FMT)) mn = sc[N * (K / G) + nn * (K / G) + gi];
            }
        }
        uint16_t * p = (uint16_t *) (blk + 1024);
        if (fmt_has_min(FMT)) { p[2 * lane] = s; p[2 * lane + 1] = mn; }
        else p[lane] = s;
    }
}

// group parameters of lane row r for the 4 MFMA steps of a block: scale and additive offset such that
// w = s * (128 + u) + boff  (sym: boff = -136 s; q4nx: boff = m - 128 s)
template <int FMT>
DEV void load_params(const uint8_t * blk, int r, float (&s)[4], float (&bo)[4]) {
    if (FMT == ONPU_G128S) {
        const float v = bf16_to_f32(*(const uint16_t *) (blk + 1024 + 2 * r));
        for (int j = 0; j < 4; j++) { s[j] = v; bo[j] = -136.0f * v; }
    } else if (FMT == ONPU_Q4NX) {
        const u32x4 p = *(const u32x4 *) (blk + 1024 + 16 * r);
        for (int j = 0; j < 4; j++) {
            s[j] = bf16_to_f32((uint16_t) (p[j] & 0xffff));
            bo[j] = bf16_to_f32((uint16_t) (p[j] >> 16)) - 128.0f * s[j];
        }
    } else {
        const u32x2 p = *(const u32x2 *) (blk + 1024 + 8 * r);
        for (int j = 0; j < 4; j++) {
            const uint32_t bits = (p[j >> 1] >> (16 * (j & 1))) & 0xffff;
            s[j] = scale_f32(FMT, bits);
            bo[j] = -136.0f * s[j];
        }
    }
}

// raw parameters for dequant (s, m) per step
template <int FMT>
DEV void load_sm(const uint8_t * blk, int r, float (&s)[4], float (&m)[4]) {
    if (FMT == ONPU_G128S) {
        const float v = bf16_to_f32(*(const uint16_t *) (blk + 1024 + 2 * r));
        for (int j = 0; j < 4; j++) { s[j] = v; m[j] = 0.f; }
    } else if (FMT == ONPU_Q4NX) {
        const u32x4 p = *(const u32x4 *) (blk + 1024 + 16 * r);
        for (int j = 0; j < 4; j++) {
            s[j] = bf16_to_f32((uint16_t) (p[j] & 0xffff));
            m[j] = bf16_to_f32((uint16_t) (p[j] >> 16));
        }
    } else {
        const u32x2 p = *(const u32x2 *) (blk + 1024 + 8 * r);
        for (int j = 0; j < 4; j++) {
            s[j] = scale_f32(FMT, (p[j >> 1] >> (16 * (j & 1))) & 0xffff);
            m[j] = 0.f;
        }
    }
}

// ------------------------------------------------------------------ dequant (parity checks)
// grid (KB, NT), 64 threads; out [N][K] fp32 (bf16 = 0) or bf16 RNE bits (bf16 = 1)
template <int FMT>
__global__ __launch_bounds__(64) void k_dequant(const uint8_t * __restrict__ W, int64_t N, int64_t K, int64_t KB,
                                                void * __restrict__ out, int bf16) {
    const int lane = threadIdx.x, q = lane >> 4, r = lane & 15;
    const int64_t b = blockIdx.x, t = blockIdx.y, n = 16 * t + r;
    const uint8_t * blk = W + (t * KB + b) * fmt_blk(FMT);
    const u32x4 dv = *(const u32x4 *) (blk + 16 * lane);
    float s[4], m[4];
    load_sm<FMT>(blk, r, s, m);
    if (n >= N) return;
    for (int j = 0; j < 4; j++)
        for (int e = 0; e < 8; e += 2) {
            const int64_t k = 128 * b + 32 * j + 8 * q + e;   // K % 32 == 0: k < K covers k + 1
            if (k >= K) continue;
            const float v0 = dq_val(FMT, code_of(dv[j], e), s[j], m[j]);
            const float v1 = dq_val(FMT, code_of(dv[j], e + 1), s[j], m[j]);
            if (bf16) *(uint32_t *) ((uint16_t *) out + n * K + k) = pack_bf16x2(v0, v1);
            else { ((float *) out)[n * K + k] = v0; ((float *) out)[n * K + k + 1] = v1; }
        }
}

// ------------------------------------------------------------------ decode GEMV family
// Per wave: RT row tiles x a run of K blocks. A operand = x rows (16 per MFMA block, MB blocks),
// B operand = unpacked biased codes. For each MFMA step j (32 k, one 32-group):
//   cg = x . (128 + u)^T,  cs = x . 1  (column sums of x, shared by all row tiles)
//   acc += s_j * cg + boff_j * cs
template <int FMT, int MB, int RT>
DEV void qacc_block(const uint8_t * const (&blk)[RT], const u32x4 (&wv)[RT], const u32x4 (&xa)[MB][4], uint32_t mag,
                    int r, f32x4 (&acc)[RT][MB]) {
    const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    if (FMT == ONPU_G128S) {
        f32x4 cs[MB];
        for (int mb = 0; mb < MB; mb++) {
            cs[mb] = z;
            for (int j = 0; j < 4; j++) cs[mb] = mfma(xa[mb][j], ones, cs[mb]);
        }
        for (int rt = 0; rt < RT; rt++) {
            if (!blk[rt]) continue;
            f32x4 cg[MB];
            for (int mb = 0; mb < MB; mb++) cg[mb] = z;
            for (int j = 0; j < 4; j++) {
                const u32x4 bw = unpack_biased(wv[rt][j], mag);
                for (int mb = 0; mb < MB; mb++) cg[mb] = mfma(xa[mb][j], bw, cg[mb]);
            }
            float s[4], bo[4];
            load_params<FMT>(blk[rt], r, s, bo);
            for (int mb = 0; mb < MB; mb++)
                for (int v = 0; v < 4; v++) acc[rt][mb][v] += s[0] * cg[mb][v] + bo[0] * cs[mb][v];
        }
    } else {
        f32x4 cs[MB][4];
        for (int mb = 0; mb < MB; mb++)
            for (int j = 0; j < 4; j++) cs[mb][j] = mfma(xa[mb][j], ones, z);
        for (int rt = 0; rt < RT; rt++) {
            if (!blk[rt]) continue;
            float s[4], bo[4];
            load_params<FMT>(blk[rt], r, s, bo);
            for (int j = 0; j < 4; j++) {
                const u32x4 bw = unpack_biased(wv[rt][j], mag);
                for (int mb = 0; mb < MB; mb++) {
                    const f32x4 cg = mfma(xa[mb][j], bw, z);
                    for (int v = 0; v < 4; v++) acc[rt][mb][v] += s[j] * cg[v] + bo[j] * cs[mb][j][v];
                }
            }
        }
    }
}

// x fragments of block b: lane (r, q) of A-block mb holds x[row(16 mb + r)][128 b + 32 j + 8 q .. +7]
template <int MB>
DEV void load_x(const uint16_t * __restrict__ x, int64_t ldx, const int32_t * xrows, int M, int64_t K, int64_t b,
                int r, int q, u32x4 (&xa)[MB][4]) {
    for (int mb = 0; mb < MB; mb++) {
        const int m = 16 * mb + r;
        int64_t row = m;
        bool ok = m < M;
        if (xrows && ok) { row = xrows[m]; ok = row >= 0; }
        for (int j = 0; j < 4; j++) {
            const int64_t k = 128 * b + 32 * j + 8 * q;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (ok && k < K) v = *(const u32x4 *) (x + row * ldx + k);
            xa[mb][j] = v;
        }
    }
}

// one wave: tiles tb[rt] (nullptr: no tile) over blocks [b0, b1), double-buffered weight loads
template <int FMT, int MB, int RT>
DEV void qacc_run(const uint8_t * const (&tb)[RT], int64_t b0, int64_t b1, const uint16_t * __restrict__ x,
                  int64_t ldx, const int32_t * xrows, int M, int64_t K, f32x4 (&acc)[RT][MB]) {
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
    const uint32_t mag = 0x43004300u;
    for (int rt = 0; rt < RT; rt++)
        for (int mb = 0; mb < MB; mb++) acc[rt][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (b0 >= b1) return;
    u32x4 wcur[RT], wnext[RT];
    for (int rt = 0; rt < RT; rt++)
        wcur[rt] = tb[rt] ? *(const u32x4 *) (tb[rt] + b0 * BLK + 16 * lane) : (u32x4){0u, 0u, 0u, 0u};
    for (int64_t b = b0; b < b1; b++) {
        if (b + 1 < b1)
            for (int rt = 0; rt < RT; rt++)
                wnext[rt] = tb[rt] ? *(const u32x4 *) (tb[rt] + (b + 1) * BLK + 16 * lane) : (u32x4){0u, 0u, 0u, 0u};
        u32x4 xa[MB][4];
        load_x<MB>(x, ldx, xrows, M, K, b, r, q, xa);
        const uint8_t * blk[RT];
        for (int rt = 0; rt < RT; rt++) blk[rt] = tb[rt] ? tb[rt] + b * BLK : nullptr;
        qacc_block<FMT, MB, RT>(blk, wcur, xa, mag, r, acc);
        for (int rt = 0; rt < RT; rt++) wcur[rt] = wnext[rt];
    }
}

// Epilogues
enum { EPI_STORE = 0, EPI_ACT = 1, EPI_SLOTSUM = 2 };

DEV void store_out(void * y, int yf32, int64_t idx, float v) {
    if (yf32) ((float *) y)[idx] = v;
    else ((uint16_t *) y)[idx] = f32_to_bf16(v);
}

DEV float silu_f(float g) { return g / (1.0f + expf(-g)); }

// grid: (tile groups, slots), block: waves * 64 threads; dynamic LDS: waves * RT * MB * 256 floats.
//   STORE  : slot = blockIdx.y; tiles blockIdx.x + rt * gridDim.x; waves split K
//   ACT    : RT = 2, tiles (t, t + gridDim.x) = (gate, up); out[m][16 t + r] = silu(g) * u
//   SLOTSUM: wave w -> slot w / ksplit (its expert and x row), K part w % ksplit; out = sum_s w_s y_s
template <int FMT, int MB, int RT, int EPI>
__global__ __launch_bounds__(MB == 1 ? 1024 : 512) void k_qgemv(QArgs a) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    // STORE / ACT: slot = blockIdx.y, every wave a K part. SLOTSUM: token blockIdx.y, wave -> slot
    // blockIdx.y * nslot + wave / ksplit and K part wave % ksplit
    int64_t slot;
    int kpart;
    if (EPI == EPI_SLOTSUM) { slot = (int64_t) blockIdx.y * a.nslot + wave / a.ksplit; kpart = wave % a.ksplit; }
    else { slot = blockIdx.y; kpart = wave; }
    const int64_t e = a.ids ? (int64_t) a.ids[slot] : 0;
    const uint8_t * W = a.W + e * a.estride;
    const uint16_t * x = a.x + (slot / a.xdiv) * a.xslot;
    const int32_t * xrows = nullptr;
    const uint8_t * tb[RT];
    int64_t tile[RT];
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    for (int rt = 0; rt < RT; rt++) {
        tile[rt] = (int64_t) blockIdx.x + (int64_t) rt * gridDim.x;
        tb[rt] = tile[rt] < a.NT ? W + tile[rt] * a.KB * BLK : nullptr;
    }
    const int64_t b0 = (int64_t) kpart * a.bpw, b1 = b0 + a.bpw < a.KB ? b0 + a.bpw : a.KB;
    f32x4 acc[RT][MB];
    qacc_run<FMT, MB, RT>(tb, b0, b1, x, a.ldx, xrows, a.M, a.K, acc);

    // cross-wave reduction through LDS: red[wave][((rt * MB + mb) * 4 + v) * 64 + lane]
    constexpr int PER = RT * MB * 256;
    for (int rt = 0; rt < RT; rt++)
        for (int mb = 0; mb < MB; mb++)
            for (int v = 0; v < 4; v++) red[wave * PER + ((rt * MB + mb) * 4 + v) * 64 + lane] = acc[rt][mb][v];
    __syncthreads();
    const int nout = EPI == EPI_ACT ? MB * 256 : PER;
    for (int o = threadIdx.x; o < nout; o += blockDim.x) {
        const int rt = o / (MB * 256), mb = (o / 256) % MB, v = (o / 64) % 4, l = o % 64;
        const int m = 16 * mb + 4 * (l >> 4) + v;
        const int64_t n = 16 * tile[rt] + (l & 15);
        if (m >= a.M) continue;
        if (EPI == EPI_SLOTSUM) {
            const float * ws = a.wslot + (int64_t) blockIdx.y * a.nslot;
            float s = 0.f;
            for (int sl = 0; sl < a.nslot; sl++) {
                float p = 0.f;
                for (int kp = 0; kp < a.ksplit; kp++) p += red[(sl * a.ksplit + kp) * PER + o];
                s += ws[sl] * p;
            }
            if (n < a.N) store_out(a.y, a.yf32, (int64_t) blockIdx.y * a.yslot + (int64_t) m * a.ldy + n, s);
        } else if (EPI == EPI_ACT) {
            float g = 0.f, u = 0.f;
            for (int w = 0; w < nw; w++) { g += red[w * PER + o]; u += red[w * PER + MB * 256 + o]; }
            if (n < a.N / 2)
                store_out(a.y, a.yf32, (int64_t) slot * a.yslot + (int64_t) m * a.ldy + n, silu_f(g) * u);
        } else {
            float s = 0.f;
            for (int w = 0; w < nw; w++) s += red[w * PER + o];
            if (n < a.N) store_out(a.y, a.yf32, (int64_t) slot * a.yslot + (int64_t) m * a.ldy + n, s);
        }
    }
}

// ------------------------------------------------------------------ prefill GEMM
// Y[M][N] = X[M][K] . deq(W)^T. WG: 4 waves, tile BM = 128 rows of X x BN = 64 * NTW row tiles... each wave
// owns NTW row tiles (16 rows each) and all 128 X rows: 8 A-blocks x NTW accumulators.
// Per K block (128): X tile (128 x 128 bf16, 32 KiB) staged in LDS as MFMA fragments
// [mb][j][lane] (16 B each); each wave loads its own weight blocks and dequantizes them to bf16
// RNE((u - 8) s) (the reference's device weight, gemv_any.cc:65,106-107) in registers.
template <int FMT, int NTW>
__global__ __launch_bounds__(256) void k_qgemm(GArgs a) {
    __shared__ u32x4 xs[8 * 4 * 64];                 // 32 KiB
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, r = lane & 15;
    // XCD-aware order: consecutive logical tiles land on the same XCD (WG i runs on XCD i % 8)
    const int64_t nwg = (int64_t) gridDim.x, wg = blockIdx.x;
    int64_t lid = wg;
    if (nwg % 8 == 0) lid = (wg % 8) * (nwg / 8) + wg / 8;
    const int64_t gm = (a.M + 127) / 128;
    const int64_t mblk = lid % gm, nblk = lid / gm;
    const int64_t m0 = mblk * 128;
    const int64_t t0 = nblk * (4 * NTW) + wave * NTW;       // first row tile of this wave
    const uint8_t * tb[NTW];
    for (int i = 0; i < NTW; i++) tb[i] = (t0 + i) < a.NT ? a.W + (t0 + i) * a.KB * BLK : nullptr;

    f32x4 acc[8][NTW];
    for (int mb = 0; mb < 8; mb++)
        for (int i = 0; i < NTW; i++) acc[mb][i] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // X tile loader: 2048 chunks of 16 B (128 rows x 16 chunks), 8 per thread
    u32x4 xr[8];
    auto load_xt = [&](int64_t b) {
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i, row = c >> 4, c16 = c & 15;
            const int64_t m = m0 + row, k = 128 * b + 8 * c16;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (m < a.M && k < a.K) v = *(const u32x4 *) (a.x + m * a.ldx + k);
            xr[i] = v;
        }
    };
    auto store_xt = [&]() {
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i, row = c >> 4, c16 = c & 15;
            const int j = c16 >> 2, qq = c16 & 3, mb = row >> 4, rr = row & 15;
            xs[(mb * 4 + j) * 64 + qq * 16 + rr] = xr[i];
        }
    };
    u32x4 wr[NTW];
    float ws[NTW][4], wm[NTW][4];
    auto load_w = [&](int64_t b) {
        for (int i = 0; i < NTW; i++) {
            if (tb[i]) {
                const uint8_t * blk = tb[i] + b * BLK;
                wr[i] = *(const u32x4 *) (blk + 16 * lane);
                load_sm<FMT>(blk, r, ws[i], wm[i]);
            } else {
                wr[i] = (u32x4){0u, 0u, 0u, 0u};
                for (int j = 0; j < 4; j++) { ws[i][j] = 0.f; wm[i][j] = 0.f; }
            }
        }
    };
    load_xt(0);
    load_w(0);
    for (int64_t b = 0; b < a.KB; b++) {
        __syncthreads();                 // previous block's reads of xs are done
        store_xt();
        // dequantize this block's weights to bf16 B operands
        u32x4 bw[NTW][4];
        for (int i = 0; i < NTW; i++)
            for (int j = 0; j < 4; j++) {
                const uint32_t d = wr[i][j];
                uint32_t o[4];
                for (int p = 0; p < 4; p++)
                    o[p] = pack_bf16x2(dq_val(FMT, code_of(d, 2 * p), ws[i][j], wm[i][j]),
                                       dq_val(FMT, code_of(d, 2 * p + 1), ws[i][j], wm[i][j]));
                bw[i][j] = (u32x4){o[0], o[1], o[2], o[3]};
            }
        __syncthreads();
        if (b + 1 < a.KB) { load_xt(b + 1); load_w(b + 1); }
        for (int j = 0; j < 4; j++)
            for (int mb = 0; mb < 8; mb++) {
                const u32x4 xa = xs[(mb * 4 + j) * 64 + lane];
                for (int i = 0; i < NTW; i++) acc[mb][i] = mfma(xa, bw[i][j], acc[mb][i]);
            }
    }
    // store: lane holds rows 4 (l >> 4) + v of A-block mb, column r of row tile t0 + i
    for (int mb = 0; mb < 8; mb++)
        for (int i = 0; i < NTW; i++) {
            const int64_t n = 16 * (t0 + i) + r;
            if (n >= a.N) continue;
            for (int v = 0; v < 4; v++) {
                const int64_t m = m0 + 16 * mb + 4 * q + v;
                if (m < a.M) store_out(a.y, a.yf32, m * a.ldy + n, acc[mb][i][v]);
            }
        }
}

// ------------------------------------------------------------------ router
// one wave per token: softmax over E <= 256 logits, top-k (ties to the lower id), renormalised
__global__ __launch_bounds__(64) void k_route(const float * __restrict__ logits, int64_t T, int E, int k, int renorm,
                                              int32_t * __restrict__ ids, float * __restrict__ w) {
    const int64_t t = blockIdx.x;
    const int lane = threadIdx.x;
    const float * l = logits + t * E;
    float v[4];
    float mx = -INFINITY;
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        v[i] = e < E ? l[e] : -INFINITY;
        mx = fmaxf(mx, v[i]);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float p[4], sum = 0.f;
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        p[i] = e < E ? expf(v[i] - mx) : 0.f;
        sum += p[i];
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    float ws = 0.f;
    for (int j = 0; j < k; j++) {
        // argmax over (p, -id)
        float bv = -1.f;
        int bi = 0x7fffffff;
        for (int i = 0; i < 4; i++) {
            const int e = lane + 64 * i;
            if (e < E && (p[i] > bv || (p[i] == bv && e < bi))) { bv = p[i]; bi = e; }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i == bi) p[i] = -2.f;        // taken
        const float pj = bv / sum;
        ws += pj;
        if (lane == 0) { ids[t * k + j] = bi; w[t * k + j] = pj; }
    }
    if (renorm && lane == 0)
        for (int j = 0; j < k; j++) w[t * k + j] = w[t * k + j] / ws;
}

// ------------------------------------------------------------------ MoE permutation
// One workgroup. entries i = t * k + j (T * k of them) sorted by expert:
//   cnt[e], off[e] (exclusive scan, off[E] = total), perm[off[e] + rank] = i,
//   work list of (expert, first position, rows <= rows_per_item) items -> items[], nitems
__global__ __launch_bounds__(1024) void k_moe_permute(const int32_t * __restrict__ ids, int64_t n, int E,
                                                      int rows_per_item, int32_t * __restrict__ off,
                                                      int32_t * __restrict__ perm, int32_t * __restrict__ items,
                                                      int32_t * __restrict__ nitems) {
    extern __shared__ int32_t sh[];
    int32_t * cnt = sh;              // [E]
    int32_t * pos = sh + E;          // [E + 1]
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) atomicAdd(&cnt[ids[i]], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t s = 0, it = 0;
        for (int e = 0; e < E; e++) {
            pos[e] = s;
            off[e] = s;
            for (int32_t r0 = 0; r0 < cnt[e]; r0 += rows_per_item) {
                items[3 * it] = e;
                items[3 * it + 1] = s + r0;
                items[3 * it + 2] = cnt[e] - r0 < rows_per_item ? cnt[e] - r0 : rows_per_item;
                it++;
            }
            s += cnt[e];
        }
        off[E] = s;
        *nitems = it;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const int32_t p = atomicAdd(&pos[ids[i]], 1);
        perm[p] = (int32_t) i;
    }
}

// grouped gate_up (+ SiLU * up) over work items: blockIdx.y = item, blockIdx.x = gate tile t.
// Rows of the item: perm[first .. first + rows) -> token = entry / k (x row), output row = position.
template <int FMT, int MB>
__global__ __launch_bounds__(MB == 1 ? 1024 : 512) void k_moe_gu(MArgs a) {
    extern __shared__ float red[];
    const int item = blockIdx.y;
    if (item >= *a.nitems) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int32_t e = a.items[3 * item], first = a.items[3 * item + 1], rows = a.items[3 * item + 2];
    const uint8_t * W = a.W + (int64_t) e * a.estride;
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    // x rows of this item: token = perm / k
    __shared__ int32_t xr[64];
    if (threadIdx.x < 64) xr[threadIdx.x] = threadIdx.x < rows ? a.perm[first + threadIdx.x] / a.k : -1;
    __syncthreads();
    const uint8_t * tb[2];
    int64_t tile[2] = {(int64_t) blockIdx.x, (int64_t) blockIdx.x + gridDim.x};
    for (int rt = 0; rt < 2; rt++) tb[rt] = tile[rt] < a.NT ? W + tile[rt] * a.KB * BLK : nullptr;
    const int64_t b0 = (int64_t) wave * a.bpw, b1 = b0 + a.bpw < a.KB ? b0 + a.bpw : a.KB;
    f32x4 acc[2][MB];
    qacc_run<FMT, MB, 2>(tb, b0, b1, a.x, a.ldx, xr, rows, a.K, acc);
    constexpr int PER = 2 * MB * 256;
    for (int rt = 0; rt < 2; rt++)
        for (int mb = 0; mb < MB; mb++)
            for (int v = 0; v < 4; v++) red[wave * PER + ((rt * MB + mb) * 4 + v) * 64 + lane] = acc[rt][mb][v];
    __syncthreads();
    for (int o = threadIdx.x; o < MB * 256; o += blockDim.x) {
        const int mb = (o / 256) % MB, v = (o / 64) % 4, l = o % 64;
        const int m = 16 * mb + 4 * (l >> 4) + v;
        const int64_t n = 16 * tile[0] + (l & 15);
        if (m >= rows || n >= a.N / 2) continue;
        float g = 0.f, u = 0.f;
        for (int w = 0; w < nw; w++) { g += red[w * PER + o]; u += red[w * PER + MB * 256 + o]; }
        ((uint16_t *) a.y)[(int64_t) (first + m) * a.ldy + n] = f32_to_bf16(silu_f(g) * u);
    }
}

// grouped down over work items: rows are act rows at positions first .. first + rows (contiguous);
// output o[position][N] fp32
template <int FMT, int MB>
__global__ __launch_bounds__(MB == 1 ? 1024 : 512) void k_moe_dn(MArgs a) {
    extern __shared__ float red[];
    const int item = blockIdx.y;
    if (item >= *a.nitems) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int32_t e = a.items[3 * item], first = a.items[3 * item + 1], rows = a.items[3 * item + 2];
    const uint8_t * W = a.W + (int64_t) e * a.estride;
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const uint8_t * tb[1];
    int64_t tile = blockIdx.x;
    tb[0] = tile < a.NT ? W + tile * a.KB * BLK : nullptr;
    const int64_t b0 = (int64_t) wave * a.bpw, b1 = b0 + a.bpw < a.KB ? b0 + a.bpw : a.KB;
    f32x4 acc[1][MB];
    qacc_run<FMT, MB, 1>(tb, b0, b1, a.x + (int64_t) first * a.ldx, a.ldx, nullptr, rows, a.K, acc);
    constexpr int PER = MB * 256;
    for (int mb = 0; mb < MB; mb++)
        for (int v = 0; v < 4; v++) red[wave * PER + (mb * 4 + v) * 64 + lane] = acc[0][mb][v];
    __syncthreads();
    for (int o = threadIdx.x; o < PER; o += blockDim.x) {
        const int mb = o / 256, v = (o / 64) % 4, l = o % 64;
        const int m = 16 * mb + 4 * (l >> 4) + v;
        const int64_t n = 16 * tile + (l & 15);
        if (m >= rows || n >= a.N) continue;
        float s = 0.f;
        for (int w = 0; w < nw; w++) s += red[w * PER + o];
        ((float *) a.y)[(int64_t) (first + m) * a.ldy + n] = s;
    }
}

// combine: y[t][n] = sum_j w[t][j] * o[inv[t * k + j]][n]; inv = inverse permutation (position of entry)
__global__ __launch_bounds__(256) void k_moe_combine(const float * __restrict__ o, const int32_t * __restrict__ inv,
                                                     const float * __restrict__ w, int64_t T, int k, int64_t N,
                                                     void * __restrict__ y, int yf32) {
    const int64_t t = blockIdx.y;
    for (int64_t n = blockIdx.x * blockDim.x + threadIdx.x; n < N; n += (int64_t) gridDim.x * blockDim.x) {
        float s = 0.f;
        for (int j = 0; j < k; j++) s += w[t * k + j] * o[(int64_t) inv[t * k + j] * N + n];
        store_out(y, yf32, t * N + n, s);
    }
}

__global__ void k_invert(const int32_t * __restrict__ perm, int64_t n, int32_t * __restrict__ inv) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) inv[perm[i]] = (int32_t) i;
}

// ------------------------------------------------------------------ argmax
// one workgroup per row: first maximum of logits[row][0..N)
__global__ __launch_bounds__(1024) void k_argmax(const float * __restrict__ v, int64_t N, int32_t * __restrict__ out) {
    const float * x = v + (int64_t) blockIdx.x * N;
    float bv = -INFINITY;
    int bi = (int) N;
    for (int n = threadIdx.x; n < (int) N; n += blockDim.x) {
        const float f = x[n];
        if (f > bv || (f == bv && n < bi)) { bv = f; bi = n; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int) (blockDim.x >> 6); w++)
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
        out[blockIdx.x] = (int32_t) bi;
    }
}

// ------------------------------------------------------------------ small helpers
__global__ void k_f32_to_bf16(const float * __restrict__ in, int64_t n, uint16_t * __restrict__ out) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(in[i]);
}

// act on host-API gate_up output h [rows][Ng] fp32 -> a [rows][Ng/2] fp32 (act 0: silu*up; 1: gpt-oss)
__global__ void k_moe_act(const float * __restrict__ h, int64_t rows, int64_t Ng, const int32_t * __restrict__ ids,
                          const float * __restrict__ bias, int act, float alpha, float limit, float * __restrict__ o) {
    const int64_t I = Ng / 2;
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * I) return;
    const int64_t r = i / I, c = i % I;
    const float * hr = h + r * Ng;
    const float * b = bias ? bias + (int64_t) ids[r] * Ng : nullptr;
    if (act == 1) {
        float g = hr[2 * c] + (b ? b[2 * c] : 0.f), u = hr[2 * c + 1] + (b ? b[2 * c + 1] : 0.f);
        g = fminf(g, limit);
        u = fmaxf(-limit, fminf(u, limit));
        o[i] = (u + 1.f) * g / (1.f + expf(-alpha * g));
    } else {
        const float g = hr[c] + (b ? b[c] : 0.f), u = hr[I + c] + (b ? b[I + c] : 0.f);
        o[i] = g / (1.f + expf(-g)) * u;
    }
}

// y[t][n] = sum_j w[t][j] (o[t][j][n] + bias[ids[t][j]][n])
__global__ void k_moe_sum(const float * __restrict__ o, int64_t T, int k, int64_t N, const int32_t * __restrict__ ids,
                          const float * __restrict__ w, const float * __restrict__ bias, float * __restrict__ y) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * N) return;
    const int64_t t = i / N, n = i % N;
    float s = 0.f;
    for (int j = 0; j < k; j++) {
        const int64_t r = t * k + j;
        s += w[r] * (o[r * N + n] + (bias ? bias[(int64_t) ids[r] * N + n] : 0.f));
    }
    y[i] = s;
}

// ================================================================== launchers
#define CHECK_LAUNCH() do { hipError_t e_ = hipGetLastError(); if (e_ != hipSuccess) return e_; } while (0)

hipError_t launch_repack(int fmt, const uint8_t * st, int64_t sstride, int64_t N, int64_t K, uint8_t * out,
                         int64_t ostride, int64_t E, hipStream_t s) {
    const Tiled g = tiled_geom(fmt, N, K);
    dim3 grid((unsigned) g.KB, (unsigned) g.NT, (unsigned) E);
    switch (fmt) {
        case ONPU_Q4NX: k_repack<ONPU_Q4NX><<<grid, 64, 0, s>>>(st, sstride, N, K, g.KB, out, ostride); break;
        case ONPU_Q4S: k_repack<ONPU_Q4S><<<grid, 64, 0, s>>>(st, sstride, N, K, g.KB, out, ostride); break;
        case ONPU_G128S: k_repack<ONPU_G128S><<<grid, 64, 0, s>>>(st, sstride, N, K, g.KB, out, ostride); break;
        case ONPU_Q4_0: k_repack<ONPU_Q4_0><<<grid, 64, 0, s>>>(st, sstride, N, K, g.KB, out, ostride); break;
        default: return hipErrorInvalidValue;
    }
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_dequant(int fmt, const uint8_t * W, int64_t N, int64_t K, void * out, int bf16, hipStream_t s) {
    const Tiled g = tiled_geom(fmt, N, K);
    dim3 grid((unsigned) g.KB, (unsigned) g.NT);
    switch (fmt) {
        case ONPU_Q4NX: k_dequant<ONPU_Q4NX><<<grid, 64, 0, s>>>(W, N, K, g.KB, out, bf16); break;
        case ONPU_Q4S: k_dequant<ONPU_Q4S><<<grid, 64, 0, s>>>(W, N, K, g.KB, out, bf16); break;
        case ONPU_G128S: k_dequant<ONPU_G128S><<<grid, 64, 0, s>>>(W, N, K, g.KB, out, bf16); break;
        case ONPU_Q4_0: k_dequant<ONPU_Q4_0><<<grid, 64, 0, s>>>(W, N, K, g.KB, out, bf16); break;
        default: return hipErrorInvalidValue;
    }
    CHECK_LAUNCH();
    return hipSuccess;
}

template <int FMT, int MB, int RT, int EPI>
static hipError_t qgemv_t(const QArgs & a, dim3 grid, int waves, hipStream_t s) {
    const size_t lds = (size_t) waves * RT * MB * 256 * sizeof(float);
    k_qgemv<FMT, MB, RT, EPI><<<grid, waves * 64, lds, s>>>(a);
    CHECK_LAUNCH();
    return hipSuccess;
}

template <int FMT, int EPI>
static hipError_t qgemv_mb(const QArgs & a, int mb, int rt, dim3 grid, int waves, hipStream_t s) {
    if (EPI == EPI_ACT) {
        if (mb == 1) return qgemv_t<FMT, 1, 2, EPI>(a, grid, waves, s);
        if (mb == 2) return qgemv_t<FMT, 2, 2, EPI>(a, grid, waves, s);
        return qgemv_t<FMT, 4, 2, EPI>(a, grid, waves, s);
    }
    if (EPI == EPI_SLOTSUM) {
        if (mb == 1) return qgemv_t<FMT, 1, 1, EPI>(a, grid, waves, s);
        return hipErrorInvalidValue;
    }
    if (mb == 1) {
        if (rt == 1) return qgemv_t<FMT, 1, 1, EPI>(a, grid, waves, s);
        if (rt == 2) return qgemv_t<FMT, 1, 2, EPI>(a, grid, waves, s);
        return qgemv_t<FMT, 1, 4, EPI>(a, grid, waves, s);
    }
    if (mb == 2) return qgemv_t<FMT, 2, 1, EPI>(a, grid, waves, s);
    return qgemv_t<FMT, 4, 1, EPI>(a, grid, waves, s);
}

template <int EPI>
static hipError_t qgemv_fmt(int fmt, const QArgs & a, int mb, int rt, dim3 grid, int waves, hipStream_t s) {
    switch (fmt) {
        case ONPU_Q4NX: return qgemv_mb<ONPU_Q4NX, EPI>(a, mb, rt, grid, waves, s);
        case ONPU_Q4S: return qgemv_mb<ONPU_Q4S, EPI>(a, mb, rt, grid, waves, s);
        case ONPU_G128S: return qgemv_mb<ONPU_G128S, EPI>(a, mb, rt, grid, waves, s);
        case ONPU_Q4_0: return qgemv_mb<ONPU_Q4_0, EPI>(a, mb, rt, grid, waves, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_qgemv(int fmt, int epi, const QArgs & a, int mb, int rt, dim3 grid, int waves, hipStream_t s) {
    if (waves < 1 || waves > 16 || (mb != 1 && mb != 2 && mb != 4)) return hipErrorInvalidValue;
    if (epi == EPI_STORE) return qgemv_fmt<EPI_STORE>(fmt, a, mb, rt, grid, waves, s);
    if (epi == EPI_ACT) return qgemv_fmt<EPI_ACT>(fmt, a, mb, rt, grid, waves, s);
    return qgemv_fmt<EPI_SLOTSUM>(fmt, a, mb, rt, grid, waves, s);
}

template <int FMT>
static hipError_t qgemm_t(const GArgs & a, int ntw, hipStream_t s) {
    const int64_t gm = (a.M + 127) / 128, gn = (a.NT + 4 * ntw - 1) / (4 * ntw);
    dim3 grid((unsigned) (gm * gn));
    if (ntw == 4) k_qgemm<FMT, 4><<<grid, 256, 0, s>>>(a);
    else k_qgemm<FMT, 2><<<grid, 256, 0, s>>>(a);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_qgemm(int fmt, const GArgs & a, int ntw, hipStream_t s) {
    switch (fmt) {
        case ONPU_Q4NX: return qgemm_t<ONPU_Q4NX>(a, ntw, s);
        case ONPU_Q4S: return qgemm_t<ONPU_Q4S>(a, ntw, s);
        case ONPU_G128S: return qgemm_t<ONPU_G128S>(a, ntw, s);
        case ONPU_Q4_0: return qgemm_t<ONPU_Q4_0>(a, ntw, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_route(const float * logits, int64_t T, int E, int k, int renorm, int32_t * ids, float * w,
                        hipStream_t s) {
    if (E > 256 || k > 16 || k > E) return hipErrorInvalidValue;
    k_route<<<dim3((unsigned) T), 64, 0, s>>>(logits, T, E, k, renorm, ids, w);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_permute(const int32_t * ids, int64_t n, int E, int rows_per_item, int32_t * off, int32_t * perm,
                              int32_t * items, int32_t * nitems, hipStream_t s) {
    k_moe_permute<<<1, 1024, (size_t) (2 * E + 1) * sizeof(int32_t), s>>>(ids, n, E, rows_per_item, off, perm, items,
                                                                          nitems);
    CHECK_LAUNCH();
    return hipSuccess;
}

template <int FMT>
static hipError_t moe_fmt(int which, const MArgs & a, int mb, dim3 grid, int waves, hipStream_t s) {
    const size_t lds = (size_t) waves * (which == 0 ? 2 : 1) * mb * 256 * sizeof(float);
    if (which == 0) {
        if (mb == 1) k_moe_gu<FMT, 1><<<grid, waves * 64, lds, s>>>(a);
        else if (mb == 2) k_moe_gu<FMT, 2><<<grid, waves * 64, lds, s>>>(a);
        else k_moe_gu<FMT, 4><<<grid, waves * 64, lds, s>>>(a);
    } else {
        if (mb == 1) k_moe_dn<FMT, 1><<<grid, waves * 64, lds, s>>>(a);
        else if (mb == 2) k_moe_dn<FMT, 2><<<grid, waves * 64, lds, s>>>(a);
        else k_moe_dn<FMT, 4><<<grid, waves * 64, lds, s>>>(a);
    }
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_grouped(int fmt, int which, const MArgs & a, int mb, dim3 grid, int waves, hipStream_t s) {
    switch (fmt) {
        case ONPU_Q4NX: return moe_fmt<ONPU_Q4NX>(which, a, mb, grid, waves, s);
        case ONPU_Q4S: return moe_fmt<ONPU_Q4S>(which, a, mb, grid, waves, s);
        case ONPU_G128S: return moe_fmt<ONPU_G128S>(which, a, mb, grid, waves, s);
        case ONPU_Q4_0: return moe_fmt<ONPU_Q4_0>(which, a, mb, grid, waves, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_invert(const int32_t * perm, int64_t n, int32_t * inv, hipStream_t s) {
    k_invert<<<dim3((unsigned) ((n + 255) / 256)), 256, 0, s>>>(perm, n, inv);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_combine(const float * o, const int32_t * inv, const float * w, int64_t T, int k, int64_t N,
                              void * y, int yf32, hipStream_t s) {
    dim3 grid((unsigned) ((N + 255) / 256), (unsigned) T);
    k_moe_combine<<<grid, 256, 0, s>>>(o, inv, w, T, k, N, y, yf32);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_argmax(const float * v, int64_t rows, int64_t N, int32_t * out, hipStream_t s) {
    k_argmax<<<dim3((unsigned) rows), 1024, 0, s>>>(v, N, out);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_f32_to_bf16(const float * in, int64_t n, uint16_t * out, hipStream_t s) {
    k_f32_to_bf16<<<dim3((unsigned) ((n + 255) / 256)), 256, 0, s>>>(in, n, out);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_act(const float * h, int64_t rows, int64_t Ng, const int32_t * ids, const float * bias, int act,
                          float alpha, float limit, float * o, hipStream_t s) {
    const int64_t n = rows * (Ng / 2);
    k_moe_act<<<dim3((unsigned) ((n + 255) / 256)), 256, 0, s>>>(h, rows, Ng, ids, bias, act, alpha, limit, o);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_sum(const float * o, int64_t T, int k, int64_t N, const int32_t * ids, const float * w,
                          const float * bias, float * y, hipStream_t s) {
    const int64_t n = T * N;
    k_moe_sum<<<dim3((unsigned) ((n + 255) / 256)), 256, 0, s>>>(o, T, k, N, ids, w, bias, y);
    CHECK_LAUNCH();
    return hipSuccess;
}

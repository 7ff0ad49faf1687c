// Templated device code of libonpu_hip for gfx950: the tiled-layout kernels instantiated once per
// weight format (onpu_fmt.hip, compiled with ONPU_FMT_ID = 0..3).
//
//   k_repack     staging layout -> tiled HBM layout (onpu_common.h), once per weight upload
//   k_dequant    tiled -> fp32 or bf16 (RNE) dequantized weights (parity checks)
//   k_qgemv      up to 64 rows: the decode GEMV family. Integer MFMA on biased codes (128 + u) in
//                bf16, group scales applied in fp32 between MFMA steps, x column sums from an
//                extra MFMA against ones; epilogues: store, SiLU(gate) * up, MoE slot sum
//   k_qgemm      prefill (and 1-64 rows of larger matrices): x tile in LDS, int4 tile dequantized
//                to bf16 RNE((u-8)s) in registers and fed to v_mfma_f32_16x16x32_bf16, fp32
//                accumulate; split along K into fp32 partials when the tiles leave CUs idle
//   k_moe_gemm   grouped expert products (MoE prompts) over a device work list
#pragma once
#include <hip/hip_runtime.h>
#include "onpu_common.h"
#include "onpu_launch.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define DEV static __device__ __forceinline__

// LDS views: pointers into the dynamic shared array travel through generic pointers; casting them
// back to address space 3 makes the accesses ds_read / ds_write (a generic "flat" access counts
// against both the vector-memory and LDS counters and forces waits on the weight prefetch)
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
// global-memory view of a pointer that came from memory rather than a kernel argument (without it
// the compiler emits flat loads, which also count against the LDS wait counter)
#define GLB(T, p) ((__attribute__((address_space(1))) T *) (p))
#define LDS_U32X4(p) ((lds_u32x4 *) (p))


DEV f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) with the other counters free, and lgkmcnt(0)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int LGKM0_IMM = 15 | (3 << 14) | (7 << 4);

// D_j -> 8 bf16 holding 128 + u (bf16 0x43XX = 128 + XX for XX < 128), in B-operand order:
// r.x = (d & M) | mag, r.y = ((d >> 4) & M) | mag, r.z = ((d >> 8) & M) | mag, r.w = ((d >> 12) & M) | mag.
// Seven VALU ops: with the mask in an SGPR and mag in a VGPR, both opaque (gfx9 VOP3 takes no
// literal), the compiler selects v_and_or_b32. Written as plain code, not inline asm, so that the compiler sees
// VALU writes and keeps its MFMA hazard rules: an asm block may be given registers that an MFMA it
// just issued still reads or writes (for M = 1 three of the four result registers of an MFMA are
// dead, and the MFMA's late write-back then lands on the asm's output).
// A value the optimizer cannot see through: an empty asm tied to its operand emits no instruction
// and writes no register (so it raises no hazard), but the constant is no longer known.
DEV uint32_t opaque_s(uint32_t v) { asm("" : "+s"(v)); return v; }
DEV uint32_t opaque_v(uint32_t v) { asm("" : "+v"(v)); return v; }

DEV u32x4 unpack_biased(uint32_t d, uint32_t mag) {
    const uint32_t M = opaque_s(0x000F000Fu), g = opaque_v(mag);
    return (u32x4){(d & M) | g, ((d >> 4) & M) | g, ((d >> 8) & M) | g, ((d >> 12) & M) | g};
}

// code u (0..15) of element e of D_j
DEV uint32_t code_of(uint32_t d, int e) { return (d >> (4 * nib_pos(e))) & 0xfu; }

DEV float scale_f32(int fmt, uint32_t bits) {
    return fmt == ONPU_Q4_0 ? f16_to_f32((uint16_t) bits) : bf16_to_f32((uint16_t) bits);
}

// dequantized weight (fp32) as the reference defines it: (u - 8) * s (exact; a negative scale
// gives -0 for u = 8, as the reference's expression does), or u * s + m for q4nx (u * s is exact
// in fp32, 4-bit times 8-bit, so fmaf rounds once, like the reference's multiply-then-add).
DEV float dq_val(int fmt, uint32_t u, float s, float m) {
    return fmt_has_min(fmt) ? fmaf((float) u, s, m) : ((float) u - 8.0f) * s;
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

// Raw group parameters of lane row r in one block for the decode kernels (loaded early, decoded at
// compute time): G128S the dword holding the u16 scales of rows r & ~1 and r | 1 plus the byte
// selector of row r's half (set from r when loaded), Q4S / Q4_0 four u16 scales, Q4NX four
// {u16 scale, u16 min} pairs.
template <int FMT> struct Par { uint32_t v[FMT == ONPU_Q4NX ? 4 : 2]; };
// The prefill GEMMs' parameters of row r: G128S the u16 scale alone (a 16-bit load), else as Par.
// A type of its own, so that the two G128S encodings cannot be mixed up.
template <int FMT> struct GPar { uint32_t v[FMT == ONPU_Q4NX ? 4 : (FMT == ONPU_G128S ? 1 : 2)]; };

// perm selector that moves the u16 of row r (the low half for even r) to the top of a dword
DEV uint32_t g128s_sel(int r) { return (r & 1) ? 0x03020c0cu : 0x01000c0cu; }

template <int FMT>
DEV Par<FMT> par_zero() {
    Par<FMT> p;
    for (auto & x : p.v) x = 0u;
    return p;
}

template <int FMT>
DEV Par<FMT> load_par(const uint8_t * blk, int r) {
    Par<FMT> p;
    // G128S: the dword holding rows r & ~1 and r | 1, and the selector of row r's half
    if (FMT == ONPU_G128S) {
        p.v[0] = *GLB(const uint32_t, blk + 1024 + 4 * (r >> 1));
        p.v[1] = g128s_sel(r);
    }
    else if (FMT == ONPU_Q4NX) {
        const u32x4 q = __builtin_nontemporal_load(GLB(const u32x4, blk + 1024 + 16 * r));
        for (int j = 0; j < 4; j++) p.v[j % (sizeof(p.v) / 4)] = q[j];
    } else {
        const u32x2 q = __builtin_nontemporal_load(GLB(const u32x2, blk + 1024 + 8 * r));
        p.v[0] = q.x;
        p.v[1 % (sizeof(p.v) / 4)] = q.y;
    }
    return p;
}

// Symmetric formats (w = s (u - 8)): the scale of each MFMA step (G128S: one for the block).
template <int FMT>
DEV void decode_scale(const Par<FMT> & p, float (&s)[4]) {
    if (FMT == ONPU_G128S) {
        // p.v[0] holds the scales of rows r & ~1 (low half) and r | 1 (high half); one byte
        // permute with the selector set at load (p.v[1]) moves row r's half to the top. A 16-bit
        // load instead lets the compiler narrow the loop's phi of loaded values to 16 bits and
        // widen it again at the loop's entry, a use that waits for the first chunk before the next
        // one is issued.
        const float v = __uint_as_float(__builtin_amdgcn_perm(p.v[0], p.v[0], p.v[1]));
        for (int j = 0; j < 4; j++) s[j] = v;
    } else {
        for (int j = 0; j < 4; j++)
            s[j] = scale_f32(FMT, (p.v[(j >> 1) % (sizeof(p.v) / 4)] >> (16 * (j & 1))) & 0xffff);
    }
}

// q4nx (w = s u + m): scale s, min m and nb = -128 s (exact) per MFMA step, for
// w = s (128 + u) + nb + m
template <int FMT>
DEV void decode_par(const Par<FMT> & p, float (&s)[4], float (&m)[4], float (&nb)[4]) {
    for (int j = 0; j < 4; j++) {
        const uint32_t pj = p.v[j % (sizeof(p.v) / 4)];
        s[j] = bf16_to_f32((uint16_t) (pj & 0xffff));
        m[j] = bf16_to_f32((uint16_t) (pj >> 16));
        nb[j] = -128.0f * s[j];
    }
}

// The factor on x's group sums as the decode kernels carry them: the symmetric formats start each
// MFMA from -136 * (sum of x over the group), so that it ends at x . (u - 8) (128 + u codes less
// the 8 of the symmetric zero point); q4nx keeps the plain sums for its offset term.
template <int FMT> constexpr float xsum_mul() { return FMT == ONPU_Q4NX ? 1.0f : -136.0f; }

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

// ------------------------------------------------------------------ router
// Wave-wide reductions with DPP inside each 16-lane row and readlane across the four rows (no LDS
// round trips): every lane gets the result.
template <int CTRL>
DEV uint32_t dpp_u(uint32_t v) { return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, CTRL, 0xf, 0xf, false); }
DEV float readlane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

DEV uint32_t wave_umax(uint32_t v) {
    v = max(v, dpp_u<0x111>(v));                      // row_shr:1 (lanes without a source see 0)
    v = max(v, dpp_u<0x112>(v));                      // row_shr:2
    v = max(v, dpp_u<0x114>(v));                      // row_shr:4
    v = max(v, dpp_u<0x118>(v));                      // row_shr:8: lane 15 of each row has the row's max
    const uint32_t a = __builtin_amdgcn_readlane(v, 15), b = __builtin_amdgcn_readlane(v, 31);
    const uint32_t c = __builtin_amdgcn_readlane(v, 47), d = __builtin_amdgcn_readlane(v, 63);
    return max(max(a, b), max(c, d));
}

DEV float wave_fsum(float v) {
    v += __uint_as_float(dpp_u<0xB1>(__float_as_uint(v)));   // quad_perm [1,0,3,2]
    v += __uint_as_float(dpp_u<0x4E>(__float_as_uint(v)));   // quad_perm [2,3,0,1]
    v += __uint_as_float(dpp_u<0x124>(__float_as_uint(v)));  // row_ror:4
    v += __uint_as_float(dpp_u<0x128>(__float_as_uint(v)));  // row_ror:8: every lane has its row's sum
    return (readlane_f(v, 0) + readlane_f(v, 16)) +
           (readlane_f(v, 32) + readlane_f(v, 48));
}

// float <-> unsigned key with the same order
DEV uint32_t ord_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
DEV float ord_val(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k); }


// Router of one token on one wave: softmax over E <= 256 logits, top-k by probability (ties to the
// lower id), renormalised when renorm (moe_runtime.py:333-341, reference.py:72-76). Lane l holds
// experts 4 l .. 4 l + 3, so the lowest lane holding the maximum also holds its lowest id. Lane j < k
// returns pick j (id and weight).
DEV void route_token(const float * __restrict__ l, int E, int k, int renorm, int & my_id, float & my_w) {
    const int lane = threadIdx.x & 63;
    float v[4];
    uint32_t mk = 0;
    for (int i = 0; i < 4; i++) {
        const int e = 4 * lane + i;
        v[i] = e < E ? l[e] : -INFINITY;
        mk = max(mk, ord_key(v[i]));
    }
    const float mx = ord_val(wave_umax(mk));
    float p[4], sum = 0.f;
    for (int i = 0; i < 4; i++) {
        const int e = 4 * lane + i;
        p[i] = e < E ? expf(v[i] - mx) : 0.f;
        sum += p[i];
    }
    sum = wave_fsum(sum);
    // selection keys: probability bits + 1 (p >= 0, so the bits order like the values); 0 = taken
    uint32_t key[4];
    for (int i = 0; i < 4; i++) key[i] = 4 * lane + i < E ? __float_as_uint(p[i]) + 1u : 0u;
    float ws = 0.f, my_p = 0.f;
    my_id = 0;
    for (int j = 0; j < k; j++) {
        uint32_t lb = 0;
        int li = 0;
        for (int i = 0; i < 4; i++)
            if (key[i] > lb) { lb = key[i]; li = i; }
        const uint32_t best = wave_umax(lb);
        const uint64_t hold = __ballot(lb == best);
        const int first = __builtin_ctzll(hold);
        const int bi = 4 * first + __builtin_amdgcn_readlane(li, first);
        for (int i = 0; i < 4; i++)
            if (lane == first && i == li) key[i] = 0u;
        const float pj = __uint_as_float(best - 1u) / sum;
        ws += pj;
        if (lane == j) { my_id = bi; my_p = pj; }
    }
    my_w = renorm ? my_p / ws : my_p;
}

// ------------------------------------------------------------------ decode GEMV family
// Per wave: RT row tiles x a run of K blocks. A operand = x rows (16 per MFMA block, MB blocks),
// B operand = unpacked biased codes 128 + u. For each MFMA step j (32 k, one 32-group), with cs the
// group sums of x times xsum_mul (shared by all row tiles):
//   symmetric formats:  cg = x . (128 + u)^T + cs = x . (u - 8)^T,   acc += s_j * cg
//                       (G128S: the four steps chain into one cg, one scale per block)
//   q4nx:               cg = x . (128 + u)^T,   acc += (s_j * cg - 128 s_j * cs) + m_j * cs
//                       (in that order: for one x row of 1 the bracket is u s exactly and the sum
//                       one rounding of u s + m, the reference's dequantized weight)
// cs[mb][j] comes from the caller (G128S: cs[mb][0] is over the whole block), in the MFMA C layout:
// lane (q, r) holds the sums of rows 16 mb + 4 q + v.
// With one A block (MB = 1) x row m sits in MFMA row perm16(m), so C element v of lane quarter q
// holds x row 4 v + q: RV (compile time) = the elements that hold rows below M (1 for M <= 4, 2 for
// M <= 8, else 4), and the accumulate touches those alone. MB > 1 keeps rows in order and all four.
// rows: the C elements that hold x rows below M (compile time), the only ones accumulated
DEV void acc4(f32x4 & acc, float s, float m, float nb, const f32x4 & cg, const f32x4 & cs, int rows) {
#pragma unroll
    for (int v = 0; v < rows; v++) acc[v] = fmaf(m, cs[v], fmaf(s, cg[v], fmaf(nb, cs[v], acc[v])));
}

DEV void acc1(f32x4 & acc, float s, const f32x4 & cg, int rows) {
#pragma unroll
    for (int v = 0; v < rows; v++) acc[v] = fmaf(s, cg[v], acc[v]);
}

// MFMA row of x row m (0..15) in a single A block: rows 0..3 go to MFMA rows 0, 4, 8, 12 (element 0
// of the four lane quarters of C), rows 4..7 to 1, 5, 9, 13, ...; the map is its own inverse.
DEV int perm16(int m) { return 4 * (m & 3) + (m >> 2); }

template <int FMT, int MB, int RT, int RV>
DEV void qacc_block(const bool (&valid)[RT], const u32x4 (&wv)[RT], const Par<FMT> (&par)[RT],
                    const u32x4 (&xa)[MB][4], const f32x4 (&cs)[MB][4], uint32_t mag, f32x4 (&acc)[RT][MB]) {
    constexpr int rows = MB == 1 ? RV : 4;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    if (FMT == ONPU_G128S) {
        for (int rt = 0; rt < RT; rt++) {
            if (!valid[rt]) continue;
            f32x4 cg[MB];
            for (int mb = 0; mb < MB; mb++) cg[mb] = cs[mb][0];
            for (int j = 0; j < 4; j++) {
                const u32x4 bw = unpack_biased(wv[rt][j], mag);
                for (int mb = 0; mb < MB; mb++) cg[mb] = mfma(xa[mb][j], bw, cg[mb]);
            }
            float s[4];
            decode_scale<FMT>(par[rt], s);
            for (int mb = 0; mb < MB; mb++) acc1(acc[rt][mb], s[0], cg[mb], rows);
        }
    } else if (FMT == ONPU_Q4NX) {
        for (int rt = 0; rt < RT; rt++) {
            if (!valid[rt]) continue;
            float s[4], m[4], nb[4];
            decode_par<FMT>(par[rt], s, m, nb);
            for (int j = 0; j < 4; j++) {
                const u32x4 bw = unpack_biased(wv[rt][j], mag);
                for (int mb = 0; mb < MB; mb++) {
                    const f32x4 cg = mfma(xa[mb][j], bw, z);
                    acc4(acc[rt][mb], s[j], m[j], nb[j], cg, cs[mb][j], rows);
                }
            }
        }
    } else {
        for (int rt = 0; rt < RT; rt++) {
            if (!valid[rt]) continue;
            float s[4];
            decode_scale<FMT>(par[rt], s);
            u32x4 bw[4];
            for (int j = 0; j < 4; j++) bw[j] = unpack_biased(wv[rt][j], mag);
            for (int mb = 0; mb < MB; mb++) {
                f32x4 cg[4];                              // four independent MFMAs, then their scales
                for (int j = 0; j < 4; j++) cg[j] = mfma(xa[mb][j], bw[j], cs[mb][j]);
                for (int j = 0; j < 4; j++) acc1(acc[rt][mb], s[j], cg[j], rows);
            }
        }
    }
}

// column sums of x for one block times xsum_mul, from an MFMA against a constant B of bf16 1 (q4nx)
// or -136 (exact in bf16, so each product is exact) (x from global memory)
template <int FMT, int MB>
DEV void xsum_mfma(const u32x4 (&xa)[MB][4], f32x4 (&cs)[MB][4]) {
    const uint32_t c = FMT == ONPU_Q4NX ? 0x3f803f80u : 0xc308c308u;
    const u32x4 ones = {c, c, c, c};
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    for (int mb = 0; mb < MB; mb++) {
        if (FMT == ONPU_G128S) {
            cs[mb][0] = z;
            for (int j = 0; j < 4; j++) cs[mb][0] = mfma(xa[mb][j], ones, cs[mb][0]);
        } else {
            for (int j = 0; j < 4; j++) cs[mb][j] = mfma(xa[mb][j], ones, z);
        }
    }
}

// Where the A operand (x rows) comes from: global rows or the workgroup's LDS copy xs[M][xls]
// (bf16, zero past K).
struct XSrc {
    const uint16_t * x;
    int64_t ldx;
    const uint16_t * xs;
    int64_t xls;
    const float * xsum;       // XL: LDS column sums [group][16] of x's 32- (G128S: 128-) groups
};

// x fragments of block b from the LDS copy: lane (r, q) of A-block mb holds
// x[row(16 mb + r)][128 b + 32 j + 8 q .. +7]. LDS rows are zero-padded to 128 KB columns; rows
// >= M read row M - 1 (their MFMA rows are never stored), so the reads need no masks.
template <int MB>
DEV void load_x_lds(const XSrc & X, int M, int64_t b, int r, int q, u32x4 (&xa)[MB][4]) {
    for (int mb = 0; mb < MB; mb++) {
        const int i = MB == 1 ? perm16(r) : 16 * mb + r, m = i < M ? i : M - 1;
        const uint16_t * base = X.xs + (uint32_t) m * (uint32_t) X.xls + (uint32_t) b * 128u + 8u * q;
        for (int j = 0; j < 4; j++) xa[mb][j] = *LDS_U32X4(base + 32 * j);
    }
}

// x fragments of block b from global rows (zero for rows >= M and columns past K), loaded just
// before the block's MFMAs, after the next chunk's weights were issued: measured faster (M = 4..8,
// K = 4096..12288) than loading a whole chunk's x first or loading it ahead with the chunk's
// weights (clamped, branch-free), which holds registers across the whole pipeline.
template <int MB>
DEV void load_x_glb(const XSrc & X, int M, int64_t K, int64_t b, int r, int q, u32x4 (&xa)[MB][4]) {
    for (int mb = 0; mb < MB; mb++) {
        const int m = MB == 1 ? perm16(r) : 16 * mb + r;
        for (int j = 0; j < 4; j++) {
            const int64_t k = 128 * b + 32 * j + 8 * q;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (m < M && k < K) v = *(const u32x4 *) (X.x + m * X.ldx + k);
            xa[mb][j] = v;
        }
    }
}

// One chunk of NB blocks x RT row tiles: weights (non-temporal: each byte is read once), parameters
// and which (block, tile) pairs are real. The loads are unconditional (an out-of-range pair reads
// the always-valid block `safe` and is flagged), so the hardware wait counts stay exact across the
// two-chunk pipeline instead of falling back to waiting for every outstanding load.
template <int FMT, int RT, int NB>
struct WChunk {
    u32x4 wv[NB][RT];
    Par<FMT> par[NB][RT];
    bool ok[NB][RT];
};

template <int FMT, int RT, int NB>
DEV void load_chunk(WChunk<FMT, RT, NB> & c, const uint8_t * const (&tb)[RT], const uint8_t * last, int64_t c0,
                    int64_t b1, int lane, int r) {
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const uint8_t * p[NB][RT];
    for (int i = 0; i < NB; i++)
        for (int rt = 0; rt < RT; rt++) {
            // a block past b1 (or of a missing tile) re-reads `last`, the wave's own last block of
            // tile 0: an address the wave fetches anyway, never one that every wave shares
            c.ok[i][rt] = tb[rt] != nullptr && (int) c0 + i < (int) b1;      // 32-bit: scalar compares
            p[i][rt] = c.ok[i][rt] ? tb[rt] + (c0 + i) * BLK : last;
        }
    for (int i = 0; i < NB; i++)
        for (int rt = 0; rt < RT; rt++) {
            c.wv[i][rt] = __builtin_nontemporal_load(GLB(const u32x4, p[i][rt] + 16 * lane));
            c.par[i][rt] = load_par<FMT>(p[i][rt], r);
        }
}

// The MFMAs of one chunk (blocks c0 .. c0 + NB - 1, those below b1)
template <int FMT, int MB, int RT, int NB, bool XL, int RV, bool MS = false>
DEV void compute_chunk(const WChunk<FMT, RT, NB> & ch, int64_t c0, int64_t b1, const XSrc & X, int M, int64_t K,
                       int r, int q, uint32_t mag, f32x4 (&acc)[RT][MB]) {
    if (XL) {                             // x from LDS, one block at a time (short latency)
        for (int i = 0; i < NB; i++) {
            if ((int) c0 + i >= (int) b1) break;
            u32x4 xa[MB][4];
            load_x_lds<MB>(X, M, c0 + i, r, q, xa);
            f32x4 cs[MB][4];
            constexpr int GPB = FMT == ONPU_G128S ? 1 : 4;
            if (!MS) {                        // the group sums the staging left in LDS
                for (int mb = 0; mb < MB; mb++)
                    for (int j = 0; j < GPB; j++)
                        cs[mb][j] = *(const __attribute__((address_space(3))) f32x4 *) (X.xsum + ((c0 + i) * GPB + j) *
                                                                                       16 + 16 * mb + 4 * q);
            } else {                          // on the matrix core (the staging skipped them)
                xsum_mfma<FMT, MB>(xa, cs);
            }
            qacc_block<FMT, MB, RT, RV>(ch.ok[i], ch.wv[i], ch.par[i], xa, cs, mag, acc);
        }
    } else {                              // x from global memory, each block's just before its MFMAs
        for (int i = 0; i < NB; i++)
            if ((int) c0 + i < (int) b1) {
                u32x4 xa[MB][4];
                load_x_glb<MB>(X, M, K, c0 + i, r, q, xa);
                f32x4 cs[MB][4];
                xsum_mfma<FMT, MB>(xa, cs);
                qacc_block<FMT, MB, RT, RV>(ch.ok[i], ch.wv[i], ch.par[i], xa, cs, mag, acc);
            }
    }
}

// the first chunk's loads (qacc_run's prologue). Returns the wave's last block (the target of
// out-of-range slots); b1 drops to b0 without a tile. The loads are issued also by a wave without
// blocks (from `safe`, a block every launch has): a load under a branch would make the compiler's
// wait counts at the join assume the branch not taken, and the first wait for x would then also
// wait for the weights just issued.
template <int FMT, int RT, int NB>
DEV const uint8_t * qacc_start(WChunk<FMT, RT, NB> & ca, const uint8_t * const (&tb)[RT], int64_t b0, int64_t & b1,
                               const uint8_t * safe) {
    const int lane = threadIdx.x & 63, r = lane & 15;
    if (tb[0] == nullptr) b1 = b0;
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const uint8_t * last = b0 < b1 ? tb[0] + (b1 - 1) * BLK : safe;
    load_chunk<FMT, RT, NB>(ca, tb, last, b0, b1, lane, r);
    return last;
}

// the chunk loop after qacc_start (acc accumulates; the caller zeroes it); b1 and last as
// qacc_start left them
template <int FMT, int MB, int RT, int NB, bool XL, int RV, bool MS = false>
DEV void qacc_rest(WChunk<FMT, RT, NB> & ca, const uint8_t * const (&tb)[RT], const uint8_t * last, int64_t b0,
                   int64_t b1, const XSrc & X, int M, int64_t K, f32x4 (&acc)[RT][MB]) {
    const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
    if (b0 >= b1) return;
    const uint32_t mag = 0x43004300u;
    WChunk<FMT, RT, NB> cb;
    const int64_t nc = (b1 - b0 + NB - 1) / NB;     // chunks; chunk i starts at b0 + i * NB
    int64_t i = 0;
    for (; i + 2 < nc; i += 2) {                     // chunks i + 1 and i + 2 exist
        load_chunk<FMT, RT, NB>(cb, tb, last, b0 + (i + 1) * NB, b1, lane, r);
        compute_chunk<FMT, MB, RT, NB, XL, RV, MS>(ca, b0 + i * NB, b1, X, M, K, r, q, mag, acc);
        load_chunk<FMT, RT, NB>(ca, tb, last, b0 + (i + 2) * NB, b1, lane, r);
        compute_chunk<FMT, MB, RT, NB, XL, RV, MS>(cb, b0 + (i + 1) * NB, b1, X, M, K, r, q, mag, acc);
    }
    if (i + 1 < nc) {                                // two chunks left: ca (loaded) and one more
        load_chunk<FMT, RT, NB>(cb, tb, last, b0 + (i + 1) * NB, b1, lane, r);
        compute_chunk<FMT, MB, RT, NB, XL, RV, MS>(ca, b0 + i * NB, b1, X, M, K, r, q, mag, acc);
        compute_chunk<FMT, MB, RT, NB, XL, RV, MS>(cb, b0 + (i + 1) * NB, b1, X, M, K, r, q, mag, acc);
    } else {
        compute_chunk<FMT, MB, RT, NB, XL, RV, MS>(ca, b0 + i * NB, b1, X, M, K, r, q, mag, acc);
    }
}

// One wave: tiles tb[rt] (nullptr: no tile) over blocks [b0, b1), in chunks of NB blocks with two
// chunk buffers: the loads of chunk i + 1 are in flight while chunk i is computed, so each wave
// streams its K range with NB..2 NB blocks (x RT tiles) outstanding. Loads are only issued for
// chunks that hold blocks, and every path into the loop head has exactly the chunk `ca`
// outstanding, so the compiler's wait counts cover just the chunk being computed. pre() runs
// before the first loads are issued and post() right after (the workgroup's LDS staging of x: its
// loads first, then the LDS writes and the barrier while the weights stream); every wave calls
// both, also one with no blocks. (Issuing both chunks before the barrier measured slower.)
template <int FMT, int MB, int RT, int NB, bool XL, int RV, bool MS, class Pre, class Post>
DEV void qacc_run(const uint8_t * const (&tb)[RT], int64_t b0, int64_t b1, const uint8_t * safe, const XSrc & X, int M,
                  int64_t K, Pre pre, Post post, f32x4 (&acc)[RT][MB]) {
    for (int rt = 0; rt < RT; rt++)
        for (int mb = 0; mb < MB; mb++) acc[rt][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
    WChunk<FMT, RT, NB> ca;
    pre();
    const uint8_t * last = qacc_start<FMT, RT, NB>(ca, tb, b0, b1, safe);
    post();
    qacc_rest<FMT, MB, RT, NB, XL, RV, MS>(ca, tb, last, b0, b1, X, M, K, acc);
}

// The workgroup's LDS copy of x [M][K] (bf16) for the XL variants, in 16 B units u = tid + i *
// blockDim; rows are zero-padded from K to Kpad = 128 * KB and followed by the column sums of x per
// 32-group (G128S: per 128) times xsum_mul, xsum[group][16 MFMA rows] (MB = 1: x row m at
// perm16(m)). pre() loads the first PRE units per thread and is called before the weight loads are
// issued; post() stores them, copies any further units and ends with a barrier, while the weights
// stream. A unit copied there is loaded after the weights, and its wait then also waits for them,
// which holds the next weight chunk back by a memory round trip: PRE = 8 covers up to 8 x rows of
// K = 4096 in a workgroup of 8 waves. The first PRE units are buffer loads over x's M rows (the
// host keeps M * ldx * 2 < 2^31):
// units past the rows or past K get an offset out of the buffer's range, which returns zeros
// without a memory access, so the loads need no branch (a load under a branch gets a wait for
// every outstanding load at the branch's end, which would hold the weight loads back by a full
// memory round trip) and no clamped address (which would send every wave to one L2 line).
template <int FMT, int MB, int PRE, bool MS>
struct XStage {
    const uint16_t * x;
    int64_t ldx, K;
    uint16_t * xs;
    int64_t xls;
    float * xsum;
    uint32_t kp8, nunits, bd, xbytes;
    bool sums;                                // MS: group sums staged (only past 8 rows)
    u32x4 xv[PRE];
    static constexpr int UPG = (FMT == ONPU_G128S ? 128 : 32) / 8;     // 16 B units per group

    __device__ __forceinline__ XStage(const uint16_t * x_, int64_t ldx_, int64_t K_, int64_t KB, int M, uint16_t * xs_,
                                      int64_t xls_, float * xsum_)
        : x(x_), ldx(ldx_), K(K_), xs(xs_), xls(xls_), xsum(xsum_), kp8((uint32_t) KB * 16),
          nunits((uint32_t) M * (uint32_t) KB * 16), bd(blockDim.x), xbytes((uint32_t) (M * ldx_ * 2)), sums(!MS || M > 8) {}

    __device__ __forceinline__ u32x4 unit(uint32_t u) const {
        const uint32_t m = u / kp8, k = (u - m * kp8) * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (k < K) v = *(const u32x4 *) (x + (int64_t) m * ldx + k);
        return v;
    }
    // row m = u / kp8 from a float reciprocal (u < 2^24, so the estimate is off by at most one).
    // Iterations past the last unit are skipped as a whole (measured 0.2-0.3 us faster per launch
    // at M = 1 than issuing all four).
    __device__ __forceinline__ void pre() {
        const float inv = 1.0f / (float) kp8;
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *) x, (short) 0, (int) xbytes, 0x00020000);
        for (int i = 0; i < PRE; i++) {
            if ((uint32_t) i * bd >= nunits) break;
            const uint32_t u = threadIdx.x + i * bd;
            uint32_t m = (uint32_t) ((float) u * inv);
            m = m * kp8 > u ? m - 1 : ((m + 1) * kp8 <= u ? m + 1 : m);
            const uint32_t k = (u - m * kp8) * 8;
            const uint32_t off = u < nunits && k < K ? (m * (uint32_t) ldx + k) * 2u : 0x80000000u;
            xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
    }
    // unit u's 8 values summed in fp32, then over the UPG consecutive lanes holding one group (the
    // units of a group are consecutive in u, and u = tid + i * blockDim keeps them in one wave)
    __device__ __forceinline__ void stage(uint32_t u, u32x4 v) {
        if (u < nunits) {
            const uint32_t m = u / kp8;
            *LDS_U32X4(xs + (int64_t) m * xls + (u - m * kp8) * 8) = v;
        }
        if (MS && !sums) return;
        float t = 0.f;
        for (int d = 0; d < 4; d++) t += __uint_as_float(v[d] << 16) + __uint_as_float(v[d] & 0xffff0000u);
        for (int o = UPG / 2; o > 0; o >>= 1) t += __shfl_xor(t, o);
        if (u < nunits && u % UPG == 0) {
            const uint32_t m = u / kp8, g = (u - m * kp8) / UPG;
            xsum[g * 16 + (MB == 1 ? perm16(m) : m)] = t * xsum_mul<FMT>();
        }
    }
    // REST: copy units past the first PRE per thread (a kernel that never has them leaves the loop
    // out: its loads would make the compiler's wait counts after it assume a pending load)
    template <bool REST = true>
    __device__ __forceinline__ void post() {
        for (int i = 0; i < PRE; i++) {
            if ((uint32_t) i * bd >= nunits) break;
            stage(threadIdx.x + i * bd, xv[i]);
        }
        if (REST)
            for (uint32_t u0 = PRE * bd; u0 < nunits; u0 += bd) {    // same trip count for every lane
                const uint32_t u = u0 + threadIdx.x;
                stage(u, u < nunits ? unit(u) : (u32x4){0u, 0u, 0u, 0u});
            }
        __syncthreads();
    }
};

// Epilogues
enum { EPI_STORE = 0, EPI_ACT = 1, EPI_SLOTSUM = 2, EPI_ARGMAX = 3 };

// argmax key of value v at index n: the value's order-preserving bits above the complement of the
// index, so the larger key is the larger value and, among equal values, the lower index. A NaN gets
// the top value bits, above +inf: a row holding a NaN gives its first NaN's index, as the reference's
// numpy / torch argmax over the logits does (npu4/engine.py:358, runtime.py:348).
DEV uint64_t argmax_key(float v, int64_t n) {
    return ((uint64_t) (v != v ? 0xffffffffu : ord_key(v)) << 32) | (uint32_t) (0xffffffffu - (uint32_t) n);
}

DEV uint64_t wave_umax64(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t u = __shfl_xor(v, o);
        v = u > v ? u : v;
    }
    return v;
}

DEV void store_out(void * y, int yf32, int64_t idx, float v) {
    if (yf32) ((float *) y)[idx] = v;
    else ((uint16_t *) y)[idx] = f32_to_bf16(v);
}

DEV float silu_f(float g) { return g / (1.0f + expf(-g)); }

constexpr int qgemv_lb(int MB, int RT, int NB, int XL) { return (MB == 1 && RT * NB <= (XL ? 4 : 2)) ? 1024 : 512; }

// grid: (tile groups, slots), block: waves * 64 threads. A workgroup holds a.tw tile groups x KW
// K parts (KW = waves / a.tw): wave w works on tile group w / KW (RT row tiles: t and t + stride,
// stride = gridDim.x * a.tw) and K part w % KW. Dynamic LDS: the cross-wave reduction buffer
// (waves * RT * MB KiB), then with XL the x rows [M][xls] bf16 shared by all waves. XL = 2 is XL = 1
// except up to 8 rows, where x's group sums come from one MFMA per group against a constant B
// instead of the staging's VALU sums, and are not kept in LDS.
//   STORE  : slot = blockIdx.y; y[m][n] = sum of the K parts
//   ACT    : RT = 2, tiles (gate t, up t + stride); out[m][16 t + r] = silu(g) * u
//   SLOTSUM: a.tw = 1; wave w -> slot w / ksplit (its expert and x row), K part w % ksplit;
//            out = sum_s w_s y_s
//   ARGMAX : as STORE (fp32 y), and each row's key over the workgroup's outputs (an LDS maximum)
//            into a.akeys[m][blockIdx.x], for k_argmax_keys to reduce. (One counter on which the
//            ~1000 workgroups of the LM head count in, the last reducing, measured ~5x slower: the
//            agent-scope increments of one address queue behind each other, ~0.2 us apiece.)
template <int FMT, int MB, int RT, int NB, int EPI, int XL>
__global__ __launch_bounds__(qgemv_lb(MB, RT, NB, XL)) void k_qgemv(QArgs a) {
    extern __shared__ __align__(16) float red[];
    // the wave index is uniform across a wave: readfirstlane lets the compiler keep tile bases,
    // block ranges and their guards in scalar registers
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const int ntw = EPI == EPI_SLOTSUM ? 1 : a.tw, KW = nw / ntw;
    int64_t slot;
    int kpart, twi;
    if (EPI == EPI_SLOTSUM) {
        slot = (int64_t) blockIdx.y * a.nslot + wave / a.ksplit;
        kpart = wave % a.ksplit;
        twi = 0;
    } else {
        slot = blockIdx.y;
        twi = wave / KW;
        kpart = wave % KW;
    }
    const uint16_t * x = a.x + (slot / a.xdiv) * a.xslot;
    constexpr int PER = RT * MB * 256;
    uint16_t * xs = (uint16_t *) (red + nw * PER);
    // XL: column sums of x per 32-group (G128S: per 128) times xsum_mul after the x rows:
    // xsum[group][16 MFMA rows] (x row m at perm16(m))
    float * xsum = (float *) (xs + (int64_t) a.M * a.xls);
    XStage<FMT, MB, MB == 1 && EPI != EPI_ACT ? 8 : 4, XL == 2> xst(x, a.ldx, a.K, a.KB, a.M, xs, a.xls, xsum);
    int64_t e = 0;
    const bool route = EPI == EPI_ACT && a.logits != nullptr;
    if (route) {
        // the slot's expert from the token's logits (wave 0, the router kernel's selection) while
        // the x loads are in flight; the weights' addresses wait for it
        __shared__ int s_expert;
        if (XL) xst.pre();
        if (wave == 0) {
            const int64_t t = slot / a.xdiv;
            const int j = (int) (slot - t * a.xdiv);
            int my_id;
            float my_w;
            route_token(a.logits + t * a.E, a.E, (int) a.xdiv, a.renorm, my_id, my_w);
            if (lane == 0) s_expert = __builtin_amdgcn_readlane(my_id, j);
            if (blockIdx.x == 0 && j == 0 && lane < a.xdiv) {
                a.rids[t * a.xdiv + lane] = my_id;
                a.rw[t * a.xdiv + lane] = my_w;
            }
        }
        __syncthreads();
        e = s_expert;
    } else if (a.ids) {
        e = a.ids[slot];
    }
    const uint8_t * W = a.W + e * a.estride;
    const uint8_t * tb[RT];
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const int64_t stride = (int64_t) gridDim.x * ntw, tg0 = (int64_t) blockIdx.x * ntw;
    for (int rt = 0; rt < RT; rt++) {
        const int64_t t = tg0 + twi + rt * stride;
        tb[rt] = t < a.NT ? W + t * a.KB * BLK : nullptr;
    }
    const int64_t b0 = (int64_t) kpart * a.bpw, b1 = b0 + a.bpw < a.KB ? b0 + a.bpw : a.KB;
    const XSrc X{x, a.ldx, XL ? xs : nullptr, a.xls, XL ? xsum : nullptr};
    auto pre = [&]() {
        if (XL && !route) xst.pre();              // (routing workgroups issued them already)
    };
    auto post = [&]() {
        if (XL) xst.post();
    };
    f32x4 acc[RT][MB];
    if (MB == 1 && a.M <= 4) qacc_run<FMT, MB, RT, NB, XL != 0, 1, XL == 2>(tb, b0, b1, W, X, a.M, a.K, pre, post, acc);
    else if (MB == 1 && a.M <= 8) qacc_run<FMT, MB, RT, NB, XL != 0, 2, XL == 2>(tb, b0, b1, W, X, a.M, a.K, pre, post, acc);
    else qacc_run<FMT, MB, RT, NB, XL != 0, 4, false>(tb, b0, b1, W, X, a.M, a.K, pre, post, acc);

    // cross-wave reduction through LDS: red[wave][((rt * MB + mb) * 4 + v) * 64 + lane]
    for (int rt = 0; rt < RT; rt++)
        for (int mb = 0; mb < MB; mb++)
            for (int v = 0; v < 4; v++) red[wave * PER + ((rt * MB + mb) * 4 + v) * 64 + lane] = acc[rt][mb][v];
    __shared__ uint64_t s_key[EPI == EPI_ARGMAX ? 64 : 1];
    if (EPI == EPI_ARGMAX && (int) threadIdx.x < a.M) s_key[threadIdx.x] = 0;    // below every key
    __syncthreads();
    const int nout = EPI == EPI_ACT ? MB * 256 : PER;
    for (int oo = threadIdx.x; oo < ntw * nout; oo += blockDim.x) {
        const int tw = oo / nout, o = oo % nout;
        const int rt = o / (MB * 256), mb = (o / 256) % MB, v = (o / 64) % 4, l = o % 64;
        const int m = MB == 1 ? 4 * v + (l >> 4) : 16 * mb + 4 * (l >> 4) + v;     // see perm16
        const int64_t n = 16 * (tg0 + tw + rt * stride) + (l & 15);
        if (m >= a.M) continue;
        const float * rp = red + (int64_t) tw * KW * PER + o;
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
            for (int kp = 0; kp < KW; kp++) { g += rp[kp * PER]; u += rp[kp * PER + MB * 256]; }
            if (n < a.N / 2)
                store_out(a.y, a.yf32, (int64_t) slot * a.yslot + (int64_t) m * a.ldy + n, silu_f(g) * u);
        } else {
            float s = 0.f;
            for (int kp = 0; kp < KW; kp++) s += rp[kp * PER];
            if (n < a.N) {
                store_out(a.y, a.yf32, (int64_t) slot * a.yslot + (int64_t) m * a.ldy + n, s);
                if (EPI == EPI_ARGMAX) atomicMax((unsigned long long *) &s_key[m], (unsigned long long) argmax_key(s, n));
            }
        }
    }
    if (EPI == EPI_ARGMAX) {
        __syncthreads();
        if ((int) threadIdx.x < a.M) a.akeys[(int64_t) threadIdx.x * gridDim.x + blockIdx.x] = s_key[threadIdx.x];
    }
}

// ------------------------------------------------------------------ prefill GEMM
// The 8 weights of dword d (B-operand order: element e at nibble (e >> 1) + 4 (e & 1)) dequantized
// to bf16 RNE(w), w = (u - 8) s or u s + m: the weight the reference device feeds its MAC
// (gemv_any.cc:65,106-107).
// Symmetric formats: each pair of codes becomes two fp16 1024 + u in one and-or (as unpack_biased),
// and v_fma_mix_f32 (an fp16 operand widened inside a fused fma) forms (1024 + u) s - 1032 s: the
// product and the sum are exact in fp32 (at most 19 significant bits), so the result is
// (u - 8) s exactly, and v_cvt_pk_bf16_f32 rounds it to nearest even: 7 + 8 + 4 = 19 VALU ops per 8
// weights. c (from par_sc) is -1032 s.
// q4nx (u s + m, one rounding): the nibbles split into bytes (lo: even nibbles, hi: odd), converted
// with v_cvt_f32_ubyteN and one fma each (u s is exact), 23 ops per 8 weights.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
DEV uint32_t dq_pair(uint32_t w16, float s, float c) {
    const f16x2 h = __builtin_bit_cast(f16x2, w16);
    return pack_bf16x2(fmaf((float) h.x, s, c), fmaf((float) h.y, s, c));
}
template <int FMT>
DEV u32x4 dequant8(uint32_t d, float s, float c) {
    if (FMT != ONPU_Q4NX) {
        const u32x4 h = unpack_biased(d, 0x64006400u);
        return (u32x4){dq_pair(h.x, s, c), dq_pair(h.y, s, c), dq_pair(h.z, s, c), dq_pair(h.w, s, c)};
    }
    // an opaque mask, so that the optimizer cannot fold each byte extraction into a 4-bit field
    // extract (v_bfe) plus v_cvt_f32_ubyte0 (two ops per weight instead of one); plain code rather
    // than an asm v_and_b32, so that MFMA hazards stay visible to the compiler
    const uint32_t M = opaque_s(0x0f0f0f0fu);
    const uint32_t lo = d & M, hi = (d >> 4) & M;
    auto f = [&](uint32_t w, int byte) { return fmaf((float) ((w >> (8 * byte)) & 0xffu), s, c); };
    return (u32x4){pack_bf16x2(f(lo, 0), f(lo, 2)), pack_bf16x2(f(hi, 0), f(hi, 2)), pack_bf16x2(f(lo, 1), f(lo, 3)),
                   pack_bf16x2(f(hi, 1), f(hi, 3))};
}

// dequant8 in parts, for spreading its VALU work: dequant_split prepares the dword (q4nx: the
// nibbles split into bytes; symmetric formats: kept whole), dequant_part(k) forms output dword k
// of dequant8 (the same operations, so the same bits)
template <int FMT>
DEV void dequant_split(uint32_t d, uint32_t & lo, uint32_t & hi) {
    if (FMT != ONPU_Q4NX) {
        lo = d;
        hi = 0;
        return;
    }
    const uint32_t M = opaque_s(0x0f0f0f0fu);
    lo = d & M;
    hi = (d >> 4) & M;
}
template <int FMT>
DEV uint32_t dequant_part(uint32_t lo, uint32_t hi, int k, float s, float c) {
    if (FMT != ONPU_Q4NX) {
        const uint32_t M = opaque_s(0x000F000Fu), g = opaque_v(0x64006400u);
        return dq_pair(((k ? lo >> (4 * k) : lo) & M) | g, s, c);
    }
    auto f = [&](uint32_t w, int byte) { return fmaf((float) ((w >> (8 * byte)) & 0xffu), s, c); };
    const uint32_t w = (k & 1) ? hi : lo;
    const int b = k >> 1;                    // dwords: (lo 0, 2), (hi 0, 2), (lo 1, 3), (hi 1, 3)
    return pack_bf16x2(f(w, b), f(w, b + 2));
}

// scale s and additive constant c of MFMA step j for dequant8: symmetric formats c = -1032 s (the
// fp16 codes carry 1024 + u), q4nx c = m (w = u s + m)
template <int FMT>
DEV void par_sc(const GPar<FMT> & p, int j, float & s, float & c) {
    if (FMT == ONPU_G128S) {
        s = bf16_to_f32((uint16_t) p.v[0]);
        c = -1032.0f * s;
    } else if (FMT == ONPU_Q4NX) {
        const uint32_t pj = p.v[j % (sizeof(p.v) / 4)];
        s = bf16_to_f32((uint16_t) (pj & 0xffff));
        c = bf16_to_f32((uint16_t) (pj >> 16));
    } else {
        s = scale_f32(FMT, (p.v[(j >> 1) % (sizeof(p.v) / 4)] >> (16 * (j & 1))) & 0xffff);
        c = -1032.0f * s;
    }
}

// Y[M][N] = X[M][K] . deq(W)^T. Workgroup: 4 waves, tile MT = 16 MB rows of X (MB = 8, or 2 / 4
// A blocks for up to 32 / 64 rows: MFMAs and LDS reads on rows past M would cost their full time)
// x 64 NTW rows of W; wave w owns NTW 16-row weight tiles and all MT X rows (MB x NTW accumulators
// of 16 x 16). Per 128-wide K block the X tile (MB x 4 KiB of MFMA A fragments [mb][j][lane]) sits
// in one of two LDS buffers. The buffers are filled straight from global memory by buffer_load_dwordx4 ... lds
// (lane l of a wave writes 16 B at base + 16 l, so one load fills one A fragment; rows past M and
// k past K read out of the buffer's range and land as zeros), so X never occupies registers.
// Each wave dequantizes its own weight blocks in registers one 32-wide K step at a time and runs
// 8 NTW MFMAs per step. The next block's X and weights are in flight while the current block
// computes; one barrier per block. Workgroups are numbered so that consecutive tiles share an XCD
// (workgroup i runs on XCD i % 8), M tile fastest: concurrent workgroups of an XCD reuse the same
// weight tiles from its L2. The host keeps M * ldx * 2 below 2^31 (32-bit buffer offsets).
typedef __attribute__((address_space(3))) void lds_void;

// one 128-wide K block of the GEMM: 4 steps of (dequantize NTW weight fragments, MBG NTW MFMAs),
// X from the LDS fragments [mb][j][lane] of MBG 16-row A blocks.
// NTW <= 3: the A fragments of step j + 1 are read from LDS before step j's MFMAs are issued, and
// step j's dequant runs while step j's reads are in flight. NTW = 4 has no registers to spare for
// that and reads each step's fragments at the step's start.
template <int FMT, int NTW, int MBG>
DEV void gemm_block(const u32x4 * xsb, const u32x4 (&wr)[NTW], const GPar<FMT> (&pr)[NTW], int lane,
                    f32x4 (&acc)[MBG][NTW]) {
    constexpr bool PIPE = NTW <= 3;
    u32x4 xa[PIPE ? 2 : 1][MBG];
    if (PIPE) {
#pragma unroll
        for (int mb = 0; mb < MBG; mb++) xa[0][mb] = *LDS_U32X4(&xsb[(mb * 4 + 0) * 64 + lane]);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int cur = PIPE ? (j & 1) : 0;
        if (!PIPE) {
#pragma unroll
            for (int mb = 0; mb < MBG; mb++) xa[0][mb] = *LDS_U32X4(&xsb[(mb * 4 + j) * 64 + lane]);
        }
        if (PIPE) {
            u32x4 bw[NTW];
#pragma unroll
            for (int i = 0; i < NTW; i++) {
                float sc, cc;
                par_sc<FMT>(pr[i], j, sc, cc);
                bw[i] = dequant8<FMT>(wr[i][j], sc, cc);
            }
            if (j < 3) {
#pragma unroll
                for (int mb = 0; mb < MBG; mb++)
                    xa[(j + 1) & 1][mb] = *LDS_U32X4(&xsb[(mb * 4 + j + 1) * 64 + lane]);
            }
#pragma unroll
            for (int mb = 0; mb < MBG; mb++)
#pragma unroll
                for (int i = 0; i < NTW; i++) acc[mb][i] = mfma(xa[cur][mb], bw[i], acc[mb][i]);
        } else {                          // one weight fragment live at a time
#pragma unroll
            for (int i = 0; i < NTW; i++) {
                float sc, cc;
                par_sc<FMT>(pr[i], j, sc, cc);
                const u32x4 bw = dequant8<FMT>(wr[i][j], sc, cc);
#pragma unroll
                for (int mb = 0; mb < MBG; mb++) acc[mb][i] = mfma(xa[0][mb], bw, acc[mb][i]);
            }
        }
        // keep each step's work within the step: hoisting later steps forward only lengthens live
        // ranges past the register budget
        __builtin_amdgcn_sched_barrier(0);
    }
}

// one 128-wide K block with the decode GEMV's arithmetic, for 16-row tiles: the codes
// enter the MFMA as the bf16 integers 128 + u (one and-or per pair), each group's MFMA starts from
// -136 (sum of x over the group) (symmetric formats; the sums from MFMAs against a constant
// fragment), so that it ends at x . (u - 8) exactly, and the group scale is applied to the fp32
// result: the exact dequant (u - 8) s, or u s + m for q4nx (m sum(x) + s x . (128 + u) - 128 s
// sum(x)), as the GEMV computes it, with ~5 VALU ops per MFMA instead of a dequant per weight
// (19-23 ops per 8 weights for one MFMA at this tile height; 151936 x 4096 g128s at 4 / 8 / 16 rows
// 80 / 78 / 77 -> 61 / 63 / 71 us)
template <int FMT, int NTW, int MBG>
DEV void gemm_block_biased(const u32x4 * xsb, const u32x4 (&wr)[NTW], const GPar<FMT> (&pr)[NTW], int lane,
                           f32x4 (&acc)[MBG][NTW]) {
    const uint32_t mag = 0x43004300u;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    u32x4 xa[MBG][4];
#pragma unroll
    for (int mb = 0; mb < MBG; mb++)
#pragma unroll
        for (int j = 0; j < 4; j++) xa[mb][j] = *LDS_U32X4(&xsb[(mb * 4 + j) * 64 + lane]);
    f32x4 cs[MBG][4];
    xsum_mfma<FMT, MBG>(xa, cs);
#pragma unroll
    for (int i = 0; i < NTW; i++) {
        if (FMT == ONPU_G128S) {
            float s, c;
            par_sc<FMT>(pr[i], 0, s, c);
            f32x4 cg[MBG];
#pragma unroll
            for (int mb = 0; mb < MBG; mb++) cg[mb] = cs[mb][0];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const u32x4 bw = unpack_biased(wr[i][j], mag);
#pragma unroll
                for (int mb = 0; mb < MBG; mb++) cg[mb] = mfma(xa[mb][j], bw, cg[mb]);
            }
#pragma unroll
            for (int mb = 0; mb < MBG; mb++) acc1(acc[mb][i], s, cg[mb], 4);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float s, m;
                par_sc<FMT>(pr[i], j, s, m);
                const u32x4 bw = unpack_biased(wr[i][j], mag);
#pragma unroll
                for (int mb = 0; mb < MBG; mb++) {
                    if (FMT == ONPU_Q4NX) acc4(acc[mb][i], s, m, -128.0f * s, mfma(xa[mb][j], bw, z), cs[mb][j], 4);
                    else acc1(acc[mb][i], s, mfma(xa[mb][j], bw, cs[mb][j]), 4);
                }
            }
        }
    }
}

// The X tile of block b (MB A blocks of 16 rows) into LDS buffer buf: wave w of 4 fills fragments
// f = MB w + i, (mb, j) = (f / 4, f % 4); lane (q, r) brings row m0 + 16 mb + r, k = 128 b + 32 j +
// 8 q. xo[i] is the lane's byte offset of its element at b = 0 (0x80000000, past the buffer, for
// rows >= M: those land as zeros); block b adds 256 b in the scalar offset. kfix: the last block
// when K % 128 != 0 (its k >= K lanes read past the buffer too).
template <int MB>
DEV void gemm_load_x(const __amdgpu_buffer_rsrc_t & xr, const uint32_t (&xo)[MB], int64_t b, bool kfix, int64_t K,
                     int wave, int q, u32x4 * buf) {
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const int f = MB * wave + i, j = f & 3;
        uint32_t off = xo[i];
        if (kfix && 128 * b + 32 * j + 8 * q >= K) off = 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void *) (buf + f * 64), 16, off, (uint32_t) (256 * b), 0, 0);
    }
}

// weight block b of the wave's NTW tiles (buffer loads: one lane offset, the block in the scalar offset)
// weight tile block b (16 B of codes per lane) and its group parameters for lane row r
template <int FMT>
DEV void gemm_load_w1(const __amdgpu_buffer_rsrc_t & wrs, int64_t b, int lane, int r, u32x4 & w, GPar<FMT> & p) {
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const uint32_t sb = (uint32_t) (b * BLK);
    w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, 16 * lane, sb, 0));
    if (FMT == ONPU_G128S) {
        p.v[0] = __builtin_amdgcn_raw_buffer_load_b16(wrs, 1024 + 2 * r, sb, 0);
    } else if (FMT == ONPU_Q4NX) {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, 1024 + 16 * r, sb, 0));
        for (int jj = 0; jj < 4; jj++) p.v[jj % (sizeof(p.v) / 4)] = v[jj];
    } else {
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrs, 1024 + 8 * r, sb, 0));
        p.v[0] = v.x;
        p.v[1 % (sizeof(p.v) / 4)] = v.y;
    }
}

template <int FMT, int NTW>
DEV void gemm_load_w(const __amdgpu_buffer_rsrc_t (&wrs)[NTW], int64_t b, int lane, int r, u32x4 (&w)[NTW],
                     GPar<FMT> (&p)[NTW]) {
#pragma unroll
    for (int i = 0; i < NTW; i++) gemm_load_w1<FMT>(wrs[i], b, lane, r, w[i], p[i]);
}

// AK: one row tile (M <= 16 MB), no split: the epilogue also leaves the workgroup's argmax key of
// each row over its columns in a.akeys[m][N block] (argmax_key: larger value, then lower column)
// DEEP (16- and 32-row tiles): weights two blocks ahead (three register sets), for grids of at
// most two workgroups per CU, where one block in flight per workgroup leaves the memory idle
template <int FMT, int NTW, int MB, bool AK = false, bool DEEP = false>
__global__ __launch_bounds__(256, MB == 8 ? 2 : 4) void k_qgemm(GArgs a) {
    __shared__ u32x4 xs0[MB * 4 * 64], xs1[MB * 4 * 64];   // 2 x MB x 4 KiB
    constexpr int MT = 16 * MB;                           // rows of the workgroup tile
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), r = lane & 15;
    const int q = lane >> 4;
    const int64_t nwg = (int64_t) gridDim.x, wg = blockIdx.x;
    int64_t lid = wg;
    if (nwg % 8 == 0) lid = (wg % 8) * (nwg / 8) + wg / 8;
    // groups of GMS M tiles x all N columns, M fastest: the 64 workgroups an XCD runs at once cover
    // GMS M tiles x 64 / GMS N columns, so each X tile and each weight tile is read by many of them
    constexpr int64_t GMS = 4;
    const int64_t gm = (a.M + MT - 1) / MT, gn = (a.NT + 4 * NTW - 1) / (4 * NTW);
    // split-K: logical workgroups split-major (an XCD's contiguous range holds whole splits, whose
    // tiles share X columns), K blocks [kb0, kb1), fp32 partials in the split's plane
    int64_t kb0 = 0, kb1 = a.KB;
    void * yo = a.y;
    int64_t ldy = a.ldy;
    int yf32 = a.yf32;
    if (a.splits > 1) {
        const int64_t sp = lid / (gm * gn);
        lid -= sp * (gm * gn);
        kb0 = sp * a.kbs;
        kb1 = kb0 + a.kbs < a.KB ? kb0 + a.kbs : a.KB;
        yo = a.ws + sp * a.M * a.N;
        ldy = a.N;
        yf32 = 1;
    }
    const int64_t grp = lid / (GMS * gn), in = lid % (GMS * gn);
    const int64_t gms = gm - grp * GMS < GMS ? gm - grp * GMS : GMS;       // M tiles in this group
    const int64_t mblk = grp * GMS + in % gms, nblk = in / gms;
    const int64_t m0 = mblk * MT;
    const int64_t t0 = nblk * (4 * NTW) + wave * NTW;     // first weight tile of this wave
    // tiles past NT (the last column of workgroups) recompute tile t0 (or 0) and are not stored
    int nt_ok = (int) (a.NT - t0 < NTW ? a.NT - t0 : NTW);
    if (nt_ok < 0) nt_ok = 0;
    __amdgpu_buffer_rsrc_t wrs[NTW];
#pragma unroll
    for (int i = 0; i < NTW; i++) {
        const int64_t t = i < nt_ok ? t0 + i : (nt_ok > 0 ? t0 : 0);
        wrs[i] = __builtin_amdgcn_make_buffer_rsrc((void *) (a.W + t * a.KB * BLK), (short) 0,
                                                   (int) (uint32_t) (a.KB * BLK), 0x00020000);
    }
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) (uint32_t) (a.M * a.ldx * 2), 0x00020000);
    uint32_t xo[MB];
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const int f = MB * wave + i, mb = f >> 2, j = f & 3;
        const int64_t m = m0 + 16 * mb + r;
        xo[i] = m < a.M ? (uint32_t) ((m * a.ldx + 32 * j + 8 * q) * 2) : 0x80000000u;
    }
    const bool ktail = a.K % 128 != 0;

    f32x4 acc[MB][NTW];
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int i = 0; i < NTW; i++) acc[mb][i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // 16-row tiles, and g128s 32-row tiles, compute as the decode GEMV does (biased codes, scales
    // after the MFMA: exact dequant); the others feed the MFMA the bf16 RNE dequantized weights,
    // whose dequant a fragment's 2-8 MFMAs share (there the biased block needs more than the 128
    // registers of four workgroups per CU; with two it measured 0-25 % slower at 17-64 rows; g128s
    // 32-row tiles fit, 151936 x 4096 at 17 / 24 rows 101.4 / 109.6 -> 91.3 / 102.7 us)
    auto blk = [&](const u32x4 * xsb, const u32x4 (&wr)[NTW], const GPar<FMT> (&pr)[NTW]) {
        if constexpr (MB == 1 || (MB == 2 && FMT == ONPU_G128S)) gemm_block_biased<FMT, NTW, MB>(xsb, wr, pr, lane, acc);
        else gemm_block<FMT, NTW, MB>(xsb, wr, pr, lane, acc);
    };
    // two register sets for the weights, alternating with the two LDS buffers (no copies)
    u32x4 wa[NTW], wb[NTW];
    GPar<FMT> pa[NTW], pb[NTW];
    if constexpr (MB <= 2 && DEEP) {
        // 16- and 32-row tiles on small grids: a block's loads are small (4 KiB of X, NTW weight blocks per
        // wave) and its compute short, so the weights stay two blocks ahead (57344 x 8192 at 4-16
        // rows 65 -> 54 us, 8192 x 28672 38 -> 33 us; the 151936 x 4096 heads, ~4.6 workgroups per
        // CU, measured 2-6 % slower and keep one block): three register sets in rotation,
        // block b + 2's weights issued before block b's compute. X (from L2) stays one block ahead
        // and is issued after each barrier: the barrier's fence waits for every LDS-DMA load issued
        // before it, so an X load issued earlier would hold it. Each stage issues its X load, then
        // (after a scheduling fence, so the order holds) its weight loads, and waits for all but
        // those before the barrier. Loads past the range re-read block kb1 - 1 (in range) into a
        // set that is not read again; the last wait drains them.
        __shared__ u32x4 xs2[MB * 4 * 64];
        u32x4 wc[NTW];
        GPar<FMT> pc[NTW];
        const int64_t bl = kb1 - 1;
        auto issue = [&](int64_t bx, u32x4 * xsb, int64_t bw, u32x4 (&w)[NTW], GPar<FMT> (&p)[NTW]) {
            const int64_t cx = bx < kb1 ? bx : bl, cw = bw < kb1 ? bw : bl;
            gemm_load_x(xr, xo, cx, ktail && cx + 1 == a.KB, a.K, wave, q, xsb);
            __builtin_amdgcn_sched_barrier(0);
            gemm_load_w<FMT, NTW>(wrs, cw, lane, r, w, p);
            __builtin_amdgcn_sched_barrier(0);
        };
        constexpr int WL = 2 * NTW;                       // weight loads of one block per wave
        gemm_load_w<FMT, NTW>(wrs, kb0, lane, r, wa, pa);
        __builtin_amdgcn_sched_barrier(0);
        issue(kb0, xs0, kb0 + 1, wb, pb);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(WL));       // X of block kb0 (and its weights) landed
        __syncthreads();
        // one exit and the same loads outstanding on every path into the loop head (the blocks
        // past the range are skipped around their compute, not by leaving the loop, so the
        // compiler's own waits stay exact)
        for (int64_t b = kb0; b < kb1; b += 3) {
            issue(b + 1, xs1, b + 2, wc, pc);
            blk(xs0, wa, pa);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(WL));   // X of block b + 1 landed
            __syncthreads();
            issue(b + 2, xs2, b + 3, wa, pa);
            if (b + 1 < kb1) blk(xs1, wb, pb);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(WL));
            __syncthreads();
            issue(b + 3, xs0, b + 4, wb, pb);
            if (b + 2 < kb1) blk(xs2, wc, pc);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(WL));
            __syncthreads();
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);               // vmcnt(0): no load still writes LDS
    } else {
    gemm_load_x(xr, xo, kb0, ktail && kb0 + 1 == a.KB, a.K, wave, q, xs0);
    gemm_load_w<FMT, NTW>(wrs, kb0, lane, r, wa, pa);
    __builtin_amdgcn_s_waitcnt(0x0f70);                  // vmcnt(0): the DMA into xs0 is done
    __syncthreads();
    // pairs of blocks, one loop exit (acc merges once); an odd last block after the loop
    int64_t b = kb0;
    for (; b + 2 <= kb1; b += 2) {
        // even block from (xs0, wa) while block b + 1 streams into (xs1, wb)
        gemm_load_x(xr, xo, b + 1, ktail && b + 2 == a.KB, a.K, wave, q, xs1);
        gemm_load_w<FMT, NTW>(wrs, b + 1, lane, r, wb, pb);
        blk(xs0, wa, pa);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
        // odd block from (xs1, wb) while block b + 2 streams into (xs0, wa)
        if (b + 2 < kb1) {
            gemm_load_x(xr, xo, b + 2, ktail && b + 3 == a.KB, a.K, wave, q, xs0);
            gemm_load_w<FMT, NTW>(wrs, b + 2, lane, r, wa, pa);
        }
        blk(xs1, wb, pb);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
    }
    if (b < kb1) blk(xs0, wa, pa);
    }
    // store: lane (q, r) holds rows 4 q + v of A-block mb, column r of weight tile t0 + i
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int i = 0; i < NTW; i++) {
            if (i >= nt_ok) continue;
            const int64_t n = 16 * (t0 + i) + r;
            if (n >= a.N) continue;
            for (int v = 0; v < 4; v++) {
                const int64_t m = m0 + 16 * mb + 4 * q + v;
                if (m < a.M) store_out(yo, yf32, m * ldy + n, acc[mb][i][v]);
            }
        }
    if constexpr (AK) {
        // per row: the maximum key over the lane's columns, then over the 16 lanes of its row group
        // (lanes 16 q .. 16 q + 15), then over the 4 waves in LDS
        __shared__ uint64_t kw[4][16 * MB];
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                uint64_t k = 0;
#pragma unroll
                for (int i = 0; i < NTW; i++) {
                    const int64_t n = 16 * (t0 + i) + r;
                    const uint64_t c = argmax_key(acc[mb][i][v], n);
                    if (i < nt_ok && n < a.N && c > k) k = c;
                }
                for (int o = 1; o < 16; o <<= 1) {
                    const uint64_t u = __shfl_xor(k, o);
                    k = u > k ? u : k;
                }
                if (r == 0) kw[wave][16 * mb + 4 * q + v] = k;
            }
        __syncthreads();
        if (threadIdx.x < 16 * MB && threadIdx.x < a.M) {
            uint64_t k = kw[0][threadIdx.x];
            for (int w = 1; w < 4; w++) k = kw[w][threadIdx.x] > k ? kw[w][threadIdx.x] : k;
            a.akeys[(int64_t) threadIdx.x * gn + nblk] = k;
        }
    }
}

// ------------------------------------------------------------------ prefill GEMM, 256-row tiles
// Y = X . deq(W)^T with a workgroup tile of MT = 16 MBG rows of X by 16 NTW WV rows of W. Wave w
// owns NTW weight tiles and all MT rows (MBG x NTW accumulators of 16 x 16), so one dequantized
// weight fragment (23 VALU ops) feeds MBG MFMAs: at MBG = 16 that is 1.4 VALU ops per
// v_mfma_f32_16x16x32_bf16, which the matrix pipe hides when two waves share a SIMD (the 128-row
// k_qgemm leaves 2.9 per MFMA, which it does not). X blocks move HBM -> LDS by buffer-to-LDS loads
// into two MBG * 4 KiB buffers, weights stream into two register sets, as in k_qgemm.
// Work split, one workgroup per CU, every CU the same number of MFMAs whatever the tile count:
//   two-phase (sched 1): F rounds in which workgroup g takes all of tile r G + g (the 32
//     workgroups of an XCD hold a block of 4 M tiles x 8 N tiles and step through K together, so
//     each X block and weight block they share is fetched into that XCD's L2 once), then the R
//     remaining tiles cut at K block s: g < R takes [0, s) of tile F G + g (again in step), the
//     other workgroups take [s, KB) of c tiles each;
//   stream-K (sched 0): the tiles' K blocks as one tile-major sequence, workgroup g takes
//     iterations [g ipw, (g + 1) ipw).
// A cut tile has two segments (the host keeps it to two): the first to finish stores its fp32
// accumulators to the tile's slot with
// agent-scope stores (coherent across the XCDs' L2 caches once complete, no cache write-back) and
// raises the slot's flag; the second waits for the flag (raised by a workgroup already in its
// epilogue, so the wait is short and bounded), adds the partial and stores Y. Two addends give
// the same fp32 sum in either order, so Y does not depend on which segment finishes first. The
// second also clears the slot's counter and flag, which are therefore zero between launches.

// X fragments of block b for a workgroup of WV waves: wave w fills FPW = 4 MBG / WV fragments
// f = FPW w + i, (mb, j) = (f / 4, f % 4). xrow[i / 4]: the lane's byte offset of row m0 + 16 mb + r
// at k = 8 q (0x80000000, past the buffer, for rows >= M); kfix as in gemm_load_x.
template <int FPW>
DEV void gemm_load_x_frag(const __amdgpu_buffer_rsrc_t & xr, const uint32_t (&xrow)[FPW / 4], int64_t b, bool kfix,
                          int64_t K, int wave, int q, u32x4 * buf, int i) {
    // step j's 64 bytes in the scalar offset (a row past M, at 0x80000000, stays past the range);
    // the K tail is checked only in the block that holds it (kfix is uniform)
    const int f = FPW * wave + i, j = i & 3;
    uint32_t off = xrow[i >> 2];
    if (kfix && 128 * b + 32 * j + 8 * q >= K) off = 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void *) (buf + f * 64), 16, off, (uint32_t) (256 * b + 64 * j), 0,
                                             0);
}
template <int FPW>
DEV void gemm_load_x_sk(const __amdgpu_buffer_rsrc_t & xr, const uint32_t (&xrow)[FPW / 4], int64_t b, bool kfix,
                        int64_t K, int wave, int q, u32x4 * buf) {
#pragma unroll
    for (int i = 0; i < FPW; i++) gemm_load_x_frag<FPW>(xr, xrow, b, kfix, K, wave, q, buf, i);
}

// one 128-wide K block, 4 steps j x MBG row blocks, with a rolling A pipeline: fragment p = (j, mb),
// in j-major order, is read PD fragments ahead of its MFMAs, so LDS latency hides behind the MFMAs
// of the PD fragments in between (20 registers of read-ahead; a double buffer of a half-step's 8
// fragments took 64, which left the compiler no room to keep the reads ahead: it issued each read
// just before its use, 4-5 % slower). A scheduling fence closes every row block, so no read can
// sink toward its use. The next step's weight fragments are dequantized one output dword per row
// block (dequant8 in four parts), spread over the current step, and the loads of the next K block
// are issued by `issue(k)`, k < NI, one per row block of step 0 (all at the block's start, 8 waves
// x 10 loads queued at once, measured 1-4 % slower).
template <int FMT, int NTW, int MBG, int NI, class Issue>
DEV void gemm_block_rp(const u32x4 * xsb, const u32x4 (&wr)[NTW], const GPar<FMT> (&pr)[NTW], int lane,
                       f32x4 (&acc)[MBG][NTW], Issue issue) {
    constexpr int PD = 4, NP = 4 * MBG, DQ = MBG / (4 * NTW);
    static_assert(MBG % (4 * NTW) == 0, "dequant spread: four parts per tile and step");
    static_assert(NI <= MBG, "one load per row block of step 0");
    u32x4 xa[PD + 1], bw[2][NTW];
    uint32_t lo[NTW], hi[NTW];
    float sc[NTW], cc[NTW];
#pragma unroll
    for (int p = 0; p < PD; p++) xa[p] = *LDS_U32X4(&xsb[((p % MBG) * 4 + p / MBG) * 64 + lane]);
#pragma unroll
    for (int i = 0; i < NTW; i++) {
        par_sc<FMT>(pr[i], 0, sc[i], cc[i]);
        bw[0][i] = dequant8<FMT>(wr[i][0], sc[i], cc[i]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int mb = 0; mb < MBG; mb++) {
            const int p = j * MBG + mb;
            if (p + PD < NP) {
                const int f = p + PD;
                xa[f % (PD + 1)] = *LDS_U32X4(&xsb[((f % MBG) * 4 + f / MBG) * 64 + lane]);
            }
            if (j + 1 < 4 && mb % DQ == 0) {                // part k of tile i for step j + 1
                const int i = (mb / DQ) / 4, k = (mb / DQ) % 4;
                if (k == 0) {
                    par_sc<FMT>(pr[i], j + 1, sc[i], cc[i]);
                    dequant_split<FMT>(wr[i][j + 1], lo[i], hi[i]);
                }
                bw[(j + 1) & 1][i][k] = dequant_part<FMT>(lo[i], hi[i], k, sc[i], cc[i]);
            }
#pragma unroll
            for (int i = 0; i < NTW; i++) acc[mb][i] = mfma(xa[p % (PD + 1)], bw[j & 1][i], acc[mb][i]);
            if (j == 0 && mb < NI) issue(mb);             // the next block's loads, one per row block
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int V> struct IC { static constexpr int value = V; };     // a compile-time int as a value

// KT: K % 128 != 0 (the last K block reads zeros past K); launched with KT = false otherwise, so
// that no block pays for the check
template <int FMT, int NTW, int MBG, int WV, bool KT>
__global__ __launch_bounds__(64 * WV, 1) void k_qgemm_sk(GArgs a) {
    extern __shared__ u32x4 gsk_lds[];                   // two X buffers of 4 MBG fragments
    __shared__ int s_old, s_tag;
    constexpr int MT = 16 * MBG, NF = 4 * MBG, FPW = NF / WV, TPW = NTW * WV;
    static_assert(FPW % 4 == 0 && MBG % 8 == 0, "fragment split");
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    constexpr uint32_t SLOT = (uint32_t) WV * MBG * NTW * 1024;       // bytes of one partial tile
    u32x4 * xs0 = gsk_lds, * xs1 = gsk_lds + NF * 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), r = lane & 15;
    const int q = lane >> 4;
    // workgroup i runs on XCD i % 8: consecutive logical indices (adjacent iteration ranges, hence
    // adjacent tiles) go to one XCD so that its L2 holds their shared X rows and weight columns
    const int64_t G = gridDim.x, wg = blockIdx.x;
    const int64_t lid = G % 8 == 0 ? (wg % 8) * (G / 8) + wg / 8 : wg;
    constexpr int64_t GMS = 4;
    const int64_t gm = (a.M + MT - 1) / MT, gn = (a.NT + TPW - 1) / TPW, total = gm * gn * a.KB;
    const int64_t itb = lid * a.ipw, ite = itb + a.ipw < total ? itb + a.ipw : total;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) (uint32_t) (a.M * a.ldx * 2), 0x00020000);
    const bool ktail = KT && a.K % 128 != 0;
    if (tid == 0) {                                       // this launch's tag: the last one's + 1, never 0
        const int32_t prev = __hip_atomic_load(a.ctl + GSK_CTL_TAG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_tag = prev == 0x7fffffff ? 1 : prev + 1;
    }                                                     // (visible after the first __syncthreads below)
    int64_t it = itb;                                     // stream-K cursor
    for (int64_t qs = 0;; qs++) {
        int64_t t, kb0, kb1, slot;                        // this segment: tile, K blocks, partial slot
        if (a.sched == 0) {
            if (it >= ite) break;
            t = it / a.KB;
            kb0 = it % a.KB;
            kb1 = a.KB - kb0 < ite - it ? a.KB : kb0 + (ite - it);
            it += kb1 - kb0;
            slot = kb0 > 0 ? lid - 1 : lid;               // the boundary that cuts the tile
        } else {
            if (qs < a.F) {
                t = qs * G + lid;
                kb0 = 0;
                kb1 = a.KB;
            } else if (lid < a.R) {
                if (qs > a.F) break;
                t = a.F * G + lid;
                kb0 = 0;
                kb1 = a.s;
            } else {
                const int64_t p = (lid - a.R) * a.c + (qs - a.F);
                if (qs - a.F >= a.c || p >= a.R) break;
                t = a.F * G + p;
                kb0 = a.s;
                kb1 = a.KB;
            }
            slot = t - a.F * G;
        }
        // tile -> (M block, N block): groups of GMS M blocks x all N blocks, M fastest
        const int64_t grp = t / (GMS * gn), in = t % (GMS * gn);
        const int64_t gms = gm - grp * GMS < GMS ? gm - grp * GMS : GMS;
        const int64_t m0 = (grp * GMS + in % gms) * MT, t0 = (in / gms) * TPW + wave * NTW;
        int nt_ok = (int) (a.NT - t0 < NTW ? a.NT - t0 : NTW);
        if (nt_ok < 0) nt_ok = 0;
        __amdgpu_buffer_rsrc_t wrs[NTW];
#pragma unroll
        for (int i = 0; i < NTW; i++) {
            const int64_t tt = i < nt_ok ? t0 + i : (nt_ok > 0 ? t0 : 0);
            wrs[i] = __builtin_amdgcn_make_buffer_rsrc((void *) (a.W + tt * a.KB * BLK), (short) 0,
                                                       (int) (uint32_t) (a.KB * BLK), 0x00020000);
        }
        uint32_t xrow[FPW / 4];
#pragma unroll
        for (int g = 0; g < FPW / 4; g++) {
            const int64_t m = m0 + 16 * ((FPW * wave) / 4 + g) + r;
            xrow[g] = m < a.M ? (uint32_t) ((m * a.ldx + 8 * q) * 2) : 0x80000000u;
        }
        f32x4 acc[MBG][NTW];
#pragma unroll
        for (int mb = 0; mb < MBG; mb++)
#pragma unroll
            for (int i = 0; i < NTW; i++) acc[mb][i] = (f32x4){0.f, 0.f, 0.f, 0.f};
        u32x4 wc[NTW], wn[NTW];
        GPar<FMT> pc[NTW], pn[NTW];
        __syncthreads();                                  // the previous segment is done with xs0 / xs1
        gemm_load_x_sk<FPW>(xr, xrow, kb0, ktail && kb0 + 1 == a.KB, a.K, wave, q, xs0);
        gemm_load_w<FMT, NTW>(wrs, kb0, lane, r, wc, pc);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
        // one block per iteration (a single MFMA code path keeps the accumulators in place): block
        // b + 1 streams into the other LDS buffer and the other register set while b computes
        u32x4 * cur = xs0, * nxt = xs1;
        for (int64_t b = kb0; b < kb1; b++) {
            // block b + 1's X fragments and weights; at the segment's last block they reload block b
            // (in range, no branch around the loads), ended by the wait below before any reuse
            const int64_t bn = b + 1 < kb1 ? b + 1 : b;
            const bool kfn = ktail && bn + 1 == a.KB;
            auto issue = [&](int k) {
                if (k < FPW) gemm_load_x_frag<FPW>(xr, xrow, bn, kfn, a.K, wave, q, nxt, k);
                else gemm_load_w1<FMT>(wrs[k - FPW], bn, lane, r, wn[k - FPW], pn[k - FPW]);
            };
            gemm_block_rp<FMT, NTW, MBG, FPW + NTW>(cur, wc, pc, lane, acc, issue);
            __builtin_amdgcn_s_waitcnt(0x0f70);
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NTW; i++) { wc[i] = wn[i]; pc[i] = pn[i]; }
            u32x4 * t_ = cur; cur = nxt; nxt = t_;
        }

        // Y from the accumulators, plus (second segment) the other segment's partial tile, added
        // at the store so that no updated copy of the accumulators has to be merged with them.
        // Stores go through a buffer resource over this tile's rows (offsets fit 32 bits: MT rows):
        // the lane's part of the offset (row 4 q, column n) once per weight tile, the row step
        // 16 mb + v in the scalar offset. A column past N, and in a tile that runs past M a row past
        // it, gets an offset past the range, so the store is dropped.
        // A blocks [MB0, MB0 + NMB); with addp the other segment's partial of exactly those blocks,
        // laid out [wave][mb - MB0][i][lane] from byte pbase of the slot
        auto store_tile = [&](auto mb0c, auto nmbc, bool addp, const __amdgpu_buffer_rsrc_t & wsr, uint32_t pbase) {
            constexpr int MB0 = decltype(mb0c)::value, NMB = decltype(nmbc)::value;
            const uint32_t es = a.yf32 ? 4u : 2u, rowb = (uint32_t) a.ldy * es;
            const int64_t rows = a.M - m0 < MT ? a.M - m0 : MT;
            const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
                (void *) ((char *) a.y + m0 * a.ldy * es), (short) 0, (int) (uint32_t) (rows * rowb), 0x00020000);
            const bool full = rows == MT;                     // no row past M in this tile
            const int rows_l = (int) rows - 4 * q;            // rows left from the lane's first
            // the other segment's partial, PF A blocks in flight ahead of the one being added (each
            // load otherwise waits a full memory latency)
            constexpr int PF = 4;
            f32x4 pl[PF][NTW];
            auto load_part = [&](int mb, f32x4 (&d)[NTW]) {
#pragma unroll
                for (int i = 0; i < NTW; i++)
                    d[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         wsr, (uint32_t) lane * 16,
                                                         pbase + (uint32_t) (((wave * NMB + mb - MB0) * NTW + i) * 1024), 16));
            };
            if (addp) {
#pragma unroll
                for (int k = 0; k < PF && k < NMB; k++) load_part(MB0 + k, pl[k]);
            }
            // lane (q, r) holds rows 4 q + v of A block mb, column r of weight tile t0 + i
#pragma unroll
            for (int mb = MB0; mb < MB0 + NMB; mb++) {
                f32x4 pc[NTW];
                if (addp) {
#pragma unroll
                    for (int i = 0; i < NTW; i++) pc[i] = pl[(mb - MB0) % PF][i];
                    if (mb + PF < MB0 + NMB) load_part(mb + PF, pl[(mb - MB0) % PF]);
                }
#pragma unroll
                for (int i = 0; i < NTW; i++) {
                    f32x4 v4 = acc[mb][i];
                    if (addp) v4 += pc[i];
                    if (i >= nt_ok) continue;
                    const int64_t n = 16 * (t0 + i) + r;
                    const uint32_t vo = n < a.N ? (uint32_t) (4 * q) * rowb + (uint32_t) n * es : 0x80000000u;
                    uint32_t vov[4];
#pragma unroll
                    for (int v = 0; v < 4; v++) vov[v] = full || 16 * mb + v < rows_l ? vo : 0x80000000u;
                    if (a.yf32) {
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v4[v]), yr, vov[v],
                                                                  (uint32_t) (16 * mb + v) * rowb, 0);
                    } else {
#pragma unroll
                        for (int v = 0; v < 4; v += 2) {
                            const uint32_t pk = pack_bf16x2(v4[v], v4[v + 1]);
                            __builtin_amdgcn_raw_buffer_store_b16((unsigned short) pk, yr, vov[v],
                                                                  (uint32_t) (16 * mb + v) * rowb, 0);
                            __builtin_amdgcn_raw_buffer_store_b16((unsigned short) (pk >> 16), yr, vov[v + 1],
                                                                  (uint32_t) (16 * mb + v + 1) * rowb, 0);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (kb0 == 0 && kb1 == a.KB) {
            store_tile(IC<0>(), IC<MBG>(), false, xr, 0);
            continue;
        }
        int32_t * sc = a.sync + slot * GSK_SYNC_STRIDE;
        const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(
            (void *) ((char *) a.ws + (int64_t) slot * SLOT), (short) 0, (int) SLOT, 0x00020000);
        if (a.sym) {
            // a tile cut into two segments that end together (sched 1, one tail piece per workgroup):
            // each publishes the half of the rows that the other finishes (A blocks MBG/2.. for the
            // head, ..MBG/2 for the tail: half the partial tile each, both at once), sets its ready
            // word to the launch's tag, waits for the other's, adds the other's half to its own
            // rows and stores them. Both publish before waiting, and every workgroup of the launch
            // is resident (one per CU), so neither waits on a workgroup that has not run.
            constexpr int MBH = MBG / 2;
            const int h = kb0 == 0 ? 0 : 1;               // 0: head, keeps A blocks [0, MBH)
            const uint32_t pub = h ? SLOT / 2 : 0u;
#pragma unroll
            for (int mb = 0; mb < MBH; mb++)
#pragma unroll
                for (int i = 0; i < NTW; i++)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, h ? acc[mb][i] : acc[MBH + mb][i]), wsr, (uint32_t) lane * 16,
                        pub + (uint32_t) (((wave * MBH + mb) * NTW + i) * 1024), 16 /* sc1: agent scope */);
            __builtin_amdgcn_s_waitcnt(0x0f70);           // the stores have completed
            __syncthreads();
            if (tid == 0) {
                __hip_atomic_store(sc + 2 + h, s_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                uint32_t polls = 0;
                // a poll limit of 0 gives up without polling (the host forces a time-out with it)
                while (a.spin == 0 || __hip_atomic_load(sc + 3 - h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != s_tag) {
                    if (++polls > a.spin) {
                        __hip_atomic_store(a.ctl + GSK_CTL_ERR, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
            __syncthreads();
            if (h == 0) store_tile(IC<0>(), IC<MBH>(), true, wsr, SLOT / 2);
            else store_tile(IC<MBH>(), IC<MBH>(), true, wsr, 0);
            continue;
        }
        // a cut tile's two segments meet at its slot: every launch adds two arrivals to the slot's
        // counter, so an even count on arrival means first. The first publishes its partial and
        // sets the slot's ready word to this launch's tag; the second waits for that tag, so a
        // ready word left by any earlier launch (also by a publisher that came after a timed-out
        // wait) never matches, and nothing has to be cleared between launches.
        if (tid == 0) s_old = __hip_atomic_fetch_add(sc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int old = s_old;
        if ((old & 1) == 0) {                             // first segment: publish the partial
#pragma unroll
            for (int mb = 0; mb < MBG; mb++)
#pragma unroll
                for (int i = 0; i < NTW; i++)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mb][i]), wsr,
                                                           (uint32_t) lane * 16,
                                                           (uint32_t) (((wave * MBG + mb) * NTW + i) * 1024),
                                                           16 /* sc1: agent scope */);
            __builtin_amdgcn_s_waitcnt(0x0f70);           // the stores have completed
            __syncthreads();
            if (tid == 0) __hip_atomic_store(sc + 1, s_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {                                          // second: wait for the partial, add, store
            if (tid == 0) {
                uint32_t polls = 0;
                while (a.spin == 0 || __hip_atomic_load(sc + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != s_tag) {
                    if (++polls > a.spin) {
                        __hip_atomic_store(a.ctl + GSK_CTL_ERR, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
            __syncthreads();
            store_tile(IC<0>(), IC<MBG>(), true, wsr, 0);
        }
    }
    if (tid == 0) {
        // the last workgroup to finish advances the tag for the next launch (every workgroup read
        // it before it could finish; the next launch on this workspace starts after this one ends)
        if (__hip_atomic_fetch_add(a.ctl + GSK_CTL_DONE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int32_t) G - 1) {
            __hip_atomic_store(a.ctl + GSK_CTL_DONE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.ctl + GSK_CTL_TAG, s_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------ MoE prefill: grouped GEMM
// Work item = (expert e, first permuted position, rows <= 64) from k_moe_permute, taken with a group
// cg of output columns by each workgroup (k_moe_gemm below maps workgroups to (item, cg) so that an
// item's column groups share one XCD). Workgroup: WV waves x 2 weight tiles, the item's
// rows of X (gathered) as MBG = ceil(rows / 16) A blocks of 16 rows, MBG chosen per item (the
// matrix cores do not overlap the dequant's VALU work, so MFMAs on rows past the item cost their
// full time: with 4096 routed rows over 128 experts an item averages ~32 rows). Per 128-wide K block
// the X tile (MBG x 4 KiB of A fragments, spread over the waves) is filled by buffer loads straight
// to LDS, each lane from its own row (rows past the item land as zeros), and each wave dequantizes
// its two weight tiles in registers (the k_qgemm scheme over one expert's weights). Every column
// group re-reads the item's X, so wider groups (WV = 8) halve that traffic.
//   WHICH 0 (gate_up + SiLU * up): wave w holds gate tile g = WV cg + w and up tile
//           g + NT / 2; act[position][16 g + r] = bf16(silu(gate) * up)
//   WHICH 1 (down): wave w holds tiles 2 WV cg + 2 w + {0, 1}; o[position][n] = bf16 (the
//           reference device's output precision per expert: its GEMV flushes each row to bf16,
//           gemv_any.cc:120-130, and the host sums the weighted rows in fp32, onpu_cpu.cpp:259-274)
// X rows: WHICH 0 token perm[position] / k of x [T][K]; WHICH 1 position of act [T k][K].
template <int FMT, int WHICH, int WV, int MBG, bool KT>
DEV void moe_gemm_item(const MArgs & a, int64_t cg, int32_t e, int32_t first, int32_t rows, u32x4 * xs0, u32x4 * xs1) {
    // X fragments f = FPW wave + i (i < FPW, f < 4 MBG): (mb, j) = (f / 4, f % 4); FPW divides 4,
    // so that a wave's fragments share one A block and each lane one row
    constexpr int NF = 4 * MBG, FPW0 = (NF + WV - 1) / WV, FPW = FPW0 <= 1 ? 1 : FPW0 <= 2 ? 2 : 4;
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), r = lane & 15;
    const int q = lane >> 4;
    const uint8_t * W = a.W + (int64_t) e * a.estride;
    int64_t t[2];
    if (WHICH == 0) { t[0] = cg * WV + wave; t[1] = t[0] + a.NT / 2; }
    else { t[0] = cg * 2 * WV + 2 * wave; t[1] = t[0] + 1; }
    const bool ok0 = WHICH == 0 ? t[0] < a.NT / 2 : t[0] < a.NT;
    const bool ok1 = WHICH == 0 ? ok0 : t[1] < a.NT;
    __amdgpu_buffer_rsrc_t wrs[2];
    for (int i = 0; i < 2; i++) {
        const int64_t tt = (i == 0 ? ok0 : ok1) ? t[i] : 0;
        wrs[i] = __builtin_amdgcn_make_buffer_rsrc((void *) (W + tt * a.KB * BLK), (short) 0,
                                                   (int) (uint32_t) (a.KB * BLK), 0x00020000);
    }
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) (uint32_t) a.xbytes, 0x00020000);
    const bool xload = FPW * wave < NF;                          // wave-uniform
    const int xmb = FPW * wave / 4, xj0 = FPW * wave % 4;
    const int row = 16 * xmb + r;
    // the lane's byte offset of its row and k = 8 q (a row past the item, 0x80000000 + 16 q, stays
    // past the buffer's range); step j's 64 bytes and block b's 256 go in the scalar offset
    uint32_t xrow = 0x80000000u + 16u * q;
    if (xload && row < rows) {
        const int64_t src = WHICH == 0 ? (int64_t) (a.perm[first + row] / a.k) : (int64_t) (first + row);
        xrow = (uint32_t) (src * a.ldx * 2) + 16u * q;
    }
    auto load_xt = [&](int64_t b, u32x4 * buf) {
        if (!xload) return;
#pragma unroll
        for (int i = 0; i < FPW; i++) {
            const int j = xj0 + i;
            uint32_t off = xrow;
            if (KT && 128 * b + 32 * j + 8 * q >= a.K) off = 0x80000000u;      // the K tail reads zeros
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void *) (buf + (FPW * wave + i) * 64), 16, off,
                                                     (uint32_t) (256 * b + 64 * j), 0, 0);
        }
    };
    f32x4 acc[MBG][2];
#pragma unroll
    for (int mb = 0; mb < MBG; mb++) acc[mb][0] = acc[mb][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
    u32x4 wa[2], wb[2];
    GPar<FMT> pa[2], pb[2];
    load_xt(0, xs0);
    gemm_load_w<FMT, 2>(wrs, 0, lane, r, wa, pa);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    int64_t b = 0;
    for (; b + 2 <= a.KB; b += 2) {
        load_xt(b + 1, xs1);
        gemm_load_w<FMT, 2>(wrs, b + 1, lane, r, wb, pb);
        gemm_block<FMT, 2, MBG>(xs0, wa, pa, lane, acc);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
        if (b + 2 < a.KB) {
            load_xt(b + 2, xs0);
            gemm_load_w<FMT, 2>(wrs, b + 2, lane, r, wa, pa);
        }
        gemm_block<FMT, 2, MBG>(xs1, wb, pb, lane, acc);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
    }
    if (b < a.KB) gemm_block<FMT, 2, MBG>(xs0, wa, pa, lane, acc);
    // bf16 stores through a buffer resource over the item's rows (rows <= 64: 32-bit offsets): the
    // lane's row 4 q and column in the vector offset, the row step 16 mb + v in the scalar offset;
    // a row past the item or a column past N gets an offset past the range, so the store is dropped
    const uint32_t rowb = (uint32_t) a.ldy * 2;
    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
        (void *) ((uint16_t *) a.y + (int64_t) first * a.ldy), (short) 0, (int) ((uint32_t) rows * rowb), 0x00020000);
    const int rows_l = rows - 4 * q;                               // rows left from the lane's first
    uint32_t vo[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const bool okc = (i == 0 ? ok0 : ok1) && 16 * t[i] + r < a.N;
        vo[i] = okc ? (uint32_t) (4 * q) * rowb + (uint32_t) (16 * t[i] + r) * 2 : 0x80000000u;
    }
    // lane (q, r) holds rows 4 q + v of A block mb, column r of its tiles
#pragma unroll
    for (int mb = 0; mb < MBG; mb++)
#pragma unroll
        for (int v = 0; v < 4; v += 2) {
            const uint32_t so0 = (uint32_t) (16 * mb + v) * rowb, so1 = so0 + rowb;
            const bool in0 = 16 * mb + v < rows_l, in1 = 16 * mb + v + 1 < rows_l;
            if (WHICH == 0) {
                const uint32_t pk = pack_bf16x2(silu_f(acc[mb][0][v]) * acc[mb][1][v],
                                                silu_f(acc[mb][0][v + 1]) * acc[mb][1][v + 1]);
                __builtin_amdgcn_raw_buffer_store_b16((unsigned short) pk, yr, in0 ? vo[0] : 0x80000000u, so0, 0);
                __builtin_amdgcn_raw_buffer_store_b16((unsigned short) (pk >> 16), yr, in1 ? vo[0] : 0x80000000u, so1, 0);
            } else {
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const uint32_t pk = pack_bf16x2(acc[mb][i][v], acc[mb][i][v + 1]);
                    __builtin_amdgcn_raw_buffer_store_b16((unsigned short) pk, yr, in0 ? vo[i] : 0x80000000u, so0, 0);
                    __builtin_amdgcn_raw_buffer_store_b16((unsigned short) (pk >> 16), yr, in1 ? vo[i] : 0x80000000u,
                                                          so1, 0);
                }
            }
        }
}

// KT: K % 128 != 0 (launched with KT = false otherwise, so that no block pays for the tail check)
template <int FMT, int WHICH, bool KT>
// grid: (column groups G, item slots, a multiple of 8). Workgroup L = x + G y runs on XCD L % 8; its
// position j = L / 8 there takes item 8 (j / G) + L % 8 and column group j % G, so the G column
// groups of an item run together on one XCD and fetch the item's X rows into that XCD's L2 once
// (items in the list's order, the longest first, one per XCD at a time)
__global__ __launch_bounds__(512, 1) void k_moe_gemm(MArgs a) {
    constexpr int WV = 8;
    __shared__ u32x4 xs0[4 * 4 * 64], xs1[4 * 4 * 64];         // 2 x 16 KiB: up to 4 A blocks
    const int64_t G = gridDim.x, L = blockIdx.x + G * blockIdx.y, j = L / 8;
    const int item = (int) (8 * (j / G) + L % 8);
    const int64_t cg = j % G;
    if (item >= *a.nitems) return;
    const int32_t e = a.items[3 * item], first = a.items[3 * item + 1], rows = a.items[3 * item + 2];
    if (rows <= 16) moe_gemm_item<FMT, WHICH, WV, 1, KT>(a, cg, e, first, rows, xs0, xs1);
    else if (rows <= 32) moe_gemm_item<FMT, WHICH, WV, 2, KT>(a, cg, e, first, rows, xs0, xs1);
    else if (rows <= 48) moe_gemm_item<FMT, WHICH, WV, 3, KT>(a, cg, e, first, rows, xs0, xs1);
    else moe_gemm_item<FMT, WHICH, WV, 4, KT>(a, cg, e, first, rows, xs0, xs1);
}


// ------------------------------------------------------------------ MoE decode in one launch
// Opt-in (ONPU_MOE_FUSED=1): measured on MI355X for Qwen3-30B-A3B at T = 1 it takes ~19 us against
// ~16 us for the router kernel plus the two GEMV launches. Routing and x staging finish at ~2.5 us,
// the expert weights are in by ~6 us, but the handoff of act between workgroups (store
// acknowledgement, arrival, poll, reload: four memory round trips) costs more than the two kernel
// boundaries it removes.
// T <= 4 tokens, k <= 8 routed experts each (the reference's fused expert FFN, onpu_api.cpp:292-496,
// gemv_any.cc:34-50, and onpu_moe_ffn's act 0 path, onpu_api.cpp:261-278 with onpu_cpu.cpp:233-274):
//   router (when logits are given): softmax -> top-k -> renorm, as k_route;
//   phase A: slot s = t k + j, expert e = ids[s]: act[s][i] = bf16(silu(g_i) * u_i) with g, u the
//            rows i and I + i of gate_up_e times x_t, for every 16-row tile pair (gate tile i / 16,
//            up tile I / 16 + i / 16) ("pairs");
//   phase B: y[t][n] = sum_j w[t][j] (down_e(j) . act[t k + j])[n] for every 16-row tile of down
//            ("units"), the k slots summed in slot order.
// One workgroup of 8 waves per CU. Workgroup g takes pairs g, g + G, ... (the 8 waves split each
// pair's K blocks and meet in LDS) and units G - 1 - g, 2 G - 1 - g, ... (wave j takes slot j), so
// with one token the workgroups with fewer pairs are the ones with a unit. All weight loads are
// issued as soon as the routing is known: the unit's down tiles first, then the pairs' tiles.
// A workgroup publishes each pair's 16 act values with two 16-byte agent-scope stores (coherent
// across the XCDs' L2 caches once complete), waits for its stores to complete and adds its pair
// count to sync[0]; a workgroup with units waits until sync[0] counts every pair (a wait on workgroups that never wait themselves,
// bounded by a.spin polls; a timeout raises sync[MD_SYNC_ERR]), reads the act rows with agent-scope
// loads and finishes its units. The last workgroup with units takes the launch's npairs off sync[0]
// and clears sync[MD_SYNC_DONE], so the counters are zero between launches (and a captured graph
// replays without resets).

// x rows [T][H] -> LDS xs[T][xl] (bf16, zero past H) and their group sums times xsum_mul,
// xg[T][KB * GPB], by the whole workgroup: thread u takes 8 elements, a group's threads are
// consecutive lanes of one wave
template <int FMT>
DEV void md_stage_x(const uint16_t * __restrict__ x, int T, int64_t H, int64_t KB, int64_t xl, uint16_t * xs,
                    float * xg) {
    constexpr int GS = FMT == ONPU_G128S ? 128 : 32, UPG = GS / 8, GPB = 128 / GS;
    const uint32_t kp8 = (uint32_t) KB * 16, nunits = (uint32_t) T * kp8;
    for (uint32_t u0 = 0; u0 < nunits; u0 += blockDim.x) {       // same trip count for the workgroup
        const uint32_t u = u0 + threadIdx.x, t = u / kp8, k = (u - t * kp8) * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (u < nunits && k < H) v = *(const u32x4 *) (x + (int64_t) t * H + k);
        if (u < nunits) *LDS_U32X4(xs + (int64_t) t * xl + k) = v;
        float sum = 0.f;
        for (int d = 0; d < 4; d++) sum += __uint_as_float(v[d] << 16) + __uint_as_float(v[d] & 0xffff0000u);
        for (int o = UPG / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (u < nunits && (k / 8) % UPG == 0) xg[(int64_t) t * KB * GPB + k / GS] = sum * xsum_mul<FMT>();
    }
}

// One wave's M = 1 products over NB blocks of RT row tiles (weights and parameters loaded earlier):
// the x row from LDS (xr, blocks b0 ..), its group sums xg; acc[rt][0] lanes 0..15 hold the partials
// of tile rows 0..15. Blocks i >= nb are skipped (their loads re-read a valid block).
template <int FMT, int RT, int NB>
DEV void md_accum(const u32x4 (&wv)[NB][RT], const Par<FMT> (&par)[NB][RT], int nb, const uint16_t * xr,
                  const float * xg, int64_t b0, f32x4 (&acc)[RT][1]) {
    const int q = (threadIdx.x & 63) >> 4;
    constexpr int GPB = FMT == ONPU_G128S ? 1 : 4;
    bool valid[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) valid[rt] = true;
#pragma unroll
    for (int i = 0; i < NB; i++) {
        if (i >= nb) break;
        const int64_t b = b0 + i;
        u32x4 xa[1][4];
#pragma unroll
        for (int j = 0; j < 4; j++) xa[0][j] = *LDS_U32X4(xr + b * 128 + 32 * j + 8 * q);
        f32x4 cs[1][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = *(const __attribute__((address_space(3))) float *) (xg + b * GPB + (j < GPB ? j : 0));
            cs[0][j] = (f32x4){v, v, v, v};
        }
        qacc_block<FMT, 1, RT, 1>(valid, wv[i], par[i], xa, cs, 0x43004300u, acc);
    }
}

// weights of NB blocks b0 .. of RT tiles (bases tb[rt]); blocks past nb re-read block b0
template <int FMT, int RT, int NB>
DEV void md_load(const uint8_t * const (&tb)[RT], int64_t b0, int nb, u32x4 (&wv)[NB][RT], Par<FMT> (&par)[NB][RT]) {
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    const int lane = threadIdx.x & 63, r = lane & 15;
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const uint8_t * p = tb[rt] + (b0 + (i < nb ? i : 0)) * BLK;
            wv[i][rt] = __builtin_nontemporal_load(GLB(const u32x4, p + 16 * lane));
            par[i][rt] = load_par<FMT>(p, r);
        }
}

// GB: gate_up K blocks per wave (the 8 waves split the H / 128 blocks); DB: down K blocks (I / 128
// rounded up), both at most as built
template <int FMT, int GB, int DB>
__global__ __launch_bounds__(512) void k_moe_decode(MDArgs a) {
    extern __shared__ __align__(16) float mds[];
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    constexpr int GS = FMT == ONPU_G128S ? 128 : 32, GPB = 128 / GS;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 15;
    const int64_t G = gridDim.x, g = blockIdx.x;
    const int k = a.k, T = a.T;
    const int64_t IT = a.I / 16;
    // LDS: ids / w, x rows and sums, the cross-wave buffer, then per wave one act row and its sums
    int32_t * sids = (int32_t *) mds;
    float * sw = mds + MD_MAX_T * MD_MAX_K;
    const int64_t xl = a.gKB * 128, al = (int64_t) DB * 128;
    uint16_t * xs = (uint16_t *) (mds + 2 * MD_MAX_T * MD_MAX_K);
    float * xg = (float *) (xs + T * xl);
    float * red = xg + (T * a.gKB * GPB + 3) / 4 * 4;          // [8][2][64], 16-byte aligned
    uint16_t * ab = (uint16_t *) (red + MD_WAVES * 2 * 64);      // [8][al]
    float * abg = (float *) (ab + MD_WAVES * al);                // [8][DB * GPB]

    // routing (wave 0) while the other waves stage x
    if (a.logits) {
        if (wave == 0)
            for (int t = 0; t < T; t++) {
                int id;
                float wt;
                route_token(a.logits + (int64_t) t * a.E, a.E, k, a.renorm, id, wt);
                if (lane < k) {
                    sids[t * k + lane] = id;
                    sw[t * k + lane] = wt;
                    if (g == 0) {
                        a.ids[t * k + lane] = id;
                        a.w[t * k + lane] = wt;
                    }
                }
            }
    } else if (threadIdx.x < T * k) {
        sids[threadIdx.x] = a.ids[threadIdx.x];
        sw[threadIdx.x] = a.w[threadIdx.x];
    }
    md_stage_x<FMT>(a.x, T, a.H, a.gKB, xl, xs, xg);
    __syncthreads();

    // the first unit's down tiles (wave j < k: slot j of the unit's token), then the first pair
    const int64_t u0 = G - 1 - g;
    u32x4 dw[DB][1];
    Par<FMT> dp[DB][1];
    auto load_unit = [&](int64_t u) {
        const int64_t t = u / a.dNT, h = u % a.dNT;
        const int j = wave < k ? wave : 0;
        const uint8_t * tb[1] = {a.Wd + (int64_t) sids[t * k + j] * a.dstride + h * a.dKB * BLK};
        md_load<FMT, 1, DB>(tb, 0, (int) a.dKB, dw, dp);
    };
    if (u0 < a.nunits) load_unit(u0);
    const int64_t gb0 = (int64_t) wave * GB, gnb = a.gKB - gb0 < GB ? (a.gKB - gb0 > 0 ? a.gKB - gb0 : 0) : GB;
    u32x4 gw[2][GB][2];
    Par<FMT> gp[2][GB][2];
    auto load_pair = [&](int64_t p, int buf) {
        const int64_t s = p / IT, gt = p % IT;
        const uint8_t * e = a.Wg + (int64_t) sids[s] * a.gstride;
        const uint8_t * tb[2] = {e + gt * a.gKB * BLK, e + (IT + gt) * a.gKB * BLK};
        md_load<FMT, 2, GB>(tb, gnb > 0 ? gb0 : 0, gnb > 0 ? (int) gnb : 1, gw[buf], gp[buf]);
    };
    auto do_pair = [&](int64_t p, const u32x4 (&wv)[GB][2], const Par<FMT> (&pv)[GB][2]) {
        f32x4 acc[2][1] = {{{0.f, 0.f, 0.f, 0.f}}, {{0.f, 0.f, 0.f, 0.f}}};
        const int64_t s = p / IT, gt = p % IT, t = s / k;
        if (gnb > 0) md_accum<FMT, 2, GB>(wv, pv, (int) gnb, xs + t * xl, xg + t * a.gKB * GPB, gb0, acc);
        red[(wave * 2 + 0) * 64 + lane] = acc[0][0][0];
        red[(wave * 2 + 1) * 64 + lane] = acc[1][0][0];
        __syncthreads();
        // wave 0: lane r < 16 forms act of tile row r; lane 0 gathers the 16 bf16 (32 bytes) and
        // publishes them with two 16-byte agent-scope stores, waits for them, and arrives
        if (wave == 0) {
            float gs = 0.f, us = 0.f;
            for (int w = 0; w < MD_WAVES; w++) { gs += red[(w * 2 + 0) * 64 + r]; us += red[(w * 2 + 1) * 64 + r]; }
            const uint32_t h = f32_to_bf16(silu_f(gs) * us);
            const uint32_t pr = h | (__shfl_down(h, 1) << 16);        // lanes 2i: rows 2i, 2i + 1
            u32x4 lo, hi;
#pragma unroll
            for (int d = 0; d < 4; d++) {
                lo[d] = __shfl(pr, 2 * d);
                hi[d] = __shfl(pr, 8 + 2 * d);
            }
            if (lane == 0) {
                const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
                    (void *) (a.act + s * a.I + gt * 16), (short) 0, 32, 0x00020000);
                __builtin_amdgcn_raw_buffer_store_b128(lo, ar, 0, 0, 16 /* sc1: agent scope */);
                __builtin_amdgcn_raw_buffer_store_b128(hi, ar, 16, 0, 16);
            }
        }
        __syncthreads();                               // red is reused by the next pair
    };
    int64_t mine = 0;                                  // pairs done by this workgroup
    // phase A: pairs g, g + G, ... alternating between the two register sets, the next pair's loads
    // in flight while the current one computes
    if (g < a.npairs) load_pair(g, 0);
    for (int64_t p = g; p < a.npairs; p += 2 * G) {
        if (p + G < a.npairs) load_pair(p + G, 1);
        do_pair(p, gw[0], gp[0]);
        mine++;
        if (p + G >= a.npairs) break;
        if (p + 2 * G < a.npairs) load_pair(p + 2 * G, 0);
        do_pair(p + G, gw[1], gp[1]);
        mine++;
    }
    // publish: this workgroup's act stores have completed, then one arrival for all its pairs
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    if (threadIdx.x == 0 && mine > 0)
        __hip_atomic_fetch_add(a.sync, (int32_t) mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (u0 >= a.nunits) return;

    // phase B: wait until every pair is published
    if (threadIdx.x == 0) {
        uint32_t polls = 0;
        // a poll limit of 0 gives up without polling (the host forces a time-out with it)
        while (a.spin == 0 || __hip_atomic_load(a.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (int32_t) a.npairs) {
            if (++polls > a.spin) {
                __hip_atomic_store(a.sync + MD_SYNC_ERR, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
    uint16_t * abw = ab + wave * al;
    float * abgw = abg + wave * DB * GPB;
    for (int64_t u = u0; u < a.nunits; u += G) {
        if (u != u0) load_unit(u);
        const int64_t t = u / a.dNT, h = u % a.dNT;
        float part = 0.f;
        if (wave < k) {
            // act row of slot t k + wave (agent-scope loads: written by other workgroups in this launch)
            // into this wave's LDS row, 8 bytes per lane per step, zero past I; group sums (times
            // xsum_mul) by shuffles
            const int64_t s = t * k + wave;
            const uint64_t * src = (const uint64_t *) (a.act + s * a.I);
            for (int64_t e0 = 0; e0 < al; e0 += 256) {
                const int64_t e = e0 + 4 * lane;
                uint64_t v = 0;
                if (e < a.I) v = __hip_atomic_load(GLB(const uint64_t, src + e / 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *(__attribute__((address_space(3))) uint64_t *) (abw + e) = v;
                float sum = 0.f;
                for (int d = 0; d < 2; d++) {
                    const uint32_t wd = (uint32_t) (v >> (32 * d));
                    sum += __uint_as_float(wd << 16) + __uint_as_float(wd & 0xffff0000u);
                }
                for (int o = GS / 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
                if ((e % GS) == 0) abgw[e / GS] = sum * xsum_mul<FMT>();
            }
            f32x4 acc[1][1] = {{{0.f, 0.f, 0.f, 0.f}}};
            md_accum<FMT, 1, DB>(dw, dp, (int) a.dKB, abw, abgw, 0, acc);
            part = sw[s] * acc[0][0][0];
        }
        red[wave * 64 + lane] = part;
        __syncthreads();
        if (threadIdx.x < 16) {
            float ys = 0.f;
            for (int j = 0; j < k; j++) ys += red[j * 64 + r];
            const int64_t n = 16 * h + r;
            if (n < a.Nd) store_out(a.y, a.yf32, t * a.Nd + n, ys);
        }
        __syncthreads();
    }
    // the last workgroup with units returns the counters to zero for the next launch: it takes this
    // launch's npairs arrivals off sync[0] instead of storing zero, so that an arrival still to come
    // (after a wait that gave up) cannot leave a count behind: every launch adds npairs in all
    if (threadIdx.x == 0) {
        const int32_t consumers = (int32_t) (a.nunits < G ? a.nunits : G);
        if (__hip_atomic_fetch_add(a.sync + MD_SYNC_DONE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == consumers - 1) {
            __hip_atomic_fetch_add(a.sync, -(int32_t) a.npairs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.sync + MD_SYNC_DONE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------ MoE decode split along I
// The step-major copy (onpu_launch.h dec_sblk): one wave per superblock (s, tq) and expert. Lane l
// gathers dword j = s % 4 of its 16 bytes in block (4 tq + d, s / 4) for the four tiles d; lanes
// 0..15 gather row r's parameters of that step for the four tiles.
template <int FMT>
__global__ __launch_bounds__(64) void k_relayout_dec(const uint8_t * __restrict__ src, int64_t sstride, int64_t NT,
                                                     int64_t KB, uint8_t * __restrict__ dst, int64_t dstride) {
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    constexpr int SB = 1024 + (FMT == ONPU_Q4NX ? 256 : 128);
    const int64_t NTq = (NT + 3) / 4, sb = blockIdx.x, st = sb / NTq, tq = sb - st * NTq, b = st / 4;
    const int j = (int) (st % 4), l = threadIdx.x, r = l & 15;
    const uint8_t * e = src + (int64_t) blockIdx.y * sstride;
    uint8_t * o = dst + (int64_t) blockIdx.y * dstride + sb * SB;
    u32x4 v;
    for (int d = 0; d < 4; d++) {
        const int64_t t = 4 * tq + d;
        v[d] = t < NT ? *(const uint32_t *) (e + (t * KB + b) * BLK + 16 * l + 4 * j) : 0u;
    }
    *(u32x4 *) (o + 16 * l) = v;
    if (l < 16) {
        if (FMT == ONPU_Q4NX) {
            u32x4 p;
            for (int d = 0; d < 4; d++) {
                const int64_t t = 4 * tq + d;
                p[d] = t < NT ? *(const uint32_t *) (e + (t * KB + b) * BLK + 1024 + 16 * r + 4 * j) : 0u;
            }
            *(u32x4 *) (o + 1024 + 16 * r) = p;
        } else {
            uint16_t p[4];
            for (int d = 0; d < 4; d++) {
                const int64_t t = 4 * tq + d;
                const int64_t off = FMT == ONPU_G128S ? 1024 + 2 * r : 1024 + 8 * r + 2 * j;
                p[d] = t < NT ? *(const uint16_t *) (e + (t * KB + b) * BLK + off) : (uint16_t) 0;
            }
            *(u32x2 *) (o + 1024 + 8 * r) = (u32x2){p[0] | ((uint32_t) p[1] << 16), p[2] | ((uint32_t) p[3] << 16)};
        }
    }
}

// x row [H] -> LDS xs (zero past H up to KB * 128) and its group sums times xsum_mul -> xg, by the
// threads from `first` on (wave 0 may be routing meanwhile). Units of 8 values; a group's units sit
// on consecutive lanes of one wave (blockDim - first is a multiple of 64).
template <int FMT>
DEV void ds_stage_x(const uint16_t * __restrict__ x, int64_t H, int64_t KB, uint16_t * xs, float * xg, int first) {
    constexpr int GS = FMT == ONPU_G128S ? 128 : 32, UPG = GS / 8;
    if ((int) threadIdx.x < first) return;
    const uint32_t nunits = (uint32_t) KB * 16, nt = blockDim.x - (uint32_t) first, tid = threadIdx.x - first;
    for (uint32_t u0 = 0; u0 < nunits; u0 += nt) {
        const uint32_t u = u0 + tid;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (u < nunits && (int64_t) u * 8 < H) v = *(const u32x4 *) (x + (int64_t) u * 8);
        if (u < nunits) *LDS_U32X4(xs + (int64_t) u * 8) = v;
        float sum = 0.f;
        for (int d = 0; d < 4; d++) sum += __uint_as_float(v[d] << 16) + __uint_as_float(v[d] & 0xffff0000u);
        for (int o = UPG / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (u < nunits && u % UPG == 0) xg[u / UPG] = sum * xsum_mul<FMT>();
    }
}

// One wave's gate / up products over GB blocks from b0 (loaded by md_load), x from LDS. Every block
// is computed: blocks past nb (re-reads of block b0) get zero parameters, so they add exact zeros
// (x finite). No use of a loaded value sits behind a branch, so the compiler keeps the loads where
// md_load issues them, all before the first MFMA, instead of sinking each to its use (one memory
// round trip per block).
template <int FMT, int GB>
DEV void ds_accum(const u32x4 (&wv)[GB][1], const Par<FMT> (&par)[GB][1], int nb, const uint16_t * xr,
                  const float * xg, int64_t b0, f32x4 (&acc)[1][1]) {
    const int q = (threadIdx.x & 63) >> 4;
    constexpr int GPB = FMT == ONPU_G128S ? 1 : 4;
    const bool valid[1] = {true};
#pragma unroll
    for (int i = 0; i < GB; i++) {
        const bool on = i < nb;
        const int64_t b = b0 + (on ? i : 0);
        Par<FMT> p[1];
        p[0] = par[i][0];
        if (!on) p[0].v[0] = 0u;
        if (FMT != ONPU_G128S && !on)
#pragma unroll
            for (int d = 1; d < (int) (sizeof(p[0].v) / 4); d++) p[0].v[d] = 0u;
        u32x4 xa[1][4];
#pragma unroll
        for (int j = 0; j < 4; j++) xa[0][j] = *LDS_U32X4(xr + b * 128 + 32 * j + 8 * q);
        f32x4 cs[1][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = *(const __attribute__((address_space(3))) float *) (xg + b * GPB + (j < GPB ? j : 0));
            cs[0][j] = (f32x4){v, v, v, v};
        }
        u32x4 w1[1] = {wv[i][0]};
        qacc_block<FMT, 1, 1, 1>(valid, w1, p, xa, cs, 0x43004300u, acc);
    }
}

// grid (S slices, T k slots), NW waves (8 or 16); SV = 32 or 16 values of I per slice. Wave 0 routes
// the slot's token (from logits) while the others stage x; then wave w loads its gate/up tile
// (w / P, P = NW / (SV / 8) K parts per tile; SV 32: gate tiles 2 s, 2 s + 1, up tiles NT / 2 + 2 s,
// + 1; SV 16: gate tile s, up tile NT / 2 + s) over K part w % P (GB blocks at most) and its down
// superblocks (quads w, w + NW, ..., DQ at most) of the slice's 32-wide K step (s, or s / 2 for SV
// 16, whose slice is half of the step: the lanes of the other two K groups load nothing), all at
// once. The gate/up partials meet in LDS, act = bf16(silu(g) u) for the slice's values (zero in the
// rest of the step), and each wave multiplies act into its down superblocks: A = act on every MFMA
// row, C starts at the act sum times xsum_mul, so lanes 0..15 end with row r of each of the four
// tiles.
template <int FMT, int GB, int DQ, int NW, int SV>
__global__ __launch_bounds__(NW * 64) void k_moe_dsplit(MSArgs a) {
    extern __shared__ __align__(16) float dsl[];
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    constexpr int SB = 1024 + (FMT == ONPU_Q4NX ? 256 : 128);
    constexpr int GS = FMT == ONPU_G128S ? 128 : 32, GPB = 128 / GS;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 15,
              q = lane >> 4;
    const int64_t s = blockIdx.x, slot = blockIdx.y, t = slot / a.k;
    const int j = (int) (slot - t * a.k);
    static_assert(SV == 32 || SV == 16, "slices of 32 or 16 values of I");
    constexpr int NTL = SV / 8;                // gate / up tiles per workgroup
    constexpr int P = NW / NTL;                // K parts of each gate / up tile
    // LDS: x row and its group sums, the gate/up partials [NW][16], act [32] bf16 and its sum
    const int64_t xl = a.gKB * 128;
    uint16_t * xs = (uint16_t *) dsl;
    float * xg = (float *) (xs + xl);
    float * red = xg + (a.gKB * GPB + 3) / 4 * 4;
    uint16_t * act = (uint16_t *) (red + NW * 16);
    float * acs = (float *) (act + 32);
    __shared__ int s_e;
    if (a.logits) {
        if (wave == 0) {
            int my_id;
            float my_w;
            route_token(a.logits + t * a.E, a.E, a.k, a.renorm, my_id, my_w);
            if (lane == 0) s_e = __builtin_amdgcn_readlane(my_id, j);
            if (s == 0 && j == 0 && lane < a.k) {
                a.ids[t * a.k + lane] = my_id;
                a.w[t * a.k + lane] = my_w;
            }
        }
        ds_stage_x<FMT>(a.x + t * a.H, a.H, a.gKB, xs, xg, 64);
    } else {
        if (threadIdx.x == 0) s_e = a.ids[slot];
        ds_stage_x<FMT>(a.x + t * a.H, a.H, a.gKB, xs, xg, 0);
    }
    __syncthreads();
    const int64_t e = s_e;
    // gate / up tile of this wave and its K part
    const int ti = wave / P, h = wave % P;
    const int64_t tile = SV == 32 ? (ti < 2 ? 0 : a.gNT / 2) + 2 * s + (ti & 1) : (ti == 0 ? 0 : a.gNT / 2) + s;
    const uint8_t * tb[1] = {a.Wg + e * a.gstride + tile * a.gKB * BLK};
    const int64_t part = (a.gKB + P - 1) / P, b0 = h * part;
    const int nb = (int) (a.gKB - b0 < part ? (a.gKB - b0 > 0 ? a.gKB - b0 : 0) : part);
    u32x4 wv[GB][1];
    Par<FMT> par[GB][1];
    md_load<FMT, 1, GB>(tb, nb > 0 ? b0 : 0, nb, wv, par);
    // down superblocks of the slice's step: quads wave + NW i (a quad past the last re-reads quad 0).
    // SV 16: the lanes of the other half of the step (K groups q / 2 != s % 2) get an offset past the
    // range, so their loads return zeros without a memory access (and act is zero there)
    const int64_t step = SV == 32 ? s : s >> 1;
    const uint8_t * wd = a.Wd + e * a.dstride + step * a.dNTq * SB;
    const __amdgpu_buffer_rsrc_t wdr =
        __builtin_amdgcn_make_buffer_rsrc((void *) wd, (short) 0, (int) (uint32_t) (a.dNTq * SB), 0x00020000);
    const uint32_t dvo = SV == 32 || (q >> 1) == (int) (s & 1) ? 16u * lane : 0x80000000u;
    u32x4 dv[DQ];
    uint32_t dp[DQ][FMT == ONPU_Q4NX ? 4 : 2];
#pragma unroll
    for (int i = 0; i < DQ; i++) {
        const int64_t tq = wave + NW * i < a.dNTq ? wave + NW * i : 0;
        if (SV == 32) dv[i] = __builtin_nontemporal_load(GLB(const u32x4, wd + tq * SB + 16 * lane));
        else dv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wdr, dvo, (uint32_t) (tq * SB), 2));
        if (FMT == ONPU_Q4NX) {
            const u32x4 p = __builtin_nontemporal_load(GLB(const u32x4, wd + tq * SB + 1024 + 16 * r));
#pragma unroll
            for (int d = 0; d < 4; d++) dp[i][d % (sizeof(dp[i]) / 4)] = p[d];
        } else {
            const u32x2 p = __builtin_nontemporal_load(GLB(const u32x2, wd + tq * SB + 1024 + 8 * r));
            dp[i][0] = p.x;
            dp[i][1 % (sizeof(dp[i]) / 4)] = p.y;
        }
    }
    // keep the down loads here, in flight during the gate / up products (the scheduler would
    // otherwise issue them after those, adding a memory round trip)
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[1][1] = {{{0.f, 0.f, 0.f, 0.f}}};
    ds_accum<FMT, GB>(wv, par, nb, xs, xg, nb > 0 ? b0 : 0, acc);
    if (q == 0) red[wave * 16 + r] = acc[0][0][0];
    __syncthreads();
    if (threadIdx.x < 32) {                     // act of the step's K position i
        // SV 32: I value 32 s + i, gate / up tile i >> 4, row i & 15; SV 16: position i holds I value
        // 16 s + (i & 15) when i >> 4 == s % 2 (row i & 15 of the slice's gate / up tile), else zero
        const int i = threadIdx.x, tt = SV == 32 ? i >> 4 : 0, rr = i & 15;
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int pp = 0; pp < P; pp++) {       // the K parts in order
            g += red[(tt * P + pp) * 16 + rr];
            u += red[((NTL / 2 + tt) * P + pp) * 16 + rr];
        }
        const uint16_t ab = SV == 32 || (i >> 4) == (int) (s & 1) ? f32_to_bf16(silu_f(g) * u) : (uint16_t) 0;
        act[i] = ab;
        float sum = bf16_to_f32(ab);
        for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (i == 0) *acs = sum * xsum_mul<FMT>();
    }
    __syncthreads();
    const u32x4 xa = *LDS_U32X4(act + 8 * q);
    const float cs1 = *acs;
    const f32x4 csv = {cs1, cs1, cs1, cs1}, z = {0.f, 0.f, 0.f, 0.f};
    const uint32_t mag = 0x43004300u;
    float * out = a.part + (slot * a.S + s) * a.dNTq * 64;
#pragma unroll
    for (int i = 0; i < DQ; i++) {             // every quad computed (no load's use behind a branch)
        const int64_t tq = wave + NW * i;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const u32x4 bw = unpack_biased(dv[i][d], mag);
            float y;
            if (FMT == ONPU_Q4NX) {
                // w = u s + m: (s (128 + u) . act - 128 s sum) + m sum, as the decode GEMV adds it
                const float sc = bf16_to_f32((uint16_t) (dp[i][d % (sizeof(dp[i]) / 4)] & 0xffff));
                const float mn = bf16_to_f32((uint16_t) (dp[i][d % (sizeof(dp[i]) / 4)] >> 16));
                const f32x4 cg = mfma(xa, bw, z);
                y = fmaf(mn, cs1, fmaf(sc, cg[0], fmaf(-128.0f * sc, cs1, 0.f)));
            } else {
                const float sc = scale_f32(FMT, (dp[i][d >> 1] >> (16 * (d & 1))) & 0xffff);
                const f32x4 cg = mfma(xa, bw, csv);
                y = sc * cg[0];
            }
            if (q == 0 && tq < a.dNTq) out[tq * 64 + 16 * d + r] = y;
        }
    }
}

// ------------------------------------------------------------------ chained decode GEMVs
// One launch runs a.n GEMVs in order (M <= 16 rows, x staged in LDS), one workgroup per CU of
// CHAIN_WAVES compute waves and CHAIN_CTRL control waves. Entry i's tile groups (tw tiles x kw K
// parts, tw kw = CHAIN_WAVES) go to workgroups g = blockIdx.x, + gridDim.x, ...
// Compute waves: weights stream through a ring of S block slots per wave, filled by buffer-to-LDS
//   loads. A wave's sequence of blocks over the whole chain is known up front (weights do not depend
//   on x), so the ring is refilled with the next block of the sequence as each block is consumed and
//   keeps S blocks in flight across entry boundaries: HBM streams while a workgroup waits for x. The
//   compute waves issue no other memory loads, so their wait counts stay exact and nothing drains
//   the ring.
// Control waves: sum the K parts of each tile group and store y; for an entry that a later entry
//   reads, also publish y as link words (bf16 value << 16 | the run's 16-bit tag) with agent-scope
//   stores. Then they stage the next entry's x into LDS: an external x with plain loads, a linked x
//   by polling the producer's link words that it reads with agent-scope loads until every one
//   carries this run's tag. Each 32-bit word is written and read whole, so a word with the tag holds
//   this run's value. This is the dependency itself, seen one memory round trip after the data
//   lands, instead of a grid barrier (store acknowledgement, arrival, poll, re-read). A poll past
//   a.spin attempts sets the error flag and proceeds (results then wrong, the kernel still ends).
// The run's tag is (epoch + 1) mod 2^16, epoch read from a.ep at the start; the last workgroup to
// finish advances the epoch and resets the done counter, so a captured launch replays with fresh
// tags and the link words never need clearing (they start at zero, epoch 0).
// Every workgroup must be resident at once (the host sizes the grid from the occupancy).

// x rows [M][K] (bf16, row stride K) of an external input into the LDS copy xs[M][xls] (zero past
// K up to 128 KB) and the column sums of each group of gs times xmul (xsum[group][perm16(row)]), by
// the T control threads (index ct): consecutive threads take consecutive 8-element units, a
// group's units in consecutive lanes of one wave, summed across them.
DEV void chain_stage_ext(const uint16_t * x, int M, int64_t K, int64_t KB, int64_t xls, int gs, float xmul,
                         uint16_t * xs, float * xsum, uint32_t ct, uint32_t T) {
    const uint32_t upg = gs / 8, kp8 = (uint32_t) KB * 16, nunits = (uint32_t) M * kp8;
    for (uint32_t u0 = 0; u0 < nunits; u0 += 2 * T) {            // same trip count for every control lane
        u32x4 v[2];
        uint32_t m[2], kk[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {                             // both loads first: one round trip
            const uint32_t u = u0 + j * T + ct;
            v[j] = (u32x4){0u, 0u, 0u, 0u};
            m[j] = u / kp8;
            kk[j] = (u - m[j] * kp8) * 8;
            if (u < nunits && kk[j] < K) v[j] = *GLB(const u32x4, x + (int64_t) m[j] * K + kk[j]);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t u = u0 + j * T + ct;
            if (u < nunits) *LDS_U32X4(xs + (int64_t) m[j] * xls + kk[j]) = v[j];
            float t = 0.f;
            for (int d = 0; d < 4; d++) t += __uint_as_float(v[j][d] << 16) + __uint_as_float(v[j][d] & 0xffff0000u);
            for (int o = upg / 2; o > 0; o >>= 1) t += __shfl_xor(t, o);
            if (u < nunits && u % upg == 0) xsum[(kk[j] / gs) * 16 + perm16((int) m[j])] = t * xmul;
        }
    }
}

// one 8-word unit of link words (agent-scope loads: coherent across the XCDs' L2 caches)
DEV void chain_link_load(const uint32_t * p, uint64_t (&v)[4]) {
    const auto * q = GLB(uint64_t, p);
    for (int d = 0; d < 4; d++) v[d] = __hip_atomic_load(q + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

DEV bool chain_link_ok(const uint64_t (&v)[4], uint32_t tag) {
    const uint64_t t2 = (uint64_t) tag | ((uint64_t) tag << 32), m2 = 0x0000ffff0000ffffull;
    return ((v[0] & m2) == t2) & ((v[1] & m2) == t2) & ((v[2] & m2) == t2) & ((v[3] & m2) == t2);
}

// poll until every lane's units (need[] false for those that need no wait) carry `tag`: the units
// are (re)loaded until the whole wave sees them. Returns false when `spin` polls ran out or, checked
// every 256 polls, another wave has already set the error flag (so one lost wait ends them all).
template <int B, class Addr>
DEV bool chain_poll(Addr addr, const bool (&need)[B], uint64_t (&v)[B][4], uint32_t tag, uint32_t spin,
                    const int32_t * err) {
    for (uint32_t polls = 0;; polls++) {
#pragma unroll
        for (int b = 0; b < B; b++)
            if (need[b]) chain_link_load(addr(b), v[b]);
        bool ok = true;
#pragma unroll
        for (int b = 0; b < B; b++) ok &= !need[b] || chain_link_ok(v[b], tag);
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
        if (polls >= spin) return false;
        if ((polls & 255u) == 255u &&
            __hip_atomic_load(GLB(const int32_t, err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
            return false;
        __builtin_amdgcn_s_sleep(2);
    }
}

// x of a linked entry from its producer's link words (row m of x = lx[m * ldl + 0 .. K)), staged
// as chain_stage_ext does, each unit once all its words carry this run's tag
DEV void chain_stage_link(const ChainEntry & E, int M, int64_t xls, int gs, float xmul, uint16_t * xs, float * xsum,
                          uint32_t tag, uint32_t spin, int32_t * err, uint32_t ct, uint32_t T) {
    constexpr int B = 4;
    const uint32_t upg = gs / 8, kp8 = (uint32_t) E.KB * 16, nunits = (uint32_t) M * kp8;
    const uint32_t K = (uint32_t) E.K, ldl = (uint32_t) E.ldl;
    bool fine = true;
    for (uint32_t u0 = 0; u0 < nunits; u0 += B * T) {            // same trip count for every control lane
        bool need[B];
        uint32_t m[B], kk[B];
        uint64_t v[B][4];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const uint32_t u = u0 + b * T + ct;
            m[b] = u / kp8;
            kk[b] = (u - m[b] * kp8) * 8;
            need[b] = u < nunits && kk[b] < K;
            for (int d = 0; d < 4; d++) v[b][d] = 0;
        }
        if (!chain_poll<B>([&](int b) { return E.lx + m[b] * ldl + kk[b]; }, need, v, tag, spin, err)) {
            fine = false;
            spin = 0;                                 // the rest of this wait gives up at once
        }
#pragma unroll
        for (int b = 0; b < B; b++) {
            const uint32_t u = u0 + b * T + ct;
            u32x4 w = {0u, 0u, 0u, 0u};              // bf16 values: the high halves of the words
            if (need[b])
                for (int d = 0; d < 4; d++)
                    w[d] = (uint32_t) (v[b][d] >> 16 & 0xffffu) | (uint32_t) (v[b][d] >> 32 & 0xffff0000u);
            if (u < nunits) *LDS_U32X4(xs + (int64_t) m[b] * xls + kk[b]) = w;
            float t = 0.f;
            for (int d = 0; d < 4; d++) t += __uint_as_float(w[d] << 16) + __uint_as_float(w[d] & 0xffff0000u);
            for (int o = upg / 2; o > 0; o >>= 1) t += __shfl_xor(t, o);
            if (u < nunits && u % upg == 0) xsum[(kk[b] / gs) * 16 + perm16((int) m[b])] = t * xmul;
        }
    }
    if (!fine) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// position in a wave's block sequence over the chain: block b (< b1) of tile t of entry e, tile
// group g; e == a.n: past the end. 32-bit throughout, so that the bookkeeping stays in scalar
// registers (a 64-bit compare goes through vector registers, and a vector write on a path that
// merges with outstanding loads makes the compiler wait for all of them)
struct ChainCur {
    int e, g, t, b, b1;
    uint32_t so;                      // byte offset of block b of tile t in entry e's weights
    __amdgpu_buffer_rsrc_t rs;        // entry e's weights (bounds: the whole matrix)
};

// the wave's tile and K blocks [b0, b1) in tile group g of entry E (empty past the last tile)
DEV void chain_range(const ChainEntry & E, int g, int wave, int & t, int & b0, int & b1) {
    const int twi = wave / E.kw, kp = wave % E.kw, KB = (int) E.KB, bpw = (int) E.bpw;
    t = g * E.tw + twi;
    b0 = kp * bpw;
    b1 = b0 + bpw < KB ? b0 + bpw : KB;
    if (t >= (int) E.NT) b1 = b0;
}

// moves c forward to the next position that holds a block, or past the end
template <int FMT>
DEV void chain_settle(ChainCur & c, const ChainEntry * __restrict__ ents, int n, int w, int P, int wave) {
    while (c.e < n && c.b >= c.b1) {
        c.g += P;
        if (c.g >= (int) ents[c.e].groups) { c.e++; c.g = w; }
        c.b = c.b1 = 0;
        if (c.e < n && c.g < (int) ents[c.e].groups) {
            const ChainEntry & E = ents[c.e];
            chain_range(E, c.g, wave, c.t, c.b, c.b1);
            c.so = (uint32_t) (c.t * (int) E.KB + c.b) * (uint32_t) fmt_blk(FMT);
            c.rs = __builtin_amdgcn_make_buffer_rsrc((void *) E.W, (short) 0, (int) (E.NT * E.KB * fmt_blk(FMT)),
                                                     0x00020000);
        }
    }
}

// two buffer-to-LDS loads of c's block into `slot`: 1 KiB of nibbles (16 bytes per lane) and the
// parameters (4 bytes per lane, the lanes they need); past the end both read out of range (zeros,
// no memory traffic), so every refill counts two loads. Within a tile's K range the next block is
// the next BLK bytes; the cursor is settled only at the range's end.
template <int FMT>
DEV void chain_issue(ChainCur & c, const ChainEntry * __restrict__ ents, int n, int w, int P, int wave,
                     uint8_t * slot, int lane) {
    constexpr int BLK = 1024 + 16 * (128 / (FMT == ONPU_G128S ? 128 : 32)) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    constexpr int PW = (BLK - 1024) / 4;
    const bool live = c.e < n;
    const uint32_t vo = live ? 16u * lane : 0x80000000u, vp = live ? 1024u + 4u * lane : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rs, (lds_void *) slot, 16, vo, c.so, 0, 0);
    if (lane < PW) __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rs, (lds_void *) (slot + 1024), 4, vp, c.so, 0, 0);
    if (live) {
        c.b++;
        c.so += BLK;
        if (c.b >= c.b1) chain_settle<FMT>(c, ents, n, w, P, wave);
    }
}

// workgroup barrier that orders LDS only: a __syncthreads here would also wait for every
// buffer-to-LDS load in flight (the ring), draining it at each barrier
DEV void chain_sync() {
    __builtin_amdgcn_s_waitcnt(LGKM0_IMM);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int FMT>
DEV Par<FMT> load_par_lds(const uint8_t * blk, int r) {
    Par<FMT> p;
    typedef __attribute__((address_space(3))) const uint32_t lds_u32;
    typedef __attribute__((address_space(3))) const u32x2 lds_u32x2;
    if (FMT == ONPU_G128S) {                                                     // as load_par
        p.v[0] = *(lds_u32 *) (blk + 1024 + 4 * (r >> 1));
        p.v[1] = g128s_sel(r);
    }
    else if (FMT == ONPU_Q4NX) {
        const u32x4 q = *LDS_U32X4(blk + 1024 + 16 * r);
        for (int j = 0; j < 4; j++) p.v[j % (sizeof(p.v) / 4)] = q[j];
    } else {
        const u32x2 q = *(lds_u32x2 *) (blk + 1024 + 8 * r);
        p.v[0] = q.x;
        p.v[1 % (sizeof(p.v) / 4)] = q.y;
    }
    return p;
}

// The two roles run separate loops with the same sequence of workgroup barriers (one after the
// first x, one per tile group, one per entry boundary), so the compiler's wait counts on the compute
// path never see the control waves' loads (a merged path makes it wait for every outstanding load,
// which would drain the ring).
template <int FMT, int S>
__global__ __launch_bounds__((CHAIN_WAVES + CHAIN_CTRL) * 64) void k_qgemv_chain(ChainArgs a,
                                                                                 const ChainEntry * __restrict__ ents) {
    constexpr int GS = FMT == ONPU_G128S ? 128 : 32;
    constexpr int BLK = 1024 + 16 * (128 / GS) * 2 * (FMT == ONPU_Q4NX ? 2 : 1);
    constexpr uint32_t CT = CHAIN_CTRL * 64;            // control threads
    static_assert(2 * (S - 1) <= 63, "ring deeper than the load counter");
    extern __shared__ __align__(16) float red[];  // [2][CHAIN_WAVES][256] partial sums, x rows, column sums, ring
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int P = (int) gridDim.x, w = (int) blockIdx.x;
    uint16_t * xs = (uint16_t *) (red + 2 * CHAIN_WAVES * 256);
    float * xsum = (float *) (xs + (int64_t) a.M * a.xls);
    if (wave < CHAIN_WAVES) {
        // ---------------- compute waves
        const int r = lane & 15, q = lane >> 4;
        uint8_t * ring = (uint8_t *) red + a.ring + wave * S * BLK;
        const XSrc X{nullptr, 0, xs, a.xls, xsum};
        ChainCur ic;                        // refills past the end read entry 0 out of range
        ic.e = 0; ic.g = w - P; ic.t = ic.b = ic.b1 = 0; ic.so = 0;
        ic.rs = __builtin_amdgcn_make_buffer_rsrc((void *) ents[0].W, (short) 0, 0, 0x00020000);
        chain_settle<FMT>(ic, ents, a.n, w, P, wave);
        for (int s = 0; s < S; s++) chain_issue<FMT>(ic, ents, a.n, w, P, wave, ring + s * BLK, lane);
        chain_sync();                                           // x of entry 0 staged
        const uint32_t mag = 0x43004300u;
        uint32_t k = 0;                     // blocks consumed: the next one sits in slot k % S
        int rb = 0;                         // partial-sum buffer of the current tile group
        for (int i = 0; i < a.n; i++) {
            const ChainEntry & E = ents[i];
            const int groups = (int) E.groups;
            for (int g = w; g < groups; g += P) {
                float * rp = red + rb * CHAIN_WAVES * 256;
                f32x4 acc[1][1];
                acc[0][0] = (f32x4){0.f, 0.f, 0.f, 0.f};
                int t, b0, b1;
                chain_range(E, g, wave, t, b0, b1);
                for (int b = b0; b < b1; b++) {
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (S - 1)));     // block k has landed
                    uint8_t * sl = ring + (k % S) * BLK;
                    WChunk<FMT, 1, 1> ch;
                    ch.ok[0][0] = true;
                    ch.wv[0][0] = *LDS_U32X4(sl + 16 * lane);
                    ch.par[0][0] = load_par_lds<FMT>(sl, r);
                    compute_chunk<FMT, 1, 1, 1, true, 4>(ch, b, b1, X, a.M, E.K, r, q, mag, acc);
                    __builtin_amdgcn_s_waitcnt(LGKM0_IMM);            // the slot's reads are done
                    chain_issue<FMT>(ic, ents, a.n, w, P, wave, sl, lane);     // refill it
                    k++;
                }
                for (int v = 0; v < 4; v++) rp[wave * 256 + v * 64 + lane] = acc[0][0][v];
                chain_sync();                                   // partial sums of the group
                rb ^= 1;
            }
            if (i + 1 == a.n) break;
            chain_sync();                                       // x of entry i + 1 staged
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));   // the ring's last (out-of-range) loads have landed
        return;
    }
    // ---------------- control waves
    const uint32_t ct = threadIdx.x - CHAIN_WAVES * 64;
    const uint32_t epoch = __hip_atomic_load(GLB(uint32_t, a.ep) + CHAIN_EP_EPOCH, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t tag = (epoch + 1u) & 0xffffu;
    chain_stage_ext(ents[0].x, a.M, ents[0].K, ents[0].KB, a.xls, GS, xsum_mul<FMT>(), xs, xsum, ct, CT);
    chain_sync();
    int rb = 0;
    for (int i = 0; i < a.n; i++) {
        const ChainEntry & E = ents[i];
        const int groups = (int) E.groups, etw = E.tw, ekw = E.kw, nout = etw * 16 * a.M;
        const int64_t eN = E.N, nl = E.NT * 16;          // link rows: whole tiles
        void * const ey = E.y;
        uint32_t * const ely = E.ly;
        for (int g = w; g < groups; g += P) {
            chain_sync();                                       // partial sums of the group
            const float * rp = red + rb * CHAIN_WAVES * 256;
            // outputs (tile g tw + ti, row m, column c), summed over the kw K parts
            for (int o = (int) ct; o < nout; o += (int) CT) {
                const int ti = o / (16 * a.M), m = (o / 16) % a.M, c = o % 16;
                const int64_t n = 16 * ((int64_t) g * etw + ti) + c;
                // the accumulator of row m, column c sits at lane c + 16 (m % 4), element m / 4
                // (x row m in MFMA row perm16(m))
                const float * src = rp + ti * ekw * 256 + (m >> 2) * 64 + c + 16 * (m & 3);
                float sum = src[0];
#pragma unroll
                for (int k2 = 1; k2 < CHAIN_WAVES; k2++)
                    if (k2 < ekw) sum += src[k2 * 256];
                if (n < eN) store_out(ey, a.yf32, (int64_t) m * eN + n, sum);
                if (ely != nullptr && n < nl) {             // zeros past N
                    const uint32_t word = ((uint32_t) (n < eN ? f32_to_bf16(sum) : 0) << 16) | tag;
                    __hip_atomic_store(GLB(uint32_t, ely) + m * nl + n, word, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            rb ^= 1;
        }
        if (i + 1 == a.n) break;
        const ChainEntry & F = ents[i + 1];
        if (F.lx != nullptr)
            chain_stage_link(F, a.M, a.xls, GS, xsum_mul<FMT>(), xs, xsum, tag, a.spin, a.ep + CHAIN_EP_ERR, ct, CT);
        else
            chain_stage_ext(F.x, a.M, F.K, F.KB, a.xls, GS, xsum_mul<FMT>(), xs, xsum, ct, CT);
        chain_sync();                                           // x of entry i + 1 staged
    }
    if (ct == 0) {
        // the last workgroup to finish advances the epoch (the next launch's tags) and resets the
        // count; every workgroup read the epoch before it could finish, and the next launch starts
        // after this one has ended
        const uint32_t done = __hip_atomic_fetch_add(GLB(uint32_t, a.ep) + CHAIN_EP_DONE, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        if (done == (uint32_t) P - 1) {
            __hip_atomic_store(GLB(uint32_t, a.ep) + CHAIN_EP_DONE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(GLB(uint32_t, a.ep) + CHAIN_EP_EPOCH, epoch + 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Kernel argument blocks and launchers shared by onpu_kernels.hip and onpu_api.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "onpu_common.h"

// k_qgemv: y = x . deq(W)^T for M <= 64 rows of x, per slot (expert) and epilogue
struct QArgs {
    const uint8_t * W;        // tiled weights; expert e at W + e * estride
    int64_t estride;
    const int32_t * ids;      // expert of each slot (nullptr: one dense matrix)
    int64_t N, K, NT, KB;
    const uint16_t * x;       // bf16 rows; slot s reads x + (s / xdiv) * xslot, row stride ldx
    int64_t ldx, xslot, xdiv;
    int M;
    void * y;                 // bf16 or fp32 (yf32); slot s writes y + s * yslot, row stride ldy
    int64_t ldy, yslot;
    int yf32;
    const float * wslot;      // EPI_SLOTSUM: routing weights [tokens][nslot]
    int nslot, ksplit;        // EPI_SLOTSUM: waves = nslot * ksplit
    int64_t bpw;              // K blocks (128 wide) per wave
    int64_t xls;              // LDS-staged x (XL variants): row stride in elements
    int tw;                   // tile groups per workgroup (waves = tw * K parts); 1 for EPI_SLOTSUM
    // EPI_ACT with logits: each workgroup routes its token (slot / xdiv, top xdiv of E experts) and
    // multiplies by the expert it picks for its slot instead of reading ids; one workgroup per token
    // writes the token's ids and weights to rids / rw (renorm as the router kernel)
    const float * logits;
    int E, renorm;
    int32_t * rids;
    float * rw;
    // EPI_ARGMAX: the workgroups' keys per row, [M][gridDim.x]
    uint64_t * akeys;
};

// k_qgemm / k_qgemm_sk: prefill, Y[M][N] = X[M][K] . deq(W)^T
struct GArgs {
    const uint8_t * W;
    int64_t NT, KB, N, K, M;
    const uint16_t * x;
    int64_t ldx;
    void * y;
    int64_t ldy;
    int yf32;
    // k_qgemm_sk only: K-block iterations per workgroup over the tile-major sequence of
    // tiles * KB; fp32 partial tiles, one slot per cut tile; per slot an arrival counter (two per
    // launch) and a ready word holding the tag of the launch that published (GSK_SYNC_STRIDE ints
    // apart, zero when allocated); ctl: the last launch's tag, the count of finished workgroups and
    // the timed-out-wait flag (GSK_CTL_* ints apart)
    int64_t ipw;
    int sym;                  // sched 1 with one tail piece per workgroup: the two segments of a cut
                              // tile exchange halves (each finishes half the rows), slot words 2, 3
    float * ws;
    int32_t * sync;
    int32_t * ctl;
    uint32_t spin;
    // sched 1 (two-phase): rounds F of one whole tile per workgroup, then the R remaining tiles
    // cut at K block s: workgroup g < R takes blocks [0, s) of tile F G + g, workgroup g >= R the
    // blocks [s, KB) of c tiles. sched 0: the ipw ranges above.
    int sched;
    int64_t F, R, s, c;
    // k_qgemm split-K (splits > 1): the workgroups of split sp take K blocks [sp kbs, (sp + 1) kbs)
    // of every tile and store fp32 partials to ws + sp M N ([M][N], row stride N); k_gemm_split_sum
    // adds the splits in order into Y
    int splits;
    int64_t kbs;
    // k_qgemm, one row tile and no split: also each workgroup's argmax key per row, akeys[m][N block]
    uint64_t * akeys;
    int deep;                 // k_qgemm 16-row tiles: weights two blocks ahead
};
constexpr int GSK_SYNC_STRIDE = 16;
constexpr int GSK_CTL_TAG = 0, GSK_CTL_DONE = 16, GSK_CTL_ERR = 32, GSK_CTL_INTS = 48;

// grouped MoE products (k_moe_gemm) over a device work list (expert, first position, rows)
struct MArgs {
    const uint8_t * W;
    int64_t estride, NT, KB, N, K;
    const uint16_t * x;       // gate_up: token rows [T][K]; down: act rows in permuted order
    int64_t ldx;
    void * y;                 // gate_up: act bf16 [T*k][N/2]; down: bf16 [T*k][N]
    int64_t ldy;
    const int32_t * perm;     // permuted position -> entry t * k + j
    const int32_t * items;    // [nitems][3]
    const int32_t * nitems;
    int k;
    int64_t xbytes;           // k_moe_gemm: bytes of x (buffer range of the gathered rows, < 2^31)
};

// MoE decode in one launch (k_moe_decode): router (optional), gate_up + SiLU * up per routed slot,
// down + routing-weighted slot sum per token. T <= MD_MAX_T tokens, k <= MD_MAX_K slots each.
struct MDArgs {
    const uint8_t * Wg;       // gate_up bank: expert e at Wg + e * gstride, [2 I][H] tiled
    int64_t gstride, gNT, gKB;
    const uint8_t * Wd;       // down bank: [Nd][I] tiled
    int64_t dstride, dNT, dKB;
    int64_t H, I, Nd;
    const uint16_t * x;       // [T][H] bf16
    const float * logits;     // [T][E] fp32 -> route in the kernel; nullptr: ids / w are inputs
    int E, k, renorm, T;
    int32_t * ids;            // [T][k]
    float * w;                // [T][k]
    uint16_t * act;           // [T k][I] bf16 scratch (written and read with agent-scope accesses)
    void * y;                 // [T][Nd]
    int yf32;
    int32_t * sync;           // [0] act tiles published, [MD_SYNC_DONE] consumers done, [MD_SYNC_ERR]
                              // timed-out wait flag; zero between launches
    int64_t npairs, nunits;   // T k (I / 16) gate/up tile pairs; T * dNT down tile rows
    uint32_t spin;            // poll limit of the wait for the act tiles
};
constexpr int MD_MAX_T = 4, MD_MAX_K = 8, MD_WAVES = 8, MD_SYNC_DONE = 16, MD_SYNC_ERR = 32, MD_SYNC_INTS = 48;
constexpr int MD_MAX_GB = 4;      // gate_up K blocks per wave (H <= 8 * 4 * 128)
constexpr int MD_MAX_DB = 8;      // down K blocks (I <= 1024)

// MoE decode split along I (k_moe_dsplit, then k_moe_dsum). Workgroup (slice s, slot t k + j) takes
// the I values [SV s, SV s + SV) of its slot's expert (SV = 32, or 16: half of a 32-wide K step):
// their gate and up rows (SV / 16 row tiles each) give act for those values, which it multiplies
// into the expert's down weights for the same K values (one MFMA K step, read from the down bank's
// step-major copy), leaving fp32 partial sums part[slot][s][n]. No workgroup waits for another.
// k_moe_dsum then forms y[t][n] = sum_j w[t][j] sum_s part[t k + j][s][n] in that order.
struct MSArgs {
    const uint8_t * Wg;       // gate_up bank: expert e at Wg + e * gstride, [2 I][H] tiled
    int64_t gstride, gNT, gKB;
    const uint8_t * Wd;       // down bank, step-major copy: expert e at Wd + e * dstride
    int64_t dstride, dNTq;    // dNTq = ceil(down row tiles / 4) superblocks per K step
    int64_t H, I, S;          // S = I / 32 slices of 32 values of I (I / 16 of 16)
    const uint16_t * x;       // [T][H] bf16
    const float * logits;     // [T][E] fp32 -> route in the kernel; nullptr: ids are inputs
    int E, k, renorm, T;
    int32_t * ids;            // [T][k]
    float * w;                // [T][k]
    float * part;             // [T k][S][dNTq * 64] fp32
};
constexpr int DS_MAX_T = 4, DS_MAX_K = 16;

// The step-major copy of a tiled matrix that k_moe_dsplit reads (per expert, dec_bytes apart):
// superblock (s, tq), s = 4 b + j one 32-wide K step, tq a quad of row tiles, at (s * NTq + tq) *
// dec_sblk. Its [0, 1024) holds for lane l (= 16 q + r) the dwords D_j of tiles 4 tq + d, d = 0..3, of
// block b (the tiled layout's dword j of lane l, zero past the last tile): the B operands of those
// four row tiles for step s. [1024, dec_sblk) holds per row r the four tiles' parameters of step s:
// u16 scales [16][4] (q4nx: {u16 scale, u16 min} [16][4]).
inline int dec_sblk(int fmt) { return 1024 + (fmt == ONPU_Q4NX ? 256 : 128); }
inline int64_t dec_bytes(int fmt, int64_t N, int64_t K) {
    const int64_t NTq = ((N + 15) / 16 + 3) / 4, S = 4 * ((K + 127) / 128);
    return (S * NTq * dec_sblk(fmt) + 255) / 256 * 256;
}

// chained decode GEMVs (k_qgemv_chain): entry i = y_i [M][N] = x_i [M][K] . W_i^T, in order. An
// entry reads an external x (bf16 rows, written before the launch) or a link: words
// (bf16 << 16 | run tag) that an earlier entry publishes for its output, rows ldl words apart
struct ChainEntry {
    const uint8_t * W;
    const uint16_t * x;       // external x [M][K] (nullptr when linked)
    void * y;
    int64_t NT, KB, N, K, bpw, groups;
    int tw, kw;               // tw * kw = CHAIN_WAVES
    uint32_t * ly;            // this entry's link words [M][NT * 16] (nullptr: no later entry reads y)
    const uint32_t * lx;      // linked x: row m at lx + m * ldl, in the producer's link words
    int64_t ldl;
};
struct ChainArgs {              // (the entries array is a kernel argument of its own)
    int n, M, yf32;
    int32_t * ep;             // CHAIN_EP_INTS ints: epoch, done counter, error flag (CHAIN_EP_* apart)
    int64_t xls;              // LDS row stride of x (elements) >= 128 KB of every entry
    int64_t ring;             // LDS byte offset of the weight ring
    uint32_t spin;            // poll limit of one wait for a link word
};
constexpr int CHAIN_WAVES = 8;    // compute waves per workgroup
constexpr int CHAIN_CTRL = 4;     // control waves per workgroup (sums, stores, x staging)
constexpr int CHAIN_RING_SLOTS[4] = {13, 10, 5, 3};   // ring depths built, deepest first
// the epoch, the count of finished workgroups and the error flag, on separate cache lines
constexpr int CHAIN_EP_EPOCH = 0, CHAIN_EP_DONE = 64, CHAIN_EP_ERR = 128, CHAIN_EP_INTS = 192;

hipError_t launch_repack(int fmt, const uint8_t * st, int64_t sstride, int64_t N, int64_t K, uint8_t * out,
                         int64_t ostride, int64_t E, hipStream_t s);
hipError_t launch_dequant(int fmt, const uint8_t * W, int64_t N, int64_t K, void * out, int bf16, hipStream_t s);
hipError_t launch_qgemv(int fmt, int epi, const QArgs & a, int mb, int rt, int nb, int xl, dim3 grid, int waves,
                        hipStream_t s);
int qgemv_has_variant(int epi, int mb, int rt, int nb, int xl);

int qgemv_max_waves(int mb, int rt, int nb, int xl);
// mb: 16-row A blocks per workgroup tile, 8 (ntw 2-4) or, with ntw 2, 1, 2 or 4 (up to 16 / 32 / 64 rows)
hipError_t launch_qgemm(int fmt, const GArgs & a, int ntw, int mb, hipStream_t s);
// Y [M][N] (row stride ldy; bf16 RNE or fp32) = the sum over s = 0 .. S-1, in that order, of
// part + s M N ([M][N] fp32)
hipError_t launch_gemm_split_sum(const float * part, int S, int64_t M, int64_t N, void * y, int64_t ldy, int yf32,
                                 hipStream_t s);
// k_qgemm_sk configuration: {weight tiles per wave, 16-row A blocks, waves}; rows and columns of the
// workgroup tile are 16 * MBG and 16 * NTW * WV. (Measured on MI355X against 256 x 64 per wave with
// one wave per SIMD and 256 x 32 with four waves: both slower, the first by ~30 %; and against
// 128 x 64 per wave with eight waves, which halves the LDS reads of X but doubles the dequantization
// per MFMA and spills: 40 % slower.)
struct GskCfg { int ntw, mbg, wv; };
constexpr GskCfg GSK_CFGS[1] = {{2, 16, 8}};
hipError_t launch_qgemm_sk(int fmt, const GArgs & a, int cfg, int grid, hipStream_t s);
hipError_t launch_route(const float * logits, int64_t T, int E, int k, int renorm, int32_t * ids, float * w,
                        hipStream_t s);
// ... and inv[i] = the position of entry i (perm's inverse)
hipError_t launch_moe_permute(const int32_t * ids, int64_t n, int E, int rows_per_item, int32_t * off, int32_t * perm,
                              int32_t * inv, int32_t * items, int32_t * nitems, hipStream_t s);
// grouped GEMM over the work items (k_moe_gemm): grid.x column groups (gate_up: NT / 8, down: NT / 8)
hipError_t launch_moe_gemm(int fmt, int which, const MArgs & a, int64_t maxitems, hipStream_t s);
// one-launch MoE decode on `grid` workgroups (one per CU); hipErrorInvalidValue when the shapes are
// outside what k_moe_decode handles (moe_decode_fits; the caller then uses the multi-launch path)
hipError_t launch_moe_decode(int fmt, const MDArgs & a, int grid, hipStream_t s);
bool moe_decode_fits(int64_t H, int64_t I, int64_t Nd, int64_t gKB, int64_t dKB, int T, int k, int E);
// MoE decode split along I (grid S x T k, then the partial sums); hipErrorInvalidValue outside what
// moe_dsplit_fits allows
bool moe_dsplit_fits(int64_t H, int64_t I, int64_t Nd, int64_t gKB, int T, int k, int E);
// sv: values of I per slice (32 or 16; a.S = a.I / sv)
hipError_t launch_moe_dsplit(int fmt, const MSArgs & a, int64_t Nd, int sv, hipStream_t s);
hipError_t launch_moe_dsum(const float * part, int64_t S, int64_t ld, const float * w, int64_t T, int k, int64_t Nd,
                           void * y, int yf32, hipStream_t s);
// experts [0, E) of a tiled matrix (src, sstride apart) -> their step-major copies (dst, dstride apart)
hipError_t launch_relayout_dec(int fmt, const uint8_t * src, int64_t sstride, int64_t N, int64_t K, uint8_t * dst,
                               int64_t dstride, int64_t E, hipStream_t s);
// the chained kernel on `grid` workgroups (all resident at once)
// (ring: CHAIN_RING_SLOTS[ring] weight blocks per compute wave)
hipError_t launch_chain(int fmt, int ring, const ChainArgs & a, const ChainEntry * ents, int grid, size_t lds,
                        hipStream_t s);
// workgroups of the chained kernel that fit one CU at this LDS size
int chain_occupancy(int fmt, int ring, size_t lds);
// experts [0, E) of the reference's NPU packing in geometry g (src, sstride apart) -> the staging
// layout (dst, dstride apart); packed row r becomes staging row rowmap[r] (r when rowmap is null)
hipError_t launch_npu_stage(int fmt, const uint8_t * src, int64_t sstride, const NpuGeom & g, const int32_t * rowmap,
                            int64_t N, int64_t K, uint8_t * dst, int64_t dstride, int64_t E, hipStream_t s);
// p[0, n) = 0 by a kernel on stream s (a graph node under capture, unlike a memset)
hipError_t launch_zero_i32(int32_t * p, int64_t n, hipStream_t s);
// y[t] = sum_j w[t][j] o[inv[t k + j]] (o bf16 rows, fp32 sum)
hipError_t launch_moe_combine(const uint16_t * o, const int32_t * inv, const float * w, int64_t T, int k, int64_t N,
                              void * y, int yf32, hipStream_t s);
// index of the largest of each row's P keys (k_qgemv's EPI_ARGMAX keys [rows][P]): one workgroup per row
hipError_t launch_argmax_keys(const uint64_t * keys, int64_t P, int64_t rows, int32_t * out, hipStream_t s);
// one launch of argmax_parts(N) workgroups per row, each over ARGMAX_CHUNK values; keys: workspace
// of rows * argmax_parts(N) * ARGMAX_PAD bytes; cnt: rows * ARGMAX_PAD bytes of counters, zero before
// the first call (each call leaves them at zero). Calls that overlap must not share keys / cnt.
constexpr int ARGMAX_THREADS = 256, ARGMAX_CHUNK = 16 * ARGMAX_THREADS, ARGMAX_PAD = 128;
int64_t argmax_parts(int64_t N);
// the argmax's counters and keys in a static device array (no allocation): ARGMAX_SCRATCH_BYTES
// per GPU, counters (zero between calls) in the first ARGMAX_SCRATCH_CNT bytes. init: once per
// device with that device current (hipGetSymbolAddress, counters zeroed); get: the current device's
// counters and keys for `rows` rows of N values, hipErrorInvalidValue past the array's size,
// hipErrorNotInitialized before init on this device.
constexpr int64_t ARGMAX_SCRATCH_BYTES = 1 << 20, ARGMAX_SCRATCH_CNT = 16384;
constexpr int ARGMAX_SCRATCH_MAX_DEVICES = 64;
hipError_t argmax_scratch_init();
hipError_t argmax_scratch_get(int64_t rows, int64_t N, uint64_t ** keys, uint32_t ** cnt);
hipError_t launch_argmax(const float * v, int64_t rows, int64_t N, int32_t * out, uint64_t * keys, uint32_t * cnt,
                         hipStream_t s);
// GPU weight codecs (onpu_codec.hip): W [ne][N][ldw] fp32 (wbf16 = 0) or bf16 -> ne staging buffers of
// format fmt, ostride bytes apart (a multiple of 16); Q4_K rows (ld bytes apart, experts bstride
// bytes apart) -> q4nx staging
hipError_t launch_quant_stage(int fmt, const void * W, int64_t ldw, int wbf16, int64_t N, int64_t K, int64_t ne,
                              uint8_t * out, int64_t ostride, hipStream_t s);
hipError_t launch_q4k_stage(const uint8_t * blocks, int64_t ld, int64_t bstride, int64_t N, int64_t K, int64_t ne,
                            uint8_t * out, int64_t ostride, hipStream_t s);
// int8 GEMV y = s * (W x) for int8 W [N][K] rows (K a multiple of 16, K * 4 bytes of x in LDS)
hipError_t launch_gemv_i8(const int8_t * W, const float * sc, int64_t N, int64_t K, const float * x, float * y,
                          hipStream_t s);
// Gated DeltaNet decode step (onpu_attn.hip): workspace of the conv outputs, and the two launches
int64_t gdn_ws_bytes(int Hk, int Hv, int Dk, int Dv);
hipError_t launch_gdn_step(const float * x, int H, const float * qkv, const float * z, const float * Wb,
                           const float * Wa, const float * conv_w, int Kc, float * conv_state, int L,
                           const float * A_log, const float * dt_bias, const float * norm_w, float eps, float * S,
                           int Hk, int Hv, int Dk, int Dv, float * out, void * ws, int64_t ws_bytes, hipStream_t s);
// decode attention (onpu_attn.hip): workspace bytes for (Hq, D, Hkv, S), and the two launches
int64_t attn_ws_bytes(int Hq, int D, int Hkv, int64_t S);
hipError_t launch_attn_step(const float * q, int Hq, int D, const void * K, const void * V, int kv_bf16, int Hkv,
                            int64_t S, int64_t hs, int64_t rs, const float * mask, const float * sinks, float scale,
                            float * out, void * ws, int64_t ws_bytes, hipStream_t s);
hipError_t launch_f32_to_bf16(const float * in, int64_t n, uint16_t * out, hipStream_t s);
hipError_t launch_moe_act(const float * h, int64_t rows, int64_t Ng, const int32_t * ids, const float * bias, int act,
                          float alpha, float limit, float * o, hipStream_t s);
hipError_t launch_moe_sum(const float * o, int64_t T, int k, int64_t N, const int32_t * ids, const float * w,
                          const float * bias, float * y, hipStream_t s);

enum { EPI_STORE_ = 0, EPI_ACT_ = 1, EPI_SLOTSUM_ = 2, EPI_ARGMAX_ = 3 };

// k_qgemv variants built for every format: X(epilogue, MB, RT, NB, XL). MB: 16-row x blocks;
// RT: row tiles per workgroup; NB: K blocks each wave loads before computing; XL: x staged in LDS.
#define ONPU_QGEMV_VARIANTS(X)                                                                          \
    X(0, 1, 1, 1, 1) X(0, 1, 1, 2, 1) X(0, 1, 1, 4, 1) X(0, 1, 2, 2, 1)                                 \
    X(0, 1, 1, 1, 0) X(0, 1, 1, 2, 0) X(0, 1, 2, 1, 0) X(0, 2, 1, 1, 0) X(0, 2, 1, 2, 0) X(0, 4, 1, 1, 0) \
    X(1, 1, 2, 1, 1) X(1, 1, 2, 2, 1) X(1, 1, 2, 1, 0) X(1, 2, 2, 1, 0) X(1, 4, 2, 1, 0)                \
    X(2, 1, 1, 1, 0) X(2, 1, 1, 2, 0) X(2, 1, 1, 3, 0)                                                   \
    X(3, 1, 1, 2, 1) X(3, 1, 1, 1, 1) X(3, 1, 1, 1, 0) X(3, 2, 1, 1, 0) X(3, 4, 1, 1, 0)                 \
    X(0, 1, 1, 1, 2) X(0, 1, 1, 2, 2) X(3, 1, 1, 1, 2) X(3, 1, 1, 2, 2)

// per-format entry points (onpu_fmt.hip compiled with ONPU_FMT_ID = id)
#define ONPU_FMT_DECL(id)                                                                                   \
    hipError_t repack_f##id(const uint8_t * st, int64_t sstride, int64_t N, int64_t K, int64_t KB, int64_t NT,  \
                            uint8_t * out, int64_t ostride, int64_t E, hipStream_t s);                    \
    hipError_t dequant_f##id(const uint8_t * W, int64_t N, int64_t K, int64_t KB, int64_t NT, void * out, int bf16, \
                             hipStream_t s);                                                              \
    hipError_t qgemv_f##id(int epi, const QArgs & a, int mb, int rt, int nb, int xl, dim3 grid, int waves,       \
                           size_t lds, hipStream_t s);                                                    \
    hipError_t qgemm_f##id(const GArgs & a, int ntw, int mb, hipStream_t s);                                       \
    hipError_t qgemm_sk_f##id(const GArgs & a, int cfg, int grid, hipStream_t s);                          \
    hipError_t moe_gemm_f##id(int which, const MArgs & a, dim3 grid, hipStream_t s);                  \
    hipError_t moe_decode_f##id(const MDArgs & a, int gb, int grid, size_t lds, hipStream_t s);       \
    hipError_t moe_dsplit_f##id(const MSArgs & a, int nw, int sv, size_t lds, hipStream_t s);         \
    hipError_t relayout_dec_f##id(const uint8_t * src, int64_t sstride, int64_t NT, int64_t KB, uint8_t * dst, \
                                  int64_t dstride, int64_t E, hipStream_t s);                          \
    hipError_t chain_f##id(int ring, const ChainArgs & a, const ChainEntry * ents, int grid, size_t lds,  \
                           hipStream_t s);                                                                \
    int chain_occ_f##id(int ring, size_t lds);
ONPU_FMT_DECL(0)
ONPU_FMT_DECL(1)
ONPU_FMT_DECL(2)
ONPU_FMT_DECL(3)

// GPU weight codecs of libonpu_hip: quantize weights already in HBM (fp32 or bf16) into the staging
// layout of a format, or transcode GGUF Q4_K super-blocks into q4nx staging, with the quantizers
// of onpu_codec.h (the same source as the host's onpu_pack / onpu_pack_q4k, so the bytes are
// equal). The host then repacks the staging into the tiled HBM layout (k_repack).
// One thread per group: the search quantizers are compute-bound (16 or 21 candidate scales, each a
// pass of divisions over the group) and every group is independent.
#include "onpu_codec.h"
#include "onpu_launch.h"

namespace {

constexpr int CODEC_THREADS = 128;

template <int G>
__device__ __forceinline__ void load_group(const void * W, int wbf16, int64_t off, float (&x)[G]) {
    if (wbf16) {
        const uint16_t * p = (const uint16_t *) W + off;
#pragma unroll
        for (int i = 0; i < G; i++) x[i] = bf16_to_f32(p[i]);
    } else {
        const float * p = (const float *) W + off;
#pragma unroll
        for (int i = 0; i < G; i++) x[i] = p[i];
    }
}

// grid (groups / CODEC_THREADS, experts): W [e][N][ldw] (elements), out [e] staging of ostride bytes
template <int FMT>
__global__ __launch_bounds__(CODEC_THREADS) void k_quant_stage(const void * __restrict__ W, int64_t ldw, int wbf16,
                                                              int64_t N, int64_t K, uint8_t * __restrict__ out,
                                                              int64_t ostride) {
    constexpr int G = FMT == ONPU_G128S ? 128 : 32;
    const int64_t ng = K / G, gid = (int64_t) blockIdx.x * CODEC_THREADS + threadIdx.x;
    if (gid >= N * ng) return;
    const int64_t e = blockIdx.y, r = gid / ng, g = gid - r * ng;
    float x[G];
    load_group<G>(W, wbf16, (e * N + r) * ldw + g * G, x);
    uint8_t q[G];
    uint8_t * o = out + e * ostride;
    if (FMT == ONPU_Q4_0) {
        uint16_t dh;
        quant_q4_0(*reinterpret_cast<float (*)[32]>(x), *reinterpret_cast<uint8_t (*)[32]>(q), dh);
        uint16_t * blk = (uint16_t *) (o + (r * ng + g) * 18);           // 18-byte blocks: 2-byte aligned
        blk[0] = dh;
#pragma unroll
        for (int j = 0; j < 8; j++)
            blk[1 + j] = (uint16_t) ((q[2 * j] | (q[16 + 2 * j] << 4)) | ((q[2 * j + 1] | (q[17 + 2 * j] << 4)) << 8));
        return;
    }
    uint16_t s = 0, m = 0;
    if (FMT == ONPU_Q4NX) quant_asym32(*reinterpret_cast<float (*)[32]>(x), *reinterpret_cast<uint8_t (*)[32]>(q), s, m);
    else quant_sym<G>(x, q, s);
    uint32_t * c = (uint32_t *) (o + r * (K / 2) + g * (G / 2));          // G / 2 bytes, 16-byte aligned
#pragma unroll
    for (int w = 0; w < G / 8; w++) {
        uint32_t v = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) v |= (uint32_t) q[8 * w + i] << (4 * i);
        c[w] = v;
    }
    uint16_t * sc = (uint16_t *) (o + N * K / 2);
    sc[r * ng + g] = s;
    if (FMT == ONPU_Q4NX) sc[N * ng + r * ng + g] = m;
}

// grid (groups / CODEC_THREADS, experts): Q4_K rows of K / 256 super-blocks, ld bytes apart,
// experts bstride bytes apart -> q4nx staging
__global__ __launch_bounds__(CODEC_THREADS) void k_q4k_stage(const uint8_t * __restrict__ blocks, int64_t ld,
                                                            int64_t bstride, int64_t N, int64_t K,
                                                            uint8_t * __restrict__ out, int64_t ostride) {
    const int64_t ng = K / 32, gid = (int64_t) blockIdx.x * CODEC_THREADS + threadIdx.x;
    if (gid >= N * ng) return;
    const int64_t e = blockIdx.y, r = gid / ng, g = gid - r * ng;
    uint8_t q[32];
    uint16_t s = 0, m = 0;
    q4k_sub(blocks + e * bstride + r * ld + (g / 8) * Q4K_BLOCK, (int) (g % 8), q, s, m);
    uint8_t * o = out + e * ostride;
    uint32_t * c = (uint32_t *) (o + r * (K / 2) + g * 16);
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t v = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) v |= (uint32_t) q[8 * w + i] << (4 * i);
        c[w] = v;
    }
    uint16_t * sc = (uint16_t *) (o + N * K / 2);
    sc[r * ng + g] = s;
    sc[N * ng + r * ng + g] = m;
}

}  // namespace

hipError_t launch_quant_stage(int fmt, const void * W, int64_t ldw, int wbf16, int64_t N, int64_t K, int64_t ne,
                              uint8_t * out, int64_t ostride, hipStream_t s) {
    const int64_t groups = N * (K / fmt_group(fmt));
    if (groups <= 0 || ne <= 0) return hipSuccess;
    if (ne > 65535 || (groups + CODEC_THREADS - 1) / CODEC_THREADS >= ((int64_t) 1 << 31) || ostride % 16 != 0)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned) ((groups + CODEC_THREADS - 1) / CODEC_THREADS), (unsigned) ne);
    switch (fmt) {
    case ONPU_Q4NX: k_quant_stage<ONPU_Q4NX><<<grid, CODEC_THREADS, 0, s>>>(W, ldw, wbf16, N, K, out, ostride); break;
    case ONPU_Q4S: k_quant_stage<ONPU_Q4S><<<grid, CODEC_THREADS, 0, s>>>(W, ldw, wbf16, N, K, out, ostride); break;
    case ONPU_G128S: k_quant_stage<ONPU_G128S><<<grid, CODEC_THREADS, 0, s>>>(W, ldw, wbf16, N, K, out, ostride); break;
    case ONPU_Q4_0: k_quant_stage<ONPU_Q4_0><<<grid, CODEC_THREADS, 0, s>>>(W, ldw, wbf16, N, K, out, ostride); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_q4k_stage(const uint8_t * blocks, int64_t ld, int64_t bstride, int64_t N, int64_t K, int64_t ne,
                            uint8_t * out, int64_t ostride, hipStream_t s) {
    const int64_t groups = N * (K / 32);
    if (groups <= 0 || ne <= 0) return hipSuccess;
    if (ne > 65535 || (groups + CODEC_THREADS - 1) / CODEC_THREADS >= ((int64_t) 1 << 31) || ostride % 16 != 0)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned) ((groups + CODEC_THREADS - 1) / CODEC_THREADS), (unsigned) ne);
    k_q4k_stage<<<grid, CODEC_THREADS, 0, s>>>(blocks, ld, bstride, N, K, out, ostride);
    return hipGetLastError();
}

/* CPU BASELINE KERNELS: test and benchmark infrastructure only (bench.py's cpu_baseline leg).
 *
 * A fused int4 GEMV / small-M GEMM on the host CPU, this build's own code in the style of the
 * reference's host int8 GEMV (llama/ggml-opennpu/onpu_cpu.cpp:276-299: one row per iteration,
 * split over a thread pool, AVX-512 FMAs into fp32 lanes, one horizontal sum per row): the honest
 * CPU-bandwidth comparison for the GPU kernels. Nothing in the product calls it.
 *
 *   g128s:  y[m][n] = sum_g s[n][g] * (sum_{k in g} u[n][k] x[m][k] - 8 sum_{k in g} x[m][k])
 *           codes u8 [N][K/2] (low nibble = even k), bf16 scales [N][K/128], x fp32 [M][K]
 *   Q4_0:   GGUF blocks of 32 (fp16 d, 16 bytes: element j = low nibble of byte j, j + 16 = high
 *           nibble), w = (q - 8) d; y as above with one scale per 32
 *
 * x is split once per call into even / odd k (g128s) so that a 64-byte group of codes multiplies
 * contiguous x; per group each row takes 8 FMAs of 16 lanes and one scaling FMA; the group sums of
 * x carry the -8 of the symmetric zero point. AVX-512 when the CPU has it (chosen at run time),
 * else AVX2, else scalar. Rows of W are split over OpenMP threads.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bf16f(uint16_t h) {
    uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float f16f(uint16_t h) {
    const uint32_t s = (uint32_t) (h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = s;
        else {                                  /* subnormal */
            float f = (float) m * (1.0f / 16777216.0f);
            return s ? -f : f;
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------ g128s */
__attribute__((target("avx512f,avx512bw"))) static void g128_rows_avx512(
    const uint8_t * codes, const uint16_t * sc, int64_t n0, int64_t n1, int64_t K, const float * xe,
    const float * xo, const float * gs, int M, float * y, int64_t N) {
    const int64_t G = K / 128;
    const __m512i m4 = _mm512_set1_epi8(0x0f);
    for (int64_t n = n0; n < n1; n++) {
        __m512 acc[8];
        float corr[8];
        for (int m = 0; m < M; m++) { acc[m] = _mm512_setzero_ps(); corr[m] = 0.f; }
        const uint8_t * c = codes + n * (K / 2);
        for (int64_t g = 0; g < G; g++) {
            const __m512i b = _mm512_loadu_si512((const void *) (c + 64 * g));
            const __m512i lo = _mm512_and_si512(b, m4), hi = _mm512_and_si512(_mm512_srli_epi16(b, 4), m4);
            __m512 ul[4], uh[4];
            for (int i = 0; i < 4; i++) {
                ul[i] = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm512_extracti32x4_epi32(lo, i)));
                uh[i] = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm512_extracti32x4_epi32(hi, i)));
            }
            const float s = bf16f(sc[n * G + g]);
            const __m512 sv = _mm512_set1_ps(s);
            for (int m = 0; m < M; m++) {
                const float * pe = xe + (int64_t) m * (K / 2) + 64 * g, * po = xo + (int64_t) m * (K / 2) + 64 * g;
                __m512 t = _mm512_mul_ps(ul[0], _mm512_loadu_ps(pe));
                t = _mm512_fmadd_ps(uh[0], _mm512_loadu_ps(po), t);
                for (int i = 1; i < 4; i++) {
                    t = _mm512_fmadd_ps(ul[i], _mm512_loadu_ps(pe + 16 * i), t);
                    t = _mm512_fmadd_ps(uh[i], _mm512_loadu_ps(po + 16 * i), t);
                }
                acc[m] = _mm512_fmadd_ps(sv, t, acc[m]);
                corr[m] += s * gs[(int64_t) m * G + g];
            }
        }
        for (int m = 0; m < M; m++) y[(int64_t) m * N + n] = _mm512_reduce_add_ps(acc[m]) - 8.0f * corr[m];
    }
}

__attribute__((target("avx2,fma"))) static void g128_rows_avx2(const uint8_t * codes, const uint16_t * sc,
                                                              int64_t n0, int64_t n1, int64_t K, const float * xe,
                                                              const float * xo, const float * gs, int M, float * y,
                                                              int64_t N) {
    const int64_t G = K / 128;
    for (int64_t n = n0; n < n1; n++) {
        __m256 acc[8];
        float corr[8];
        for (int m = 0; m < M; m++) { acc[m] = _mm256_setzero_ps(); corr[m] = 0.f; }
        const uint8_t * c = codes + n * (K / 2);
        for (int64_t g = 0; g < G; g++) {
            const float s = bf16f(sc[n * G + g]);
            const __m256 sv = _mm256_set1_ps(s);
            __m256 t[8];
            for (int m = 0; m < M; m++) t[m] = _mm256_setzero_ps();
            for (int i = 0; i < 8; i++) {               /* 8 bytes = 16 codes per step */
                const __m128i b = _mm_loadl_epi64((const __m128i *) (c + 64 * g + 8 * i));
                const __m128i lo = _mm_and_si128(b, _mm_set1_epi8(0x0f));
                const __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), _mm_set1_epi8(0x0f));
                const __m256 ul = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(lo));
                const __m256 uh = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(hi));
                for (int m = 0; m < M; m++) {
                    const int64_t o = (int64_t) m * (K / 2) + 64 * g + 8 * i;
                    t[m] = _mm256_fmadd_ps(ul, _mm256_loadu_ps(xe + o), t[m]);
                    t[m] = _mm256_fmadd_ps(uh, _mm256_loadu_ps(xo + o), t[m]);
                }
            }
            for (int m = 0; m < M; m++) {
                acc[m] = _mm256_fmadd_ps(sv, t[m], acc[m]);
                corr[m] += s * gs[(int64_t) m * G + g];
            }
        }
        for (int m = 0; m < M; m++) {
            float v[8];
            _mm256_storeu_ps(v, acc[m]);
            float r = 0.f;
            for (int i = 0; i < 8; i++) r += v[i];
            y[(int64_t) m * N + n] = r - 8.0f * corr[m];
        }
    }
}

static void g128_rows_scalar(const uint8_t * codes, const uint16_t * sc, int64_t n0, int64_t n1, int64_t K,
                             const float * xe, const float * xo, const float * gs, int M, float * y, int64_t N) {
    const int64_t G = K / 128;
    for (int64_t n = n0; n < n1; n++)
        for (int m = 0; m < M; m++) {
            float r = 0.f;
            for (int64_t g = 0; g < G; g++) {
                float t = 0.f;
                for (int j = 0; j < 64; j++) {
                    const uint8_t b = codes[n * (K / 2) + 64 * g + j];
                    t += (float) (b & 15) * xe[(int64_t) m * (K / 2) + 64 * g + j] +
                         (float) (b >> 4) * xo[(int64_t) m * (K / 2) + 64 * g + j];
                }
                r += bf16f(sc[n * G + g]) * (t - 8.0f * gs[(int64_t) m * G + g]);
            }
            y[(int64_t) m * N + n] = r;
        }
}

/* y [M][N] = x [M][K] . W^T for g128s W (staging layout: codes then scales); M <= 8. isa_max caps
 * the instruction set (2 AVX-512, 1 AVX2, 0 scalar; the best the CPU has below it is used). Returns
 * the instruction set used, -1 on bad arguments. */
int cpu_g128s_mv(const uint8_t * st, int64_t N, int64_t K, const float * x, int M, float * y, int threads,
                 int isa_max) {
    if (K % 128 || M < 1 || M > 8 || N < 1) return -1;
    const uint8_t * codes = st;
    const uint16_t * sc = (const uint16_t *) (st + N * K / 2);
    const int64_t G = K / 128, H = K / 2;
    float * xe = (float *) malloc(sizeof(float) * (size_t) (M * H));
    float * xo = (float *) malloc(sizeof(float) * (size_t) (M * H));
    float * gs = (float *) malloc(sizeof(float) * (size_t) (M * G));
    for (int m = 0; m < M; m++) {
        for (int64_t j = 0; j < H; j++) {
            xe[m * H + j] = x[(int64_t) m * K + 2 * j];
            xo[m * H + j] = x[(int64_t) m * K + 2 * j + 1];
        }
        for (int64_t g = 0; g < G; g++) {
            float t = 0.f;
            for (int j = 0; j < 128; j++) t += x[(int64_t) m * K + 128 * g + j];
            gs[m * G + g] = t;
        }
    }
    int isa = __builtin_cpu_supports("avx512bw") ? 2 : (__builtin_cpu_supports("avx2") ? 1 : 0);
    if (isa > isa_max) isa = isa_max;
    const int64_t chunk = 64;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int64_t n0 = 0; n0 < N; n0 += chunk) {
        const int64_t n1 = n0 + chunk < N ? n0 + chunk : N;
        if (isa == 2) g128_rows_avx512(codes, sc, n0, n1, K, xe, xo, gs, M, y, N);
        else if (isa == 1) g128_rows_avx2(codes, sc, n0, n1, K, xe, xo, gs, M, y, N);
        else g128_rows_scalar(codes, sc, n0, n1, K, xe, xo, gs, M, y, N);
    }
    free(xe);
    free(xo);
    free(gs);
    return isa;
}

/* ------------------------------------------------------------------ GGUF Q4_0 */
__attribute__((target("avx512f,avx512bw"))) static void q40_rows_avx512(const uint8_t * st, int64_t n0, int64_t n1,
                                                                        int64_t K, const float * x,
                                                                        const float * bs, int M, float * y, int64_t N) {
    const int64_t B = K / 32;
    const __m128i m4 = _mm_set1_epi8(0x0f);
    for (int64_t n = n0; n < n1; n++) {
        __m512 acc[8];
        float corr[8];
        for (int m = 0; m < M; m++) { acc[m] = _mm512_setzero_ps(); corr[m] = 0.f; }
        for (int64_t b = 0; b < B; b++) {
            const uint8_t * blk = st + (n * B + b) * 18;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            const float d = f16f(dh);
            const __m128i q = _mm_loadu_si128((const __m128i *) (blk + 2));
            const __m512 ul = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm_and_si128(q, m4)));
            const __m512 uh = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm_and_si128(_mm_srli_epi16(q, 4), m4)));
            const __m512 dv = _mm512_set1_ps(d);
            for (int m = 0; m < M; m++) {
                const float * px = x + (int64_t) m * K + 32 * b;
                const __m512 t = _mm512_fmadd_ps(uh, _mm512_loadu_ps(px + 16), _mm512_mul_ps(ul, _mm512_loadu_ps(px)));
                acc[m] = _mm512_fmadd_ps(dv, t, acc[m]);
                corr[m] += d * bs[(int64_t) m * B + b];
            }
        }
        for (int m = 0; m < M; m++) y[(int64_t) m * N + n] = _mm512_reduce_add_ps(acc[m]) - 8.0f * corr[m];
    }
}

static void q40_rows_scalar(const uint8_t * st, int64_t n0, int64_t n1, int64_t K, const float * x, const float * bs,
                            int M, float * y, int64_t N) {
    const int64_t B = K / 32;
    for (int64_t n = n0; n < n1; n++)
        for (int m = 0; m < M; m++) {
            float r = 0.f;
            for (int64_t b = 0; b < B; b++) {
                const uint8_t * blk = st + (n * B + b) * 18;
                uint16_t dh;
                memcpy(&dh, blk, 2);
                float t = 0.f;
                for (int j = 0; j < 16; j++)
                    t += (float) (blk[2 + j] & 15) * x[(int64_t) m * K + 32 * b + j] +
                         (float) (blk[2 + j] >> 4) * x[(int64_t) m * K + 32 * b + 16 + j];
                r += f16f(dh) * (t - 8.0f * bs[(int64_t) m * B + b]);
            }
            y[(int64_t) m * N + n] = r;
        }
}

/* y [M][N] = x [M][K] . W^T for GGUF Q4_0 rows; M <= 8; isa_max as above. Returns 2 (AVX-512),
 * 0 (scalar) or -1. */
int cpu_q4_0_mv(const uint8_t * st, int64_t N, int64_t K, const float * x, int M, float * y, int threads,
                int isa_max) {
    if (K % 32 || M < 1 || M > 8 || N < 1) return -1;
    const int64_t B = K / 32;
    float * bs = (float *) malloc(sizeof(float) * (size_t) (M * B));
    for (int m = 0; m < M; m++)
        for (int64_t b = 0; b < B; b++) {
            float t = 0.f;
            for (int j = 0; j < 32; j++) t += x[(int64_t) m * K + 32 * b + j];
            bs[m * B + b] = t;
        }
    int isa = __builtin_cpu_supports("avx512bw") ? 2 : 0;
    if (isa > isa_max) isa = isa_max < 2 ? 0 : 2;
    const int64_t chunk = 256;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int64_t n0 = 0; n0 < N; n0 += chunk) {
        const int64_t n1 = n0 + chunk < N ? n0 + chunk : N;
        if (isa == 2) q40_rows_avx512(st, n0, n1, K, x, bs, M, y, N);
        else q40_rows_scalar(st, n0, n1, K, x, bs, M, y, N);
    }
    free(bs);
    return isa;
}

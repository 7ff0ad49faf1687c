// Format-independent kernels of libonpu_hip (router, MoE permutation and combine, argmax, input
// conversion, the host-API MoE helpers) and the launchers that dispatch the per-format ones.
#include "onpu_kern.h"

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
    switch (fmt) {
        case 0: return repack_f0(st, sstride, N, K, g.KB, g.NT, out, ostride, E, s);
        case 1: return repack_f1(st, sstride, N, K, g.KB, g.NT, out, ostride, E, s);
        case 2: return repack_f2(st, sstride, N, K, g.KB, g.NT, out, ostride, E, s);
        case 3: return repack_f3(st, sstride, N, K, g.KB, g.NT, out, ostride, E, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_dequant(int fmt, const uint8_t * W, int64_t N, int64_t K, void * out, int bf16, hipStream_t s) {
    const Tiled g = tiled_geom(fmt, N, K);
    switch (fmt) {
        case 0: return dequant_f0(W, N, K, g.KB, g.NT, out, bf16, s);
        case 1: return dequant_f1(W, N, K, g.KB, g.NT, out, bf16, s);
        case 2: return dequant_f2(W, N, K, g.KB, g.NT, out, bf16, s);
        case 3: return dequant_f3(W, N, K, g.KB, g.NT, out, bf16, s);
    }
    return hipErrorInvalidValue;
}

int qgemv_has_variant(int epi, int mb, int rt, int nb, int xl) {
#define X(e_, mb_, rt_, nb_, xl_) if (epi == e_ && mb == mb_ && rt == rt_ && nb == nb_ && xl == xl_) return 1;
    ONPU_QGEMV_VARIANTS(X)
#undef X
    return 0;
}

int qgemv_max_waves(int mb, int rt, int nb, int xl) { return qgemv_lb(mb, rt, nb, xl) / 64; }

// LDS per workgroup: the reduction buffer plus, with xl, the staged x rows and their column sums
// (<= 64 KiB together)
hipError_t launch_qgemv(int fmt, int epi, const QArgs & a, int mb, int rt, int nb, int xl, dim3 grid, int waves,
                        hipStream_t s) {
    if (waves < 1 || waves > qgemv_max_waves(mb, rt, nb, xl) || !qgemv_has_variant(epi, mb, rt, nb, xl))
        return hipErrorInvalidValue;
    const size_t red = (size_t) waves * rt * mb * 1024;
    // x rows, then the column sums [KB * groups per block][16] floats
    const size_t xb = xl ? (size_t) a.M * a.xls * 2 + (size_t) a.KB * (fmt == 2 ? 1 : 4) * 64 : 0;
    if (xl && a.M > 16) return hipErrorInvalidValue;
    if (red > 32768 || red + xb > 65536) return hipErrorInvalidValue;
    if (xl && a.xls < a.KB * 128) return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return qgemv_f0(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
        case 1: return qgemv_f1(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
        case 2: return qgemv_f2(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
        case 3: return qgemv_f3(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_qgemm(int fmt, const GArgs & a, int ntw, hipStream_t s) {
    switch (fmt) {
        case 0: return qgemm_f0(a, ntw, s);
        case 1: return qgemm_f1(a, ntw, s);
        case 2: return qgemm_f2(a, ntw, s);
        case 3: return qgemm_f3(a, ntw, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_moe_grouped(int fmt, int which, const MArgs & a, int mb, dim3 grid, int waves, hipStream_t s) {
    if ((size_t) waves * (which == 0 ? 2 : 1) * mb * 1024 > 32768) return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return moe_f0(which, a, mb, grid, waves, s);
        case 1: return moe_f1(which, a, mb, grid, waves, s);
        case 2: return moe_f2(which, a, mb, grid, waves, s);
        case 3: return moe_f3(which, a, mb, grid, waves, s);
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

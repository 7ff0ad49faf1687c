// Format-independent kernels of libonpu_hip (router, MoE permutation and combine, argmax, input
// conversion, the host-API MoE helpers) and the launchers that dispatch the per-format ones.
#include <mutex>

#include "onpu_kern.h"

// one wave per token: softmax over E <= 256 logits, top-k by probability (ties to the lower id),
// renormalised (moe_runtime.py:333-341).
__global__ __launch_bounds__(64) void k_route(const float * __restrict__ logits, int64_t T, int E, int k, int renorm,
                                              int32_t * __restrict__ ids, float * __restrict__ w) {
    const int64_t t = blockIdx.x;
    int my_id;
    float my_w;
    route_token(logits + t * E, E, k, renorm, my_id, my_w);
    if ((int) threadIdx.x < k) {
        ids[t * k + threadIdx.x] = my_id;
        w[t * k + threadIdx.x] = my_w;
    }
}

// ------------------------------------------------------------------ MoE permutation
// One workgroup. entries i = t * k + j (T * k of them) sorted by expert:
//   cnt[e], off[e] (exclusive scan, off[E] = total), perm[off[e] + rank] = i and inv[i] = its position,
//   work list of (expert, first position, rows <= rows_per_item) items -> items[], nitems
// Items are listed by A blocks (ceil(rows / 16), rows_per_item <= 64), most first: the grouped GEMMs
// take one item per grid row, so the longest items are dispatched first and the short ones fill
// the end of the launch. (The order changes no result: every item's rows are computed alone.)
__global__ __launch_bounds__(1024) void k_moe_permute(const int32_t * __restrict__ ids, int64_t n, int E,
                                                      int rows_per_item, int32_t * __restrict__ off,
                                                      int32_t * __restrict__ perm, int32_t * __restrict__ inv,
                                                      int32_t * __restrict__ items, int32_t * __restrict__ nitems) {
    extern __shared__ __align__(16) int32_t sh[];
    int32_t * cnt = sh;              // [E]
    int32_t * pos = sh + E;          // [E + 1]
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) atomicAdd(&cnt[ids[i]], 1);
    __syncthreads();
    if (threadIdx.x < 64) {
        // wave 0: lane l owns experts [l * EP, (l + 1) * EP); exclusive scans of rows and of items
        // per class c = A blocks - 1 (classes listed from 3 down to 0)
        const int lane = threadIdx.x, EP = (E + 63) / 64, e0 = lane * EP, e1 = e0 + EP < E ? e0 + EP : E;
        auto cls = [](int32_t rows) { return (rows + 15) / 16 - 1; };
        int32_t rs = 0, is[4] = {0, 0, 0, 0};
        for (int e = e0; e < e1; e++) {
            rs += cnt[e];
            for (int32_t r0 = 0; r0 < cnt[e]; r0 += rows_per_item)
                is[cls(cnt[e] - r0 < rows_per_item ? cnt[e] - r0 : rows_per_item)]++;
        }
        int32_t ri = rs, ii[4] = {is[0], is[1], is[2], is[3]};     // inclusive scans across lanes
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t a = __shfl_up(ri, o);
            int32_t b[4];
            for (int c = 0; c < 4; c++) b[c] = __shfl_up(ii[c], o);
            if (lane >= o) {
                ri += a;
                for (int c = 0; c < 4; c++) ii[c] += b[c];
            }
        }
        int32_t tot[4], it[4];
        for (int c = 0; c < 4; c++) tot[c] = __shfl(ii[c], 63);
        for (int c = 3, base = 0; c >= 0; base += tot[c], c--) it[c] = base + ii[c] - is[c];
        int32_t s = ri - rs;                          // exclusive: this lane's first row
        for (int e = e0; e < e1; e++) {
            pos[e] = s;
            off[e] = s;
            for (int32_t r0 = 0; r0 < cnt[e]; r0 += rows_per_item) {
                const int32_t rows = cnt[e] - r0 < rows_per_item ? cnt[e] - r0 : rows_per_item;
                const int c = cls(rows);
                items[3 * it[c]] = e;
                items[3 * it[c] + 1] = s + r0;
                items[3 * it[c] + 2] = rows;
                it[c]++;
            }
            s += cnt[e];
        }
        if (lane == 63) {
            off[E] = ri;
            *nitems = tot[0] + tot[1] + tot[2] + tot[3];
        }
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const int32_t p = atomicAdd(&pos[ids[i]], 1);
        perm[p] = (int32_t) i;
        inv[i] = p;
    }
}

// combine: y[t][n] = sum_j w[t][j] * o[inv[t * k + j]][n]; inv = inverse permutation (position of entry)
__global__ __launch_bounds__(256) void k_moe_combine(const uint16_t * __restrict__ o, const int32_t * __restrict__ inv,
                                                     const float * __restrict__ w, int64_t T, int k, int64_t N,
                                                     void * __restrict__ y, int yf32) {
    // token blockIdx.y, 8 consecutive outputs per thread: a 16-byte load of each of the k rows
    const int64_t t = blockIdx.y;
    const int64_t n0 = 8 * ((int64_t) blockIdx.x * blockDim.x + threadIdx.x);
    if (n0 >= N) return;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (N % 8 == 0) {
        for (int j = 0; j < k; j++) {
            const float wj = w[t * k + j];
            const uint4 v = *(const uint4 *) (o + (int64_t) inv[t * k + j] * N + n0);
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
            for (int i = 0; i < 4; i++) {
                s[2 * i] += wj * __uint_as_float(d[i] << 16);
                s[2 * i + 1] += wj * __uint_as_float(d[i] & 0xffff0000u);
            }
        }
    } else {
        for (int j = 0; j < k; j++) {
            const float wj = w[t * k + j];
            const uint16_t * row = o + (int64_t) inv[t * k + j] * N;
            for (int i = 0; i < 8 && n0 + i < N; i++) s[i] += wj * bf16_to_f32(row[n0 + i]);
        }
    }
    for (int i = 0; i < 8 && n0 + i < N; i++) store_out(y, yf32, t * N + n0 + i, s[i]);
}

// ------------------------------------------------------------------ argmax
// first maximum of v[row][0..N) in one launch. Each of a row's gridDim.x workgroups reduces
// ARGMAX_CHUNK values (a thread issues all of its loads before its first compare) to one key: the
// value's order-preserving bits above the complement of the index, so the larger key is the larger
// value and, among equal values, the lower index. A NaN key has the top value bits, so a row with a
// NaN gives its first NaN's index (numpy's and torch's argmax rule). The workgroup publishes its key and counts in on the row's
// counter; the one that arrives last reduces the row's keys, writes the index and puts the counter
// back to zero, so the counters are zero between calls with no clearing step (graph replays too).
// Keys and counters sit ARGMAX_PAD bytes apart: atomics of different workgroups on one cache line
// queue behind each other.
// workgroup maximum of the threads' keys; the result is valid in thread 0
DEV uint64_t block_umax64(uint64_t k, uint64_t * wk) {
    k = wave_umax64(k);
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < ARGMAX_THREADS / 64; w++) k = wk[w] > k ? wk[w] : k;
    return k;
}

__global__ __launch_bounds__(ARGMAX_THREADS) void k_argmax(const float * __restrict__ v, int64_t N,
                                                           uint64_t * __restrict__ keys, uint32_t * __restrict__ cnt,
                                                           int32_t * __restrict__ out) {
    constexpr int PT = ARGMAX_CHUNK / ARGMAX_THREADS, KS = ARGMAX_PAD / 8, CS = ARGMAX_PAD / 4;
    const int64_t row = blockIdx.y;
    const uint32_t P = gridDim.x;
    const float * x = v + row * N;
    const int64_t n0 = (int64_t) blockIdx.x * ARGMAX_CHUNK + threadIdx.x;
    float val[PT];
#pragma unroll
    for (int j = 0; j < PT; j++) {
        const int64_t n = n0 + (int64_t) j * ARGMAX_THREADS;
        val[j] = n < N ? x[n] : 0.f;
    }
    uint64_t k = 0;                                     // below every key of a value in range
#pragma unroll
    for (int j = 0; j < PT; j++) {
        const int64_t n = n0 + (int64_t) j * ARGMAX_THREADS;
        const uint64_t kj = n < N ? argmax_key(val[j], n) : 0;
        k = kj > k ? kj : k;
    }
    __shared__ uint64_t wk[ARGMAX_THREADS / 64];
    __shared__ uint32_t last;
    k = block_umax64(k, wk);
    if (threadIdx.x == 0) {
        // the release orders the key before the count; the acquire of the last arrival orders the
        // other workgroups' keys before its reads
        __hip_atomic_store(keys + (row * P + blockIdx.x) * KS, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = __hip_atomic_fetch_add(cnt + row * CS, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == P - 1;
    }
    __syncthreads();
    if (!last) return;
    uint64_t r = 0;
    for (uint32_t p = threadIdx.x; p < P; p += ARGMAX_THREADS) {
        const uint64_t kp = __hip_atomic_load(keys + (row * P + p) * KS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        r = kp > r ? kp : r;
    }
    __syncthreads();                                    // wk is reused
    r = block_umax64(r, wk);
    if (threadIdx.x == 0) {
        out[row] = (int32_t) (0xffffffffu - (uint32_t) r);
        __hip_atomic_store(cnt + row * CS, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// the first maximum of each row from the LM-head GEMV's keys (one per workgroup, [row][P]); the key
// order is the value order with ties to the lower index, as in k_argmax
// A thread issues its (up to) 4 loads of a pass before comparing, so a row of up to 4096 keys costs
// one memory round trip.
constexpr int AKEY_THREADS = 1024, AKEY_U = 4;
__global__ __launch_bounds__(AKEY_THREADS) void k_argmax_keys(const uint64_t * __restrict__ keys, int64_t P,
                                                              int32_t * __restrict__ out) {
    const int64_t row = blockIdx.x;
    const uint64_t * kr = keys + row * P;
    uint64_t k = 0;
    for (int64_t p0 = 0; p0 < P; p0 += AKEY_THREADS * AKEY_U) {
        uint64_t v[AKEY_U];
#pragma unroll
        for (int u = 0; u < AKEY_U; u++) {
            const int64_t p = p0 + u * AKEY_THREADS + threadIdx.x;
            v[u] = p < P ? kr[p] : 0;
        }
#pragma unroll
        for (int u = 0; u < AKEY_U; u++) k = v[u] > k ? v[u] : k;
    }
    __shared__ uint64_t wk[AKEY_THREADS / 64];
    k = wave_umax64(k);
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x < 64) {
        k = threadIdx.x < AKEY_THREADS / 64 ? wk[threadIdx.x] : 0;
        k = wave_umax64(k);
        if (threadIdx.x == 0) out[row] = (int32_t) (0xffffffffu - (uint32_t) k);
    }
}

// ------------------------------------------------------------------ int8 GEMV
// y[n] = s[n] * sum_k W[n][k] x[k] for int8 W [N][K] (the reference's host onpu_gemv_i8,
// onpu_cpu.cpp:276-299, for a MoE's shared expert). Rows go in groups of 4; a group's K range is
// split into ks slices (4 below 8192 groups, then 2, then 1), one wave per (group,
// slice), 4 / ks groups per workgroup. In a wave a row is read by 16 consecutive lanes, 16 bytes
// each (a wave instruction covers the 4 rows, 1 KiB), GI8_U loads per lane in flight per batch.
// x sits in LDS (copied once per workgroup with its sum); the four rows' lanes read the same x (a
// broadcast). The bytes are biased to u = w + 128 by one xor per dword and converted by
// v_cvt_f32_ubyteN, so a weight costs a convert and an fma, and 128 sum(x) is subtracted once.
// The 16 lanes of a row sum by DPP, the slices in LDS.
constexpr int GI8_T = 256, GI8_U = 8;

template <int CTRL> DEV float dpp_fl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__global__ __launch_bounds__(GI8_T) void k_gemv_i8(const int8_t * __restrict__ W, const float * __restrict__ s,
                                                   int64_t N, int64_t K, int ks, int64_t Kw,
                                                   const float * __restrict__ x, float * __restrict__ y) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float wsx[GI8_T / 64];
    __shared__ float red[GI8_T / 64][4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, li = lane & 15, slot = lane >> 4;
    // x to LDS: all of a thread's loads of a batch issued before the stores (8 x 1024 floats per
    // batch). Buffer loads over x's K floats (the host keeps K * 4 < 2^31): past K they return
    // zeros, so the loads need no branch (a load under a branch is waited for where the branch
    // rejoins, which would serialize the batch).
    float part = 0.f;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *) x, (short) 0, (int) (K * 4), 0x00020000);
    for (int64_t k0 = 4 * t; k0 < K; k0 += 8 * 4 * GI8_T) {
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int64_t k = k0 + (int64_t) i * 4 * GI8_T;
            v[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t) (k * 4), 0, 0));
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int64_t k = k0 + (int64_t) i * 4 * GI8_T;
            if (k < K) *(float4 *) (xs + k) = v[i];
            part += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        }
    }
    for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
    if (lane == 0) wsx[wave] = part;
    __syncthreads();
    const float xsum = (wsx[0] + wsx[1]) + (wsx[2] + wsx[3]);
    const int gpw = 4 / ks;
    const int64_t grp = (int64_t) blockIdx.x * gpw + wave / ks, row = grp * 4 + slot;
    const int64_t k0 = (wave % ks) * Kw, k1 = k0 + Kw < K ? k0 + Kw : K;
    const int8_t * wr = W + (row < N ? row : 0) * K;
    float acc = 0.f;
    // all GI8_U loads of a step unconditional: past k1 a lane re-reads its own first 16 bytes of
    // the step (never used: the products below stop at k1)
    for (int64_t kb = k0 + 16 * li; kb < k1; kb += 256 * GI8_U) {
        uint4 q[GI8_U];
#pragma unroll
        for (int u = 0; u < GI8_U; u++) {
            const int64_t k = kb + 256 * u;
            q[u] = *(const uint4 *) (wr + (k < k1 ? k : kb));
        }
#pragma unroll
        for (int u = 0; u < GI8_U; u++) {
            const int64_t k = kb + 256 * u;
            if (k >= k1) break;
            const uint32_t d[4] = {q[u].x ^ 0x80808080u, q[u].y ^ 0x80808080u, q[u].z ^ 0x80808080u,
                                   q[u].w ^ 0x80808080u};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 xv = *(const float4 *) (xs + k + 4 * i);
                acc += (float) (d[i] & 0xffu) * xv.x;
                acc += (float) ((d[i] >> 8) & 0xffu) * xv.y;
                acc += (float) ((d[i] >> 16) & 0xffu) * xv.z;
                acc += (float) (d[i] >> 24) * xv.w;
            }
        }
    }
    acc += dpp_fl<0xB1>(acc);               // quad_perm [1, 0, 3, 2]
    acc += dpp_fl<0x4E>(acc);               // quad_perm [2, 3, 0, 1]
    acc += dpp_fl<0x141>(acc);              // row_half_mirror
    acc += dpp_fl<0x140>(acc);              // row_mirror
    if (ks == 1) {
        if (li == 0 && row < N) y[row] = (acc - 128.0f * xsum) * s[row];
        return;
    }
    if (li == 0) red[wave][slot] = acc;
    __syncthreads();
    if (t < 4 * gpw) {
        const int gl = t / 4;
        const int64_t r = ((int64_t) blockIdx.x * gpw + gl) * 4 + (t & 3);
        float sum = 0.f;
        for (int sl = 0; sl < ks; sl++) sum += red[gl * ks + sl][t & 3];
        if (r < N) y[r] = (sum - 128.0f * xsum) * s[r];
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
// (<= 160 KiB together)
hipError_t launch_qgemv(int fmt, int epi, const QArgs & a, int mb, int rt, int nb, int xl, dim3 grid, int waves,
                        hipStream_t s) {
    if (waves < 1 || waves > qgemv_max_waves(mb, rt, nb, xl) || !qgemv_has_variant(epi, mb, rt, nb, xl))
        return hipErrorInvalidValue;
    const size_t red = (size_t) waves * rt * mb * 1024;
    // x rows, then the column sums [KB * groups per block][16] floats (not with xl = 2 up to 8 rows,
    // which sums on the MFMAs)
    const bool sums = xl == 1 || (xl == 2 && a.M > 8);
    const size_t xb = xl ? (size_t) a.M * a.xls * 2 + (sums ? (size_t) a.KB * (fmt == 2 ? 1 : 4) * 64 : 0) : 0;
    if (xl && (a.M > 16 || (int64_t) a.M * a.ldx * 2 >= ((int64_t) 1 << 31))) return hipErrorInvalidValue;
    // gfx950: 160 KiB per workgroup (the argmax epilogue's row keys take 1 KiB of static LDS)
    if (red > 32768 || red + xb + (epi == EPI_ARGMAX_ ? 1024 : 0) > 163840) return hipErrorInvalidValue;
    if (xl && a.xls < a.KB * 128) return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return qgemv_f0(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
        case 1: return qgemv_f1(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
        case 2: return qgemv_f2(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
        case 3: return qgemv_f3(epi, a, mb, rt, nb, xl, grid, waves, red + xb, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_qgemm(int fmt, const GArgs & a, int ntw, int mb, hipStream_t s) {
    if (!(mb == 8 && ntw >= 2 && ntw <= 4) && !((mb == 1 || mb == 2 || mb == 4) && ntw == 2)) return hipErrorInvalidValue;
    // argmax keys: tiles of at most 64 rows that hold every row, no split, fp32 logits
    if (a.akeys && (mb == 8 || a.M > 16 * mb || a.splits > 1 || !a.yf32)) return hipErrorInvalidValue;
    // split-K: every split holds at least one K block, the splits cover all KB, the grid fits 32 bits
    if (a.splits > 1 && (!a.ws || a.kbs < 1 || (a.splits - 1) * a.kbs >= a.KB || a.splits * a.kbs < a.KB ||
                         ((a.M + 16 * mb - 1) / (16 * mb)) * ((a.NT + 4 * ntw - 1) / (4 * ntw)) * a.splits >=
                             ((int64_t) 1 << 31)))
        return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return qgemm_f0(a, ntw, mb, s);
        case 1: return qgemm_f1(a, ntw, mb, s);
        case 2: return qgemm_f2(a, ntw, mb, s);
        case 3: return qgemm_f3(a, ntw, mb, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_qgemm_sk(int fmt, const GArgs & a, int cfg, int grid, hipStream_t s) {
    if (cfg != 0 || grid <= 0 || a.ipw <= 0 || !a.ws || !a.sync || !a.ctl) return hipErrorInvalidValue;
    if (a.sched == 1 && (a.R < 0 || a.R > grid || (a.R > 0 && (a.c <= 0 || a.s <= 0 || a.s >= a.KB))))
        return hipErrorInvalidValue;
    if (a.M * a.ldx * 2 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;     // 32-bit X offsets
    if (256 * a.ldy * 4 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;     // 32-bit Y offsets per tile
    switch (fmt) {
        case 0: return qgemm_sk_f0(a, cfg, grid, s);
        case 1: return qgemm_sk_f1(a, cfg, grid, s);
        case 2: return qgemm_sk_f2(a, cfg, grid, s);
        case 3: return qgemm_sk_f3(a, cfg, grid, s);
    }
    return hipErrorInvalidValue;
}

bool moe_decode_fits(int64_t H, int64_t I, int64_t Nd, int64_t gKB, int64_t dKB, int T, int k, int E) {
    return T >= 1 && T <= MD_MAX_T && k >= 1 && k <= MD_MAX_K && E >= k && E <= 256 && I % 16 == 0 && I >= 16 &&
           Nd >= 1 && gKB >= 1 && (gKB + MD_WAVES - 1) / MD_WAVES <= MD_MAX_GB && dKB >= 1 && dKB <= MD_MAX_DB &&
           (H * 2) % 16 == 0;
}

hipError_t launch_moe_decode(int fmt, const MDArgs & a, int grid, hipStream_t s) {
    if (!moe_decode_fits(a.H, a.I, a.Nd, a.gKB, a.dKB, a.T, a.k, a.E) || grid <= 0 || !a.act || !a.sync)
        return hipErrorInvalidValue;
    if (a.gNT * 16 != 2 * a.I || a.npairs != (int64_t) a.T * a.k * (a.I / 16) || a.nunits != a.T * a.dNT)
        return hipErrorInvalidValue;
    const int gb = (int) ((a.gKB + MD_WAVES - 1) / MD_WAVES);
    const int GPB = fmt == ONPU_G128S ? 1 : 4;
    const int db = (gb == 2 && a.dKB <= 6) ? 6 : MD_MAX_DB;
    const size_t lds = (size_t) 2 * MD_MAX_T * MD_MAX_K * 4 + (size_t) a.T * a.gKB * 128 * 2 +
                       (size_t) ((a.T * a.gKB * GPB + 3) / 4 * 4) * 4 + (size_t) MD_WAVES * 2 * 64 * 4 +
                       (size_t) MD_WAVES * db * 128 * 2 + (size_t) MD_WAVES * db * GPB * 4;
    if (lds > 163840) return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return moe_decode_f0(a, gb, grid, lds, s);
        case 1: return moe_decode_f1(a, gb, grid, lds, s);
        case 2: return moe_decode_f2(a, gb, grid, lds, s);
        case 3: return moe_decode_f3(a, gb, grid, lds, s);
    }
    return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ MoE decode split along I
bool moe_dsplit_fits(int64_t H, int64_t I, int64_t Nd, int64_t gKB, int T, int k, int E) {
    const int64_t NTq = ((Nd + 15) / 16 + 3) / 4;
    return T >= 1 && T <= DS_MAX_T && k >= 1 && k <= DS_MAX_K && k <= E && E <= 256 && I >= 32 && I % 32 == 0 &&
           H >= 8 && H % 8 == 0 && gKB >= 1 && (gKB + 1) / 2 <= 16 && Nd >= 1 && NTq <= 8 * 8;
}

hipError_t launch_moe_dsplit(int fmt, const MSArgs & a, int64_t Nd, int sv, hipStream_t s) {
    if (!moe_dsplit_fits(a.H, a.I, Nd, a.gKB, a.T, a.k, a.E) || (sv != 32 && sv != 16) || a.S != a.I / sv ||
        a.gNT * 16 != 2 * a.I ||
        a.dNTq != ((Nd + 15) / 16 + 3) / 4 || !a.part || (a.logits && (!a.ids || !a.w)) || (!a.logits && !a.ids))
        return hipErrorInvalidValue;
    // 16 waves where each then holds at most 8 blocks and 4 quads (measured against 8 on MI355X), else 8
    const char * ev = getenv("ONPU_DS_WAVES");
    int nw = ev && *ev ? atoi(ev) : 16;
    if (nw != 8 && ((a.gKB + 3) / 4 > 8 || (a.dNTq + 15) / 16 > 4)) nw = 8;
    const int GPB = fmt == ONPU_G128S ? 1 : 4;
    const size_t lds = (size_t) a.gKB * 128 * 2 + (size_t) ((a.gKB * GPB + 3) / 4 * 4) * 4 + (size_t) nw * 16 * 4 +
                       32 * 2 + 16;
    switch (fmt) {
        case 0: return moe_dsplit_f0(a, nw, sv, lds, s);
        case 1: return moe_dsplit_f1(a, nw, sv, lds, s);
        case 2: return moe_dsplit_f2(a, nw, sv, lds, s);
        case 3: return moe_dsplit_f3(a, nw, sv, lds, s);
    }
    return hipErrorInvalidValue;
}

constexpr int DS_SUM_MAX = 32;       // partials per lane in flight at once, at most (I <= 1024 in one round)
constexpr int DS_SUM_N = 16;         // outputs per workgroup of k_moe_dsum (64 B of each partial row)

// y[t][n] = sum_j w[t][j] (sum_s part[t k + j][s][n]), the sums in that order. grid (ceil(Nd / 16), T),
// 16 k threads: thread 16 j + c sums slot j's S partials of output 16 blockIdx.x + c (all its loads in
// flight at once, rounds of U with the index clamped to the last partial), then threads c < 16 weight
// and add the k slots. U is the smallest of 8, 16, 24 and 32 that holds S (larger S in rounds of
// 32): a clamped load is a wasted one (U = 32 at S = 24 took the Qwen3-30B-A3B layer 0.27 us more). Small workgroups spread the partials' reads over the GPU (one CU
// keeps only so many loads in flight); 16 outputs read 64 B pieces of each partial row (8 outputs
// fetched twice the bytes they used).
template <int U>
__global__ __launch_bounds__(DS_SUM_N * DS_MAX_K) void k_moe_dsum(const float * __restrict__ part, int64_t S,
                                                                        int64_t ld, const float * __restrict__ w, int k,
                                                                        int64_t Nd, void * y, int yf32) {
    __shared__ float sp[DS_MAX_K * DS_SUM_N];
    const int j = threadIdx.x / DS_SUM_N, c = threadIdx.x % DS_SUM_N;
    const int64_t t = blockIdx.y, n = (int64_t) blockIdx.x * DS_SUM_N + c;
    const float * p = part + (t * k + j) * S * ld + n;
    float acc = 0.f;
    for (int64_t s0 = 0; s0 < S; s0 += U) {
        float v[U];
#pragma unroll
        for (int i = 0; i < U; i++) v[i] = p[(s0 + i < S ? s0 + i : S - 1) * ld];
#pragma unroll
        for (int i = 0; i < U; i++)
            if (s0 + i < S) acc += v[i];
    }
    sp[j * DS_SUM_N + c] = acc;
    __syncthreads();
    if ((int) threadIdx.x < DS_SUM_N && n < Nd) {
        float v = 0.f;
        for (int i = 0; i < k; i++) v += w[t * k + i] * sp[i * DS_SUM_N + c];
        store_out(y, yf32, t * Nd + n, v);
    }
}

hipError_t launch_moe_dsum(const float * part, int64_t S, int64_t ld, const float * w, int64_t T, int k, int64_t Nd,
                           void * y, int yf32, hipStream_t s) {
    if (T < 1 || T > DS_MAX_T || k < 1 || k > DS_MAX_K || S < 1 || ld % 64 || Nd > ld) return hipErrorInvalidValue;
    const dim3 grid((unsigned) ((Nd + DS_SUM_N - 1) / DS_SUM_N), (unsigned) T);
    const unsigned th = (unsigned) (DS_SUM_N * k);
    if (S <= 8) k_moe_dsum<8><<<grid, th, 0, s>>>(part, S, ld, w, k, Nd, y, yf32);
    else if (S <= 16) k_moe_dsum<16><<<grid, th, 0, s>>>(part, S, ld, w, k, Nd, y, yf32);
    else if (S <= 24) k_moe_dsum<24><<<grid, th, 0, s>>>(part, S, ld, w, k, Nd, y, yf32);
    else k_moe_dsum<DS_SUM_MAX><<<grid, th, 0, s>>>(part, S, ld, w, k, Nd, y, yf32);
    return hipGetLastError();
}

hipError_t launch_relayout_dec(int fmt, const uint8_t * src, int64_t sstride, int64_t N, int64_t K, uint8_t * dst,
                               int64_t dstride, int64_t E, hipStream_t s) {
    const Tiled g = tiled_geom(fmt, N, K);
    if (E <= 0 || E > 65535 || dstride < dec_bytes(fmt, N, K)) return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return relayout_dec_f0(src, sstride, g.NT, g.KB, dst, dstride, E, s);
        case 1: return relayout_dec_f1(src, sstride, g.NT, g.KB, dst, dstride, E, s);
        case 2: return relayout_dec_f2(src, sstride, g.NT, g.KB, dst, dstride, E, s);
        case 3: return relayout_dec_f3(src, sstride, g.NT, g.KB, dst, dstride, E, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_moe_gemm(int fmt, int which, const MArgs & a, int64_t maxitems, hipStream_t s) {
    if (a.xbytes <= 0 || a.xbytes >= ((int64_t) 1 << 31) || maxitems <= 0 || maxitems > 65528) return hipErrorInvalidValue;
    if (which == 0 && (a.NT % 2 || a.N != 16 * a.NT)) return hipErrorInvalidValue;   // gate | up halves of whole tiles
    constexpr int wv = 8;                                   // k_moe_gemm: 8 waves x 2 weight tiles
    const int64_t gx = which == 0 ? (a.NT / 2 + wv - 1) / wv : (a.NT + 2 * wv - 1) / (2 * wv);
    const dim3 grid((unsigned) gx, (unsigned) ((maxitems + 7) / 8 * 8));   // item slots: whole XCD rounds
    switch (fmt) {
        case 0: return moe_gemm_f0(which, a, grid, s);
        case 1: return moe_gemm_f1(which, a, grid, s);
        case 2: return moe_gemm_f2(which, a, grid, s);
        case 3: return moe_gemm_f3(which, a, grid, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_chain(int fmt, int ring, const ChainArgs & a, const ChainEntry * ents, int grid, size_t lds,
                        hipStream_t s) {
    if (a.n <= 0 || a.M < 1 || a.M > 16 || grid < 1 || lds > 163840 || ring < 0 || ring > 3)
        return hipErrorInvalidValue;
    switch (fmt) {
        case 0: return chain_f0(ring, a, ents, grid, lds, s);
        case 1: return chain_f1(ring, a, ents, grid, lds, s);
        case 2: return chain_f2(ring, a, ents, grid, lds, s);
        case 3: return chain_f3(ring, a, ents, grid, lds, s);
    }
    return hipErrorInvalidValue;
}

int chain_occupancy(int fmt, int ring, size_t lds) {
    switch (fmt) {
        case 0: return chain_occ_f0(ring, lds);
        case 1: return chain_occ_f1(ring, lds);
        case 2: return chain_occ_f2(ring, lds);
        case 3: return chain_occ_f3(ring, lds);
    }
    return 0;
}

hipError_t launch_route(const float * logits, int64_t T, int E, int k, int renorm, int32_t * ids, float * w,
                        hipStream_t s) {
    if (E > 256 || k > 16 || k > E) return hipErrorInvalidValue;
    k_route<<<dim3((unsigned) T), 64, 0, s>>>(logits, T, E, k, renorm, ids, w);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_permute(const int32_t * ids, int64_t n, int E, int rows_per_item, int32_t * off, int32_t * perm,
                              int32_t * inv, int32_t * items, int32_t * nitems, hipStream_t s) {
    k_moe_permute<<<1, 1024, (size_t) (2 * E + 1) * sizeof(int32_t), s>>>(ids, n, E, rows_per_item, off, perm, inv,
                                                                          items, nitems);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_moe_combine(const uint16_t * o, const int32_t * inv, const float * w, int64_t T, int k, int64_t N,
                              void * y, int yf32, hipStream_t s) {
    dim3 grid((unsigned) ((N + 8 * 256 - 1) / (8 * 256)), (unsigned) T);
    k_moe_combine<<<grid, 256, 0, s>>>(o, inv, w, T, k, N, y, yf32);
    CHECK_LAUNCH();
    return hipSuccess;
}

__global__ void k_zero_i32(int32_t * p, int64_t n) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x)
        p[i] = 0;
}

hipError_t launch_zero_i32(int32_t * p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    k_zero_i32<<<(unsigned) std::min<int64_t>((n + 255) / 256, 1024), 256, 0, s>>>(p, n);
    CHECK_LAUNCH();
    return hipSuccess;
}

// split-K GEMM epilogue: four consecutive columns of a row per thread, the planes added in order
// (the same fp32 sum whatever the launch shape)
// U (>= S up to 16): a thread's first U planes are loaded at once, then added in plane order (one
// load in flight per thread left the launch at ~3.9 TB/s: too few bytes in flight for HBM)
template <int U>
__global__ __launch_bounds__(256) void k_gemm_split_sum(const float * __restrict__ part, int S, int64_t M, int64_t N,
                                                        void * __restrict__ y, int64_t ldy, int yf32) {
    const int64_t plane = M * N, nq = (N + 3) / 4;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < M * nq; i += (int64_t) gridDim.x * blockDim.x) {
        const int64_t m = i / nq, n0 = 4 * (i % nq);
        const float * p = part + m * N + n0;
        if (N % 4 == 0) {                                  // planes and rows 16-byte aligned
            f32x4 v[U];
#pragma unroll
            for (int s = 0; s < U; s++)
                if (s < S) v[s] = *(const f32x4 *) (p + s * plane);
            f32x4 acc = v[0];
#pragma unroll
            for (int s = 1; s < U; s++)
                if (s < S) acc += v[s];
            for (int s = U; s < S; s++) acc += *(const f32x4 *) (p + s * plane);
            for (int v = 0; v < 4; v++) store_out(y, yf32, m * ldy + n0 + v, acc[v]);
        } else {
            for (int v = 0; v < 4 && n0 + v < N; v++) {
                float acc = p[v];
                for (int s = 1; s < S; s++) acc += p[s * plane + v];
                store_out(y, yf32, m * ldy + n0 + v, acc);
            }
        }
    }
}

hipError_t launch_gemm_split_sum(const float * part, int S, int64_t M, int64_t N, void * y, int64_t ldy, int yf32,
                                 hipStream_t s) {
    if (S < 1 || M < 0 || N < 0 || ldy < N) return hipErrorInvalidValue;
    const int64_t n4 = M * ((N + 3) / 4);
    if (n4 == 0) return hipSuccess;
    const unsigned g = (unsigned) std::min<int64_t>((n4 + 255) / 256, 8192);
    if (S <= 2) k_gemm_split_sum<2><<<g, 256, 0, s>>>(part, S, M, N, y, ldy, yf32);
    else if (S <= 4) k_gemm_split_sum<4><<<g, 256, 0, s>>>(part, S, M, N, y, ldy, yf32);
    else if (S <= 8) k_gemm_split_sum<8><<<g, 256, 0, s>>>(part, S, M, N, y, ldy, yf32);
    else k_gemm_split_sum<16><<<g, 256, 0, s>>>(part, S, M, N, y, ldy, yf32);
    CHECK_LAUNCH();
    return hipSuccess;
}

int64_t argmax_parts(int64_t N) { return (N + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK; }

// The reference's NPU packing (onpu_common.h) -> the staging layout (q4nx, q4s). One workgroup per
// (packed row r, 512 columns) of expert blockIdx.y: thread j gathers the codes of columns 2j, 2j + 1
// into one staging byte, threads 0..15 the scale (and min) of the chunk's groups. Packed row r is
// staging row rowmap[r] (r without a map).
__global__ __launch_bounds__(256) void k_npu_stage(const uint8_t * __restrict__ src, int64_t sstride, NpuGeom g,
                                                   int sym, const int32_t * __restrict__ rowmap, int64_t N, int64_t K,
                                                   int64_t kch, uint8_t * __restrict__ dst, int64_t dstride) {
    const int64_t r = blockIdx.x / kch, c0 = (int64_t) (blockIdx.x % kch) * 512;
    const uint8_t * S = src + (int64_t) blockIdx.y * sstride;
    uint8_t * D = dst + (int64_t) blockIdx.y * dstride;
    const int64_t n = rowmap ? rowmap[r] : r;
    const int64_t k = c0 + 2 * (int64_t) threadIdx.x;
    if (k < K) {
        int s0, s1;
        const int64_t o0 = npu_code_byte(g, r, k, s0), o1 = npu_code_byte(g, r, k + 1, s1);
        D[n * (K / 2) + k / 2] = (uint8_t) (((S[o0] >> s0) & 15) | (((S[o1] >> s1) & 15) << 4));
    }
    const int64_t kg = c0 + 32 * (int64_t) threadIdx.x;
    if (threadIdx.x < 16 && kg < K) {
        const int64_t so = npu_scale_off(g, r, kg), G = K / 32;
        uint16_t * sc = (uint16_t *) (D + N * K / 2);
        sc[n * G + kg / 32] = (uint16_t) (S[so] | (S[so + 1] << 8));
        if (!sym) sc[N * G + n * G + kg / 32] = (uint16_t) (S[so + 1024] | (S[so + 1025] << 8));
    }
}

hipError_t launch_npu_stage(int fmt, const uint8_t * src, int64_t sstride, const NpuGeom & g, const int32_t * rowmap,
                            int64_t N, int64_t K, uint8_t * dst, int64_t dstride, int64_t E, hipStream_t s) {
    if ((fmt != ONPU_Q4NX && fmt != ONPU_Q4S) || N <= 0 || K <= 0 || K % 32 || E <= 0 || E > 65535 ||
        dstride < stage_bytes(fmt, N, K) || g.S * g.ks < K)
        return hipErrorInvalidValue;
    const int64_t kch = (K + 511) / 512;
    if (N * kch > INT32_MAX) return hipErrorInvalidValue;
    k_npu_stage<<<dim3((unsigned) (N * kch), (unsigned) E), 256, 0, s>>>(src, sstride, g, fmt == ONPU_Q4S, rowmap, N,
                                                                        K, kch, dst, dstride);
    CHECK_LAUNCH();
    return hipSuccess;
}

// ------------------------------------------------------------------ argmax scratch without allocation
// For callers that cannot allocate (graph capture, serving loops): the argmax's row counters and
// per-workgroup keys live in this file-scope array, ARGMAX_SCRATCH_BYTES per GPU, held until the
// process ends. Counters first (ARGMAX_SCRATCH_CNT bytes, zeroed once per device at set-up; every
// call leaves them at zero), then the keys. In host code `scratch` is only a stand-in for the
// device array: kernels get the address that hipGetSymbolAddress returns for the current device.
// Calls that overlap on one GPU share the array and race.
static __device__ __align__(256) uint8_t scratch[ARGMAX_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void * g_scratch_dev[ARGMAX_SCRATCH_MAX_DEVICES];      // the array's address on each device
}

hipError_t argmax_scratch_init() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= ARGMAX_SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_dev[dev]) return hipSuccess;
    void * p = nullptr;
    if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
    if ((e = hipMemset(p, 0, ARGMAX_SCRATCH_CNT)) != hipSuccess) return e;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
    g_scratch_dev[dev] = p;
    return hipSuccess;
}

hipError_t argmax_scratch_get(int64_t rows, int64_t N, uint64_t ** keys, uint32_t ** cnt) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= ARGMAX_SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    void * p = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch_dev[dev];
    }
    if (!p) return hipErrorNotInitialized;      // set-up (argmax_scratch_init) not run on this device
    if (rows * ARGMAX_PAD > ARGMAX_SCRATCH_CNT ||
        rows * argmax_parts(N) * ARGMAX_PAD > (int64_t) (ARGMAX_SCRATCH_BYTES - ARGMAX_SCRATCH_CNT))
        return hipErrorInvalidValue;
    *cnt = (uint32_t *) p;
    *keys = (uint64_t *) ((uint8_t *) p + ARGMAX_SCRATCH_CNT);
    return hipSuccess;
}

hipError_t launch_argmax(const float * v, int64_t rows, int64_t N, int32_t * out, uint64_t * keys, uint32_t * cnt,
                         hipStream_t s) {
    if (rows <= 0 || N <= 0) return hipSuccess;
    if (rows > 65535 || N >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    k_argmax<<<dim3((unsigned) argmax_parts(N), (unsigned) rows), ARGMAX_THREADS, 0, s>>>(v, N, keys, cnt, out);
    CHECK_LAUNCH();
    return hipSuccess;
}

hipError_t launch_argmax_keys(const uint64_t * keys, int64_t P, int64_t rows, int32_t * out, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (rows > 65535 || P <= 0) return hipErrorInvalidValue;
    k_argmax_keys<<<dim3((unsigned) rows), AKEY_THREADS, 0, s>>>(keys, P, out);
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

hipError_t launch_gemv_i8(const int8_t * W, const float * sc, int64_t N, int64_t K, const float * x, float * y,
                          hipStream_t s) {
    if (N <= 0 || K <= 0) return hipSuccess;
    if (K % 16 || K * 4 > 128 * 1024 || ((uintptr_t) W | (uintptr_t) x) % 16) return hipErrorInvalidValue;
    const int64_t ng = (N + 3) / 4;
    // K parts per row: more, shorter waves win, except that a row of one full step (256 GI8_U
    // bytes) stays whole (11264 x 2048: 15.1 us against 15.9 with 4 parts; 2048 x 5632 keeps 4
    // parts: 8.8 us against 9.4 with 2)
    const int ks = K <= 256 * GI8_U ? 1 : (ng >= 16384 ? 1 : (ng >= 8192 ? 2 : 4));
    const int64_t Kw = (K + (int64_t) ks * 256 - 1) / ((int64_t) ks * 256) * 256;
    const int64_t grid = (ng + 4 / ks - 1) / (4 / ks);
    if (grid >= ((int64_t) 1 << 31) || K * 4 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    k_gemv_i8<<<(unsigned) grid, GI8_T, (size_t) K * 4, s>>>(W, sc, N, K, ks, Kw, x, y);
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

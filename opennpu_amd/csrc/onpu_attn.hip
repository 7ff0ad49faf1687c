// Decode attention for one token (grouped-query), the step the reference runs on the host beside
// its int4 matmuls: onpu_attn_step / onpu_attn_step_bf16 (onpu_cpu.cpp:173-229): for query head h
// (kv head g = h / (Hq / Hkv)), s_j = scale * q_h . K[g][j] + mask[j], softmax over j (with an
// optional per-head sink logit that takes probability mass but has no value), out_h = sum_j p_j
// V[g][j]. fp32 arithmetic; the KV cache is fp32 or bf16 (widened exactly).
//
// Split over the sequence (HBM-bound: K and V are read once). k_attn_part: workgroup (c, g) takes
// rows [c C, c C + C) of kv head g for all rep = Hq / Hkv query heads that share it, so each K and
// V row is read once for rep heads. Phase 1: thread t scores its rows (a row's D values streamed in
// 16-byte loads, q from LDS), the chunk's max and exp-sum per head through LDS. Phase 2: threads
// own pairs of d and row groups, accumulate p_j V[j][d] (a row's D values read by consecutive
// lanes), reduce the row groups in LDS and write the chunk's (max, sum, o[rep][D]) partials.
// k_attn_combine: one workgroup per query head rescales the chunks' partials to the global max
// (and the sink) and divides by the total mass.
#include "onpu_launch.h"

namespace {

constexpr int ATT_T = 256;                   // threads per workgroup
constexpr int ATT_RPT = 4;                   // rows per thread at most in phase 1 (C <= 1024)

struct AttnArgs {
    const float * q;
    const void * K, * V;
    const float * mask, * sinks;
    float * ws, * out;
    int64_t S, hs, rs;
    float scale;
    int Hq, D, Hkv, rep, C, nch;
};

template <typename KV> __device__ __forceinline__ void load8(const KV * p, float (&v)[8]);
template <> __device__ __forceinline__ void load8<uint16_t>(const uint16_t * p, float (&v)[8]) {
    const uint4 u = *(const uint4 *) p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
template <> __device__ __forceinline__ void load8<float>(const float * p, float (&v)[8]) {
    const float4 a = *(const float4 *) p, b = *(const float4 *) (p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <typename KV> __device__ __forceinline__ void load2(const KV * p, float & v0, float & v1);
template <> __device__ __forceinline__ void load2<uint16_t>(const uint16_t * p, float & v0, float & v1) {
    const uint32_t w = *(const uint32_t *) p;
    v0 = __uint_as_float(w << 16);
    v1 = __uint_as_float(w & 0xffff0000u);
}
template <> __device__ __forceinline__ void load2<float>(const float * p, float & v0, float & v1) {
    const float2 f = *(const float2 *) p;
    v0 = f.x;
    v1 = f.y;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// LDS: qs [RP][D], P [RP][C], red [ATT_T / (D / 2)][RP][D], small [2][4][RP]
template <typename KV, int RP>
__global__ __launch_bounds__(ATT_T) void k_attn_part(AttnArgs a) {
    extern __shared__ float lds[];
    const int D = a.D, C = a.C, c = blockIdx.x, g = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    float * qs = lds, * P = qs + RP * D, * red = P + RP * C;
    float * wmax = red + (ATT_T / (D / 2)) * RP * D, * wsum = wmax + 4 * RP;
    const int rep = a.rep;
    for (int i = t; i < RP * D; i += ATT_T) {
        const int h = i / D;
        qs[i] = h < rep ? a.q[(int64_t) (g * rep + h) * D + (i - h * D)] : 0.f;
    }
    __syncthreads();
    const KV * Kg = (const KV *) a.K + (int64_t) g * a.hs;
    const KV * Vg = (const KV *) a.V + (int64_t) g * a.hs;
    const int64_t j0 = (int64_t) c * C;
    const int rows = (int) (a.S - j0 < C ? a.S - j0 : C);

    // phase 1: scores of this thread's rows t, t + 256, ...
    float mloc[RP];
#pragma unroll
    for (int h = 0; h < RP; h++) mloc[h] = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < ATT_RPT; i++) {
        const int jl = t + i * ATT_T;
        if (jl >= C) break;
        float sc[RP];
#pragma unroll
        for (int h = 0; h < RP; h++) sc[h] = 0.f;
        if (jl < rows) {
            const KV * kr = Kg + (j0 + jl) * a.rs;
            for (int d0 = 0; d0 < D; d0 += 8) {
                float kv[8];
                load8<KV>(kr + d0, kv);
#pragma unroll
                for (int h = 0; h < RP; h++) {
                    const float4 qa = *(const float4 *) (qs + h * D + d0), qb = *(const float4 *) (qs + h * D + d0 + 4);
                    sc[h] += qa.x * kv[0]; sc[h] += qa.y * kv[1]; sc[h] += qa.z * kv[2]; sc[h] += qa.w * kv[3];
                    sc[h] += qb.x * kv[4]; sc[h] += qb.y * kv[5]; sc[h] += qb.z * kv[6]; sc[h] += qb.w * kv[7];
                }
            }
            const float mk = a.mask ? a.mask[j0 + jl] : 0.f;
#pragma unroll
            for (int h = 0; h < RP; h++) {
                sc[h] = sc[h] * a.scale + mk;
                mloc[h] = fmaxf(mloc[h], sc[h]);
            }
        } else {
#pragma unroll
            for (int h = 0; h < RP; h++) sc[h] = -__builtin_inff();
        }
#pragma unroll
        for (int h = 0; h < RP; h++) P[h * C + jl] = sc[h];
    }
#pragma unroll
    for (int h = 0; h < RP; h++) {
        const float m = wave_max(mloc[h]);
        if (lane == 0) wmax[wave * RP + h] = m;
    }
    __syncthreads();
    float mc[RP];
#pragma unroll
    for (int h = 0; h < RP; h++)
        mc[h] = fmaxf(fmaxf(wmax[h], wmax[RP + h]), fmaxf(wmax[2 * RP + h], wmax[3 * RP + h]));
    float lloc[RP];
#pragma unroll
    for (int h = 0; h < RP; h++) lloc[h] = 0.f;
#pragma unroll
    for (int i = 0; i < ATT_RPT; i++) {
        const int jl = t + i * ATT_T;
        if (jl >= C) break;
#pragma unroll
        for (int h = 0; h < RP; h++) {
            // a chunk whose rows are all masked (-inf) keeps p = 0 instead of exp(-inf + inf)
            const float p = mc[h] == -__builtin_inff() ? 0.f : expf(P[h * C + jl] - mc[h]);
            P[h * C + jl] = p;
            lloc[h] += p;
        }
    }
#pragma unroll
    for (int h = 0; h < RP; h++) {
        const float s = wave_sum(lloc[h]);
        if (lane == 0) wsum[wave * RP + h] = s;
    }
    __syncthreads();

    // phase 2: o[h][d] = sum_j P[h][j] V[j][d]; thread (row group rg, d pair dp)
    const int ndp = D / 2, tpd = ATT_T / ndp, dp = t % ndp, rg = t / ndp;
    float acc[RP][2];
#pragma unroll
    for (int h = 0; h < RP; h++) acc[h][0] = acc[h][1] = 0.f;
    if (rg < tpd) {
        const KV * vb = Vg + j0 * a.rs + 2 * dp;
        int j = rg;
        for (; j + 3 * tpd < rows; j += 4 * tpd) {            // four rows' loads in flight
            float v[4][2];
#pragma unroll
            for (int u = 0; u < 4; u++) load2<KV>(vb + (int64_t) (j + u * tpd) * a.rs, v[u][0], v[u][1]);
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int h = 0; h < RP; h++) {
                    const float p = P[h * C + j + u * tpd];
                    acc[h][0] += p * v[u][0];
                    acc[h][1] += p * v[u][1];
                }
        }
        for (; j < rows; j += tpd) {
            float v0, v1;
            load2<KV>(vb + (int64_t) j * a.rs, v0, v1);
#pragma unroll
            for (int h = 0; h < RP; h++) {
                const float p = P[h * C + j];
                acc[h][0] += p * v0;
                acc[h][1] += p * v1;
            }
        }
#pragma unroll
        for (int h = 0; h < RP; h++) {
            red[(rg * RP + h) * D + 2 * dp] = acc[h][0];
            red[(rg * RP + h) * D + 2 * dp + 1] = acc[h][1];
        }
    }
    __syncthreads();
    // partials of (g, c): m [RP], l [RP], o [RP][D]
    float * wp = a.ws + ((int64_t) g * a.nch + c) * (RP * (2 + D));
    for (int i = t; i < RP * D; i += ATT_T) {
        const int h = i / D, d = i - h * D;
        float s = 0.f;
        for (int r = 0; r < tpd; r++) s += red[(r * RP + h) * D + d];
        wp[2 * RP + i] = s;
    }
    if (t < RP) {
        wp[t] = fmaxf(fmaxf(wmax[t], wmax[RP + t]), fmaxf(wmax[2 * RP + t], wmax[3 * RP + t]));
        wp[RP + t] = wsum[t] + wsum[RP + t] + wsum[2 * RP + t] + wsum[3 * RP + t];
    }
}

// grid Hq, D threads: out[h][d] = sum_c e^(m_c - M) o_c[d] / (sum_c e^(m_c - M) l_c + e^(sink - M))
template <int RP>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
    const int h = blockIdx.x, g = h / a.rep, hi = h - g * a.rep, d = threadIdx.x;
    const float * wp = a.ws + (int64_t) g * a.nch * (RP * (2 + a.D));
    const int64_t st = RP * (2 + a.D);
    float M = a.sinks ? a.sinks[h] : -__builtin_inff();
    for (int c = 0; c < a.nch; c++) M = fmaxf(M, wp[c * st + hi]);
    float den = a.sinks ? expf(a.sinks[h] - M) : 0.f, num = 0.f;
    for (int c = 0; c < a.nch; c++) {
        const float mc = wp[c * st + hi];
        const float f = mc == -__builtin_inff() ? 0.f : expf(mc - M);
        den += f * wp[c * st + RP + hi];
        if (d < a.D) num += f * wp[c * st + 2 * RP + hi * a.D + d];
    }
    if (d < a.D) a.out[(int64_t) h * a.D + d] = num / den;
}

int next_pow2(int v) {
    int p = 1;
    while (p < v) p *= 2;
    return p;
}

// rows per chunk: a multiple of 256 up to 1024 with P [RP][C] <= 32 KiB, aiming at >= 512
// workgroups
int attn_chunk(int RP, int Hkv, int64_t S) {
    int C = 256;
    while (C < 1024 && RP * C * 2 <= 8192 && (S + 2 * C - 1) / (2 * C) * Hkv >= 512) C *= 2;
    return C;
}

size_t attn_lds(int RP, int D, int C) {
    return sizeof(float) * ((size_t) RP * D + (size_t) RP * C + (size_t) (ATT_T / (D / 2)) * RP * D + 8 * RP);
}

template <typename KV, int RP>
hipError_t run_attn(AttnArgs a, hipStream_t s) {
    const size_t lds = attn_lds(RP, a.D, a.C);
    k_attn_part<KV, RP><<<dim3((unsigned) a.nch, (unsigned) a.Hkv), ATT_T, lds, s>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_attn_combine<RP><<<dim3((unsigned) a.Hq), 256, 0, s>>>(a);
    return hipGetLastError();
}

template <typename KV>
hipError_t run_attn_rp(int RP, const AttnArgs & a, hipStream_t s) {
    switch (RP) {
    case 1: return run_attn<KV, 1>(a, s);
    case 2: return run_attn<KV, 2>(a, s);
    case 4: return run_attn<KV, 4>(a, s);
    case 8: return run_attn<KV, 8>(a, s);
    case 16: return run_attn<KV, 16>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int64_t attn_ws_bytes(int Hq, int D, int Hkv, int64_t S) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || S <= 0) return 0;
    const int RP = next_pow2(Hq / Hkv);
    const int C = attn_chunk(RP, Hkv, S);
    return (int64_t) Hkv * ((S + C - 1) / C) * RP * (2 + D) * (int64_t) sizeof(float);
}

hipError_t launch_attn_step(const float * q, int Hq, int D, const void * K, const void * V, int kv_bf16, int Hkv,
                            int64_t S, int64_t hs, int64_t rs, const float * mask, const float * sinks, float scale,
                            float * out, void * ws, int64_t ws_bytes, hipStream_t s) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || S <= 0 || D <= 0 || D > 256 || D % 8) return hipErrorInvalidValue;
    const int rep = Hq / Hkv, RP = next_pow2(rep);
    if (RP > 16) return hipErrorInvalidValue;
    const int64_t al = kv_bf16 ? 8 : 4;             // 16-byte row starts for the vector loads
    if (rs % al || hs % al || ((uintptr_t) K | (uintptr_t) V) % 16) return hipErrorInvalidValue;
    if (ws_bytes < attn_ws_bytes(Hq, D, Hkv, S)) return hipErrorInvalidValue;
    AttnArgs a;
    a.q = q; a.K = K; a.V = V; a.mask = mask; a.sinks = sinks; a.ws = (float *) ws; a.out = out;
    a.S = S; a.hs = hs; a.rs = rs; a.scale = scale;
    a.Hq = Hq; a.D = D; a.Hkv = Hkv; a.rep = rep;
    a.C = attn_chunk(RP, Hkv, S);
    a.nch = (int) ((S + a.C - 1) / a.C);
    if ((int64_t) a.nch * a.C < S || a.nch > 0x7fffffff) return hipErrorInvalidValue;
    return kv_bf16 ? run_attn_rp<uint16_t>(RP, a, s) : run_attn_rp<float>(RP, a, s);
}

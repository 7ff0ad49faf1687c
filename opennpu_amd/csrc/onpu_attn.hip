// Decode attention for one token (grouped-query), the step the reference runs on the host beside
// its int4 matmuls: onpu_attn_step / onpu_attn_step_bf16 (onpu_cpu.cpp:173-229): for query head h
// (kv head g = h / (Hq / Hkv)), s_j = scale * q_h . K[g][j] + mask[j], softmax over j (with an
// optional per-head sink logit that takes probability mass but has no value), out_h = sum_j p_j
// V[g][j]. fp32 arithmetic; the KV cache is fp32 or bf16 (widened exactly).
//
// Split over the sequence; HBM-bound at long context (K and V are read once). k_attn_part:
// workgroup (c, g, z) takes rows [c C, c C + C) of kv head g for HG of the query heads that share
// it (group z), so each K and V row is read once for HG heads. A row is read by LPR = D / 8
// consecutive lanes, 16 bytes each (one wave instruction covers 64 / LPR consecutive rows), with
// AU rows per lane group in flight. Phase 1 scores the chunk's rows into LDS (a lane's 8 products
// per head, summed across its LPR lanes by DPP); the chunk's max and exp-sum per head follow from
// LDS while the first V loads fly; phase 2 accumulates p_j V[j] in registers (8 values of d per lane
// and head), sums the row slots of a wave by shuffles and the waves in LDS, and writes the chunk's
// (max, sum, o[HG][D]). k_attn_combine: per query head, the chunks' partials rescaled to the
// global max (and the sink) and divided by the total mass.
#include "onpu_launch.h"

namespace {

constexpr int AT = 512;                      // threads per workgroup (8 waves)
constexpr int AW = AT / 64;
constexpr int AU = 4;                        // rows per lane group in flight
constexpr int AP_MAX = 16384;                // floats of P per workgroup (64 KiB)
constexpr int TARGET_WG = 512;
constexpr int ATT_MAX_CH = 4096;             // chunks per kv head at most (the combine's LDS)

struct AttnArgs {
    const float * q;
    const void * K, * V;
    const float * mask, * sinks;
    float * ws, * out;
    int64_t S, hs, rs;
    float scale;
    int Hq, D, Hkv, rep, ngrp, C, nch;
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

// sum over aligned groups of L lanes (L = 8, 16, 32), every lane of a group left with the sum: DPP
// within a row of 16 (xor 1 and 2 by quad permutes, then the half-row and row mirrors, which pair
// lanes of equal partial sums), one cross-row shuffle for 32
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int L> __device__ __forceinline__ float group_sum(float x) {
    x += dpp_f<0xB1>(x);                     // quad_perm [1, 0, 3, 2]
    x += dpp_f<0x4E>(x);                     // quad_perm [2, 3, 0, 1]
    x += dpp_f<0x141>(x);                    // row_half_mirror: lane i <-> 7 - i
    if (L >= 16) x += dpp_f<0x140>(x);       // row_mirror: lane i <-> 15 - i
    if (L >= 32) x += __shfl_xor(x, 16);
    return x;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// LDS: P [HG][C], red [AW][HG][D], wmax / wsum [AW][HG], qs [HG][D]
template <typename KV, int LPR, int HG>
__global__ __launch_bounds__(AT) void k_attn_part(AttnArgs a) {
    constexpr int RPW = 64 / LPR, RIT = AW * RPW * AU;          // row slots per wave; rows per pass
    extern __shared__ __align__(16) float lds[];
    const int D = a.D, C = a.C, c = blockIdx.x, g = blockIdx.y, z = blockIdx.z, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, li = lane % LPR, slot = lane / LPR;
    float * P = lds, * red = P + HG * C, * wmax = red + AW * HG * D, * wsum = wmax + AW * HG, * qs = wsum + AW * HG;
    const bool dl = 8 * li < D;                                  // this lane's 8 values of d exist
    const int64_t j0 = (int64_t) c * C;
    const int rows = (int) (a.S - j0 < C ? a.S - j0 : C);
    // lanes past D read column 0 (their values meet zero q and are never stored)
    const KV * Kg = (const KV *) a.K + (int64_t) g * a.hs + j0 * a.rs + 8 * (dl ? li : 0);
    const KV * Vg = (const KV *) a.V + (int64_t) g * a.hs + j0 * a.rs + 8 * (dl ? li : 0);
    // q of the group's heads: coalesced 16-byte loads (0 past rep), stored to LDS after the first
    // pass's K loads are issued; the barrier then waits for LDS only (a __syncthreads would also
    // wait for the K loads)
    const int nq = HG * D / 4, hq0 = z * HG, hqn = a.rep - hq0 < HG ? a.rep - hq0 : HG;
    // (loads unconditional, from clamped addresses, and masked where used: a load under a branch is
    // waited for where the branch rejoins, which would serialize the loads)
    const bool qok = t < nq && t * 4 < hqn * D;
    const float4 qv = *(const float4 *) (a.q + (int64_t) (g * a.rep + hq0) * D + (qok ? 4 * t : 0));
    // Row of (pass r0, step u, wave, slot): consecutive slots and waves take consecutive rows, so one
    // wave instruction reads RPW consecutive rows.
    float kv[AU][8];
    auto issue = [&](const KV * base, int r0) {
#pragma unroll
        for (int u = 0; u < AU; u++) {
            // rows past the chunk re-read its last row: their scores are not stored, their V rows
            // not accumulated
            const int row = r0 + (u * AW + wave) * RPW + slot;
            load8<KV>(base + (int64_t) (row < rows ? row : rows - 1) * a.rs, kv[u]);
        }
    };
    issue(Kg, 0);
    if (t < nq) *(float4 *) (qs + 4 * t) = qok ? qv : make_float4(0.f, 0.f, 0.f, 0.f);
    __builtin_amdgcn_s_waitcnt(0xc07f);                                 // lgkmcnt(0): the LDS stores
    __builtin_amdgcn_s_barrier();
    float qr[HG][8];
#pragma unroll
    for (int h = 0; h < HG; h++) {
        const float4 a0 = dl ? *(const float4 *) (qs + h * D + 8 * li) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 a1 = dl ? *(const float4 *) (qs + h * D + 8 * li + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        qr[h][0] = a0.x; qr[h][1] = a0.y; qr[h][2] = a0.z; qr[h][3] = a0.w;
        qr[h][4] = a1.x; qr[h][5] = a1.y; qr[h][6] = a1.z; qr[h][7] = a1.w;
    }

    // phase 1: scores into P
    for (int r0 = 0; r0 < rows; r0 += RIT) {
        if (r0 > 0) issue(Kg, r0);
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int row = r0 + (u * AW + wave) * RPW + slot;
            float sc[HG];
#pragma unroll
            for (int h = 0; h < HG; h++) {
                float x = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) x += qr[h][e] * kv[u][e];
                sc[h] = group_sum<LPR>(x);                                   // the row's lanes
            }
            if (li == 0 && row < rows) {
                const float mk = a.mask ? a.mask[j0 + row] : 0.f;
#pragma unroll
                for (int h = 0; h < HG; h++) P[h * C + row] = sc[h] * a.scale + mk;
            }
        }
    }
    issue(Vg, 0);                           // phase 2's first V loads fly during the softmax
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    // chunk max and exp-sum per head (a chunk whose rows are all -inf keeps p = 0)
#pragma unroll
    for (int h = 0; h < HG; h++) {
        float mx = -__builtin_inff();
        for (int r = t; r < rows; r += AT) mx = fmaxf(mx, P[h * C + r]);
        mx = wave_max(mx);
        if (lane == 0) wmax[wave * HG + h] = mx;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int h = 0; h < HG; h++) {
        float mx = wmax[h];
#pragma unroll
        for (int w = 1; w < AW; w++) mx = fmaxf(mx, wmax[w * HG + h]);
        float l = 0.f;
        for (int r = t; r < rows; r += AT) {
            const float p = mx == -__builtin_inff() ? 0.f : expf(P[h * C + r] - mx);
            P[h * C + r] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) wsum[wave * HG + h] = l;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();

    // phase 2: o[h][d] = sum_j P[h][j] V[j][d]
    float acc[HG][8];
#pragma unroll
    for (int h = 0; h < HG; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.f;
    for (int r0 = 0; r0 < rows; r0 += RIT) {
        if (r0 > 0) issue(Vg, r0);
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int row = r0 + (u * AW + wave) * RPW + slot;
            if (row < rows) {
#pragma unroll
                for (int h = 0; h < HG; h++) {
                    const float p = P[h * C + row];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[h][e] += p * kv[u][e];
                }
            }
        }
    }
    // sum the wave's row slots (lanes LPR apart), then the waves
#pragma unroll
    for (int h = 0; h < HG; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float x = acc[h][e];
#pragma unroll
            for (int o = LPR; o < 64; o <<= 1) x += __shfl_xor(x, o);
            acc[h][e] = x;
        }
    if (slot == 0 && dl) {
#pragma unroll
        for (int h = 0; h < HG; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) red[(wave * HG + h) * D + 8 * li + e] = acc[h][e];
    }
    __syncthreads();
    float * wp = a.ws + (((int64_t) g * a.ngrp + z) * a.nch + c) * (HG * (2 + D));
    for (int i = t; i < HG * D; i += AT) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < AW; w++) sum += red[w * HG * D + i];
        wp[2 * HG + i] = sum;
    }
    if (t < HG) {
        float mx = wmax[t], l = 0.f;
#pragma unroll
        for (int w = 1; w < AW; w++) mx = fmaxf(mx, wmax[w * HG + t]);
#pragma unroll
        for (int w = 0; w < AW; w++) l += wsum[w * HG + t];
        wp[t] = mx;
        wp[HG + t] = l;
    }
}

// grid Hq, 256 threads: out[h][d] = sum_c e^(m_c - M) o_c[d] / (sum_c e^(m_c - M) l_c + e^(sink - M)).
// Thread (group gi, d pair dp) sums chunks gi, gi + G, ... (G = 256 / (D / 2) groups), then LDS.
template <int HG>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
    __shared__ float sred[256 * 2];
    __shared__ float sm[4];
    __shared__ float fw[ATT_MAX_CH];                 // e^(m_c - M) per chunk
    const int h = blockIdx.x, g = h / a.rep, hr = h - g * a.rep, z = hr / HG, hh = hr - z * HG, t = threadIdx.x;
    const int64_t st = HG * (2 + a.D);
    const float * wp = a.ws + ((int64_t) g * a.ngrp + z) * a.nch * st;
    float M = a.sinks ? a.sinks[h] : -__builtin_inff();
    for (int c = t; c < a.nch; c += 256) M = fmaxf(M, wp[c * st + hh]);
    M = wave_max(M);
    if ((t & 63) == 0) sm[t >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    float den = 0.f;
    for (int c = t; c < a.nch; c += 256) {
        const float mc = wp[c * st + hh];
        const float f = mc == -__builtin_inff() ? 0.f : expf(mc - M);
        fw[c] = f;
        den += f * wp[c * st + HG + hh];
    }
    den = wave_sum(den);
    __syncthreads();
    if ((t & 63) == 0) sm[t >> 6] = den;
    __syncthreads();
    den = sm[0] + sm[1] + sm[2] + sm[3] + (a.sinks ? expf(a.sinks[h] - M) : 0.f);
    const int np = a.D / 2, G = 256 / np, dp = t % np, gi = t / np;
    float n0 = 0.f, n1 = 0.f;
    if (gi < G) {
#pragma unroll 4
        for (int c = gi; c < a.nch; c += G) {
            const float2 o = *(const float2 *) (wp + c * st + 2 * HG + hh * a.D + 2 * dp);
            n0 += fw[c] * o.x;
            n1 += fw[c] * o.y;
        }
    }
    sred[2 * t] = n0;
    sred[2 * t + 1] = n1;
    __syncthreads();
    if (t < np) {
        float s0 = 0.f, s1 = 0.f;
        for (int i = 0; i < G; i++) { s0 += sred[2 * (i * np + t)]; s1 += sred[2 * (i * np + t) + 1]; }
        a.out[(int64_t) h * a.D + 2 * t] = s0 / den;
        a.out[(int64_t) h * a.D + 2 * t + 1] = s1 / den;
    }
}

int next_pow2(int v) {
    int p = 1;
    while (p < v) p *= 2;
    return p;
}

struct AttnPlan { int LPR, HG, ngrp, C, nch; };

// chunk rows: enough chunks for ~TARGET_WG workgroups, at least 64 rows each, P within AP_MAX
AttnPlan attn_plan(int Hq, int D, int Hkv, int64_t S) {
    AttnPlan p;
    const int rep = Hq / Hkv;
    p.LPR = next_pow2(D / 8) < 8 ? 8 : next_pow2(D / 8);
    p.HG = next_pow2(rep) > 8 ? 8 : next_pow2(rep);
    p.ngrp = (rep + p.HG - 1) / p.HG;
    int64_t nch = (TARGET_WG + (int64_t) Hkv * p.ngrp - 1) / ((int64_t) Hkv * p.ngrp);
    const int64_t nmax = (S + 63) / 64;
    if (nch > nmax) nch = nmax;
    if (nch < 1) nch = 1;
    int64_t C = ((S + nch - 1) / nch + 63) / 64 * 64;
    if (C > AP_MAX / p.HG) C = AP_MAX / p.HG;
    p.C = (int) C;
    p.nch = (int) ((S + C - 1) / C);
    return p;                                 // nch <= ATT_MAX_CH is checked by the launcher
}

size_t attn_lds(const AttnPlan & p, int D) {
    return sizeof(float) * ((size_t) p.HG * p.C + (size_t) AW * p.HG * D + 2 * AW * p.HG + (size_t) p.HG * D);
}

template <typename KV, int LPR, int HG>
hipError_t run_attn(const AttnArgs & a, const AttnPlan & p, hipStream_t s) {
    k_attn_part<KV, LPR, HG><<<dim3((unsigned) a.nch, (unsigned) a.Hkv, (unsigned) a.ngrp), AT, attn_lds(p, a.D), s>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_attn_combine<HG><<<dim3((unsigned) a.Hq), 256, 0, s>>>(a);
    return hipGetLastError();
}

template <typename KV, int LPR>
hipError_t run_attn_hg(const AttnArgs & a, const AttnPlan & p, hipStream_t s) {
    switch (p.HG) {
    case 1: return run_attn<KV, LPR, 1>(a, p, s);
    case 2: return run_attn<KV, LPR, 2>(a, p, s);
    case 4: return run_attn<KV, LPR, 4>(a, p, s);
    case 8: return run_attn<KV, LPR, 8>(a, p, s);
    default: return hipErrorInvalidValue;
    }
}

template <typename KV>
hipError_t run_attn_lpr(const AttnArgs & a, const AttnPlan & p, hipStream_t s) {
    switch (p.LPR) {
    case 8: return run_attn_hg<KV, 8>(a, p, s);
    case 16: return run_attn_hg<KV, 16>(a, p, s);
    case 32: return run_attn_hg<KV, 32>(a, p, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int64_t attn_ws_bytes(int Hq, int D, int Hkv, int64_t S) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || S <= 0) return 0;
    const AttnPlan p = attn_plan(Hq, D, Hkv, S);
    return (int64_t) Hkv * p.ngrp * p.nch * p.HG * (2 + D) * (int64_t) sizeof(float);
}

hipError_t launch_attn_step(const float * q, int Hq, int D, const void * K, const void * V, int kv_bf16, int Hkv,
                            int64_t S, int64_t hs, int64_t rs, const float * mask, const float * sinks, float scale,
                            float * out, void * ws, int64_t ws_bytes, hipStream_t s) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || S <= 0 || D <= 0 || D > 256 || D % 8) return hipErrorInvalidValue;
    if (Hq / Hkv > 16) return hipErrorInvalidValue;
    const int64_t al = kv_bf16 ? 8 : 4;             // 16-byte row starts for the vector loads
    if (rs % al || hs % al || ((uintptr_t) K | (uintptr_t) V | (uintptr_t) q) % 16) return hipErrorInvalidValue;
    if (ws_bytes < attn_ws_bytes(Hq, D, Hkv, S)) return hipErrorInvalidValue;
    const AttnPlan p = attn_plan(Hq, D, Hkv, S);
    AttnArgs a;
    a.q = q; a.K = K; a.V = V; a.mask = mask; a.sinks = sinks; a.ws = (float *) ws; a.out = out;
    a.S = S; a.hs = hs; a.rs = rs; a.scale = scale;
    a.Hq = Hq; a.D = D; a.Hkv = Hkv; a.rep = Hq / Hkv; a.ngrp = p.ngrp; a.C = p.C; a.nch = p.nch;
    if (Hkv > 65535 || p.ngrp > 65535 || p.nch > ATT_MAX_CH) return hipErrorInvalidValue;
    return kv_bf16 ? run_attn_lpr<uint16_t>(a, p, s) : run_attn_lpr<float>(a, p, s);
}

// ------------------------------------------------------------------ Gated DeltaNet decode step
// One decode token of a Gated DeltaNet layer: the reference's host onpu_gdn_step (onpu_cpu.cpp:107-
// 171). k_gdn_conv: one thread per channel c of qkv: causal conv over the last Kc inputs (the same
// order of products as the reference), SiLU into co, and the conv state shifts by one. k_gdn_head:
// one workgroup per value head h: q, k of its key head L2-normalised (q also / sqrt Dk), beta =
// sigmoid(Wb x), decay = exp(-exp(A_log) softplus(Wa x + dt_bias)); the head's state S [Dk][Dv]
// goes to LDS scaled by decay while thread (d-column j, row group g) sums kv_j = sum_i S_ij k_i;
// delta = beta (v - kv); S += k delta^T and o = S^T q in a second pass over LDS, S written back;
// out = norm_w * o / sqrt(mean(o^2) + eps) * silu(z). Sums are block reductions (another order than
// the reference's sequential loops).
namespace {

__device__ __forceinline__ float gdn_silu(float v) { return v / (1.f + expf(-v)); }

__global__ __launch_bounds__(256) void k_gdn_conv(const float * __restrict__ qkv, const float * __restrict__ conv_w,
                                                  int Kc, float * __restrict__ conv_state, int L, int C,
                                                  float * __restrict__ co) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    float * st = conv_state + (int64_t) c * L;
    const float * w = conv_w + (int64_t) c * Kc;
    float s = w[Kc - 1] * qkv[c];
    for (int j = 0; j < Kc - 1; j++) s += w[j] * st[L - (Kc - 1) + j];
    co[c] = gdn_silu(s);
    for (int j = 0; j + 1 < L; j++) st[j] = st[j + 1];
    st[L - 1] = qkv[c];
}

// block sum over 256 threads (every thread gets the sum); red: 8 floats of LDS
__device__ __forceinline__ float gdn_block_sum(float v, float * red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

struct GdnArgs {
    const float * x, * z, * Wb, * Wa, * A_log, * dt_bias, * norm_w, * co;
    float * S, * out;
    float eps;
    int H, Hk, Hv, Dk, Dv;
};

// LDS: Sl [Dk][Dv], vec [4][max(Dk, Dv)] (q, k, delta / o), part [256 / Dv][Dv], red [8]
__global__ __launch_bounds__(256) void k_gdn_head(GdnArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int h = blockIdx.x, t = threadIdx.x, Dk = a.Dk, Dv = a.Dv, rep = a.Hv / a.Hk, kh = h / rep;
    const int key_dim = a.Hk * Dk, mx = Dk > Dv ? Dk : Dv, G = 256 / Dv, j = t % Dv, g = t / Dv;
    float * Sl = lds, * qv = Sl + Dk * Dv, * kvec = qv + mx, * dv = kvec + mx, * ov = dv + mx;
    float * part = ov + mx, * red = part + G * Dv;
    float qq = 0.f, kk = 0.f;
    for (int i = t; i < Dk; i += 256) {
        const float qi = a.co[kh * Dk + i], ki = a.co[key_dim + kh * Dk + i];
        qv[i] = qi;
        kvec[i] = ki;
        qq += qi * qi;
        kk += ki * ki;
    }
    float pb = 0.f, pa = 0.f;
    for (int i = t; i < a.H; i += 256) {
        pb += a.Wb[(int64_t) h * a.H + i] * a.x[i];
        pa += a.Wa[(int64_t) h * a.H + i] * a.x[i];
    }
    qq = gdn_block_sum(qq, red);
    kk = gdn_block_sum(kk, red);
    const float b = gdn_block_sum(pb, red), av = gdn_block_sum(pa, red);
    const float qn = 1.f / sqrtf(qq + 1e-6f) / sqrtf((float) Dk), kn = 1.f / sqrtf(kk + 1e-6f);
    const float beta = 1.f / (1.f + expf(-b));
    const float ad = av + a.dt_bias[h];
    const float sp = ad > 20.f ? ad : log1pf(expf(ad));
    const float decay = expf(-expf(a.A_log[h]) * sp);
    // pass 1: S <- decay S into LDS, kv_j = sum_i S_ij k_i (row groups g, g + G, ...)
    float * Sh = a.S + (int64_t) h * Dk * Dv;
    float kv = 0.f;
    if (g < G)
        for (int i = g; i < Dk; i += G) {
            const float r = Sh[(int64_t) i * Dv + j] * decay;
            Sl[i * Dv + j] = r;
            kv += r * (kvec[i] * kn);
        }
    if (g < G) part[g * Dv + j] = kv;
    __syncthreads();
    if (t < Dv) {
        float s = 0.f;
        for (int r = 0; r < G; r++) s += part[r * Dv + t];
        dv[t] = (a.co[2 * key_dim + (int64_t) h * Dv + t] - s) * beta;
    }
    __syncthreads();
    // pass 2: S += k delta^T, o_j = sum_i S_ij q_i; S back to HBM
    float o = 0.f;
    if (g < G)
        for (int i = g; i < Dk; i += G) {
            const float r = Sl[i * Dv + j] + (kvec[i] * kn) * dv[j];
            Sh[(int64_t) i * Dv + j] = r;
            o += r * (qv[i] * qn);
        }
    if (g < G) part[g * Dv + j] = o;
    __syncthreads();
    float oj = 0.f;
    if (t < Dv) {
        for (int r = 0; r < G; r++) oj += part[r * Dv + t];
        ov[t] = oj;
    }
    const float ms = gdn_block_sum(t < Dv ? oj * oj : 0.f, red) / Dv;
    const float rn = 1.f / sqrtf(ms + a.eps);
    if (t < Dv) a.out[(int64_t) h * Dv + t] = a.norm_w[t] * (oj * rn) * gdn_silu(a.z[(int64_t) h * Dv + t]);
}

}  // namespace

int64_t gdn_ws_bytes(int Hk, int Hv, int Dk, int Dv) {
    return (int64_t) (2 * Hk * Dk + Hv * Dv) * (int64_t) sizeof(float);
}

hipError_t launch_gdn_step(const float * x, int H, const float * qkv, const float * z, const float * Wb,
                           const float * Wa, const float * conv_w, int Kc, float * conv_state, int L,
                           const float * A_log, const float * dt_bias, const float * norm_w, float eps, float * S,
                           int Hk, int Hv, int Dk, int Dv, float * out, void * ws, int64_t ws_bytes, hipStream_t s) {
    if (H <= 0 || Hk <= 0 || Hv <= 0 || Hv % Hk || Dk <= 0 || Dv <= 0 || 256 % Dv || Dv < 4 || Kc < 1 ||
        L < Kc - 1 || L < 1 || (int64_t) Dk * Dv > 32768)
        return hipErrorInvalidValue;
    if (ws_bytes < gdn_ws_bytes(Hk, Hv, Dk, Dv)) return hipErrorInvalidValue;
    const int C = 2 * Hk * Dk + Hv * Dv;
    float * co = (float *) ws;
    k_gdn_conv<<<(C + 255) / 256, 256, 0, s>>>(qkv, conv_w, Kc, conv_state, L, C, co);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GdnArgs a;
    a.x = x; a.z = z; a.Wb = Wb; a.Wa = Wa; a.A_log = A_log; a.dt_bias = dt_bias; a.norm_w = norm_w; a.co = co;
    a.S = S; a.out = out; a.eps = eps; a.H = H; a.Hk = Hk; a.Hv = Hv; a.Dk = Dk; a.Dv = Dv;
    const int mx = Dk > Dv ? Dk : Dv;
    const size_t lds = sizeof(float) * ((size_t) Dk * Dv + 4 * (size_t) mx + (size_t) (256 / Dv) * Dv + 8);
    k_gdn_head<<<Hv, 256, lds, s>>>(a);
    return hipGetLastError();
}

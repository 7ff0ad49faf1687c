// Ceiling probes for the benchmark (libonpu_probe.so; not part of the C ABI the reference binds):
// what this MI355X delivers to simple kernels, so that the int4 kernels' rates can be read against
// measured ceilings as well as the published peaks.
//   onpu_probe_read  HBM streaming read: every byte of a buffer read once with 16-byte loads,
//                    4 or 16 in flight per lane, one contiguous range per workgroup of 256 lanes
//   onpu_probe_lds   LDS read rate: ds_read_b128 with consecutive lanes on consecutive 16 bytes
//                    (no bank conflicts), eight reads in flight per lane
//   onpu_probe_mfma  v_mfma_f32_16x16x32_bf16 issue rate: eight independent accumulators per wave
//   onpu_probe_coissue  VALU issue beside MFMAs on the same SIMD: waves 0-3 of a workgroup run
//                    independent v_fma_f32 chains, waves 4-7 (one per SIMD again) stream MFMAs
// Each kernel's wave 0 of workgroup 0 records the shader clock counter (s_memtime) and the constant
// 100 MHz counter (s_memrealtime) at its start and end, so the host derives the effective clock.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

// clk[0..3] = memtime start, realtime start, memtime end, realtime end (written by one lane)
static __device__ __forceinline__ void stamp(uint64_t * clk, int end) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        uint64_t t = __builtin_amdgcn_s_memtime();
        uint64_t r = __builtin_amdgcn_s_memrealtime();
        clk[2 * end] = t;
        clk[2 * end + 1] = r;
    }
}

// each workgroup streams one contiguous range (as a GEMV's row tiles do), U 16-byte loads in
// flight per lane; a grid-stride walk measured 6.3-6.5 TB/s against 7.0-7.1 for this
template <int U>
__global__ __launch_bounds__(256) void k_probe_read(const u32x4 * __restrict__ p, int64_t n16, uint32_t * out,
                                                    uint64_t * clk) {
    stamp(clk, 0);
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = (int64_t) blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
    u32x4 acc = {0, 0, 0, 0};
    int64_t i = b0 + threadIdx.x;
    for (; i + (U - 1) * 256 < b1; i += U * 256) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(p + i + u * 256);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u];
    }
    for (; i < b1; i += 256) acc ^= p[i];
    uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (v == 0x9e3779b9u) out[0] = v;     // keeps the loads; the buffer never xors to this
    __syncthreads();
    stamp(clk, 1);
}

__global__ __launch_bounds__(1024) void k_probe_lds(int iters, uint32_t * out, uint64_t * clk) {
    __shared__ u32x4 buf[4096];           // 64 KiB
    for (int i = threadIdx.x; i < 4096; i += blockDim.x) buf[i] = u32x4{(uint32_t) i, (uint32_t) i * 3u, ~(uint32_t) i, 7u};
    __syncthreads();
    stamp(clk, 0);
    lds_u32x4 * b = (lds_u32x4 *) buf;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 acc = {0, 0, 0, 0};
    int base = (wave * 512 + lane) & 4095;
    for (int it = 0; it < iters; ++it) {
        u32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = b[(base + 64 * j) & 4095];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[j];
        base = (base + 512 + 64 * (it & 7)) & 4095;
        asm volatile("" ::: "memory");    // the next iteration reads LDS again (no instruction)
    }
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (r == 0x9e3779b9u) out[0] = r;
    __syncthreads();
    stamp(clk, 1);
}

__global__ __launch_bounds__(512) void k_probe_mfma(int iters, float * out, uint64_t * clk) {
    stamp(clk, 0);
    const uint32_t t = threadIdx.x;
    u32x4 a = {0x3f803f80u ^ (t & 1u), 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    u32x4 b = {0x3f003f00u, 0x3f003f00u ^ (t & 2u), 0x3f003f00u, 0x3f003f00u};
    f32x4 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = f32x4{0.f, 0.f, 0.f, (float) j};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                           c[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += c[j].x + c[j].y + c[j].z + c[j].w;
    if (s == -1.f) out[0] = s;           // never true: all products are positive
    __syncthreads();
    stamp(clk, 1);
}

// mode 0: waves 0-3 run iters x 48 v_fma_f32 (8 independent chains), waves 4-7 idle; mode 1: waves
// 4-7 run iters x 8 MFMAs (8 independent accumulators), waves 0-3 idle; mode 2: both. Wave w and
// wave w + 4 share a SIMD. cyc[0] / cyc[1]: shader-clock cycles of wave 0 / wave 4 of workgroup 0.
template <int MODE>
__global__ __launch_bounds__(512) void k_probe_coissue(int iters, float * out, uint64_t * cyc) {
    const uint32_t t = threadIdx.x, wave = t >> 6;
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    float s = 0.f;
    if (wave < 4 && MODE != 1) {
        const float k0 = 0.999f + 1e-7f * (float) t, k1 = 1e-3f;
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (float) (j + t);
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < 6; ++u)
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] = fmaf(r[j], k0, k1);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s += r[j];
    } else if (wave >= 4 && MODE != 0) {
        u32x4 a = {0x3f803f80u ^ (t & 1u), 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
        u32x4 b = {0x3f003f00u, 0x3f003f00u ^ (t & 2u), 0x3f003f00u, 0x3f003f00u};
        f32x4 c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = f32x4{0.f, 0.f, 0.f, (float) j};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                               __builtin_bit_cast(bf16x8, b), c[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s += c[j].x + c[j].y + c[j].z + c[j].w;
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    if (s == -1.f) out[0] = s;           // never true: the chains stay positive
    if (blockIdx.x == 0 && (t == 0 || t == 256)) cyc[t == 0 ? 0 : 1] = t1 - t0;
}

extern "C" {

// n_bytes must be a multiple of 16; unroll 4 or 16 loads in flight per lane; returns 0 or the HIP
// error code of the launch
int onpu_probe_read(const void * p, int64_t n_bytes, int grid, int unroll, void * out, void * clk, void * stream) {
    if (n_bytes % 16 || grid <= 0 || (unroll != 4 && unroll != 16)) return -1;
    if (unroll == 4)
        hipLaunchKernelGGL(k_probe_read<4>, dim3(grid), dim3(256), 0, (hipStream_t) stream, (const u32x4 *) p,
                           n_bytes / 16, (uint32_t *) out, (uint64_t *) clk);
    else
        hipLaunchKernelGGL(k_probe_read<16>, dim3(grid), dim3(256), 0, (hipStream_t) stream, (const u32x4 *) p,
                           n_bytes / 16, (uint32_t *) out, (uint64_t *) clk);
    return (int) hipGetLastError();
}

// grid workgroups of `waves` waves (1..16), each lane `iters` x 8 reads of 16 bytes
int onpu_probe_lds(int grid, int waves, int iters, void * out, void * clk, void * stream) {
    if (grid <= 0 || waves < 1 || waves > 16 || iters <= 0) return -1;
    hipLaunchKernelGGL(k_probe_lds, dim3(grid), dim3(64 * waves), 0, (hipStream_t) stream, iters, (uint32_t *) out,
                       (uint64_t *) clk);
    return (int) hipGetLastError();
}

// grid workgroups of `waves` waves (1..8), each wave iters x 8 MFMAs of 16 x 16 x 32
int onpu_probe_mfma(int grid, int waves, int iters, void * out, void * clk, void * stream) {
    if (grid <= 0 || waves < 1 || waves > 8 || iters <= 0) return -1;
    hipLaunchKernelGGL(k_probe_mfma, dim3(grid), dim3(64 * waves), 0, (hipStream_t) stream, iters, (float *) out,
                       (uint64_t *) clk);
    return (int) hipGetLastError();
}

// mode 0, 1 or 2 (k_probe_coissue); grid workgroups of 8 waves
int onpu_probe_coissue(int mode, int grid, int iters, void * out, void * cyc, void * stream) {
    if (grid <= 0 || iters <= 0 || mode < 0 || mode > 2) return -1;
    hipStream_t st = (hipStream_t) stream;
    if (mode == 0) hipLaunchKernelGGL(k_probe_coissue<0>, dim3(grid), dim3(512), 0, st, iters, (float *) out, (uint64_t *) cyc);
    else if (mode == 1) hipLaunchKernelGGL(k_probe_coissue<1>, dim3(grid), dim3(512), 0, st, iters, (float *) out, (uint64_t *) cyc);
    else hipLaunchKernelGGL(k_probe_coissue<2>, dim3(grid), dim3(512), 0, st, iters, (float *) out, (uint64_t *) cyc);
    return (int) hipGetLastError();
}

}  // extern "C"

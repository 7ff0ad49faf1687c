// The format-specific kernels of libonpu_hip: compiled once per weight format with
// -DONPU_FMT_ID=<0..3> (onpu_common.h OnpuFmt), so the variants build in parallel.
#include "onpu_kern.h"

#ifndef ONPU_FMT_ID
#error "compile with -DONPU_FMT_ID=<format>"
#endif
#define ONPU_CAT2(a, b) a##b
#define ONPU_CAT(a, b) ONPU_CAT2(a, b)
#define FN(name) ONPU_CAT(name##_f, ONPU_FMT_ID)

static constexpr int F = ONPU_FMT_ID;

hipError_t FN(repack)(const uint8_t * st, int64_t sstride, int64_t N, int64_t K, int64_t KB, int64_t NT, uint8_t * out,
                      int64_t ostride, int64_t E, hipStream_t s) {
    k_repack<F><<<dim3((unsigned) KB, (unsigned) NT, (unsigned) E), 64, 0, s>>>(st, sstride, N, K, KB, out, ostride);
    return hipGetLastError();
}

hipError_t FN(dequant)(const uint8_t * W, int64_t N, int64_t K, int64_t KB, int64_t NT, void * out, int bf16,
                       hipStream_t s) {
    k_dequant<F><<<dim3((unsigned) KB, (unsigned) NT), 64, 0, s>>>(W, N, K, KB, out, bf16);
    return hipGetLastError();
}

hipError_t FN(qgemv)(int epi, const QArgs & a, int mb, int rt, int nb, int xl, dim3 grid, int waves, size_t lds,
                     hipStream_t s) {
#define X(e_, mb_, rt_, nb_, xl_)                                                           \
    if (epi == e_ && mb == mb_ && rt == rt_ && nb == nb_ && xl == xl_) {                   \
        k_qgemv<F, mb_, rt_, nb_, e_, xl_><<<grid, waves * 64, lds, s>>>(a);               \
        return hipGetLastError();                                                          \
    }
    ONPU_QGEMV_VARIANTS(X)
#undef X
    return hipErrorInvalidValue;
}

hipError_t FN(qgemm)(const GArgs & a, int ntw, int mb, hipStream_t s) {
    const int64_t gm = (a.M + 16 * mb - 1) / (16 * mb), gn = (a.NT + 4 * ntw - 1) / (4 * ntw);
    const dim3 grid((unsigned) (gm * gn * (a.splits > 1 ? a.splits : 1)));
    if (a.akeys) {                            // argmax keys: one row tile, no split (host checked)
        if (mb == 1 && a.deep) k_qgemm<F, 2, 1, true, true><<<grid, 256, 0, s>>>(a);
        else if (mb == 1) k_qgemm<F, 2, 1, true><<<grid, 256, 0, s>>>(a);
        else if (mb == 2 && a.deep) k_qgemm<F, 2, 2, true, true><<<grid, 256, 0, s>>>(a);
        else if (mb == 2) k_qgemm<F, 2, 2, true><<<grid, 256, 0, s>>>(a);
        else k_qgemm<F, 2, 4, true><<<grid, 256, 0, s>>>(a);
    } else if (mb == 1 && ntw == 2 && a.deep) k_qgemm<F, 2, 1, false, true><<<grid, 256, 0, s>>>(a);
    else if (mb == 2 && ntw == 2 && a.deep) k_qgemm<F, 2, 2, false, true><<<grid, 256, 0, s>>>(a);
    else if (mb == 1 && ntw == 2) k_qgemm<F, 2, 1><<<grid, 256, 0, s>>>(a);
    else if (mb == 2 && ntw == 2) k_qgemm<F, 2, 2><<<grid, 256, 0, s>>>(a);
    else if (mb == 4 && ntw == 2) k_qgemm<F, 2, 4><<<grid, 256, 0, s>>>(a);
    else if (mb != 8) return hipErrorInvalidValue;
    else if (ntw == 4) k_qgemm<F, 4, 8><<<grid, 256, 0, s>>>(a);
    else if (ntw == 3) k_qgemm<F, 3, 8><<<grid, 256, 0, s>>>(a);
    else k_qgemm<F, 2, 8><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t FN(qgemm_sk)(const GArgs & a, int cfg, int grid, hipStream_t s) {
    const size_t lds = (size_t) 2 * 4 * GSK_CFGS[cfg].mbg * 1024;
    if (cfg != 0) return hipErrorInvalidValue;
    if (a.K % 128) k_qgemm_sk<F, 2, 16, 8, true><<<grid, 512, lds, s>>>(a);
    else k_qgemm_sk<F, 2, 16, 8, false><<<grid, 512, lds, s>>>(a);
    return hipGetLastError();
}

hipError_t FN(moe_decode)(const MDArgs & a, int gb, int grid, size_t lds, hipStream_t s) {
    if (gb == 2 && a.dKB <= 6) k_moe_decode<F, 2, 6><<<grid, 512, lds, s>>>(a);
    else if (gb <= 4 && a.dKB <= MD_MAX_DB) k_moe_decode<F, MD_MAX_GB, MD_MAX_DB><<<grid, 512, lds, s>>>(a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t FN(moe_dsplit)(const MSArgs & a, int nw, int sv, size_t lds, hipStream_t s) {
    const dim3 grid((unsigned) a.S, (unsigned) (a.T * a.k));
    const int64_t dq8 = (a.dNTq + 7) / 8, dq16 = (a.dNTq + 15) / 16;
    if (sv == 32) {
        const int64_t gb8 = (a.gKB + 1) / 2, gb16 = (a.gKB + 3) / 4;
        if (nw == 16 && gb16 <= 4 && dq16 <= 2) k_moe_dsplit<F, 4, 2, 16, 32><<<grid, 1024, lds, s>>>(a);
        else if (nw == 16 && gb16 <= 8 && dq16 <= 4) k_moe_dsplit<F, 8, 4, 16, 32><<<grid, 1024, lds, s>>>(a);
        else if (gb8 <= 8 && dq8 <= 4) k_moe_dsplit<F, 8, 4, 8, 32><<<grid, 512, lds, s>>>(a);
        else if (gb8 <= 16 && dq8 <= 8) k_moe_dsplit<F, 16, 8, 8, 32><<<grid, 512, lds, s>>>(a);
        else return hipErrorInvalidValue;
    } else if (sv == 16) {
        const int64_t gb8 = (a.gKB + 3) / 4, gb16 = (a.gKB + 7) / 8;
        if (nw == 16 && gb16 <= 2 && dq16 <= 2) k_moe_dsplit<F, 2, 2, 16, 16><<<grid, 1024, lds, s>>>(a);
        else if (nw == 16 && gb16 <= 4 && dq16 <= 4) k_moe_dsplit<F, 4, 4, 16, 16><<<grid, 1024, lds, s>>>(a);
        else if (gb8 <= 4 && dq8 <= 4) k_moe_dsplit<F, 4, 4, 8, 16><<<grid, 512, lds, s>>>(a);
        else if (gb8 <= 8 && dq8 <= 8) k_moe_dsplit<F, 8, 8, 8, 16><<<grid, 512, lds, s>>>(a);
        else return hipErrorInvalidValue;
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t FN(relayout_dec)(const uint8_t * src, int64_t sstride, int64_t NT, int64_t KB, uint8_t * dst,
                            int64_t dstride, int64_t E, hipStream_t s) {
    const int64_t nsb = 4 * KB * ((NT + 3) / 4);
    k_relayout_dec<F><<<dim3((unsigned) nsb, (unsigned) E), 64, 0, s>>>(src, sstride, NT, KB, dst, dstride);
    return hipGetLastError();
}

hipError_t FN(moe_gemm)(int which, const MArgs & a, dim3 grid, hipStream_t s) {
    const bool kt = a.K % 128 != 0;
    if (which == 0) {
        if (kt) k_moe_gemm<F, 0, true><<<grid, 512, 0, s>>>(a);
        else k_moe_gemm<F, 0, false><<<grid, 512, 0, s>>>(a);
    } else {
        if (kt) k_moe_gemm<F, 1, true><<<grid, 512, 0, s>>>(a);
        else k_moe_gemm<F, 1, false><<<grid, 512, 0, s>>>(a);
    }
    return hipGetLastError();
}

template <int S>
static hipError_t chain_s(const ChainArgs & a, const ChainEntry * ents, int grid, size_t lds, hipStream_t s) {
    k_qgemv_chain<F, S><<<grid, (CHAIN_WAVES + CHAIN_CTRL) * 64, lds, s>>>(a, ents);
    return hipGetLastError();
}

hipError_t FN(chain)(int ring, const ChainArgs & a, const ChainEntry * ents, int grid, size_t lds, hipStream_t s) {
    switch (ring) {
        case 0: return chain_s<CHAIN_RING_SLOTS[0]>(a, ents, grid, lds, s);
        case 1: return chain_s<CHAIN_RING_SLOTS[1]>(a, ents, grid, lds, s);
        case 2: return chain_s<CHAIN_RING_SLOTS[2]>(a, ents, grid, lds, s);
        case 3: return chain_s<CHAIN_RING_SLOTS[3]>(a, ents, grid, lds, s);
    }
    return hipErrorInvalidValue;
}

template <int S>
static int chain_occ_s(size_t lds) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_qgemv_chain<F, S>, (CHAIN_WAVES + CHAIN_CTRL) * 64, lds) !=
        hipSuccess)
        return 0;
    return nb;
}

int FN(chain_occ)(int ring, size_t lds) {
    switch (ring) {
        case 0: return chain_occ_s<CHAIN_RING_SLOTS[0]>(lds);
        case 1: return chain_occ_s<CHAIN_RING_SLOTS[1]>(lds);
        case 2: return chain_occ_s<CHAIN_RING_SLOTS[2]>(lds);
        case 3: return chain_occ_s<CHAIN_RING_SLOTS[3]>(lds);
    }
    return 0;
}

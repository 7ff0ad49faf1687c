// Host-side helpers of libonpu_hip (onpu_quant.cpp).
#pragma once
#include <cstdint>
#include <functional>

namespace onpu {

struct RefGeom {                  // the reference Mat: R, S, tiles, kc, ks, rows_col, cb, nbytes
    int64_t R = 0, S = 0, tiles = 0, kc = 0, ks = 0, rows_col = 0, cb = 0, nbytes = 0;
    bool ok = false;
};

RefGeom ref_geometry(int64_t N, int64_t K, int ncols, bool sym);
bool pack_staging(int fmt, const float * W, int64_t N, int64_t K, uint8_t * out, int threads);
// GGUF Q4_K rows (K / 256 super-blocks of 144 bytes each, rows ld bytes apart) -> q4nx staging
bool pack_q4k_staging(const uint8_t * blocks, int64_t ld, int64_t N, int64_t K, uint8_t * out, int threads);
void dequant_staging(int fmt, const uint8_t * st, int64_t N, int64_t K, float * out, int threads);
// W [N][K] -> the reference's NPU packing (q4s when sym, else q4nx) in geometry rg (rg.nbytes bytes)
bool pack_npu(int sym, const float * W, int64_t N, int64_t K, const RefGeom & rg, uint8_t * out, int threads);

}  // namespace onpu

// ORACLE CHECKER — test infrastructure only; nothing in the product links or calls it.
//
// The reference's own bf16 rounding, `Mat` geometry, per-32 search quantizers, NPU packing and
// output gather, compiled from the reference checkout: oracle/Makefile copies lines 37-254 of
// llama/ggml-opennpu/opennpu_core.hpp (namespace onpu: constants, f2bf / bf2f, Mat, quant_asym32,
// quant_sym32, pack_block_fn, pack_block, pack_mat) and lines 540-561 (gather) unedited into
// oracle/_ref/opennpu_core_37_254.inc and opennpu_core_540_561.inc at build time. Those lines use
// only the standard headers below; the header's XRT includes (lines 6-9) belong to the device code
// between and after them, which is not compiled. This file adds the standard headers, closes the
// namespace that line 37 opens, and exports plain C entry points over many groups at once.
//
// Built twice (oracle/Makefile): as written (-ffp-contract=off, every operation rounded as the
// source states it) and with the reference's own flags (llama/build.sh:74: -O3 -march=native,
// which lets GCC fuse multiply-adds). tests/test_quant_ref.py compares the oracle and the library
// against both.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

#include "opennpu_core_37_254.inc"
#include "opennpu_core_540_561.inc"
}  // namespace onpu (opened by opennpu_core.hpp:37)

extern "C" {

// geometry of Mat(N, K, ncols, sym): R, S, tiles, kc, ks, rows_col, cb, nbytes; zeros if none
void ref_geometry(int64_t N, int64_t K, int ncols, int sym, int64_t * out) {
    const onpu::Mat m(N, K, ncols, sym != 0);
    const int64_t v[8] = {m.R, m.S, m.tiles, m.kc, m.ks, m.rows_col, (int64_t) m.cb, (int64_t) m.nbytes};
    for (int i = 0; i < 8; i++) out[i] = m.ok ? v[i] : 0;
}

// quant_sym32 over `groups` consecutive groups of 32 floats: codes q[groups][32], bf16 d[groups]
void ref_quant_sym32_n(const float * x, int64_t groups, uint8_t * q, uint16_t * d) {
    for (int64_t g = 0; g < groups; g++) onpu::quant_sym32(x + 32 * g, q + 32 * g, d[g]);
}

// quant_asym32 over `groups` groups: codes q[groups][32], bf16 s[groups] and m[groups]
void ref_quant_asym32_n(const float * x, int64_t groups, uint8_t * q, uint16_t * s, uint16_t * m) {
    for (int64_t g = 0; g < groups; g++) onpu::quant_asym32(x + 32 * g, q + 32 * g, s[g], m[g]);
}

// pack_mat(Mat(N, K, ncols, sym), W rows of K, one thread) into out (nbytes); returns nbytes, 0 when
// Mat has no geometry
int64_t ref_pack_mat(const float * W, int64_t N, int64_t K, int ncols, int sym, uint8_t * out) {
    const onpu::Mat m(N, K, ncols, sym != 0);
    if (!m.ok) return 0;
    onpu::pack_mat(m, W, K, out, 1);
    return (int64_t) m.nbytes;
}

// gather(Mat(N, K, ncols, sym), y, 0, 1, out): one matrix's NPU output vector (bf16, R S columns of
// out_tiles(tiles) * 4 * 64 values) -> out [N]
void ref_gather(int64_t N, int64_t K, int ncols, int sym, const uint16_t * y, float * out) {
    const onpu::Mat m(N, K, ncols, sym != 0);
    if (m.ok) onpu::gather(m, y, 0, 1, out);
}

// f2bf over n floats
void ref_f2bf_n(const float * x, int64_t n, uint16_t * out) {
    for (int64_t i = 0; i < n; i++) out[i] = onpu::f2bf(x[i]);
}

}  // extern "C"

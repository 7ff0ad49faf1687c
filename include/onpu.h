/*
 * libonpu_hip: the int4 weight-only matmul operator surface of OpenNPU, implemented for one AMD
 * Instinct MI355X (gfx950) with HIP kernels. It is a drop-in for the reference's libonpu C ABI
 * (llama/ggml-opennpu/onpu_api.cpp, onpu_cpu.cpp), which opennpu/native/npu4/model.py binds with
 * ctypes in clib() (model.py:281-335): set OPENNPU_LIBONPU to this library.
 *
 * Conventions (as in the reference):
 *   - x and y of the host-pointer calls are row-major fp32; x is rounded to bf16 (nearest even)
 *     before the product, y is overwritten and the call is synchronous.
 *   - weights: a handle owns a host buffer (*_buf) that the caller fills (onpu_pack writes it), then
 *     *_sync uploads it to HBM and repacks it into the GPU layout. For q4nx and q4s the buffers of
 *     the reference calls (onpu_dense_new2 on 8 columns, onpu_bank_new2 on ncols, onpu_ffn_new on 1)
 *     hold the reference's NPU packing below, byte for byte, so that bytes packed by the reference
 *     or cached by it (npu4's PackCache, model.py:712-759) load unchanged; the other formats and
 *     the *_new3 handles take the staging layout.
 *   - construction returns NULL for an unsupported shape or format; a HIP failure inside a void
 *     call prints the error and aborts the process (the reference throws across extern "C").
 *     onpu_last_error() reports the last failure of an int-returning call on this thread.
 *   - every call is thread-safe (one library mutex for the host-pointer calls; the *_dev calls
 *     run on the caller's stream).
 *
 * Weight formats (the `sym` argument of the reference calls; 0 and 1 are the reference's):
 *   ONPU_FMT_Q4NX  0  asymmetric, w = u*s + m, 32-wide groups along K, bf16 s and m   (q4nx)
 *   ONPU_FMT_Q4S   1  symmetric,  w = (u-8)*s, 32-wide groups, bf16 s                 (q4s)
 *   ONPU_FMT_G128S 2  symmetric,  w = (u-8)*s, 128-wide groups, bf16 s
 *   ONPU_FMT_Q4_0  3  GGUF Q4_0:  w = (u-8)*d, 32-wide blocks, fp16 d
 * Staging layout of one [N][K] matrix (K % 32 == 0; G128S: K % 128 == 0):
 *   Q4NX : codes u8 [N][K/2] (low nibble = even k), scales bf16 [N][K/32], mins bf16 [N][K/32]
 *   Q4S  : codes u8 [N][K/2], scales bf16 [N][K/32]
 *   G128S: codes u8 [N][K/2], scales bf16 [N][K/128]
 *   Q4_0 : GGUF block_q4_0 rows [N][K/32] x {fp16 d, u8 qs[16]} (element j <- qs[j] & 15,
 *          element j+16 <- qs[j] >> 4)
 * NPU packing of one matrix (pack_mat, opennpu_core.hpp:174-254), in the geometry onpu_geometry2
 * reports (R row blocks of rows_col rows x S K slices of ks columns, cb bytes per column block):
 * column block c = r*S + s at c*cb, all zero if it holds no weight; inside it, packets of 64 rows x
 * 256 columns in the order [tile t][K step kk][core row cr] (rows cr*tiles*64 + t*64 + [0, 64)),
 * each: codes [8 row octets][32 column octets][8 columns][4 bytes of a row pair, even row low],
 * then bf16 scales [8 groups][64 rows], then (q4nx) mins likewise; past the matrix, code 8 (q4s)
 * or 0 (q4nx) and zero parameters.
 * Handles made by the reference calls keep the reference's buffer sizes (onpu_geometry2's nbytes,
 * which the staging layout of formats 2 and 3 always fits in); *_new3 handles use
 * onpu_stage_bytes().
 */
#ifndef ONPU_H
#define ONPU_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ONPU_FMT_Q4NX = 0, ONPU_FMT_Q4S = 1, ONPU_FMT_G128S = 2, ONPU_FMT_Q4_0 = 3 };

/* ---- device (onpu_api.cpp:59-60) */
int onpu_ok(void);                 /* 1 when a gfx950 GPU is usable */
int onpu_batched_ok(void);         /* 1: several rows per call are supported */

/* ---- geometry (onpu_api.cpp:64-69): the reference's Mat (model.py:151-187), so that
 * check_geometry (model.py:353-360) accepts this library; formats 2 and 3 report the q4s sizes */
void onpu_geometry2(int64_t N, int64_t K, int ncols, int sym, int64_t * out /* [8] */);
void onpu_geometry(int64_t N, int64_t K, int ncols, int64_t * out);

/* ---- stats (onpu_api.cpp:72-80) and shapes (:82-84) */
void onpu_stats(int64_t * calls, double * wait_s);
int onpu_has_shape(int tiles, int kc, int batched);

/* ---- dense matrices (onpu_api.cpp:87-156) */
void * onpu_dense_new2(int64_t N, int64_t K, int sym);
void * onpu_dense_new(int64_t N, int64_t K);
uint8_t * onpu_dense_buf(void * h);
int64_t onpu_dense_bytes(void * h);
void onpu_dense_sync(void * h);
void onpu_dense_free(void * h);
/* rows > 64 run the split-K GEMM, whose bounded waits are checked after the call's synchronisation:
 * one that gave up aborts with the reason (the reference's ONPU_ASSERT, opennpu_core.hpp:30-32), or
 * with ONPU_WAIT_TIMEOUT=error sets y to NaN and onpu_last_error */
void onpu_dense_mv(void * h, const float * x, int64_t rows, float * y);

/* ---- expert banks: E experts of [N][K], expert e's staging at e * onpu_bank_expert_bytes
 * (onpu_api.cpp:159-250) */
void * onpu_bank_new2(int64_t N, int64_t K, int64_t E, int ncols, int sym);
void * onpu_bank_new(int64_t N, int64_t K, int64_t E, int ncols);
uint8_t * onpu_bank_buf(void * h);
int64_t onpu_bank_expert_bytes(void * h);
void onpu_bank_sync(void * h);
void onpu_bank_free(void * h);
/* y [T][k][N]: slot (t, j) -> expert ids[t*k+j] applied to x [T][K] (x_per_slot 0) or [T][k][K] */
void onpu_bank_run(void * h, const float * x, int x_per_slot, int64_t T, const int32_t * ids, int k, float * y);

/* ---- routed-expert FFN (onpu_api.cpp:261-278): y [T][N of dn] = sum_j w[t*k+j] *
 * dn_e(act(gu_e x_t + gu_bias[e]) ) + dn_bias[e]; act 0: silu(h[:I]) * h[I:], act 1: gpt-oss */
void onpu_moe_ffn(void * gu, void * dn, const float * x, int64_t T, const int32_t * ids, int k, const float * w,
                  int act, float alpha, float limit, const float * gu_bias, const float * dn_bias, float * y);
/* the CPU helpers of onpu_cpu.cpp:233-274, computed on the GPU (host pointers in and out) */
void onpu_moe_act(const float * h, int64_t rows, int64_t Ng, const int32_t * ids, const float * gu_bias, int act,
                  float alpha, float limit, float * a);
void onpu_moe_sum(const float * o, int64_t T, int k, int64_t N, const int32_t * ids, const float * w,
                  const float * bias, float * y);

/* ---- fused expert FFN (onpu_api.cpp:292-496): gate_up, SiLU * up and down of a token's experts
 * without host round trips. onpu_ffn_perm: the gate_up row the caller packs at each row of gu's
 * buffer; where the reference fuses the shape (onpu_api.cpp:307-322), its order, so that packed
 * banks and cached files carry the reference's bytes (the upload restores the [gate | up] order),
 * else the identity. */
void * onpu_ffn_new(int64_t Ng, int64_t Kg, int64_t Nd, int64_t Kd, int64_t E, int sym);
void * onpu_ffn_gu(void * h);
void * onpu_ffn_dn(void * h);
int onpu_ffn_fused(void * h);
void onpu_ffn_perm(void * h, int32_t * out /* [Ng] */);
/* 1 done, 0 not done (the FFN shape cannot be fused, or, with ONPU_WAIT_TIMEOUT=error, the opt-in
 * one-launch decode's bounded wait gave up: y is then NaN and onpu_last_error says why; without that
 * setting such a wait aborts, as the reference does on a device failure) */
int onpu_ffn_run(void * h, const float * x, const int32_t * ids, int k, const float * w, float * y);
int onpu_ffn_run_many(void * h, const float * x, int64_t T, const int32_t * ids, int k, const float * w, float * y);
void onpu_ffn_free(void * h);

/* ---- packing (onpu_api.cpp:499-529): quantize fp32 W [N][K] with the reference's search
 * quantizers (q4nx / q4s per 32; g128s per 128; Q4_0 as ggml): q4nx and q4s into the reference's
 * NPU packing for ncols columns (its pack_mat's bytes), g128s and Q4_0 into the staging layout,
 * zero-padded; returns onpu_geometry2's nbytes (0: unsupported) */
int64_t onpu_pack(const float * W, int64_t N, int64_t K, int ncols, int sym, uint8_t * out, int threads);
void onpu_quant_dequant(const float * W, int64_t N, int64_t K, int sym, float * out, int threads);

/* ================================================================ MI355X-native extensions
 * No counterpart in the reference: device-pointer entry points for callers whose activations
 * already live in HBM (torch tensors, a serving loop), plus introspection for parity checks. */
const char * onpu_last_error(void);
int64_t onpu_stage_bytes(int fmt, int64_t N, int64_t K);
/* handles whose staging stride is onpu_stage_bytes (no reference padding) */
void * onpu_dense_new3(int64_t N, int64_t K, int fmt);
void * onpu_bank_new3(int64_t N, int64_t K, int64_t E, int fmt);
void * onpu_ffn_new3(int64_t Ng, int64_t Kg, int64_t Nd, int64_t Kd, int64_t E, int fmt);
/* upload staging-layout bytes from caller memory without keeping a staging copy;
 * bank: experts [e0, e0 + n), stage holds n consecutive experts of onpu_stage_bytes each */
int onpu_dense_load(void * h, const void * stage);
int onpu_bank_load(void * h, int64_t e0, int64_t n, const void * stage);
/* the decode-GEMV launch plan (host only): mb, rt, nb, xl, tw, kw, bpw, grid x, built, max waves
 * for an [N][K] matrix of fmt at M rows over `slots` slots; epi 0 store, 1 SiLU-gate, 2 slot sum */
void onpu_plan_gemv(int fmt, int64_t N, int64_t K, int M, int64_t slots, int epi, int64_t * out /* [10] */);
/* what onpu_dense_mv_dev runs for M rows of an [N][K] matrix (host only; no counterpart in the
 * reference, whose NPU dispatch has no such choice): path (0 the decode GEMV, 1 the GEMM with tiles
 * of 16 mb rows, 2 the 256-row stream-K GEMM), mb, weight tiles per wave, K ranges S, K blocks per
 * range, workgroups per range, and 1 if 16-row tiles keep the weights two blocks ahead */
void onpu_plan_mv(int fmt, int64_t N, int64_t K, int64_t M, int64_t * out /* [7] */);
/* N, K, fmt, E, row tiles, K blocks, HBM bytes per expert, HBM base address */
void onpu_dense_info(void * h, int64_t * out /* [8] */);
/* dequantized weights of expert e as the GPU stores them: fp32 (bf16 = 0) or bf16 RNE bits */
int onpu_dense_dequant(void * h, int64_t e, void * out_host, int bf16);
/* y [M][N] = x [M][K] . W^T on `stream` (hipStream_t; NULL: the default stream); x bf16 in HBM,
 * y bf16 (y_f32 = 0) or fp32 in HBM. M <= 64 runs the GEMV kernels (for larger matrices, from 1-64
 * rows up depending on N and K, the MFMA GEMM, which is faster there: onpu_plan_mv), larger M the
 * MFMA GEMM. */
int onpu_dense_mv_dev(void * h, const void * x, int64_t M, void * y, int y_f32, void * stream);
/* Workspace of the calls above. The MFMA GEMM splits K (fp32 partials of K ranges, or the partial
 * tiles and slot words of its 256-row stream-K form above 128 rows) in a workspace of about 64 MiB (kept until the process ends): one per stream for eager
 * calls, one per capture for calls captured into a HIP graph. Its first use allocates it (relaxed
 * capture mode) and clears its slot words with a kernel, both legal under capture, so a first GEMM
 * may be captured (the clearing kernel becomes a node of the graph). The argmax keeps its keys per
 * handle (sized once for 64 rows); when the rows run the GEMM its counters grow with the rows and are cleared by
 * a kernel. Outgrown workspace buffers are kept until the handle is freed, so a graph captured at a
 * small M keeps valid pointers. Argmax calls on one handle share its keys: order them on one
 * stream. */
/* 1 if a split-K GEMM gave up waiting for its partner workgroup since the last call (the flag is then
 * cleared and that launch's Y is invalid), 0 if not, -1 on error; synchronises the device */
int onpu_gemm_status(void);
/* frees the device staging of the host-pointer calls (it grows to the largest call; one set for the
 * library, shared by every handle) */
void onpu_release_scratch(void);
/* logits fp32 [M][N] and argmax [M] (first maximum) */
int onpu_dense_argmax_dev(void * h, const void * x, int64_t M, float * logits, int32_t * argmax, void * stream);
/* onpu_dense_argmax_dev for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc); no counterpart in the reference. It allocates nothing:
 * the argmax's counters and keys live in a 1 MiB device array of the library, one per GPU, set up
 * when the library initialises. Limits: M <= 64 (the GEMV path) and M * ceil(N / 4096) <= 8064;
 * beyond them it returns -1 with the reason in onpu_last_error. Calls that overlap on one GPU
 * share the array and race: order them on one stream. */
int onpu_dense_argmax_dev_noalloc(void * h, const void * x, int64_t M, float * logits, int32_t * argmax,
                                  void * stream);
/* router: logits fp32 [T][E] -> ids [T][k], w [T][k] (softmax, top-k by probability, ties to the
 * lower id, renormalised when renorm != 0) */
int onpu_moe_route_dev(const float * logits, int64_t T, int E, int k, int renorm, int32_t * ids, float * w,
                       void * stream);
/* routed-expert FFN on device data: x bf16 [T][Kg], ids/w [T][k] -> y [T][Nd] (bf16 or fp32).
 * h: an onpu_ffn_new / onpu_ffn_new3 handle. Uses workspace owned by h. */
int onpu_moe_ffn_dev(void * h, const void * x, int64_t T, const int32_t * ids, int k, const float * w, void * y,
                     int y_f32, void * stream);
/* MoE decode step from router logits: logits fp32 [T][E] and x bf16 [T][Kg] in HBM -> ids / w [T][k]
 * (written) and y [T][Nd]. Replaces the reference's host routing plus onpu_ffn_run
 * (onpu_api.cpp:292-496; moe_runtime.py:333-341 for the router) with device work only. T <= 4
 * (ONPU_MOE_DECODE_MAX), k <= 16, E <= 256: two launches, the gate+up GEMV routing its own token in
 * each workgroup (ids / w written there) and the down GEMV with the weighted slot sum; with
 * ONPU_MOE_FUSED=1, k <= 8 and expert shapes that fit, one launch doing all of it (slower on MI355X:
 * its cross-workgroup handoff costs more than the kernel boundary it saves); longer prompts: the
 * router kernel, then onpu_moe_ffn_dev's launches. Calls on one handle must be ordered on one stream
 * (they share the handle's workspace). */
int onpu_moe_decode_dev(void * h, const float * logits, const void * x, int64_t T, int E, int k, int renorm,
                        int32_t * ids, float * w, void * y, int y_f32, void * stream);
/* 1 when a one-launch MoE decode on h gave up waiting for its act tiles since the last call (results
 * invalid; the flag is cleared), 0 otherwise, -1 on error. Synchronises the device. */
int onpu_moe_status(void * h);

/* ---- weight codecs on the GPU (load time). The reference quantizes on the host (onpu_pack,
 * onpu_api.cpp:499-504, with the search quantizers of opennpu_core.hpp:103-169) and transcodes GGUF
 * Q4_K for its ggml backend on the host (ggml-opennpu.cpp:103-138); these run the same codecs on
 * weights already in HBM and write the handle's tiled layout directly. They allocate a temporary
 * staging buffer (at most 256 MiB, or one expert) and return after their launches on `stream`
 * completed; calls on one handle are serialised by the library mutex. 0 ok, -1 error
 * (onpu_last_error). */
/* experts [e0, e0 + n) of a dense (E = 1) or bank handle from W [n][N][ldw] (row stride ldw >= K
 * elements), fp32 (w_bf16 = 0) or bf16 (1), with the handle's format: the codes and parameters
 * onpu_pack writes */
int onpu_quantize_dev(void * h, int64_t e0, int64_t n, const void * W, int64_t ldw, int w_bf16, void * stream);
/* q4nx handle, K a multiple of 256: experts [e0, e0 + n) from GGUF Q4_K rows of K / 256 super-blocks
 * (144 bytes each), rows ld bytes apart, experts N * ld bytes apart */
int onpu_transcode_q4k_dev(void * h, int64_t e0, int64_t n, const void * blocks, int64_t ld, void * stream);
/* the same transcode on the host (replaces ggml-opennpu.cpp:103-138's QuantFn for Q4_K groups):
 * rows of K / 256 super-blocks -> q4nx staging bytes; returns onpu_stage_bytes(q4nx, N, K), 0 when
 * K is not a multiple of 256 */
int64_t onpu_pack_q4k(const uint8_t * blocks, int64_t N, int64_t K, uint8_t * out, int threads);

/* ---- int8 GEMV on the GPU: the reference's host onpu_gemv_i8 (onpu_cpu.cpp:276-299, a MoE's
 * shared expert) with device pointers: y [N] = s[n] * sum_k W[n][k] x[k], W int8 [N][K] (rows of K
 * bytes), s, x, y fp32; K a multiple of 16 and at most 32768, W and x 16-byte aligned. On `stream`;
 * capturable. 0 ok, -1 error (onpu_last_error). */
int onpu_gemv_i8_dev(const int8_t * W, const float * s, int64_t N, int64_t K, const float * x, float * y,
                     void * stream);

/* ---- Gated DeltaNet decode step on the GPU: the reference's host onpu_gdn_step (onpu_cpu.cpp:107-
 * 171, bound by npu4 at model.py:386-391, 646-649) with device pointers and the same arguments:
 * x [H], qkv [C = 2 Hk Dk + Hv Dv], z [Hv Dv], Wb / Wa [Hv][H], conv_w [C][Kc], conv_state [C][L]
 * (updated), A_log / dt_bias [Hv], norm_w [Dv], S [Hv][Dk][Dv] (updated), out [Hv Dv]; plus a
 * device workspace of onpu_gdn_ws_bytes(Hk, Hv, Dk, Dv) bytes. Hv a multiple of Hk, Dv dividing
 * 256, Dk * Dv <= 32768. On `stream`; capturable. 0 ok, -1 error (onpu_last_error). */
int64_t onpu_gdn_ws_bytes(int Hk, int Hv, int Dk, int Dv);
int onpu_gdn_step_dev(const float * x, int H, const float * qkv, const float * z, const float * Wb, const float * Wa,
                      const float * conv_w, int Kc, float * conv_state, int L, const float * A_log,
                      const float * dt_bias, const float * norm_w, float eps, float * S, int Hk, int Hv, int Dk,
                      int Dv, float * out, void * ws, int64_t ws_bytes, void * stream);

/* ---- decode attention on the GPU: the reference's host onpu_attn_step / onpu_attn_step_bf16
 * (onpu_cpu.cpp:173-229, bound by npu4 at model.py:392-397, 612-615) with device pointers, on
 * `stream`. q fp32 [Hq][D]; K, V: Hkv heads of S rows of D values, fp32 (kv_bf16 = 0) or bf16 (1),
 * head stride hs and row stride rs in elements (shared by K and V, rows 16-byte aligned); mask fp32
 * [S] additive or NULL; sinks fp32 [Hq] or NULL (an extra logit per head with no value); out fp32
 * [Hq][D] (q, K and V 16-byte aligned). Hq a multiple of Hkv with Hq / Hkv <= 16, D <= 256 and a multiple of 8. ws: device
 * workspace of onpu_attn_ws_bytes(Hq, D, Hkv, S) bytes (calls in flight together need their own).
 * Capturable in a HIP graph. 0 ok, -1 error (onpu_last_error). */
int64_t onpu_attn_ws_bytes(int Hq, int D, int Hkv, int64_t S);
int onpu_attn_step_dev(const float * q, int Hq, int D, const void * K, const void * V, int kv_bf16, int Hkv, int64_t S,
                       int64_t hs, int64_t rs, const float * mask, const float * sinks, float scale, float * out,
                       void * ws, int64_t ws_bytes, void * stream);

/* ---- chained decode GEMVs (no counterpart in the reference's ABI; the reference's fused decode
 * engine likewise runs a token's products in one NPU dispatch). A chain is n dense GEMVs
 * y_i [M][N_i] = x_i [M][K_i] . W_i^T fixed at creation (handles, x and y device pointers; one
 * weight format; 1 <= M <= 16; y bf16 or fp32); onpu_chain_run executes them in order in ONE launch
 * on `stream`. An x_j that lies in an earlier entry's bf16 output y_i (the whole of y_i with
 * K_j == N_i, or at M = 1 a range of it starting on an 8-element boundary) is read once entry i has
 * written that part of y_i in this run: workgroups wait on the data itself, not on a grid barrier. Every
 * other x is read as it was when the launch started; onpu_chain_new refuses (NULL) an x that
 * overlaps an output in any other way and outputs that overlap. Weights stream ahead through each
 * workgroup's LDS while it waits. All workgroups must be resident together: do not run other kernels
 * concurrently with a chain on the same GPU, and keep runs of one chain ordered on one stream. A
 * wait that exceeds its poll limit (about 0.1 s) gives up rather than hanging; onpu_chain_status
 * then reports 1 (results invalid). The launch is capturable in a HIP graph. */
void * onpu_chain_new(void * const * handles, const void * const * xs, void * const * ys, int n, int64_t M,
                      int y_f32);
int onpu_chain_run(void * chain, void * stream);
/* synchronises the device; 0 ok, 1 a wait timed out since the last call (the flag is then cleared),
 * -1 error */
int onpu_chain_status(void * chain);
void onpu_chain_info(void * chain, int64_t * out /* [6]: n, workgroups, LDS bytes, x row stride,
                                                   weight-ring blocks per wave, runs completed
                                                   (synchronises) */);
void onpu_chain_free(void * chain);

#ifdef __cplusplus
}
#endif
#endif

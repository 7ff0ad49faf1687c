// libonpu_hip: the reference's libonpu C ABI (llama/ggml-opennpu/onpu_api.cpp, onpu_cpu.cpp) over
// HIP on one MI355X, plus device-pointer entry points. Declarations and conventions:
// include/onpu.h.
//
// A handle (Mat4) holds one matrix or an expert bank: the weights in HBM in the tiled layout of
// onpu_common.h, and (lazily) a host staging buffer in the staging layout that *_sync uploads.
// Host-pointer calls take the library mutex and run on the library's stream; *_dev calls run on
// the caller's stream and touch only the handle's own workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "onpu.h"
#include "onpu_codec.h"
#include "onpu_common.h"
#include "onpu_host.h"
#include "onpu_launch.h"

using namespace onpu;

namespace {

std::mutex g_mu;                          // serialises host-pointer calls (as onpu_api.cpp:53)
thread_local std::string g_err;
std::atomic<int64_t> g_calls{0};
double g_wait_s = 0;                      // guarded by g_mu

[[noreturn]] void die(const char * what, hipError_t e) {
    std::fprintf(stderr, "libonpu_hip: %s failed: %s\n", what, hipGetErrorString(e));
    std::abort();
}
void set_err(const char * what, hipError_t e) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
}
void set_err(const char * what) { g_err = what; }

// void calls abort on a HIP failure (the reference throws across extern "C"); int calls return -1
#define HIPX(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) die(#call, e_); } while (0)
#define HIPR(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { set_err(#call, e_); return -1; } } while (0)

struct Device {
    int ok = 0;
    int cus = 0;
    hipStream_t stream = nullptr;
    hipError_t scratch = hipErrorNotInitialized;   // set-up of the argmax scratch array on device 0
};

Device & device() {
    static Device d;
    static std::once_flag once;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, 0) != hipSuccess) return;
        if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {
            std::fprintf(stderr, "libonpu_hip: device 0 is %s; this library is built for gfx950 only\n",
                         p.gcnArchName);
            return;
        }
        if (hipSetDevice(0) != hipSuccess) return;
        d.cus = p.multiProcessorCount;
        if (hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking) != hipSuccess) return;
        // the no-allocation argmax's scratch array on device 0: its address and zeroed counters
        d.scratch = argmax_scratch_init();
        d.ok = 1;
    });
    return d;
}

// Grow-only device buffer, freed with its owner. Buffers of the device-pointer calls (which a caller
// may capture into a HIP graph) keep every allocation they outgrow until release(): a graph captured
// at a smaller size holds the old pointer, and later calls at a larger size must not free it under
// the graph's replays. Allocation runs in relaxed capture mode (hipMalloc is not stream-ordered), so
// a first call may come under capture.
struct DBuf {
    void * p = nullptr;
    size_t n = 0;
    bool keep = false;                     // keep outgrown allocations until release()
    std::vector<void *> old;
    hipError_t ensure(size_t bytes) {
        if (bytes <= n) return hipSuccess;
        if (p) {
            if (keep) old.push_back(p);
            else (void) hipFree(p);
        }
        p = nullptr;
        n = 0;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        hipError_t e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return e;
        e = hipMalloc(&p, std::max<size_t>(bytes, 256));
        (void) hipThreadExchangeStreamCaptureMode(&mode);
        if (e == hipSuccess) n = std::max<size_t>(bytes, 256);
        else p = nullptr;
        return e;
    }
    void release() {
        if (p) (void) hipFree(p);
        for (void * q : old) (void) hipFree(q);
        old.clear();
        p = nullptr;
        n = 0;
    }
    template <class T> T * as(size_t byte_off = 0) const { return (T *) ((char *) p + byte_off); }
};

// staging of the host-pointer calls (x, ids, w, biases, outputs on the device): one set for the
// library, since those calls hold g_mu and run one at a time on the library's stream; it grows to
// the largest call and is released by onpu_release_scratch
DBuf g_hws[12];

struct Mat4 {                              // one [N][K] matrix (E = 1) or a bank of E experts
    int fmt = 0;
    int64_t N = 0, K = 0, E = 1;
    Tiled g{};
    int64_t dstride = 0;                   // HBM bytes per expert (tiled layout, 256-aligned)
    uint8_t * dev = nullptr;
    uint8_t * stage = nullptr;             // host staging, E * sstride bytes (lazy)
    int64_t sstride = 0;
    // handles of the reference's constructors for q4nx / q4s: *_buf holds the reference's NPU
    // packing in geometry rg (sstride = rg.nbytes per expert), turned into the staging layout on the
    // device at *_sync; rowmap (device, N entries, or null): the staging row of each packed row
    bool npu = false;
    RefGeom rg{};
    int32_t * rowmap = nullptr;
    // argmax workspace of the _dev calls on this handle (kept across growth: see DBuf)
    DBuf am_keys{nullptr, 0, true};        // per-workgroup keys of the GEMV's or the small GEMM's epilogue
    DBuf am_big{nullptr, 0, true};         // keys of the argmax launch over the logits
    DBuf am_cnt{nullptr, 0, true};         // its row counters (zeroed once; each call leaves them zero)
    // the step-major copy of every expert (the down bank of a fused FFN; k_moe_dsplit reads it),
    // dec_stride bytes per expert, kept equal to the tiled weights by every write of them
    uint8_t * dec = nullptr;
    int64_t dec_stride = 0;
};

struct Ffn {
    Mat4 * gu = nullptr, * dn = nullptr;
    bool fused = false;
    // ffn_core: decode act; prompt permutation, items, act, o. k_moe_decode: act rows, counters
    // (zeroed once). All on the device-pointer calls' paths: kept across growth (see DBuf).
    DBuf ws[7] = {{nullptr, 0, true}, {nullptr, 0, true}, {nullptr, 0, true}, {nullptr, 0, true},
                  {nullptr, 0, true}, {nullptr, 0, true}, {nullptr, 0, true}};
    DBuf md_act{nullptr, 0, true}, md_sync{nullptr, 0, true};
    DBuf ds_part{nullptr, 0, true};        // k_moe_dsplit partial sums, sized once for its largest call
    std::vector<int32_t> perm;             // gate_up row packed at each row of gu's buffer (onpu_ffn_perm)
};

int64_t round_up(int64_t a, int64_t b) { return (a + b - 1) / b * b; }

Mat4 * make_mat(int64_t N, int64_t K, int64_t E, int fmt, int64_t sstride) {
    if (!device().ok) { set_err("no usable gfx950 GPU"); return nullptr; }
    if (!fmt_valid(fmt) || N <= 0 || K <= 0 || E <= 0 || K % fmt_group(fmt) != 0) {
        set_err("matrix shape or weight format not supported");
        return nullptr;
    }
    if (sstride < stage_bytes(fmt, N, K)) { set_err("staging buffer smaller than the staging layout"); return nullptr; }
    auto * m = new Mat4;
    m->fmt = fmt;
    m->N = N;
    m->K = K;
    m->E = E;
    m->g = tiled_geom(fmt, N, K);
    m->dstride = round_up(m->g.bytes, 256);
    m->sstride = sstride;
    if (const hipError_t e = hipMalloc((void **) &m->dev, (size_t) (m->dstride * E)); e != hipSuccess) {
        set_err("hipMalloc of the weights", e);
        delete m;
        return nullptr;
    }
    return m;
}

void free_mat(Mat4 * m) {
    if (!m) return;
    if (m->dev) (void) hipFree(m->dev);
    if (m->dec) (void) hipFree(m->dec);
    if (m->rowmap) (void) hipFree(m->rowmap);
    std::free(m->stage);
    m->am_keys.release();
    m->am_big.release();
    m->am_cnt.release();
    delete m;
}

uint8_t * stage_of(Mat4 * m) {
    if (!m->stage) {
        m->stage = (uint8_t *) std::calloc((size_t) (m->E * m->sstride), 1);
        if (!m->stage) { std::fprintf(stderr, "libonpu_hip: out of host memory for staging\n"); std::abort(); }
    }
    return m->stage;
}

// experts [e0, e0 + n) of the step-major copy from the tiled weights (nothing without a copy)
hipError_t refresh_dec(Mat4 * m, int64_t e0, int64_t n, hipStream_t s) {
    if (!m->dec || n <= 0) return hipSuccess;
    return launch_relayout_dec(m->fmt, m->dev + e0 * m->dstride, m->dstride, m->N, m->K, m->dec + e0 * m->dec_stride,
                               m->dec_stride, n, s);
}

// experts [e0, e0 + n) from host bytes (stride src_stride per expert) -> HBM tiled layout. The bytes
// are the staging layout, or (npu_src) the reference's NPU packing of m->rg, which a kernel first
// turns into the staging layout. Through a device temporary of at most 256 MiB (or one expert),
// freed before returning.
hipError_t upload(Mat4 * m, int64_t e0, int64_t n, const uint8_t * src, int64_t src_stride, bool npu_src,
                  hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t sb = round_up(stage_bytes(m->fmt, m->N, m->K), 256);
    const int64_t chunk = std::max<int64_t>(
        1, std::min<int64_t>(n, ((int64_t) 256 << 20) / (src_stride + (npu_src ? sb : 0))));
    const int64_t raw_bytes = round_up(chunk * src_stride, 256);
    void * tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, (size_t) (raw_bytes + (npu_src ? chunk * sb : 0)));
    if (e != hipSuccess) return e;
    uint8_t * raw = (uint8_t *) tmp, * st = raw + raw_bytes;
    const NpuGeom g = npu_geom(m->rg.S, m->rg.tiles, m->rg.kc, m->rg.ks, m->rg.rows_col, m->rg.cb, m->fmt == ONPU_Q4S);
    for (int64_t c = 0; c < n && e == hipSuccess; c += chunk) {
        const int64_t k = std::min(chunk, n - c);
        e = hipMemcpyAsync(raw, src + c * src_stride, (size_t) (k * src_stride), hipMemcpyHostToDevice, s);
        if (e == hipSuccess && npu_src)
            e = launch_npu_stage(m->fmt, raw, src_stride, g, m->rowmap, m->N, m->K, st, sb, k, s);
        if (e == hipSuccess)
            e = launch_repack(m->fmt, npu_src ? st : raw, npu_src ? sb : src_stride, m->N, m->K,
                              m->dev + (e0 + c) * m->dstride, m->dstride, k, s);
        if (e == hipSuccess) e = refresh_dec(m, e0 + c, k, s);
    }
    const hipError_t es = hipStreamSynchronize(s);
    (void) hipFree(tmp);
    return e == hipSuccess ? es : e;
}

// ------------------------------------------------------------------ launch plans
int env_int(const char * name, int dflt) {
    const char * v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

// poll limit of the kernels' bounded waits (split-K exchange, one-launch MoE decode). ONPU_SPIN_LIMIT
// overrides it; 0 makes every such wait give up without polling, so that a test can force the
// timed-out path from the host while every kernel still ends normally.
uint32_t spin_limit(uint32_t dflt) {
    const char * v = std::getenv("ONPU_SPIN_LIMIT");
    return v && *v ? (uint32_t) std::strtoul(v, nullptr, 10) : dflt;
}

struct Plan {
    int mb = 1, rt = 1, nb = 2, xl = 0, tw = 1, kw = 1;
    int64_t bpw = 1, gx = 1;                 // K blocks per wave; grid.x (tile groups / tw)
    int waves() const { return tw * kw; }
};

// Workgroup = tw tile groups x kw K parts; each wave streams bpw K blocks of its tile group (rt row
// tiles) through a two-chunk pipeline of nb blocks. The plan aims at ~4096 waves with an equal
// contiguous share of 4..8 blocks (4..8 KiB of nibbles) each (up to 32, a whole row tile, when
// there are 4096 or more tile groups, as for a vocabulary-sized LM head), at most 2 tile groups per
// workgroup (4 with several x rows, whose LDS staging then serves more tiles; 8 for the vocabulary-
// sized case, where the x copy per workgroup is the cost to share) with at least 512 workgroups,
// and x staged in LDS (xl) when M rows of K and their column sums fit in 52 KiB (112 KiB with
// 1024 or more tile groups).
// ACT pairs gate tile t with up tile t + NT/2, so tw divides NT/2 there. (Sweeps of kw, tw and nb
// over the Qwen3-8B and 151936-row LM-head shapes on MI355X put the optimum there.)
Plan plan_gemv(int fmt, int64_t NT, int64_t KB, int M, int64_t slots, int epi) {
    Plan p;
    p.mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    const bool act = epi == EPI_ACT_;
    p.rt = act ? 2 : 1;
    // two row tiles per wave for a plain store (tile t and t + stride, sharing each x fragment)
    const int ert = env_int("ONPU_GEMV_RT", 0);
    if (ert == 2 && epi == EPI_STORE_ && p.mb == 1 && slots == 1) p.rt = 2;
    const int64_t xbytes = (int64_t) M * (KB * 128 + 8) * 2 + KB * (fmt == ONPU_G128S ? 1 : 4) * 64;
    // gfx950 gives a workgroup up to 160 KiB of LDS. x in LDS up to 52 KiB keeps several workgroups
    // per CU; up to 112 KiB (one workgroup per CU) only pays off with many tile groups to share it
    const int64_t groups0 = act ? NT / 2 : (p.rt == 2 ? (NT + 1) / 2 : NT);
    p.xl = (p.mb == 1 && (xbytes <= 52 * 1024 || (xbytes <= 112 * 1024 && groups0 * slots >= 1024))) ? 1 : 0;
    const int ex = env_int("ONPU_GEMV_XL", -1);
    if (ex == 0) p.xl = 0;
    if ((ex == 1 || ex == 2) && p.mb == 1 && xbytes <= 144 * 1024) p.xl = ex;
    const int64_t groups = groups0;
    // vocabulary-sized matrices (>= 4096 tile groups) stream whole rows per wave (up to 32 blocks)
    // in workgroups of up to 8 tile groups sharing one x copy: measured on the 151936 x 4096 LM head,
    // M = 5: 65.7 us against 75.0 us with two K parts per tile and 4 tiles (M = 1: equal)
    const bool vocab = groups * slots >= 4096;
    // (4096 x 12288 at M = 1: 6 blocks per wave, 8.19 us, against 8.74 us with 12, interleaved on one
    // box; at M = 4 and 8 the two are equal)
    int64_t per = std::min<int64_t>(vocab ? 32 : 8, std::max<int64_t>(4, (groups * slots * KB + 4095) / 4096));
    int64_t kw = std::min<int64_t>(16, std::max<int64_t>(1, (KB + per - 1) / per));
    // K parts a power of two (more blocks per wave up to 8 until they are): 10240 x 4096 and
    // 12288 x 4096 at M = 1 took 8.61 / 8.62 us with 7 and 6 K parts of 5 and 6 blocks, 7.68 / 7.98
    // with 4 of 8 (graphs of 36 copies, one box)
    while (!vocab && per < 8 && (kw & (kw - 1)) != 0) {
        per++;
        kw = std::min<int64_t>(16, std::max<int64_t>(1, (KB + per - 1) / per));
    }
    const int ekw = env_int("ONPU_GEMV_KW", 0);
    if (ekw > 0) kw = std::min<int64_t>(ekw, KB);
    p.bpw = (KB + kw - 1) / kw;
    p.kw = (int) ((KB + p.bpw - 1) / p.bpw);
    p.nb = p.bpw >= 2 ? 2 : 1;
    const int en = env_int("ONPU_GEMV_NB", 0);
    if (en > 0) p.nb = en;
    // the largest built chunk size not above the wish, with x in LDS if built, else from global;
    // (rt, nb = 1, xl = 0) is built for every epilogue and MB
    int pick = 0;
    for (int xl : {p.xl, 0}) {
        for (int nb = p.nb; nb >= 1 && !pick; nb--)
            if (qgemv_has_variant(epi, p.mb, p.rt, nb, xl)) { p.nb = nb; p.xl = xl; pick = 1; }
        if (pick) break;
    }
    if (!pick) { p.nb = 1; p.xl = 0; }
    // the reduction buffer (waves x rt x mb KiB) <= 32 KiB and, with x in LDS, <= 160 KiB together
    const int64_t red_kib =
        p.xl ? std::min<int64_t>(32, (163840 - xbytes - (epi == EPI_ARGMAX_ ? 1024 : 0)) / 1024) : 32;
    const int maxw = std::max(1, std::min(qgemv_max_waves(p.mb, p.rt, p.nb, p.xl), (int) (red_kib / (p.rt * p.mb))));
    if (p.kw > maxw) {                               // more K per wave
        p.kw = maxw;
        p.bpw = (KB + p.kw - 1) / p.kw;
        p.kw = (int) ((KB + p.bpw - 1) / p.bpw);
    }
    int tw = std::max(1, std::min(vocab ? 8 : (M > 1 ? 4 : 2), maxw / p.kw));
    while (tw > 1 && (tw * p.kw * p.rt * p.mb > red_kib || (groups + tw - 1) / tw * slots < 512 ||
                      (act && groups % tw != 0)))
        tw--;
    const int etw = env_int("ONPU_GEMV_TW", 0);
    if (etw > 0 && etw * p.kw <= maxw && etw * p.kw * p.rt * p.mb <= red_kib && !(act && groups % etw))
        tw = etw;
    // One x row, plans measured on MI355X for the shapes of larger models (graphs of 36 copies, us per
    // launch against the rule above; the Qwen3-8B matrices and the LM head keep theirs):
    //   >= 2048 tile groups: 4 K parts of more blocks (57344 x 8192: 40.9 against 50.6; 34816 x 5120:
    //     19.4 against 21.8; 51200 x 5120: 26.2 against 29.6)
    //   x too long for LDS: single-block chunks over 8 K parts, two tile groups per workgroup
    //     (8192 x 28672: 32.9 against 38.2; 5120 x 25600: 28.2 against 31.6)
    //   one to two workgroups per CU of at least 5 blocks per wave: twice the tile groups per
    //     workgroup, so that each CU holds one (5120 x 17408: 13.7 against 17.4; 7168 x 5120: 7.1
    //     against 7.6; 5120 x 5120: 6.9 against 7.0; 8192 x 8192: 9.1 against 9.2)
    if (M == 1 && p.mb == 1 && (epi == EPI_STORE_ || epi == EPI_ARGMAX_) && !vocab && slots == 1 && ekw == 0 &&
        etw == 0 && en == 0 && ex < 0 && ert == 0) {
        const int64_t cus = device().cus > 0 ? device().cus : 256;
        int ckw = 0, ctw = 0;
        if (groups >= 2048) {
            ckw = 4;
        } else if (p.xl == 0) {
            ckw = 8;
            ctw = 2;
            if (qgemv_has_variant(epi, p.mb, p.rt, 1, 0)) p.nb = 1;
        } else if ((groups + tw - 1) / tw > cus && (groups + tw - 1) / tw <= 2 * cus && p.bpw >= 5) {
            if (2 * tw * p.kw <= maxw) ctw = 2 * tw;
            else if (p.kw >= 2) { ckw = p.kw / 2; ctw = 2 * tw; }
        }
        if (ckw) {
            p.bpw = (KB + ckw - 1) / ckw;
            p.kw = (int) ((KB + p.bpw - 1) / p.bpw);
            tw = std::max(1, std::min(tw, maxw / p.kw));
        }
        if (ctw && ctw * p.kw <= maxw && ctw * p.kw * p.rt * p.mb <= red_kib) tw = ctw;
    }
    // Several x rows (M > 1, one A block, plain store): plans measured per shape class on MI355X (the
    // Qwen3-8B matrices at M = 4 / 8, graphs of 36 copies, us per launch against the rule above). The
    // x copy per workgroup grows with M, so fewer and wider workgroups share it, and long K streams in
    // single-block chunks:
    //   <= 256 tile groups, K <= 4096 (4096 x 4096): 16 K parts of 2 blocks, x from global memory,
    //     5.61 / 6.07 against 6.80 / 6.49
    //   <= 512 tile groups (6144 x 4096): two tile groups per workgroup sharing x in LDS (up to
    //     112 KiB), 6.92 / 8.29 against 8.07 / 8.76
    //   >= 1024 tile groups at M > 4 (24576 x 4096): six tile groups of 2 K parts, 15.06 against 15.50
    //   K >= 8192 (4096 x 12288): single-block chunks, 10.07 / 10.71 against 10.48 / 11.33; with
    //     x too long for LDS and K >= 16384, 8 K parts of more blocks (8192 x 28672: 33.0 / 36.9
    //     against 34.4 / 38.4; 5120 x 17408: 20.5 / 23.3 against 22.3 / 24.7)
    //   >= 2048 tile groups, up to 8 rows (57344 x 8192, 34816 x 5120): six tile groups of 2 K
    //     parts, x staged with the MFMA group sums where it fits, 48.6 / 61.3 against 67.5 / 79.1 and
    //     21.9 / 26.9 against 25.5 / 29.0
    // The argmax epilogue takes the same plans, so that its logits equal those of a plain store
    // followed by the separate argmax launch, bit for bit.
    if (M > 1 && p.mb == 1 && (epi == EPI_STORE_ || epi == EPI_ARGMAX_) && !vocab && slots == 1 && ekw == 0 &&
        etw == 0 && en == 0 && ex < 0 && ert == 0) {
        int ckw = 0, ctw = 0, cnb = 0, cxl = -1;
        // x rows without their sums, as the MFMA-sum variant (up to 8 rows) stages them
        const int64_t xrows = (int64_t) M * (KB * 128 + 8) * 2;
        if (groups >= 2048 && M <= 8) {
            ckw = 2;
            ctw = 6;
            if (xrows + 12 * 1024 + (epi == EPI_ARGMAX_ ? 1024 : 0) <= 163840) cxl = 2;
        }
        else if (groups <= 256 && KB <= 32) { ckw = 16; ctw = 1; cnb = 1; cxl = 0; }
        else if (KB >= 64) {
            cnb = 1;
            if (p.xl == 0 && KB >= 128) ckw = 8;
        }
        else if (groups <= 512) { ctw = 2; cxl = xbytes <= 112 * 1024 ? 1 : -1; }
        else if (groups >= 1024 && M > 4) { ckw = 2; ctw = 6; }
        if (ckw) {
            p.bpw = (KB + ckw - 1) / ckw;
            p.kw = (int) ((KB + p.bpw - 1) / p.bpw);
        }
        if (cnb && qgemv_has_variant(epi, p.mb, p.rt, cnb, cxl >= 0 ? cxl : p.xl)) p.nb = cnb;
        if (cxl >= 0 && qgemv_has_variant(epi, p.mb, p.rt, p.nb, cxl)) p.xl = cxl;
        if (ctw) tw = ctw;
        if (tw * p.kw > qgemv_max_waves(p.mb, p.rt, p.nb, p.xl) || tw * p.kw * p.rt * p.mb > red_kib) {
            tw = std::max(1, std::min(tw, qgemv_max_waves(p.mb, p.rt, p.nb, p.xl) / p.kw));
            while (tw > 1 && tw * p.kw * p.rt * p.mb > red_kib) tw--;
        }
    }
    // x in LDS, up to 8 rows: the variant that sums x's groups on the MFMAs and leaves them out of
    // LDS, where it measured faster with the plan pinned (Qwen3-8B shapes, per launch, staged xl = 1
    // against xl = 2 alternating in one process, repeated on several boxes):
    //   per-32 formats (q4nx, q4s, Q4_0; four staged sums per block): 0.1-1.0 us faster at every
    //     shape and row count;
    //   g128s: 0.4-0.9 us faster at 2-8 rows for waves of at most 4 blocks (QKV), 0.8 / 1.6 us at
    //     4 / 8 rows for waves of 5 (7168 x 5120); 0.2 us slower at one row; for gate+up (8-16 blocks
    //     per wave) -1.4 to +1.4 us from box to box, so that keeps the staged sums;
    //   the 151936 x 4096 LM head (Q4_0): 0.6-1.3 us faster at 4-7 rows, 87.4 -> 68.7 us at 8 (its
    //     workgroup then fits twice per CU), 0.6-1.0 us slower at 1-2 rows.
    const bool msums = M <= 8 && (vocab ? M >= 4 : fmt != ONPU_G128S || (M > 1 && p.bpw < 8));
    if (p.xl == 1 && msums && ex < 0 && qgemv_has_variant(epi, p.mb, p.rt, p.nb, 2)) p.xl = 2;
    // vocabulary-sized matrices with K parts (K > 4096): single-block chunks (128256 x 8192 and
    // 151936 x 5120: 83.8 / 63.7 us against 92.8 / 74.9 at M = 1, 100.1 / 73.6 against 101.8 / 81.8
    // at M = 5; at K = 4096, one K part, the two-block chunks stay faster)
    if (vocab && p.kw >= 2 && en == 0 && qgemv_has_variant(epi, p.mb, p.rt, 1, p.xl)) p.nb = 1;
    p.tw = tw;
    p.gx = (groups + tw - 1) / tw;
    return p;
}

// MoE decode down projection with the weighted slot sum: one workgroup per row tile holds the k
// slots x ksplit K parts (kw = k * ksplit waves, returned in kw); kw = 0 when k slots do not fit
Plan plan_slotsum(int64_t KB, int k) {
    Plan p;
    p.rt = 1;
    p.tw = 1;
    int ksplit = 1;
    while (k * ksplit * 2 <= 16 && ksplit * 2 <= KB) ksplit *= 2;
    p.bpw = (KB + ksplit - 1) / ksplit;
    p.kw = 0;
    for (int nb : {3, 2, 1})                         // largest chunk whose launch bound holds the waves
        if (nb <= std::max<int64_t>(1, p.bpw) && qgemv_has_variant(EPI_SLOTSUM_, 1, 1, nb, 0) &&
            k * ksplit <= qgemv_max_waves(1, 1, nb, 0)) {
            p.nb = nb;
            p.kw = k * ksplit;
            break;
        }
    return p;
}

// y [M][N] = x [M][K] (bf16, device) . W_e^T, M rows
// Stream-K plan of k_qgemm_sk for M rows: configuration, grid and K-block iterations per workgroup.
// Every CU gets one workgroup and an equal share of the tiles * KB iterations when there are at least
// as many tiles as CUs; with half as many, each tile is split in two K halves. False (use k_qgemm)
// when neither holds or when some tile would be cut by more than one workgroup boundary.
bool plan_gsk(int64_t M, int64_t NT, int64_t KB, int cus, int & cfg, int64_t & grid, GArgs & a) {
    cfg = 0;
    if (cus <= 0) return false;
    const GskCfg c = GSK_CFGS[cfg];
    const int64_t MT = 16 * c.mbg, TPW = (int64_t) c.ntw * c.wv;
    const int64_t tiles = ((M + MT - 1) / MT) * ((NT + TPW - 1) / TPW), total = tiles * KB;
    // two-phase: whole tiles in step, then the remainder cut once per tile at s. A head piece
    // (blocks 0 .. s) and c = ceil(R / (cus - R)) tail pieces of KB - s blocks per workgroup each end
    // in a partial-tile exchange that takes about E blocks' time (publishing or adding 256 KiB of
    // fp32: 8-9 us against 3.9 us per block, Llama-3.1-8B FFN on MI355X), so s + E = c (KB - s + E)
    constexpr int64_t E = 2;
    const int64_t F = tiles / cus, R = tiles % cus;
    if (env_int("ONPU_GSK_SCHED", 1) == 1 && (F > 0 || 2 * R >= cus) && (R == 0 || KB >= 2)) {
        a.sched = 1;
        a.F = F;
        a.R = R;
        a.c = R ? (R + (cus - R) - 1) / (cus - R) : 0;
        a.s = R ? std::min<int64_t>(KB - 1, std::max<int64_t>(1, (a.c * KB + (a.c - 1) * E + (a.c + 1) / 2) / (a.c + 1)))
                : KB;
        a.ipw = KB;
        a.sym = R > 0 && a.c == 1 && env_int("ONPU_GSK_SYM", 1) ? 1 : 0;
        grid = cus;
        return true;
    }
    a.sched = 0;
    a.sym = 0;
    int64_t & ipw = a.ipw;
    if (tiles >= cus) ipw = (total + cus - 1) / cus;
    else if (2 * tiles >= cus && KB % 2 == 0) ipw = KB / 2;
    else return false;
    grid = (total + ipw - 1) / ipw;
    if (grid > cus) return false;
    int64_t last = -1;                     // tile of the previous interior boundary
    for (int64_t j = 1; j < grid; j++) {
        const int64_t B = j * ipw;
        if (B % KB == 0) continue;
        if (B / KB == last) return false;
        last = B / KB;
    }
    return true;
}

// k_qgemm_sk workspace: partial tiles, the slot words and the control words. Eager launches use
// their stream's (launches on one stream run in order, so they share it safely; launches on
// different streams get different workspaces); a launch captured into a graph uses a workspace of
// its own capture, so graphs captured on one stream (torch.cuda.graph without stream= captures
// every graph on one side stream) never share one, whatever streams they are replayed on.
struct GskWs { DBuf part, sync; };
struct GskKey {
    hipStream_t s;
    unsigned long long capture;            // capture id, 0 for eager launches
    bool operator==(const GskKey & o) const { return s == o.s && capture == o.capture; }
};
std::mutex g_gsk_mu;
std::vector<std::pair<GskKey, GskWs *>> g_gsk;           // a few streams and graphs: a linear search

// The split-K workspace of stream s (or of its capture in progress), created on the first split-K
// call at its full size (a partial tile for every CU: a launch cuts at most one tile per workgroup
// and runs at most one workgroup per CU), so it never moves: a graph that captured a GEMM keeps
// valid pointers. Its sync words are cleared by a kernel on s (under capture, a node of the graph
// ahead of the GEMM), so the first call may be captured. Each one is 64 MiB, held until the process
// ends.
// bytes of a split-K workspace's partials: a 256 x 256 fp32 partial tile per CU
size_t gsk_part_bytes(int cus) {
    size_t slot = 0;
    for (const GskCfg & c : GSK_CFGS) slot = std::max(slot, (size_t) c.wv * c.mbg * c.ntw * 1024);
    return slot * (size_t) std::max(cus, 0);
}

hipError_t gsk_workspace(hipStream_t s, int64_t cut, float ** part, int32_t ** sync, int32_t ** ctl) {
    if (cut > device().cus) return hipErrorInvalidValue;
    hipStreamCaptureStatus cst = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (const hipError_t e = hipStreamGetCaptureInfo(s, &cst, &cid); e != hipSuccess) return e;
    const GskKey key{s, cst == hipStreamCaptureStatusActive ? cid : 0ull};
    std::lock_guard<std::mutex> lk(g_gsk_mu);
    GskWs * w = nullptr;
    for (auto & p : g_gsk)
        if (p.first == key) w = p.second;
    if (!w) {
        w = new GskWs;
        const int64_t ints = (int64_t) device().cus * GSK_SYNC_STRIDE + GSK_CTL_INTS;
        // hipMalloc is not stream-ordered: relaxed mode lets it run while this thread captures
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        hipError_t e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) {
            delete w;
            return e;
        }
        e = w->part.ensure(gsk_part_bytes(device().cus));
        if (e == hipSuccess) e = w->sync.ensure((size_t) ints * 4);
        (void) hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess || (e = launch_zero_i32(w->sync.as<int32_t>(), ints, s)) != hipSuccess) {
            w->part.release();
            w->sync.release();
            delete w;
            return e;
        }
        g_gsk.emplace_back(key, w);
    }
    *part = w->part.as<float>();
    *sync = w->sync.as<int32_t>();
    *ctl = w->sync.as<int32_t>((size_t) device().cus * GSK_SYNC_STRIDE * 4);
    return hipSuccess;
}

int32_t * gsk_err_word(GskWs * w) {
    return w->sync.as<int32_t>(((size_t) device().cus * GSK_SYNC_STRIDE + GSK_CTL_ERR) * 4);
}

// the timed-out-wait flag of stream s's eager workspace, read after the stream has finished: 1 if
// set (then cleared), 0 if not or if s has none, -1 on a HIP failure
int gsk_take_flag(hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_gsk_mu);
    for (auto & p : g_gsk) {
        if (!(p.first == GskKey{s, 0ull})) continue;
        int32_t flag = 0;
        if (hipMemcpy(&flag, gsk_err_word(p.second), 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
        if (flag && hipMemset(gsk_err_word(p.second), 0, 4) != hipSuccess) return -1;
        return flag != 0;
    }
    return 0;
}

// the timed-out-wait flags of every split-K workspace: 1 if any was set (then cleared)
int gsk_status() {
    std::lock_guard<std::mutex> lk(g_gsk_mu);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    int any = 0;
    for (auto & p : g_gsk) {
        int32_t * f = gsk_err_word(p.second);
        int32_t flag = 0;
        if (hipMemcpy(&flag, f, 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
        if (flag && hipMemset(f, 0, 4) != hipSuccess) return -1;
        any |= flag != 0;
    }
    return any;
}

// the decode GEMV (M <= 64 rows): no workspace
hipError_t gemv_core(Mat4 * m, int64_t e, const uint16_t * x, int64_t M, void * y, int yf32, hipStream_t s) {
    const Plan p = plan_gemv(m->fmt, m->g.NT, m->g.KB, (int) M, 1, EPI_STORE_);
    QArgs a{};
    a.W = m->dev + e * m->dstride; a.estride = 0; a.ids = nullptr;
    a.N = m->N; a.K = m->K; a.NT = m->g.NT; a.KB = m->g.KB;
    a.x = x; a.ldx = m->K; a.xslot = 0; a.xdiv = 1; a.M = (int) M;
    a.y = y; a.ldy = m->N; a.yslot = 0; a.yf32 = yf32;
    a.bpw = p.bpw; a.tw = p.tw; a.xls = m->g.KB * 128 + 8;
    return launch_qgemv(m->fmt, EPI_STORE_, a, p.mb, p.rt, p.nb, p.xl, dim3((unsigned) p.gx, 1), p.waves(), s);
}

// LM-head GEMV whose epilogue also leaves each workgroup's key per row (EPI_ARGMAX; fp32 logits
// [M][N]), then the small launch that reduces those keys to argmax [M]: the logits are not read
// again. Keys: the handle's argmax workspace.
hipError_t argmax_gemv(Mat4 * m, const uint16_t * x, int64_t M, float * logits, int32_t * argmax, hipStream_t s) {
    const Plan p = plan_gemv(m->fmt, m->g.NT, m->g.KB, (int) M, 1, EPI_ARGMAX_);
    if (m->am_keys.n == 0) {               // sized once for the largest row count (64) it serves
        size_t most = 0;
        for (int r = 1; r <= 64; r++)
            most = std::max(most, (size_t) r * (size_t) plan_gemv(m->fmt, m->g.NT, m->g.KB, r, 1, EPI_ARGMAX_).gx * 8);
        if (const hipError_t e = m->am_keys.ensure(most); e != hipSuccess) return e;
    }
    hipError_t e = m->am_keys.ensure((size_t) (M * p.gx * 8));
    if (e != hipSuccess) return e;
    QArgs a{};
    a.W = m->dev; a.estride = 0; a.ids = nullptr;
    a.N = m->N; a.K = m->K; a.NT = m->g.NT; a.KB = m->g.KB;
    a.x = x; a.ldx = m->K; a.xslot = 0; a.xdiv = 1; a.M = (int) M;
    a.y = logits; a.ldy = m->N; a.yslot = 0; a.yf32 = 1;
    a.bpw = p.bpw; a.tw = p.tw; a.xls = m->g.KB * 128 + 8;
    a.akeys = m->am_keys.as<uint64_t>();
    e = launch_qgemv(m->fmt, EPI_ARGMAX_, a, p.mb, p.rt, p.nb, p.xl, dim3((unsigned) p.gx, 1), p.waves(), s);
    if (e != hipSuccess) return e;
    return launch_argmax_keys(a.akeys, p.gx, M, argmax, s);
}

// Up to 64 rows: the decode GEMV, whose time grows with the rows, unless the GEMM with a tile of
// 16-64 rows split along K (about the same time from 1 to 16 rows) is faster. Crossovers measured
// on MI355X over >= 600 MB of distinct weight copies (g128s unless named, us GEMV -> GEMM):
// 4096 x 4096 at 64 rows 19.6 -> 17.5 (48: 15.2 / 16.2 stays); 6144 x 4096 at 24 rows 16.4 -> 13.8
// (16: 12.0 / 12.4 stays); 4096 x 12288 at 16 rows 16.6 -> 16.6, 14336 x 4096 20.5 -> 15.3, 24576 x
// 4096 27.5 -> 22.4 (12: 16.4 / 22.0 stays), q4nx 24576 x 4096 28.3 -> 24.5; at 12 rows 151936 x 4096
// 97.0 -> 66.7 (Q4_0 98.4 -> 81.1), 57344 x 8192 106.6 -> 64.1, 8192 x 28672 52.6 -> 37.1. With the
// 16-row tile's weights two blocks ahead (same process, alternating): K >= 16384 from one row
// (4096 x 28672 31.5 -> 21.9, 5120 x 25600 28.7 -> 21.9, 8192 x 28672 34.3 -> 30.9, Q4_0 36.5 ->
// 33.2, 16384 x 16384 34.2 -> 31.8), K = 8192 with N K >= 2e8 from 4 rows (28672 x 8192 39.3 -> 30.8,
// 57344 x 8192 49.2 / 50.4 at 4, 61.7 -> 51.4 at 8; at 1-2 rows the GEMV: 40.9 / 50.1).
// ONPU_FORCE_GEMM = 1 takes the GEMM, -1 the GEMV.
bool rows_take_gemv(int64_t M, int64_t N, int64_t K) {
    const int f = env_int("ONPU_FORCE_GEMM", 0);
    if (M > 64 || f == 1) return false;
    if (f == -1) return true;
    const int64_t nk = N * K;
    return !((M >= 64 && nk >= 16000000) || (M >= 24 && nk >= 24000000) || (M >= 16 && nk >= 40000000) ||
             (M >= 12 && nk >= 200000000) || (M >= 4 && K >= 8192 && nk >= 200000000) ||
             (K >= 16384 && nk >= 64000000));
}

// mv_core's choice for M rows: the decode GEMV (path 0), k_qgemm with mb A blocks of 16 rows and ntw
// weight tiles per wave, in S ranges of kbs K blocks (path 1), or k_qgemm_sk (path 2); wgs: k_qgemm's
// workgroups per K range; deep: 16-row tiles with the weights two blocks ahead
struct MvPlan { int path, mb, ntw; int64_t S, kbs, wgs; int deep; };

MvPlan plan_mv(int fmt, int64_t N, int64_t K, int64_t NT, int64_t KB, int64_t M, int cus) {
    MvPlan p{0, 8, 2, 1, KB, 0, 0};
    if (rows_take_gemv(M, N, K)) return p;
    int cfg = 0;
    int64_t grid = 0;
    GArgs ga{};
    // the 256-row tiles of k_qgemm_sk compute at least half padding at M <= 128, where k_qgemm's
    // 128-row tiles (split along K below) are faster: 57344 x 8192 at M = 96 140 us against 194 us
    if (M > 128 && env_int("ONPU_GEMM_SK", 1) && plan_gsk(M, NT, KB, cus, cfg, grid, ga) && M * K * 2 < ((int64_t) 1 << 31)) {
        p.path = 2;
        return p;
    }
    p.path = 1;
    // A blocks of 16 rows per workgroup tile: 1 / 2 / 4 up to 16 / 32 / 64 rows, else 8 (128 rows).
    // MFMAs and LDS reads on rows past M cost their full time: the 151936 x 4096 LM head at 16 / 32
    // / 64 rows 171 / 176 / 184 us with 128-row tiles, 73 / 94 / 134 us with 16- / 32- / 64-row tiles
    p.mb = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
    const int emb = env_int("ONPU_GEMM_MB", 0);
    if (emb == 1 || emb == 2 || emb == 4 || emb == 8) p.mb = emb;
    // 3 weight tiles per wave (workgroup tile 128 x 192) when that still fills every CU with two
    // workgroups, else 2 (128 x 128); 4 (128 x 256) runs out of registers and is slower
    const int64_t wg3 = ((M + 127) / 128) * ((NT + 11) / 12);
    p.ntw = p.mb == 8 && wg3 >= 512 ? 3 : 2;
    const int entw = env_int("ONPU_GEMM_NTW", 0);
    if (entw >= 2 && entw <= 4) p.ntw = entw;
    if (p.ntw != 2) p.mb = 8;
    // the kernel addresses X with 32-bit buffer offsets: launches of at most 2^31 bytes of X rows
    const int64_t rows_max = std::max<int64_t>(128, (((int64_t) 1 << 31) - 1) / (K * 2) / 128 * 128);
    // split-K when the tiles leave CUs without work: S K ranges, S x the workgroups (two per CU,
    // at least 4 K blocks each), fp32 partials in the split-K workspace, then their sum. A sweep of
    // S over 1-16 (65-512 rows, seven shapes; 1-64 rows, thirteen shapes and formats) put this rule
    // 1.5-2 % from the best S on average
    p.wgs = ((M + 16 * p.mb - 1) / (16 * p.mb)) * ((NT + 4 * p.ntw - 1) / (4 * p.ntw));
    if (M <= rows_max) {
        const int es = env_int("ONPU_GEMM_SPLIT", 0);
        int64_t S = es >= 1 ? es : std::min<int64_t>(KB / 4, 2 * (int64_t) cus / p.wgs);
        S = std::max<int64_t>(1, std::min<int64_t>(S, KB));
        while (S > 1 && (size_t) (S * M * N * 4) > gsk_part_bytes(cus)) S--;
        if (S > 1) {
            p.kbs = (KB + S - 1) / S;
            p.S = (KB + p.kbs - 1) / p.kbs;
        }
    }
    // weights two blocks ahead with at most two workgroups per CU (one block in flight per
    // workgroup leaves the memory idle there): 16-row tiles, and g128s 32-row tiles of larger
    // matrices (57344 x 8192 at 17-32 rows 81-84 -> 74-80 us, 24576 x 4096 24.1-25.3 -> 22.5-24.0;
    // the per-32 formats and matrices below 1e8 weights measured 1-7 % slower there)
    const int ed = env_int("ONPU_GEMM_DEEP", -1);
    const bool dtile = p.mb == 1 || (p.mb == 2 && fmt == ONPU_G128S && N * K >= 100000000);
    p.deep = p.ntw == 2 && p.mb <= 2 && (ed >= 0 ? ed != 0 : dtile && p.S * p.wgs <= 2 * (int64_t) cus);
    return p;
}

hipError_t mv_core(Mat4 * m, int64_t e, const uint16_t * x, int64_t M, void * y, int yf32, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    const uint8_t * W = m->dev + e * m->dstride;
    const MvPlan p = plan_mv(m->fmt, m->N, m->K, m->g.NT, m->g.KB, M, device().cus);
    if (p.path == 0) return gemv_core(m, e, x, M, y, yf32, s);
    if (p.path == 2) {
        int cfg = 0;
        int64_t grid = 0;
        GArgs ga{};
        if (!plan_gsk(M, m->g.NT, m->g.KB, device().cus, cfg, grid, ga)) return hipErrorInvalidValue;
        // cut tiles: the R tail tiles (two-phase split) or the workgroup boundaries (stream-K)
        const int64_t cut = ga.sched == 1 ? ga.R : grid;
        hipError_t e = gsk_workspace(s, cut, &ga.ws, &ga.sync, &ga.ctl);
        if (e != hipSuccess) return e;
        ga.W = W; ga.NT = m->g.NT; ga.KB = m->g.KB; ga.N = m->N; ga.K = m->K; ga.M = M;
        ga.x = x; ga.ldx = m->K; ga.y = y; ga.ldy = m->N; ga.yf32 = yf32;
        ga.spin = spin_limit(1u << 22);
        return launch_qgemm_sk(m->fmt, ga, cfg, (int) grid, s);
    }
    if (p.S > 1) {
        GArgs a{};
        int32_t * sync = nullptr, * ctl = nullptr;
        hipError_t e = gsk_workspace(s, 0, &a.ws, &sync, &ctl);
        if (e != hipSuccess) return e;
        a.W = W; a.NT = m->g.NT; a.KB = m->g.KB; a.N = m->N; a.K = m->K; a.M = M;
        a.x = x; a.ldx = m->K; a.ldy = m->N; a.yf32 = 1; a.y = a.ws;
        a.splits = (int) p.S; a.kbs = p.kbs; a.deep = p.deep;
        if ((e = launch_qgemm(m->fmt, a, p.ntw, p.mb, s)) != hipSuccess) return e;
        return launch_gemm_split_sum(a.ws, (int) p.S, M, m->N, y, m->N, yf32, s);
    }
    const int64_t rows_max = std::max<int64_t>(128, (((int64_t) 1 << 31) - 1) / (m->K * 2) / 128 * 128);
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        GArgs a{};
        a.W = W; a.NT = m->g.NT; a.KB = m->g.KB; a.N = m->N; a.K = m->K; a.M = std::min(rows_max, M - r0);
        a.x = x + r0 * m->K; a.ldx = m->K; a.ldy = m->N; a.yf32 = yf32;
        a.y = (char *) y + r0 * m->N * (yf32 ? 4 : 2);
        a.deep = p.deep;
        const hipError_t e = launch_qgemm(m->fmt, a, p.ntw, p.mb, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// per-slot products: slot r = t * k + j -> expert ids[r] on x row (x_per_slot ? r : t); y [T*k][N]
hipError_t bank_core(Mat4 * m, const uint16_t * x, int x_per_slot, int64_t T, const int32_t * ids, int k, void * y,
                     int yf32, hipStream_t s) {
    const int64_t slots = T * k, chunk = (65535 / k) * k;     // grid.y limit; chunks start on a token
    const Plan p = plan_gemv(m->fmt, m->g.NT, m->g.KB, 1, slots, EPI_STORE_);
    for (int64_t s0 = 0; s0 < slots; s0 += chunk) {
        const int64_t ns = std::min<int64_t>(chunk, slots - s0);
        QArgs a{};
        a.W = m->dev; a.estride = m->dstride; a.ids = ids + s0;
        a.N = m->N; a.K = m->K; a.NT = m->g.NT; a.KB = m->g.KB;
        // slot r of this chunk reads x row r / xdiv from the chunk's first row
        a.xdiv = x_per_slot ? 1 : k;
        a.x = x + (x_per_slot ? s0 : s0 / k) * m->K;
        a.ldx = m->K; a.xslot = m->K; a.M = 1;
        a.y = (char *) y + s0 * m->N * (yf32 ? 4 : 2); a.ldy = m->N; a.yslot = m->N; a.yf32 = yf32;
        a.bpw = p.bpw; a.tw = p.tw; a.xls = m->g.KB * 128 + 8;
        hipError_t e = launch_qgemv(m->fmt, EPI_STORE_, a, p.mb, p.rt, p.nb, p.xl, dim3((unsigned) p.gx, (unsigned) ns),
                                    p.waves(), s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// MoE decode in one launch (k_moe_decode; opt-in with ONPU_MOE_FUSED=1, slower than the router
// kernel plus two GEMV launches on MI355X) when the shapes fit it: route from logits (non-null;
// ids / w are then written) or take ids / w, then both expert products and the weighted sum.
// hipErrorNotSupported: use the multi-launch path.
hipError_t moe_decode_core(Ffn * f, const float * logits, const uint16_t * x, int64_t T, int k, int renorm, int E,
                           int32_t * ids, float * w, void * y, int yf32, hipStream_t s) {
    Mat4 * gu = f->gu, * dn = f->dn;
    const int64_t I = gu->N / 2;
    if (!env_int("ONPU_MOE_FUSED", 0) || gu->fmt != dn->fmt || gu->N % 2 ||
        !moe_decode_fits(gu->K, I, dn->N, gu->g.KB, dn->g.KB, (int) T, k, E) || dn->K != I)
        return hipErrorNotSupported;
    hipError_t e = f->md_act.ensure((size_t) (MD_MAX_T * MD_MAX_K) * (size_t) I * 2);
    if (e != hipSuccess) return e;
    if (f->md_sync.n == 0) {              // zeroed once by a kernel on s (capturable); calls leave it zero
        if ((e = f->md_sync.ensure(MD_SYNC_INTS * 4)) != hipSuccess) return e;
        if ((e = launch_zero_i32(f->md_sync.as<int32_t>(), MD_SYNC_INTS, s)) != hipSuccess) return e;
    }
    MDArgs a{};
    a.Wg = gu->dev; a.gstride = gu->dstride; a.gNT = gu->g.NT; a.gKB = gu->g.KB;
    a.Wd = dn->dev; a.dstride = dn->dstride; a.dNT = dn->g.NT; a.dKB = dn->g.KB;
    a.H = gu->K; a.I = I; a.Nd = dn->N;
    a.x = x; a.logits = logits; a.E = E; a.k = k; a.renorm = renorm; a.T = (int) T;
    a.ids = ids; a.w = w; a.act = f->md_act.as<uint16_t>(); a.y = y; a.yf32 = yf32;
    a.sync = f->md_sync.as<int32_t>();
    a.npairs = T * k * (I / 16); a.nunits = T * dn->g.NT;
    a.spin = spin_limit(1u << 20);
    return launch_moe_decode(gu->fmt, a, device().cus, s);
}

// MoE decode split along I (k_moe_dsplit + k_moe_dsum): route from logits (non-null; ids / w are then
// written) or take ids / w. hipErrorNotSupported when the FFN has no step-major down copy, the shapes
// are outside the kernel's, or T is above ONPU_MOE_DSPLIT_MAX_T (default 1: at Qwen3-30B-A3B shapes on
// MI355X the split path takes 12.0 us per layer at T = 1 against 15.8 us for the two launches, but
// 19.5 / 29.9 us at T = 2 / 4 against 17.9 / 26.2); the caller then takes the two-launch path.
hipError_t moe_dsplit_core(Ffn * f, const float * logits, const uint16_t * x, int64_t T, int k, int renorm, int E,
                           int32_t * ids, float * w, void * y, int yf32, hipStream_t s) {
    Mat4 * gu = f->gu, * dn = f->dn;
    // values of I per workgroup: 16 while every workgroup still gets a CU of its own (a workgroup's
    // ~100 KB of loads in flight arrive at a fixed rate per CU, so halving them halves that phase),
    // else 32. Measured at Qwen3-30B-A3B, T = 1 (I 768; k slots: 48 k workgroups of 16 values against
    // 24 k of 32): 12.4-13.8 against 14.2-15.9 us for k = 1..5, 18.0 against 16.1 us at k = 6 (with
    // the dynamic LDS 16-byte aligned: 14.4 against 12.3 us at k = 8)
    const int64_t I = gu->N / 2;
    const int esv = env_int("ONPU_DS_SV", 0);
    const int sv = esv == 16 || esv == 32 ? esv : (T * k * (I / 16) <= device().cus ? 16 : 32);
    const int64_t S = I / sv, NTq = (dn->g.NT + 3) / 4;
    if (T > env_int("ONPU_MOE_DSPLIT_MAX_T", 1) || !dn->dec || gu->fmt != dn->fmt || dn->K != I || !moe_dsplit_fits(gu->K, I, dn->N, gu->g.KB, (int) T, k, E))
        return hipErrorNotSupported;
    // only while its workgroups (of 32 values) fit one per CU: past that each CU runs several
    // ~100-200 KB workgroups in turn and the partial sums grow with I, so the two launches win
    // (measured at T = 1: Qwen3-235B-A22B experts 30.4 against 26.5 us, Mixtral-8x7B 69.8
    // against 48.0 us, E 32 / H 3072 / I 3072 / k 4 27.3 against 22.6 us; Qwen3-30B-A3B 12.3
    // against 15.8 us)
    if (esv == 0 && T * k * (I / 32) > device().cus) return hipErrorNotSupported;
    hipError_t e = f->ds_part.ensure((size_t) (DS_MAX_T * DS_MAX_K) * (size_t) (S * NTq * 64) * 4);
    if (e != hipSuccess) return e;
    MSArgs a{};
    a.Wg = gu->dev; a.gstride = gu->dstride; a.gNT = gu->g.NT; a.gKB = gu->g.KB;
    a.Wd = dn->dec; a.dstride = dn->dec_stride; a.dNTq = NTq;
    a.H = gu->K; a.I = I; a.S = S;
    a.x = x; a.logits = logits; a.E = E; a.k = k; a.renorm = renorm; a.T = (int) T;
    a.ids = ids; a.w = w; a.part = f->ds_part.as<float>();
    if ((e = launch_moe_dsplit(gu->fmt, a, dn->N, sv, s)) != hipSuccess) return e;
    return launch_moe_dsum(a.part, S, NTq * 64, w, T, k, dn->N, y, yf32, s);
}

// MoE decode (T <= 4 tokens) in two launches: gate_up with SiLU(gate) * up per slot, then down with
// the routing-weighted slot sum per token. act: bf16 [T k][I] in the FFN's workspace. With logits
// (E <= 256 experts, k <= 16), the gate_up launch also routes: each of its workgroups picks its slot's
// expert from the token's logits, and ids / w are written there for the down launch and the caller.
hipError_t moe_decode_two(Ffn * f, const uint16_t * x, int64_t T, int k, const int32_t * ids, const float * w,
                          void * y, int yf32, hipStream_t s, const float * logits = nullptr, int E = 0,
                          int renorm = 1) {
    Mat4 * gu = f->gu, * dn = f->dn;
    const int64_t I = gu->N / 2, Nd = dn->N, n = T * k;
    // act rows, sized once for 4 tokens of 16 slots (more only if ONPU_MOE_DECODE_MAX raises T)
    hipError_t e = f->ws[0].ensure((size_t) (std::max<int64_t>(n, 4 * 16) * I * 2));
    if (e != hipSuccess) return e;
    uint16_t * act = f->ws[0].as<uint16_t>();
    const Plan pg = plan_gemv(gu->fmt, gu->g.NT, gu->g.KB, 1, n, EPI_ACT_);
    QArgs a{};
    a.W = gu->dev; a.estride = gu->dstride; a.ids = ids;
    a.N = gu->N; a.K = gu->K; a.NT = gu->g.NT; a.KB = gu->g.KB;
    a.x = x; a.ldx = gu->K; a.xslot = gu->K; a.xdiv = k; a.M = 1;
    a.y = act; a.ldy = I; a.yslot = I; a.yf32 = 0; a.bpw = pg.bpw; a.tw = pg.tw;
    a.xls = gu->g.KB * 128 + 8;
    if (logits != nullptr) {
        if (E > 256 || k > 16 || k > E) return hipErrorInvalidValue;
        a.logits = logits; a.E = E; a.renorm = renorm;
        a.rids = const_cast<int32_t *>(ids); a.rw = const_cast<float *>(w);
        a.ids = nullptr;
    }
    e = launch_qgemv(gu->fmt, EPI_ACT_, a, 1, 2, pg.nb, pg.xl, dim3((unsigned) pg.gx, (unsigned) n), pg.waves(), s);
    if (e != hipSuccess) return e;
    const Plan pd = plan_slotsum(dn->g.KB, k);
    if (!pd.kw) return hipErrorInvalidValue;
    QArgs b{};
    b.W = dn->dev; b.estride = dn->dstride; b.ids = ids;
    b.N = Nd; b.K = dn->K; b.NT = dn->g.NT; b.KB = dn->g.KB;
    b.x = act; b.ldx = I; b.xslot = I; b.xdiv = 1; b.M = 1;
    b.y = y; b.ldy = Nd; b.yslot = Nd; b.yf32 = yf32;
    b.wslot = w; b.nslot = k; b.ksplit = pd.kw / k; b.tw = 1;
    b.bpw = pd.bpw;
    return launch_qgemv(dn->fmt, EPI_SLOTSUM_, b, 1, 1, pd.nb, 0, dim3((unsigned) dn->g.NT, (unsigned) T), pd.kw, s);
}

// routed-expert FFN on device data (act 0, no biases): x bf16 [T][H], ids/w [T][k] -> y [T][Nd]
hipError_t ffn_core(Ffn * f, const uint16_t * x, int64_t T, const int32_t * ids, int k, const float * w, void * y,
                    int yf32, hipStream_t s) {
    Mat4 * gu = f->gu, * dn = f->dn;
    const int64_t I = gu->N / 2, Nd = dn->N;
    const int64_t n = T * k;
    const int decode_max = env_int("ONPU_MOE_DECODE_MAX", 4);
    hipError_t e;
    if (T <= decode_max && k <= 16) {
        e = moe_decode_core(f, nullptr, x, T, k, 1, (int) gu->E, const_cast<int32_t *>(ids),
                            const_cast<float *>(w), y, yf32, s);
        if (e != hipErrorNotSupported) return e;
        e = moe_dsplit_core(f, nullptr, x, T, k, 1, (int) gu->E, const_cast<int32_t *>(ids), const_cast<float *>(w),
                            y, yf32, s);
        if (e != hipErrorNotSupported) return e;
        return moe_decode_two(f, x, T, k, ids, w, y, yf32, s);
    }
    // prompts: tokens grouped per expert (one pass over each routed expert's weights per 64 rows)
    const int rows_per_item = 64;                 // the grouped GEMM's 4 A blocks of 16 rows
    const int64_t E = gu->E, maxitems = n / rows_per_item + E;
    if ((e = f->ws[1].ensure((size_t) (E + 1) * 4)) != hipSuccess) return e;
    if ((e = f->ws[2].ensure((size_t) n * 4)) != hipSuccess) return e;
    if ((e = f->ws[3].ensure((size_t) n * 4)) != hipSuccess) return e;
    if ((e = f->ws[4].ensure((size_t) (maxitems * 3 + 1) * 4)) != hipSuccess) return e;
    if ((e = f->ws[5].ensure((size_t) (n * I * 2))) != hipSuccess) return e;
    if ((e = f->ws[6].ensure((size_t) (n * Nd * 2))) != hipSuccess) return e;
    int32_t * off = f->ws[1].as<int32_t>(), * perm = f->ws[2].as<int32_t>(), * inv = f->ws[3].as<int32_t>();
    int32_t * items = f->ws[4].as<int32_t>(), * nitems = items + maxitems * 3;
    uint16_t * act = f->ws[5].as<uint16_t>();
    uint16_t * o = f->ws[6].as<uint16_t>();
    if ((e = launch_moe_permute(ids, n, (int) E, rows_per_item, off, perm, inv, items, nitems, s)) != hipSuccess)
        return e;
    MArgs a{};
    a.W = gu->dev; a.estride = gu->dstride; a.NT = gu->g.NT; a.KB = gu->g.KB; a.N = gu->N; a.K = gu->K;
    a.x = x; a.ldx = gu->K; a.y = act; a.ldy = I; a.perm = perm; a.items = items; a.nitems = nitems; a.k = k;
    a.xbytes = T * gu->K * 2;
    // grouped GEMMs: X tiles in LDS, weights dequantized in registers
    MArgs b{};
    b.W = dn->dev; b.estride = dn->dstride; b.NT = dn->g.NT; b.KB = dn->g.KB; b.N = Nd; b.K = dn->K;
    b.x = act; b.ldx = I; b.y = o; b.ldy = Nd; b.perm = perm; b.items = items; b.nitems = nitems; b.k = k;
    b.xbytes = n * I * 2;
    if ((e = launch_moe_gemm(gu->fmt, 0, a, maxitems, s)) != hipSuccess) return e;
    if ((e = launch_moe_gemm(dn->fmt, 1, b, maxitems, s)) != hipSuccess) return e;
    return launch_moe_combine(o, inv, w, T, k, Nd, y, yf32, s);
}

// expert ids from the caller index HBM: reject out-of-range ids before any launch
void check_ids(const int32_t * ids, int64_t n, int64_t E, const char * who) {
    for (int64_t i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= E) {
            std::fprintf(stderr, "libonpu_hip: %s: expert id %d at %lld outside [0, %lld)\n", who, (int) ids[i],
                         (long long) i, (long long) E);
            std::abort();
        }
}

// host fp32 rows -> bf16 on the device (the reference converts on the host, opennpu_core.hpp:418-424)
hipError_t x_to_dev(DBuf & fbuf, DBuf & bbuf, const float * x, int64_t n, hipStream_t s) {
    hipError_t e = fbuf.ensure((size_t) n * 4);
    if (e == hipSuccess) e = bbuf.ensure((size_t) n * 2);
    if (e == hipSuccess) e = hipMemcpyAsync(fbuf.p, x, (size_t) n * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = launch_f32_to_bf16(fbuf.as<float>(), n, bbuf.as<uint16_t>(), s);
    return e;
}

// A bounded wait inside one of the call's kernels gave up (its poll limit ran out), so the call's
// results are invalid. The reference aborts on a device failure (ONPU_ASSERT throws across
// extern "C", opennpu_core.hpp:30-32, and run.wait's timeout is one, :429), and so does this library,
// unless ONPU_WAIT_TIMEOUT=error: then the n floats of y are set to NaN, onpu_last_error says why, and
// the call returns (onpu_ffn_run / _many then return 0, "not done", whose caller falls back to its
// unfused path).
void wait_failed(const char * who, const char * what, float * y, int64_t n) {
    const std::string msg = std::string(who) + ": " + what + " gave up at its poll limit; the results are invalid";
    const char * mode = std::getenv("ONPU_WAIT_TIMEOUT");
    if (!(mode && std::strcmp(mode, "error") == 0)) {
        std::fprintf(stderr, "libonpu_hip: %s\n", msg.c_str());
        std::abort();
    }
    for (int64_t i = 0; i < n; i++) y[i] = __builtin_nanf("");
    g_err = msg;
}

// the one-launch MoE decode kernel's timed-out-wait flag, read after its stream has finished: 1 if
// set (then cleared), 0 if not or if the FFN never ran that kernel, -1 on a HIP failure
int md_take_flag(Ffn * f) {
    if (f->md_sync.n == 0) return 0;
    int32_t flag = 0;
    if (hipMemcpy(&flag, f->md_sync.as<int32_t>(MD_SYNC_ERR * 4), 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (flag && hipMemset(f->md_sync.as<int32_t>(MD_SYNC_ERR * 4), 0, 4) != hipSuccess) return -1;
    return flag != 0;
}

struct Timer {
    std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
    ~Timer() {
        g_wait_s += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        g_calls++;
    }
};

}  // namespace

extern "C" {

const char * onpu_last_error(void) { return g_err.c_str(); }

int onpu_ok(void) { return device().ok; }
int onpu_batched_ok(void) { return device().ok; }

void onpu_geometry2(int64_t N, int64_t K, int ncols, int sym, int64_t * out) {
    const RefGeom g = ref_geometry(N, K, ncols, sym != 0);
    const int64_t v[8] = {g.R, g.S, g.tiles, g.kc, g.ks, g.rows_col, g.cb, g.nbytes};
    for (int i = 0; i < 8; i++) out[i] = g.ok ? v[i] : 0;
}
void onpu_geometry(int64_t N, int64_t K, int ncols, int64_t * out) { onpu_geometry2(N, K, ncols, 0, out); }

int onpu_gemm_status(void) { return gsk_status(); }

void onpu_release_scratch(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!device().ok) return;
    (void) hipStreamSynchronize(device().stream);
    for (auto & b : g_hws) b.release();
}

void onpu_stats(int64_t * calls, double * wait_s) {
    std::lock_guard<std::mutex> lk(g_mu);
    *calls = g_calls.load();
    *wait_s = g_wait_s;
}

// every (tiles, kc) is served: the HIP kernels take any shape
int onpu_has_shape(int, int, int) { return device().ok; }

// the GEMV launch plan for an [N][K] matrix of fmt at M rows over `slots` (host only, no GPU):
// out = mb, rt, nb, xl, tw, kw, bpw, gx, built (1 if that kernel variant exists), max waves
void onpu_plan_mv(int fmt, int64_t N, int64_t K, int64_t M, int64_t * out) {
    const Tiled g = tiled_geom(fmt, N, K);
    const MvPlan p = plan_mv(fmt, N, K, g.NT, g.KB, M, device().cus > 0 ? device().cus : 256);
    const int64_t v[7] = {p.path, p.mb, p.ntw, p.S, p.kbs, p.wgs, p.deep};
    for (int i = 0; i < 7; i++) out[i] = v[i];
}

void onpu_plan_gemv(int fmt, int64_t N, int64_t K, int M, int64_t slots, int epi, int64_t * out) {
    const Tiled g = tiled_geom(fmt, N, K);
    const Plan p = epi == EPI_SLOTSUM_ ? plan_slotsum(g.KB, (int) slots) : plan_gemv(fmt, g.NT, g.KB, M, slots, epi);
    const int64_t v[10] = {p.mb, p.rt, p.nb, p.xl, p.tw, p.kw, p.bpw, p.gx,
                           qgemv_has_variant(epi, p.mb, p.rt, p.nb, p.xl), qgemv_max_waves(p.mb, p.rt, p.nb, p.xl)};
    for (int i = 0; i < 10; i++) out[i] = v[i];
}

int64_t onpu_stage_bytes(int fmt, int64_t N, int64_t K) {
    return fmt_valid(fmt) && K % fmt_group(fmt) == 0 ? stage_bytes(fmt, N, K) : 0;
}

// ---------------------------------------------------------------- dense
// a handle whose *_buf memory takes the reference's NPU packing in geometry g (q4nx, q4s) or, for
// this library's own formats, the staging layout in g.nbytes bytes per expert
static Mat4 * make_ref_mat(int64_t N, int64_t K, int64_t E, int fmt, const RefGeom & g) {
    Mat4 * m = make_mat(N, K, E, fmt, g.nbytes);
    if (m) {
        m->npu = fmt == ONPU_Q4NX || fmt == ONPU_Q4S;
        m->rg = g;
    }
    return m;
}

void * onpu_dense_new2(int64_t N, int64_t K, int sym) {
    const RefGeom g = ref_geometry(N, K, 8, sym != 0);
    if (!g.ok) { set_err("onpu_dense_new2: the shape has no reference geometry"); return nullptr; }
    return make_ref_mat(N, K, 1, sym, g);
}
void * onpu_dense_new(int64_t N, int64_t K) { return onpu_dense_new2(N, K, 0); }
void * onpu_dense_new3(int64_t N, int64_t K, int fmt) {
    if (!fmt_valid(fmt) || K % fmt_group(fmt) != 0) return nullptr;
    return make_mat(N, K, 1, fmt, stage_bytes(fmt, N, K));
}
uint8_t * onpu_dense_buf(void * h) { return stage_of((Mat4 *) h); }
int64_t onpu_dense_bytes(void * h) { return ((Mat4 *) h)->sstride; }

void onpu_dense_sync(void * h) {
    auto * m = (Mat4 *) h;
    std::lock_guard<std::mutex> lk(g_mu);
    HIPX(upload(m, 0, m->E, stage_of(m), m->sstride, m->npu, device().stream));
}

void onpu_dense_free(void * h) {
    std::lock_guard<std::mutex> lk(g_mu);
    free_mat((Mat4 *) h);
}

int onpu_dense_load(void * h, const void * stage) {
    auto * m = (Mat4 *) h;
    std::lock_guard<std::mutex> lk(g_mu);
    HIPR(upload(m, 0, 1, (const uint8_t *) stage, stage_bytes(m->fmt, m->N, m->K), false, device().stream));
    return 0;
}

void onpu_dense_info(void * h, int64_t * out) {
    auto * m = (Mat4 *) h;
    const int64_t v[8] = {m->N, m->K, m->fmt, m->E, m->g.NT, m->g.KB, m->dstride, (int64_t) (uintptr_t) m->dev};
    for (int i = 0; i < 8; i++) out[i] = v[i];
}

int onpu_dense_dequant(void * h, int64_t e, void * out_host, int bf16) {
    auto * m = (Mat4 *) h;
    if (e < 0 || e >= m->E) { set_err("onpu_dense_dequant: expert out of range"); return -1; }
    std::lock_guard<std::mutex> lk(g_mu);
    const hipStream_t s = device().stream;
    const size_t bytes = (size_t) (m->N * m->K * (bf16 ? 2 : 4));
    HIPR(g_hws[0].ensure(bytes));
    HIPR(launch_dequant(m->fmt, m->dev + e * m->dstride, m->N, m->K, g_hws[0].p, bf16, s));
    HIPR(hipMemcpyAsync(out_host, g_hws[0].p, bytes, hipMemcpyDeviceToHost, s));
    HIPR(hipStreamSynchronize(s));
    return 0;
}

void onpu_dense_mv(void * h, const float * x, int64_t rows, float * y) {
    auto * m = (Mat4 *) h;
    if (rows <= 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    Timer tm;
    const hipStream_t s = device().stream;
    HIPX(x_to_dev(g_hws[0], g_hws[1], x, rows * m->K, s));
    HIPX(g_hws[2].ensure((size_t) (rows * m->N * 4)));
    HIPX(mv_core(m, 0, g_hws[1].as<uint16_t>(), rows, g_hws[2].p, 1, s));
    HIPX(hipMemcpyAsync(y, g_hws[2].p, (size_t) (rows * m->N * 4), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
    // more than 128 rows may run the stream-K GEMM, whose partial-tile exchange waits are bounded
    const int timed_out = rows > 128 ? gsk_take_flag(s) : 0;
    if (timed_out < 0) die("onpu_dense_mv: reading the split-K wait flag", hipErrorUnknown);
    if (timed_out) wait_failed("onpu_dense_mv", "a split-K partial-tile wait", y, rows * m->N);
}

int onpu_dense_mv_dev(void * h, const void * x, int64_t M, void * y, int y_f32, void * stream) {
    auto * m = (Mat4 *) h;
    HIPR(mv_core(m, 0, (const uint16_t *) x, M, y, y_f32, (hipStream_t) stream));
    return 0;
}

// LM head at rows that run the GEMM with one row tile of at most 64 rows and no split along K: its
// epilogue leaves each workgroup's key per row (keys [M][N blocks], the handle's argmax workspace)
// and k_argmax_keys reduces them, so the logits are not read again (Q4_0 151936 x 4096 at 16 rows:
// the argmax launch over the logits took 13.7 us of 96)
static hipError_t argmax_gemm(Mat4 * m, const MvPlan & p, const uint16_t * x, int64_t M, float * logits,
                              int32_t * argmax, hipStream_t s) {
    const int64_t gn = (m->g.NT + 4 * p.ntw - 1) / (4 * p.ntw);
    if (const hipError_t e = m->am_keys.ensure((size_t) (M * gn * 8)); e != hipSuccess) return e;
    GArgs a{};
    a.W = m->dev; a.NT = m->g.NT; a.KB = m->g.KB; a.N = m->N; a.K = m->K; a.M = M;
    a.x = x; a.ldx = m->K; a.y = logits; a.ldy = m->N; a.yf32 = 1;
    a.akeys = m->am_keys.as<uint64_t>();
    a.deep = p.deep;
    if (const hipError_t e = launch_qgemm(m->fmt, a, p.ntw, p.mb, s); e != hipSuccess) return e;
    return launch_argmax_keys(a.akeys, gn, M, argmax, s);
}

int onpu_dense_argmax_dev(void * h, const void * x, int64_t M, float * logits, int32_t * argmax, void * stream) {
    auto * m = (Mat4 *) h;
    if (M <= 0) return 0;
    // The argmax workspace belongs to the handle (calls that overlap on one handle must not share
    // it). Rows that run the GEMV: per-workgroup keys from its epilogue, sized once for 64 rows.
    // Otherwise (or with ONPU_ARGMAX_FUSED=0) the argmax launch over the logits, with its keys and
    // per-row counters (grown to the rows of the call; new counters zeroed by a kernel on the stream,
    // and each call leaves them zero). Outgrown buffers are kept, so graphs keep valid pointers.
    const bool fused = env_int("ONPU_ARGMAX_FUSED", 1) != 0;
    if (rows_take_gemv(M, m->N, m->K) && fused) {
        HIPR(argmax_gemv(m, (const uint16_t *) x, M, logits, argmax, (hipStream_t) stream));
        return 0;
    }
    const MvPlan p = plan_mv(m->fmt, m->N, m->K, m->g.NT, m->g.KB, M, device().cus);
    if (fused && p.path == 1 && p.S == 1 && p.mb <= 4 && p.ntw == 2 && M <= 16 * p.mb) {
        HIPR(argmax_gemm(m, p, (const uint16_t *) x, M, logits, argmax, (hipStream_t) stream));
        return 0;
    }
    if (m->am_cnt.n < (size_t) M * ARGMAX_PAD) {
        HIPR(m->am_cnt.ensure((size_t) M * ARGMAX_PAD));
        HIPR(launch_zero_i32(m->am_cnt.as<int32_t>(), (int64_t) (m->am_cnt.n / 4), (hipStream_t) stream));
    }
    HIPR(m->am_big.ensure((size_t) (M * argmax_parts(m->N) * ARGMAX_PAD)));
    HIPR(mv_core(m, 0, (const uint16_t *) x, M, logits, 1, (hipStream_t) stream));
    HIPR(launch_argmax(logits, M, m->N, argmax, m->am_big.as<uint64_t>(), m->am_cnt.as<uint32_t>(),
                       (hipStream_t) stream));
    return 0;
}

int onpu_dense_argmax_dev_noalloc(void * h, const void * x, int64_t M, float * logits, int32_t * argmax,
                                  void * stream) {
    auto * m = (Mat4 *) h;
    if (M <= 0) return 0;
    if (M > 64) {
        set_err("onpu_dense_argmax_dev_noalloc: at most 64 rows (more would run the prefill GEMM, whose "
                "workspace is allocated)");
        return -1;
    }
    uint64_t * keys = nullptr;
    uint32_t * cnt = nullptr;
    if (const hipError_t e = argmax_scratch_get(M, m->N, &keys, &cnt); e != hipSuccess) {
        if (e == hipErrorInvalidValue)
            set_err("onpu_dense_argmax_dev_noalloc: M x ceil(N / 4096) exceeds the 8064 keys of the 1 MiB "
                    "scratch array");
        else
            set_err("onpu_dense_argmax_dev_noalloc: scratch array", e);
        return -1;
    }
    HIPR(gemv_core(m, 0, (const uint16_t *) x, M, logits, 1, (hipStream_t) stream));
    HIPR(launch_argmax(logits, M, m->N, argmax, keys, cnt, (hipStream_t) stream));
    return 0;
}

// ---------------------------------------------------------------- banks
void * onpu_bank_new2(int64_t N, int64_t K, int64_t E, int ncols, int sym) {
    const RefGeom g = ref_geometry(N, K, ncols, sym != 0);
    if (!g.ok) { set_err("onpu_bank_new2: the shape has no reference geometry"); return nullptr; }
    return make_ref_mat(N, K, E, sym, g);
}
void * onpu_bank_new(int64_t N, int64_t K, int64_t E, int ncols) { return onpu_bank_new2(N, K, E, ncols, 0); }
void * onpu_bank_new3(int64_t N, int64_t K, int64_t E, int fmt) {
    if (!fmt_valid(fmt) || K % fmt_group(fmt) != 0) return nullptr;
    return make_mat(N, K, E, fmt, stage_bytes(fmt, N, K));
}
uint8_t * onpu_bank_buf(void * h) { return stage_of((Mat4 *) h); }
int64_t onpu_bank_expert_bytes(void * h) { return ((Mat4 *) h)->sstride; }
void onpu_bank_sync(void * h) { onpu_dense_sync(h); }
void onpu_bank_free(void * h) { onpu_dense_free(h); }

int onpu_bank_load(void * h, int64_t e0, int64_t n, const void * stage) {
    auto * m = (Mat4 *) h;
    if (e0 < 0 || n < 0 || e0 + n > m->E) { set_err("onpu_bank_load: experts out of range"); return -1; }
    std::lock_guard<std::mutex> lk(g_mu);
    HIPR(upload(m, e0, n, (const uint8_t *) stage, stage_bytes(m->fmt, m->N, m->K), false, device().stream));
    return 0;
}

void onpu_bank_run(void * h, const float * x, int x_per_slot, int64_t T, const int32_t * ids, int k, float * y) {
    auto * m = (Mat4 *) h;
    if (T <= 0 || k <= 0) return;
    check_ids(ids, T * k, m->E, "onpu_bank_run");
    std::lock_guard<std::mutex> lk(g_mu);
    Timer tm;
    const hipStream_t s = device().stream;
    const int64_t xrows = x_per_slot ? T * k : T;
    HIPX(x_to_dev(g_hws[0], g_hws[1], x, xrows * m->K, s));
    HIPX(g_hws[2].ensure((size_t) (T * k * 4)));
    HIPX(hipMemcpyAsync(g_hws[2].p, ids, (size_t) (T * k * 4), hipMemcpyHostToDevice, s));
    HIPX(g_hws[3].ensure((size_t) (T * k * m->N * 4)));
    HIPX(bank_core(m, g_hws[1].as<uint16_t>(), x_per_slot, T, g_hws[2].as<int32_t>(), k, g_hws[3].p, 1, s));
    HIPX(hipMemcpyAsync(y, g_hws[3].p, (size_t) (T * k * m->N * 4), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
}

void onpu_moe_ffn(void * gu_h, void * dn_h, const float * x, int64_t T, const int32_t * ids, int k, const float * w,
                  int act, float alpha, float limit, const float * gu_bias, const float * dn_bias, float * y) {
    auto * gu = (Mat4 *) gu_h, * dn = (Mat4 *) dn_h;
    if (T <= 0 || k <= 0) return;
    check_ids(ids, T * k, std::min(gu->E, dn->E), "onpu_moe_ffn");
    std::lock_guard<std::mutex> lk(g_mu);
    Timer tm;
    const hipStream_t s = device().stream;
    const int64_t n = T * k, Ng = gu->N, I = Ng / 2, Nd = dn->N, E = gu->E;
    DBuf * b = g_hws;                      // x f32/bf16, ids, h, a (f32, bf16)
    DBuf * c = g_hws + 6;                  // w, o, y, biases
    HIPX(x_to_dev(b[0], b[1], x, T * gu->K, s));
    HIPX(b[2].ensure((size_t) n * 4));
    HIPX(hipMemcpyAsync(b[2].p, ids, (size_t) n * 4, hipMemcpyHostToDevice, s));
    HIPX(b[3].ensure((size_t) (n * Ng * 4)));
    HIPX(bank_core(gu, b[1].as<uint16_t>(), 0, T, b[2].as<int32_t>(), k, b[3].p, 1, s));
    const float * gb = nullptr, * db = nullptr;
    if (gu_bias) {
        HIPX(c[3].ensure((size_t) (E * Ng * 4)));
        HIPX(hipMemcpyAsync(c[3].p, gu_bias, (size_t) (E * Ng * 4), hipMemcpyHostToDevice, s));
        gb = c[3].as<float>();
    }
    if (dn_bias) {
        HIPX(c[4].ensure((size_t) (E * Nd * 4)));
        HIPX(hipMemcpyAsync(c[4].p, dn_bias, (size_t) (E * Nd * 4), hipMemcpyHostToDevice, s));
        db = c[4].as<float>();
    }
    HIPX(b[4].ensure((size_t) (n * I * 4)));
    HIPX(launch_moe_act(b[3].as<float>(), n, Ng, b[2].as<int32_t>(), gb, act, alpha, limit, b[4].as<float>(), s));
    HIPX(b[5].ensure((size_t) (n * I * 2)));
    HIPX(launch_f32_to_bf16(b[4].as<float>(), n * I, b[5].as<uint16_t>(), s));
    HIPX(c[0].ensure((size_t) n * 4));
    HIPX(hipMemcpyAsync(c[0].p, w, (size_t) n * 4, hipMemcpyHostToDevice, s));
    HIPX(c[1].ensure((size_t) (n * Nd * 4)));
    HIPX(bank_core(dn, b[5].as<uint16_t>(), 1, T, b[2].as<int32_t>(), k, c[1].p, 1, s));
    HIPX(c[2].ensure((size_t) (T * Nd * 4)));
    HIPX(launch_moe_sum(c[1].as<float>(), T, k, Nd, b[2].as<int32_t>(), c[0].as<float>(), db, c[2].as<float>(), s));
    HIPX(hipMemcpyAsync(y, c[2].p, (size_t) (T * Nd * 4), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
}

// the CPU helpers of onpu_cpu.cpp:233-274, computed on the GPU
void onpu_moe_act(const float * h, int64_t rows, int64_t Ng, const int32_t * ids, const float * gu_bias, int act,
                  float alpha, float limit, float * a) {
    if (rows <= 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    static DBuf bh, bi, bb, ba;
    const hipStream_t s = device().stream;
    int64_t E = 0;
    if (gu_bias)
        for (int64_t r = 0; r < rows; r++) E = std::max<int64_t>(E, (int64_t) ids[r] + 1);
    HIPX(bh.ensure((size_t) (rows * Ng * 4)));
    HIPX(hipMemcpyAsync(bh.p, h, (size_t) (rows * Ng * 4), hipMemcpyHostToDevice, s));
    if (gu_bias) {
        HIPX(bi.ensure((size_t) rows * 4));
        HIPX(hipMemcpyAsync(bi.p, ids, (size_t) rows * 4, hipMemcpyHostToDevice, s));
        HIPX(bb.ensure((size_t) (E * Ng * 4)));
        HIPX(hipMemcpyAsync(bb.p, gu_bias, (size_t) (E * Ng * 4), hipMemcpyHostToDevice, s));
    }
    HIPX(ba.ensure((size_t) (rows * (Ng / 2) * 4)));
    HIPX(launch_moe_act(bh.as<float>(), rows, Ng, gu_bias ? bi.as<int32_t>() : nullptr,
                        gu_bias ? bb.as<float>() : nullptr, act, alpha, limit, ba.as<float>(), s));
    HIPX(hipMemcpyAsync(a, ba.p, (size_t) (rows * (Ng / 2) * 4), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
}

void onpu_moe_sum(const float * o, int64_t T, int k, int64_t N, const int32_t * ids, const float * w,
                  const float * bias, float * y) {
    if (T <= 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    static DBuf bo, bi, bw, bb, by;
    const hipStream_t s = device().stream;
    const int64_t n = T * k;
    int64_t E = 0;
    for (int64_t r = 0; r < n; r++) E = std::max<int64_t>(E, (int64_t) ids[r] + 1);
    HIPX(bo.ensure((size_t) (n * N * 4)));
    HIPX(hipMemcpyAsync(bo.p, o, (size_t) (n * N * 4), hipMemcpyHostToDevice, s));
    HIPX(bi.ensure((size_t) n * 4));
    HIPX(hipMemcpyAsync(bi.p, ids, (size_t) n * 4, hipMemcpyHostToDevice, s));
    HIPX(bw.ensure((size_t) n * 4));
    HIPX(hipMemcpyAsync(bw.p, w, (size_t) n * 4, hipMemcpyHostToDevice, s));
    if (bias) {
        HIPX(bb.ensure((size_t) (E * N * 4)));
        HIPX(hipMemcpyAsync(bb.p, bias, (size_t) (E * N * 4), hipMemcpyHostToDevice, s));
    }
    HIPX(by.ensure((size_t) (T * N * 4)));
    HIPX(launch_moe_sum(bo.as<float>(), T, k, N, bi.as<int32_t>(), bw.as<float>(), bias ? bb.as<float>() : nullptr,
                        by.as<float>(), s));
    HIPX(hipMemcpyAsync(y, by.p, (size_t) (T * N * 4), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
}

// ---------------------------------------------------------------- fused expert FFN
static void * ffn_make(Mat4 * gu, Mat4 * dn, int64_t Nd, int64_t Kd, int64_t E, int fmt) {
    if (!gu || !dn) { free_mat(gu); free_mat(dn); return nullptr; }
    const int64_t Ng = gu->N;
    auto * f = new Ffn;
    f->gu = gu;
    f->dn = dn;
    // the fused kernels pair gate row tile t with up row tile t + I/16
    f->fused = Ng % 32 == 0 && Kd == Ng / 2;
    f->perm.resize((size_t) Ng);
    for (int64_t r = 0; r < Ng; r++) f->perm[r] = (int32_t) r;
    // decode split along I (k_moe_dsplit) reads the down bank in a step-major copy: one more
    // down-bank-sized allocation, filled with the weights (ONPU_MOE_DSPLIT=0: no copy, two launches)
    if (f->fused && Kd % 32 == 0 && env_int("ONPU_MOE_DSPLIT", 1)) {
        dn->dec_stride = dec_bytes(fmt, Nd, Kd);
        if (hipMalloc((void **) &dn->dec, (size_t) (dn->dec_stride * E)) != hipSuccess) {
            dn->dec = nullptr;
            dn->dec_stride = 0;
        }
    }
    return f;
}

// The gate_up row order of the reference's fused FFN (onpu_api.cpp:307-322 of the reference): when
// its rule holds (one row block and one K slice per matrix, I = Ng / 2 = Kd a multiple of 256, all
// Ng rows in one column, Kg <= 2048, an even tile count), its NPU writes the outputs of a column in
// [tile pair][core row][128 rows] order, so the caller packs gate_up row perm[r] at row r. The same
// order is given here, so that packed banks, the reference's cache files included, carry the same
// bytes; the upload puts packed row r back at row perm[r].
static bool ref_ffn_order(int64_t Ng, int64_t Kg, int64_t Nd, int64_t Kd, const RefGeom & gg, const RefGeom & gd,
                          std::vector<int32_t> & perm) {
    const int64_t I = Ng / 2;
    if (!(gg.R == 1 && gg.S == 1 && gd.R == 1 && gd.S == 1 && Ng % 2 == 0 && Kd == I && I % 256 == 0 &&
          gg.rows_col == Ng && Kg <= 2048 && gg.tiles % 2 == 0))
        return false;
    (void) Nd;
    const int64_t pairs = gg.tiles / 2;
    for (int64_t t2 = 0; t2 < pairs; t2++)
        for (int64_t cr = 0; cr < 4; cr++)
            for (int64_t i = 0; i < 128; i++)
                perm[(size_t) (cr * gg.tiles * 64 + t2 * 128 + i)] = (int32_t) ((t2 * 4 + cr) * 128 + i);
    return true;
}

void * onpu_ffn_new(int64_t Ng, int64_t Kg, int64_t Nd, int64_t Kd, int64_t E, int sym) {
    const RefGeom gg = ref_geometry(Ng, Kg, 1, sym != 0), gd = ref_geometry(Nd, Kd, 1, sym != 0);
    if (!gg.ok || !gd.ok) { set_err("onpu_ffn_new: a shape has no reference geometry"); return nullptr; }
    auto * f = (Ffn *) ffn_make(make_ref_mat(Ng, Kg, E, sym, gg), make_ref_mat(Nd, Kd, E, sym, gd), Nd, Kd, E, sym);
    if (f && f->fused && f->gu->npu && ref_ffn_order(Ng, Kg, Nd, Kd, gg, gd, f->perm)) {
        const size_t bytes = f->perm.size() * sizeof(int32_t);
        hipError_t e = hipMalloc((void **) &f->gu->rowmap, bytes);
        if (e == hipSuccess) e = hipMemcpy(f->gu->rowmap, f->perm.data(), bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            set_err("onpu_ffn_new: the gate_up row order", e);
            onpu_ffn_free(f);
            return nullptr;
        }
    }
    return f;
}
void * onpu_ffn_new3(int64_t Ng, int64_t Kg, int64_t Nd, int64_t Kd, int64_t E, int fmt) {
    if (!fmt_valid(fmt) || Kg % fmt_group(fmt) != 0 || Kd % fmt_group(fmt) != 0) return nullptr;
    return ffn_make(make_mat(Ng, Kg, E, fmt, stage_bytes(fmt, Ng, Kg)), make_mat(Nd, Kd, E, fmt, stage_bytes(fmt, Nd, Kd)),
                    Nd, Kd, E, fmt);
}
void * onpu_ffn_gu(void * h) { return ((Ffn *) h)->gu; }
void * onpu_ffn_dn(void * h) { return ((Ffn *) h)->dn; }
int onpu_ffn_fused(void * h) { return ((Ffn *) h)->fused ? 1 : 0; }
void onpu_ffn_perm(void * h, int32_t * out) {
    const auto & p = ((Ffn *) h)->perm;
    std::copy(p.begin(), p.end(), out);
}
void onpu_ffn_free(void * h) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto * f = (Ffn *) h;
    free_mat(f->gu);
    free_mat(f->dn);
    for (auto & b : f->ws) b.release();
    f->md_act.release();
    f->md_sync.release();
    delete f;
}

static int ffn_host(Ffn * f, const float * x, int64_t T, const int32_t * ids, int k, const float * w, float * y) {
    if (!f->fused) return 0;
    check_ids(ids, T * k, f->gu->E, "onpu_ffn_run");
    std::lock_guard<std::mutex> lk(g_mu);
    Timer tm;
    const hipStream_t s = device().stream;
    DBuf * b = g_hws;
    const int64_t n = T * k, Nd = f->dn->N;
    HIPX(x_to_dev(b[0], b[1], x, T * f->gu->K, s));
    HIPX(b[2].ensure((size_t) n * 8));
    HIPX(hipMemcpyAsync(b[2].p, ids, (size_t) n * 4, hipMemcpyHostToDevice, s));
    HIPX(hipMemcpyAsync(b[2].as<char>((size_t) n * 4), w, (size_t) n * 4, hipMemcpyHostToDevice, s));
    HIPX(b[3].ensure((size_t) (T * Nd * 4)));
    HIPX(ffn_core(f, b[1].as<uint16_t>(), T, b[2].as<int32_t>(), k, b[2].as<float>((size_t) n * 4), b[3].p, 1, s));
    HIPX(hipMemcpyAsync(y, b[3].p, (size_t) (T * Nd * 4), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
    // the one-launch decode kernel (ONPU_MOE_FUSED=1) waits, bounded, for the act rows
    const int timed_out = md_take_flag(f);
    if (timed_out < 0) die("onpu_ffn_run: reading the MoE decode wait flag", hipErrorUnknown);
    if (timed_out) {
        wait_failed("onpu_ffn_run", "the one-launch MoE decode's wait for its act rows", y, T * Nd);
        return 0;
    }
    return 1;
}

int onpu_ffn_run(void * h, const float * x, const int32_t * ids, int k, const float * w, float * y) {
    return ffn_host((Ffn *) h, x, 1, ids, k, w, y);
}
int onpu_ffn_run_many(void * h, const float * x, int64_t T, const int32_t * ids, int k, const float * w, float * y) {
    return T > 0 ? ffn_host((Ffn *) h, x, T, ids, k, w, y) : 1;
}

int onpu_moe_route_dev(const float * logits, int64_t T, int E, int k, int renorm, int32_t * ids, float * w,
                       void * stream) {
    HIPR(launch_route(logits, T, E, k, renorm, ids, w, (hipStream_t) stream));
    return 0;
}

int onpu_moe_ffn_dev(void * h, const void * x, int64_t T, const int32_t * ids, int k, const float * w, void * y,
                     int y_f32, void * stream) {
    auto * f = (Ffn *) h;
    if (!f->fused) { set_err("onpu_moe_ffn_dev: this FFN shape has no fused path"); return -1; }
    HIPR(ffn_core(f, (const uint16_t *) x, T, ids, k, w, y, y_f32, (hipStream_t) stream));
    return 0;
}

int onpu_moe_decode_dev(void * h, const float * logits, const void * x, int64_t T, int E, int k, int renorm,
                        int32_t * ids, float * w, void * y, int y_f32, void * stream) {
    auto * f = (Ffn *) h;
    if (!f->fused) { set_err("onpu_moe_decode_dev: this FFN shape has no fused path"); return -1; }
    if (E != f->gu->E) { set_err("onpu_moe_decode_dev: E differs from the bank's expert count"); return -1; }
    hipError_t e = moe_decode_core(f, logits, (const uint16_t *) x, T, k, renorm, E, ids, w, y, y_f32,
                                   (hipStream_t) stream);
    if (e == hipErrorNotSupported && T <= env_int("ONPU_MOE_DECODE_MAX", 4))
        e = moe_dsplit_core(f, logits, (const uint16_t *) x, T, k, renorm, E, ids, w, y, y_f32, (hipStream_t) stream);
    if (e != hipErrorNotSupported) {
        HIPR(e);
        return 0;
    }
    if (T <= env_int("ONPU_MOE_DECODE_MAX", 4) && k <= 16 && E <= 256 && k <= E && plan_slotsum(f->dn->g.KB, k).kw) {
        HIPR(moe_decode_two(f, (const uint16_t *) x, T, k, ids, w, y, y_f32, (hipStream_t) stream, logits, E, renorm));
        return 0;
    }
    HIPR(launch_route(logits, T, E, k, renorm, ids, w, (hipStream_t) stream));
    HIPR(ffn_core(f, (const uint16_t *) x, T, ids, k, w, y, y_f32, (hipStream_t) stream));
    return 0;
}

int onpu_moe_status(void * h) {
    auto * f = (Ffn *) h;
    if (f->md_sync.n == 0) return 0;
    int32_t flag = 0;
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(&flag, f->md_sync.as<int32_t>(MD_SYNC_ERR * 4), 4, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (flag && hipMemset(f->md_sync.as<int32_t>(MD_SYNC_ERR * 4), 0, 4) != hipSuccess) return -1;
    return flag ? 1 : 0;
}

// ---------------------------------------------------------------- chained decode GEMVs
struct Chain {
    int fmt = 0, n = 0, M = 0, yf32 = 0, grid = 0, ring = 0;
    size_t lds = 0;
    int64_t xls = 0, ring_off = 0;
    DBuf entries, ep, links;
};

namespace {
struct Span { uintptr_t a, b; };          // byte range [a, b)
bool overlap(Span u, Span v) { return u.a < v.b && v.a < u.b; }
}

void * onpu_chain_new(void * const * handles, const void * const * xs, void * const * ys, int n, int64_t M,
                      int y_f32) {
    if (!device().ok || n < 1 || M < 1 || M > 16) { set_err("onpu_chain_new: needs a GPU, n >= 1, 1 <= M <= 16"); return nullptr; }
    const int fmt = ((Mat4 *) handles[0])->fmt;
    int64_t kbmax = 0;
    std::vector<ChainEntry> es((size_t) n);
    std::vector<Span> xr((size_t) n), yr((size_t) n);
    for (int i = 0; i < n; i++) {
        const Mat4 * m = (const Mat4 *) handles[i];
        if (m->fmt != fmt || m->E != 1) { set_err("onpu_chain_new: entries need one format and dense handles"); return nullptr; }
        if (m->g.NT * m->g.KB * fmt_blk(fmt) > (int64_t) UINT32_MAX) {
            set_err("onpu_chain_new: a chained matrix must be under 4 GiB");
            return nullptr;
        }
        ChainEntry & e = es[(size_t) i];
        e = ChainEntry{};
        e.W = m->dev; e.x = (const uint16_t *) xs[i]; e.y = ys[i];
        e.NT = m->g.NT; e.KB = m->g.KB; e.N = m->N; e.K = m->K;
        // K split across 8 waves for up to 512 row tiles, else 4 (2 tiles per workgroup), else 2
        e.kw = e.NT <= 512 ? 8 : (e.NT <= 4096 ? 4 : 2);
        while (e.kw > 1 && e.kw > e.KB) e.kw /= 2;
        e.tw = CHAIN_WAVES / e.kw;
        e.bpw = (e.KB + e.kw - 1) / e.kw;
        e.groups = (e.NT + e.tw - 1) / e.tw;
        kbmax = std::max(kbmax, e.KB);
        xr[(size_t) i] = {(uintptr_t) xs[i], (uintptr_t) xs[i] + (uintptr_t) (M * m->K * 2)};
        yr[(size_t) i] = {(uintptr_t) ys[i], (uintptr_t) ys[i] + (uintptr_t) (M * m->N * (y_f32 ? 4 : 2))};
    }
    // x_j that lies in an earlier y_i reads it through y_i's link words: the whole row (x_j == y_i,
    // K_j == N_i) or, at M = 1, a range of it starting on an 8-element boundary. Any other overlap of
    // an x with a y, or of two ys, would be read while written and is refused.
    std::vector<int> src((size_t) n, -1);
    std::vector<int64_t> xoff((size_t) n, 0);
    for (int j = 0; j < n; j++) {
        for (int i = 0; i < n; i++) {
            if (i != j && overlap(yr[(size_t) i], yr[(size_t) j])) {
                set_err("onpu_chain_new: two entries' outputs overlap");
                return nullptr;
            }
            if (!overlap(xr[(size_t) j], yr[(size_t) i])) continue;
            const ChainEntry & P = es[(size_t) i];
            const ChainEntry & C = es[(size_t) j];
            const uintptr_t d = xr[(size_t) j].a - yr[(size_t) i].a;
            const bool inside = xr[(size_t) j].a >= yr[(size_t) i].a && xr[(size_t) j].b <= yr[(size_t) i].b;
            const bool whole = d == 0 && C.K == P.N;
            const bool range = M == 1 && inside && d % 16 == 0 && (int64_t) (d / 2) + C.K <= P.N;
            if (i >= j || y_f32 || !(whole || range) || src[(size_t) j] >= 0) {
                set_err(i >= j ? "onpu_chain_new: an entry reads memory that it or a later entry writes"
                               : "onpu_chain_new: an entry reads part of an earlier output in a layout the chain "
                                 "cannot link (bf16 outputs; the whole output, or at M = 1 a range of it starting "
                                 "on an 8-element boundary)");
                return nullptr;
            }
            src[(size_t) j] = i;
            xoff[(size_t) j] = (int64_t) (d / 2);
        }
    }
    if (src[0] >= 0) { set_err("onpu_chain_new: the first entry cannot read a chained output"); return nullptr; }
    for (int j = 0; j < n; j++)
        if (src[(size_t) j] < 0 && xr[(size_t) j].a % 16 != 0) {
            set_err("onpu_chain_new: an input x must start on a 16-byte boundary");
            return nullptr;
        }
    // link words for every output that a later entry reads: rows of whole tiles
    std::vector<int64_t> loff((size_t) n, -1);
    int64_t lbytes = 0;
    for (int j = 0; j < n; j++)
        if (src[(size_t) j] >= 0 && loff[(size_t) src[(size_t) j]] < 0) {
            const int i = src[(size_t) j];
            loff[(size_t) i] = lbytes;
            lbytes += M * es[(size_t) i].NT * 16 * 4;
        }
    auto * c = new Chain;
    c->fmt = fmt; c->n = n; c->M = (int) M; c->yf32 = y_f32;
    c->xls = kbmax * 128 + 8;
    // LDS: partial sums (two buffers), x rows, column sums, then the deepest weight ring that fits
    c->ring_off = (int64_t) 2 * CHAIN_WAVES * 256 * 4 + M * c->xls * 2 + kbmax * (fmt == ONPU_G128S ? 1 : 4) * 64;
    const int64_t blk = fmt_blk(fmt);
    c->ring = -1;
    for (int ri = 0; ri < 4 && c->ring < 0; ri++) {
        const size_t lds = (size_t) (c->ring_off + (int64_t) CHAIN_WAVES * CHAIN_RING_SLOTS[ri] * blk);
        if (lds <= 163840 && chain_occupancy(fmt, ri, lds) >= 1) { c->ring = ri; c->lds = lds; }
    }
    if (c->ring < 0) { set_err("onpu_chain_new: x rows do not fit in LDS"); delete c; return nullptr; }
    c->grid = device().cus;                // one workgroup per CU: the ring takes most of its LDS
    hipError_t e = c->ep.ensure(sizeof(int32_t) * (size_t) CHAIN_EP_INTS);
    if (e == hipSuccess) e = hipMemset(c->ep.p, 0, sizeof(int32_t) * (size_t) CHAIN_EP_INTS);
    if (e == hipSuccess && lbytes > 0) e = c->links.ensure((size_t) lbytes);
    if (e == hipSuccess && lbytes > 0) e = hipMemset(c->links.p, 0, (size_t) lbytes);   // epoch 0: no run's tag
    if (e == hipSuccess) {
        for (int i = 0; i < n; i++)
            if (loff[(size_t) i] >= 0) es[(size_t) i].ly = c->links.as<uint32_t>((size_t) loff[(size_t) i]);
        for (int j = 0; j < n; j++) {
            const int i = src[(size_t) j];
            if (i < 0) continue;
            ChainEntry & C = es[(size_t) j];
            C.ldl = es[(size_t) i].NT * 16;
            C.lx = es[(size_t) i].ly + xoff[(size_t) j];
            C.x = nullptr;
        }
        e = c->entries.ensure(sizeof(ChainEntry) * (size_t) n);
    }
    if (e == hipSuccess) e = hipMemcpy(c->entries.p, es.data(), sizeof(ChainEntry) * (size_t) n, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        c->entries.release(); c->ep.release(); c->links.release();
        delete c;
        return nullptr;
    }
    return c;
}

int onpu_chain_run(void * h, void * stream) {
    auto * c = (Chain *) h;
    ChainArgs a{};
    a.n = c->n; a.M = c->M; a.yf32 = c->yf32;
    a.ep = c->ep.as<int32_t>(); a.xls = c->xls; a.ring = c->ring_off;
    a.spin = 1u << 17;                     // polls of one wait: ~0.1-0.3 s, then the error flag
    HIPR(launch_chain(c->fmt, c->ring, a, c->entries.as<ChainEntry>(), c->grid, c->lds, (hipStream_t) stream));
    return 0;
}

int onpu_chain_status(void * h) {
    auto * c = (Chain *) h;
    int32_t flag = 0;
    int32_t * fp = c->ep.as<int32_t>(sizeof(int32_t) * CHAIN_EP_ERR);
    if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(&flag, fp, 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (flag && hipMemset(fp, 0, 4) != hipSuccess) return -1;
    return flag ? 1 : 0;
}

void onpu_chain_info(void * h, int64_t * out) {
    auto * c = (Chain *) h;
    out[0] = c->n; out[1] = c->grid; out[2] = (int64_t) c->lds; out[3] = c->xls;
    out[4] = CHAIN_RING_SLOTS[c->ring];
    uint32_t epoch = 0;
    out[5] = hipDeviceSynchronize() == hipSuccess &&
                     hipMemcpy(&epoch, c->ep.p, 4, hipMemcpyDeviceToHost) == hipSuccess
                 ? (int64_t) epoch
                 : -1;                     // runs completed (mod 2^32)
}

void onpu_chain_free(void * h) {
    auto * c = (Chain *) h;
    if (!c) return;
    c->entries.release();
    c->ep.release();
    c->links.release();
    delete c;
}

// ---------------------------------------------------------------- packing
// q4nx and q4s (sym 0 / 1): the reference's NPU packing, byte for byte (pack_mat,
// opennpu_core.hpp:174-254), which the handles of the reference calls take in their *_buf memory;
// this library's formats 2 and 3: their staging layout, zero-padded to nbytes
int64_t onpu_pack(const float * W, int64_t N, int64_t K, int ncols, int sym, uint8_t * out, int threads) {
    const RefGeom g = ref_geometry(N, K, ncols, sym != 0);
    if (!g.ok || !fmt_valid(sym) || K % fmt_group(sym) != 0) return 0;
    if (sym == ONPU_Q4NX || sym == ONPU_Q4S) return pack_npu(sym, W, N, K, g, out, threads) ? g.nbytes : 0;
    const int64_t sb = stage_bytes(sym, N, K);
    if (sb > g.nbytes) return 0;
    if (!pack_staging(sym, W, N, K, out, threads)) return 0;
    std::memset(out + sb, 0, (size_t) (g.nbytes - sb));
    return g.nbytes;
}

void onpu_quant_dequant(const float * W, int64_t N, int64_t K, int sym, float * out, int threads) {
    if (!fmt_valid(sym) || K % fmt_group(sym) != 0) return;
    std::vector<uint8_t> st((size_t) stage_bytes(sym, N, K));
    pack_staging(sym, W, N, K, st.data(), threads);
    dequant_staging(sym, st.data(), N, K, out, threads);
}

int64_t onpu_pack_q4k(const uint8_t * blocks, int64_t N, int64_t K, uint8_t * out, int threads) {
    if (!blocks || !out || !pack_q4k_staging(blocks, K / 256 * Q4K_BLOCK, N, K, out, threads)) return 0;
    return stage_bytes(ONPU_Q4NX, N, K);
}
}  // extern "C"

// ---------------------------------------------------------------- GPU weight codecs
// Experts [e0, e0 + n) of m from a device source: fill(e, k, staging, stride) writes the staging of
// experts e .. e + k - 1 (stride bytes apart) on stream s, which is then repacked into the tiled
// layout. The staging is a temporary of at most 256 MiB (or one expert), freed before returning,
// so the call waits for its launches.
template <class Fill>
static int codec_load(Mat4 * m, int64_t e0, int64_t n, hipStream_t s, Fill fill) {
    const int64_t sb = round_up(stage_bytes(m->fmt, m->N, m->K), 256);
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(n, ((int64_t) 256 << 20) / sb));
    if (n == 0) return 0;
    void * tmp = nullptr;
    HIPR(hipMalloc(&tmp, (size_t) (chunk * sb)));
    hipError_t e = hipSuccess;
    for (int64_t c = 0; c < n && e == hipSuccess; c += chunk) {
        const int64_t k = std::min(chunk, n - c);
        e = fill(e0 + c, k, (uint8_t *) tmp, sb);
        if (e == hipSuccess)
            e = launch_repack(m->fmt, (const uint8_t *) tmp, sb, m->N, m->K, m->dev + (e0 + c) * m->dstride, m->dstride,
                              k, s);
        if (e == hipSuccess) e = refresh_dec(m, e0 + c, k, s);
    }
    const hipError_t es = hipStreamSynchronize(s);
    (void) hipFree(tmp);
    if (e == hipSuccess) e = es;
    if (e != hipSuccess) { set_err("weight codec", e); return -1; }
    return 0;
}

extern "C" {

int onpu_quantize_dev(void * h, int64_t e0, int64_t n, const void * W, int64_t ldw, int w_bf16, void * stream) {
    auto * m = (Mat4 *) h;
    if (!m || !W || e0 < 0 || n < 0 || e0 + n > m->E || ldw < m->K || (w_bf16 != 0 && w_bf16 != 1)) {
        set_err("onpu_quantize_dev: bad arguments");
        return -1;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const hipStream_t s = (hipStream_t) stream;
    const int64_t es = m->N * ldw * (w_bf16 ? 2 : 4);           // bytes per expert of W
    return codec_load(m, e0, n, s, [&](int64_t e, int64_t k, uint8_t * st, int64_t sb) {
        return launch_quant_stage(m->fmt, (const char *) W + (e - e0) * es, ldw, w_bf16, m->N, m->K, k, st, sb, s);
    });
}

int onpu_gemv_i8_dev(const int8_t * W, const float * sc, int64_t N, int64_t K, const float * x, float * y,
                     void * stream) {
    if (!W || !sc || !x || !y || N < 0 || K < 0) {
        set_err("onpu_gemv_i8_dev: bad arguments");
        return -1;
    }
    const hipError_t e = launch_gemv_i8(W, sc, N, K, x, y, (hipStream_t) stream);
    if (e != hipSuccess) {
        set_err("onpu_gemv_i8_dev (K a multiple of 16 and at most 32768, W and x 16-byte aligned)", e);
        return -1;
    }
    return 0;
}

int64_t onpu_gdn_ws_bytes(int Hk, int Hv, int Dk, int Dv) { return gdn_ws_bytes(Hk, Hv, Dk, Dv); }

int onpu_gdn_step_dev(const float * x, int H, const float * qkv, const float * z, const float * Wb, const float * Wa,
                      const float * conv_w, int Kc, float * conv_state, int L, const float * A_log,
                      const float * dt_bias, const float * norm_w, float eps, float * S, int Hk, int Hv, int Dk,
                      int Dv, float * out, void * ws, int64_t ws_bytes, void * stream) {
    if (!x || !qkv || !z || !Wb || !Wa || !conv_w || !conv_state || !A_log || !dt_bias || !norm_w || !S || !out ||
        !ws) {
        set_err("onpu_gdn_step_dev: bad arguments");
        return -1;
    }
    const hipError_t e = launch_gdn_step(x, H, qkv, z, Wb, Wa, conv_w, Kc, conv_state, L, A_log, dt_bias, norm_w, eps,
                                         S, Hk, Hv, Dk, Dv, out, ws, ws_bytes, (hipStream_t) stream);
    if (e != hipSuccess) {
        set_err("onpu_gdn_step_dev (Hv a multiple of Hk, Dv dividing 256, Dk * Dv <= 32768, L >= Kc - 1, "
                "workspace of onpu_gdn_ws_bytes)", e);
        return -1;
    }
    return 0;
}

int64_t onpu_attn_ws_bytes(int Hq, int D, int Hkv, int64_t S) { return attn_ws_bytes(Hq, D, Hkv, S); }

int onpu_attn_step_dev(const float * q, int Hq, int D, const void * K, const void * V, int kv_bf16, int Hkv, int64_t S,
                       int64_t hs, int64_t rs, const float * mask, const float * sinks, float scale, float * out,
                       void * ws, int64_t ws_bytes, void * stream) {
    if (!q || !K || !V || !out || !ws || (kv_bf16 != 0 && kv_bf16 != 1)) {
        set_err("onpu_attn_step_dev: bad arguments");
        return -1;
    }
    const hipError_t e = launch_attn_step(q, Hq, D, K, V, kv_bf16, Hkv, S, hs, rs, mask, sinks, scale, out, ws, ws_bytes,
                                          (hipStream_t) stream);
    if (e != hipSuccess) {
        set_err("onpu_attn_step_dev (Hq a multiple of Hkv with Hq / Hkv <= 16, D <= 256 and a multiple of 8, "
                "16-byte aligned rows, workspace of onpu_attn_ws_bytes)", e);
        return -1;
    }
    return 0;
}

int onpu_transcode_q4k_dev(void * h, int64_t e0, int64_t n, const void * blocks, int64_t ld, void * stream) {
    auto * m = (Mat4 *) h;
    if (!m || !blocks || m->fmt != ONPU_Q4NX || m->K % 256 != 0 || e0 < 0 || n < 0 || e0 + n > m->E ||
        ld < m->K / 256 * Q4K_BLOCK) {
        set_err("onpu_transcode_q4k_dev: bad arguments (a q4nx handle, K a multiple of 256, rows of K / 256 blocks)");
        return -1;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const hipStream_t s = (hipStream_t) stream;
    const int64_t es = m->N * ld;                                 // bytes per expert of the blocks
    return codec_load(m, e0, n, s, [&](int64_t e, int64_t k, uint8_t * st, int64_t sb) {
        return launch_q4k_stage((const uint8_t *) blocks + (e - e0) * es, ld, es, m->N, m->K, k, st, sb, s);
    });
}

}  // extern "C"

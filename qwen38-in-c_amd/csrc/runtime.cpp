// runtime.cpp -- host side of libq35mm.so: device state, weight residency,
// kernel dispatch, and the two C ABIs (include/q35/q35_mm.h, the drop-in for
// qwen35-c/include/q35/q35_mm.h; include/q35mm/q35mm.h, the device API).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "q35/q35_mm.h"
#include "q35mm/q35mm.h"
#include "q35mm_internal.h"
#include "safetensors.h"

#include <unistd.h>

#define Q35MM_API extern "C" __attribute__((visibility("default")))

using namespace q35mm;

struct q35mm_weight {
    Weight w;
    size_t bytes = 0;
};

struct q35mm_st {
    st::Archive a;
};

struct q35mm_chain {
    void *mem = nullptr;     // step table, item lists, zeros, counters, flags, error word
    ChainParams p{};
};

namespace {

thread_local std::string t_last_error;

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_last_error = buf;
    return code;
}

#define HIP_TRY(expr)                                                                      \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess)                                                              \
            return set_error(Q35MM_EHIP, "%s failed: %s (%s:%d)", #expr,                  \
                             hipGetErrorString(e_), __FILE__, __LINE__);                   \
    } while (0)

[[noreturn]] void die(const char *where) {
    fprintf(stderr, "libq35mm: %s: %s\n", where, t_last_error.c_str());
    fflush(stderr);
    abort();
}

uint32_t env_u32(const char *name, uint32_t dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    return (uint32_t)strtoul(v, nullptr, 10);
}

// ---------------------------------------------------------------------
// Device state
// ---------------------------------------------------------------------
struct DevBuf {
    void *ptr = nullptr;
    size_t cap = 0;
};

// Scratch a launch sequence uses between its kernels.  One set per stream:
// work queued on different streams may run concurrently, and a shared set
// would let one call's kernels overwrite another's partials, counters or
// staged activations.
struct Scratch {
    DevBuf ws;        // split-K partials (float)
    DevBuf cnt;       // arrival counters (uint32, zero between launches)
    DevBuf xb;        // bf16 lane-order activations for the GEMM
    DevBuf mlp;       // MLP block intermediates (xn, gate, up, y)
    // Set for q35mm_matmul_noalloc: the device address of the fixed scratch
    // array (noalloc.hip); nothing is allocated, oversized requests fail.
    uint8_t *fixed = nullptr;
    // Set once a call captured into a HIP graph used this set: the graph
    // holds its buffers' addresses, so from then on they are never freed
    // before q35mm_shutdown -- growth allocates new buffers and retires the
    // old ones (a replay after a free would write into memory that may by
    // then belong to anything else, another stream's counters included).
    bool captured = false;
    // The current call's stream is being captured: it cannot allocate.
    bool capturing = false;
};

struct Device {
    int id = -1;
    hipStream_t stream = nullptr;
    std::unordered_map<hipStream_t, Scratch> scratch;
    Scratch *last_scratch = nullptr;   // of the most recent call outside graph capture
    std::vector<void *> retired;       // buffers a captured graph may still use (freed at shutdown)
    DevBuf dx, dy;    // activation staging for the host-pointer ABI
    void *up_pin[4] = {};        // pinned chunks of the file -> HBM upload ring
    void *up_dev[4] = {};        // device side of each chunk (+ room for its codes)
    hipEvent_t up_ev[4] = {};
    hipEvent_t xfer_ev[16] = {};   // chunks of a large host-pointer output copy
    void *pin = nullptr;   // pinned host staging
    size_t pin_cap = 0;
    uint32_t *done = nullptr;   // pinned completion word of host-pointer calls
    uint32_t done_seq = 0;
    uint32_t *done_cnt = nullptr;   // device counter of the in-kernel completion (zero between launches)
    // A host-pointer call's completion word, for the call's last launch to
    // store if it is a row-split GEMV (taken: it was attached to one).
    struct DoneReq {
        uint32_t *word = nullptr;
        uint32_t value = 0;
        bool taken = false;
    } done_req;
    bool done_spin = true;      // Q35MM_HOST_WAIT=sync: hipStreamSynchronize instead
    uint32_t gemm_min_m = 64;
    bool gemm_narrow = true;    // Q35MM_GEMM_NARROW=0: 256-token tiles for every m
    bool gemm_pair = true;      // Q35MM_GEMM_PAIR=0: two weights of one shape as separate tiles
    size_t xfer_chunk = 2u << 20;   // Q35MM_XFER_CHUNK_KB: chunk of a large host transfer (0: one piece)
    uint32_t cus = 256;
    uint32_t gemv_per_cu = kGemvCtasPerCu;
    bool trust_pointers = false;
    bool verify_full = false;   // Q35MM_VERIFY_WEIGHTS=full: fingerprint every byte of a reused host weight
    bool mlp_unfused = false;   // Q35MM_MLP_UNFUSED=1: separate neighbour kernels on the GEMV path
    uint32_t mlp_pair = 1;      // Q35MM_MLP_PAIR=0: row-split gate and up as plain GEMV launches;
                                //   2: paired, with the RMSNorm as its own kernel
    bool gemv_rows = true;      // Q35MM_GEMV_ROWSPLIT=0: every weight on the stream-K GEMV
    uint32_t rows_depth = 0;    // Q35MM_ROWS_DEPTH: ring depth of the row-split GEMV (0: by launch)
    uint32_t rows_waves = 4;    // Q35MM_ROWS_WAVES: wavefronts per row-split workgroup (4 or 8)
};

std::recursive_mutex g_mu;
Device g_dev;

int ensure_device() {
    if (g_dev.id >= 0) return Q35MM_OK;
    int dev = (int)env_u32("Q35MM_DEVICE", 0);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return set_error(Q35MM_ENODEV, "no HIP device visible");
    if (dev >= n) return set_error(Q35MM_ENODEV, "Q35MM_DEVICE=%d but %d devices", dev, n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(Q35MM_ENODEV, "device %d is %s; libq35mm is built for gfx950 only", dev,
                         prop.gcnArchName);
    HIP_TRY(hipSetDevice(dev));
    HIP_TRY(hipStreamCreateWithFlags(&g_dev.stream, hipStreamNonBlocking));
    HIP_TRY(noalloc_setup(dev, g_dev.stream));
    g_dev.id = dev;
    g_dev.gemm_min_m = env_u32("Q35MM_GEMM_MIN_M", 64);
    g_dev.gemm_narrow = env_u32("Q35MM_GEMM_NARROW", 1) != 0;
    g_dev.gemm_pair = env_u32("Q35MM_GEMM_PAIR", 1) != 0;
    g_dev.xfer_chunk = (size_t)env_u32("Q35MM_XFER_CHUNK_KB", 2048) << 10;
    g_dev.trust_pointers = env_u32("Q35MM_TRUST_POINTERS", 0) != 0;
    {
        const char *v = getenv("Q35MM_VERIFY_WEIGHTS");
        g_dev.verify_full = v && strcmp(v, "full") == 0;
    }
    g_dev.mlp_unfused = env_u32("Q35MM_MLP_UNFUSED", 0) != 0;
    g_dev.mlp_pair = env_u32("Q35MM_MLP_PAIR", 1);
    {
        const char *v = getenv("Q35MM_HOST_WAIT");
        g_dev.done_spin = !(v && strcmp(v, "sync") == 0);
    }
    g_dev.cus = (uint32_t)prop.multiProcessorCount;
    g_dev.gemv_per_cu = std::max(1u, env_u32("Q35MM_GEMV_CTAS_PER_CU", kGemvCtasPerCu));
    g_dev.gemv_rows = env_u32("Q35MM_GEMV_ROWSPLIT", 1) != 0;
    g_dev.rows_depth = env_u32("Q35MM_ROWS_DEPTH", 0);
    g_dev.rows_waves = env_u32("Q35MM_ROWS_WAVES", 4) == 8 ? 8 : 4;
    return Q35MM_OK;
}

// Device-API streams follow the HIP convention: NULL is the null stream.
hipStream_t pick_stream(void *s) { return (hipStream_t)s; }

// The scratch of stream st.  A stream first seen while it is being captured
// into a graph cannot allocate: it shares the scratch of the most recent
// call made outside capture (its warm-up, in the usual capture pattern), so
// such a graph and eager work on that stream must not run at the same time.
// A set used under capture is marked captured (its buffers are never freed
// before q35mm_shutdown, see Scratch).
Scratch &scratch_for(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    Scratch *s = nullptr;
    auto it = g_dev.scratch.find(st);
    if (it != g_dev.scratch.end())
        s = &it->second;
    else if (capturing && g_dev.last_scratch)
        s = g_dev.last_scratch;
    else
        s = &g_dev.scratch.emplace(st, Scratch()).first->second;
    s->capturing = capturing;
    if (capturing)
        s->captured = true;
    else
        g_dev.last_scratch = s;
    return *s;
}

// Grows a device buffer; waits for the device first because kernels queued
// on any stream may still use the old allocation.  owner: the scratch set
// the buffer belongs to (null for the host-pointer ABI's own buffers): under
// capture nothing can be allocated, and a set a graph has captured keeps its
// old buffer alive (retired) instead of freeing it.
int grow(DevBuf &b, size_t bytes, bool zero, Scratch *owner = nullptr) {
    if (b.cap >= bytes) return Q35MM_OK;
    if (owner && owner->capturing)
        return set_error(Q35MM_EINVAL, "%zu bytes of scratch needed while the stream is being captured into a "
                         "graph (%zu available): a capture cannot allocate -- make the same call once outside "
                         "capture first", bytes, b.cap);
    size_t cap = std::max(bytes, b.cap * 2);
    cap = (cap + 4095) & ~(size_t)4095;
    HIP_TRY(hipDeviceSynchronize());
    if (b.ptr) {
        if (owner && owner->captured)
            g_dev.retired.push_back(b.ptr);
        else
            HIP_TRY(hipFree(b.ptr));
    }
    b.ptr = nullptr;
    b.cap = 0;
    if (hipMalloc(&b.ptr, cap) != hipSuccess) {
        b.ptr = nullptr;
        return set_error(Q35MM_ENOMEM, "hipMalloc(%zu) failed", cap);
    }
    if (zero) HIP_TRY(hipMemset(b.ptr, 0, cap));
    b.cap = cap;
    return Q35MM_OK;
}

int grow_pinned(size_t bytes) {
    if (g_dev.pin_cap >= bytes) return Q35MM_OK;
    size_t cap = std::max(bytes, g_dev.pin_cap * 2);
    cap = (cap + 4095) & ~(size_t)4095;
    if (g_dev.pin) HIP_TRY(hipHostFree(g_dev.pin));
    g_dev.pin = nullptr;
    g_dev.pin_cap = 0;
    if (hipHostMalloc(&g_dev.pin, cap, hipHostMallocDefault) != hipSuccess) {
        g_dev.pin = nullptr;
        return set_error(Q35MM_ENOMEM, "hipHostMalloc(%zu) failed", cap);
    }
    g_dev.pin_cap = cap;
    return Q35MM_OK;
}

// Stream-K partials and arrival counters of one launch.
int scratch_splitk(Scratch &s, size_t ws_bytes, size_t cnt_bytes, float **ws, uint32_t **cnt) {
    if (s.fixed) {
        if (cnt_bytes > kNoAllocCntBytes || ws_bytes > kNoAllocBytes)
            return set_error(Q35MM_EINVAL, "no-alloc scratch: %zu bytes of partials and %zu of counters needed, "
                             "%zu and %zu available", ws_bytes, cnt_bytes, kNoAllocBytes, kNoAllocCntBytes);
        *cnt = reinterpret_cast<uint32_t *>(s.fixed);
        *ws = reinterpret_cast<float *>(s.fixed + kNoAllocCntBytes);
        return Q35MM_OK;
    }
    int rc = grow(s.ws, ws_bytes, false, &s);
    if (!rc) rc = grow(s.cnt, cnt_bytes, true, &s);
    if (rc) return rc;
    *ws = (float *)s.ws.ptr;
    *cnt = (uint32_t *)s.cnt.ptr;
    return Q35MM_OK;
}

// The GEMM's lane-order bf16 activations and K-slice partials.
int scratch_gemm(Scratch &s, size_t xb_bytes, size_t ws_bytes, uint16_t **xb, float **ws) {
    if (s.fixed) {
        const size_t xb_al = (xb_bytes + 255) & ~(size_t)255;
        if (xb_al + ws_bytes > kNoAllocBytes)
            return set_error(Q35MM_EINVAL, "no-alloc scratch: %zu bytes of activations and %zu of partials "
                             "needed, %zu available", xb_bytes, ws_bytes, kNoAllocBytes);
        *xb = reinterpret_cast<uint16_t *>(s.fixed + kNoAllocCntBytes);
        *ws = reinterpret_cast<float *>(s.fixed + kNoAllocCntBytes + xb_al);
        return Q35MM_OK;
    }
    int rc = grow(s.xb, xb_bytes, false, &s);
    if (!rc && ws_bytes) rc = grow(s.ws, ws_bytes, false, &s);
    if (rc) return rc;
    *xb = (uint16_t *)s.xb.ptr;
    *ws = (float *)s.ws.ptr;
    return Q35MM_OK;
}

// ---------------------------------------------------------------------
// Weight upload
// ---------------------------------------------------------------------
// Allocates a resident weight and lets fill() write its lane-order tiles
// and fp32 block scales (asynchronously on st); synchronises st.
template <typename Fill>
int weight_alloc_fill(uint32_t rows, uint32_t cols, q35mm_weight **out, Fill fill) {
    if (!out) return set_error(Q35MM_EINVAL, "null argument");
    if (rows == 0 || cols == 0) return set_error(Q35MM_EINVAL, "empty weight %ux%u", rows, cols);
    int rc = ensure_device();
    if (rc) return rc;
    const uint32_t nb = (rows + 127) / 128, kb = (cols + 127) / 128;
    auto *h = new q35mm_weight();
    h->w.rows = rows;
    h->w.cols = cols;
    h->w.nb = nb;
    h->w.kb = kb;
    const size_t tiled_bytes = (size_t)nb * kb * kBlockBytes;
    const size_t scale_bytes = (size_t)nb * kb * sizeof(float);
    auto fail = [&](int code) {
        (void)hipStreamSynchronize(g_dev.stream);
        if (h->w.codes) (void)hipFree(h->w.codes);
        if (h->w.scale) (void)hipFree(h->w.scale);
        delete h;
        return code;
    };
    if (hipMalloc(&h->w.codes, tiled_bytes) != hipSuccess) {
        h->w.codes = nullptr;
        return fail(set_error(Q35MM_ENOMEM, "hipMalloc(%zu) for weight codes failed", tiled_bytes));
    }
    if (hipMalloc(&h->w.scale, scale_bytes) != hipSuccess) {
        h->w.scale = nullptr;
        return fail(set_error(Q35MM_ENOMEM, "hipMalloc(%zu) for scales failed", scale_bytes));
    }
    hipStream_t st = g_dev.stream;
    rc = fill(h->w, st);
    if (rc) return fail(rc);
    if (hipStreamSynchronize(st) != hipSuccess)
        return fail(set_error(Q35MM_EHIP, "weight upload failed: %s", hipGetErrorString(hipGetLastError())));
    // the spread of live scales per row group, from the resident fp32 scales
    // (whatever produced them: host arrays, a checkpoint, the device quantizer)
    {
        std::vector<float> sc((size_t)nb * kb);
        if (hipMemcpy(sc.data(), h->w.scale, scale_bytes, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(set_error(Q35MM_EHIP, "scale read-back failed"));
        for (uint32_t g = 0; g < nb && !h->w.wide_scales; g++) {
            float lo = INFINITY, hi = 0.0f;
            for (uint32_t j = 0; j < kb; j++) {
                const float v = std::fabs(sc[(size_t)g * kb + j]);
                if (v == 0.0f || v != v) continue;
                lo = std::min(lo, v);
                hi = std::max(hi, v);
            }
            h->w.wide_scales = hi > 0.0f && (std::isinf(hi) || hi / lo > kGemmScaleSpan);
        }
    }
    h->bytes = tiled_bytes + scale_bytes;
    *out = h;
    return Q35MM_OK;
}

// As weight_alloc_fill, with fill() writing row-major e4m3 codes into a
// device staging buffer raw, which is then repacked into the tiles.
template <typename Fill>
int weight_build(uint32_t rows, uint32_t cols, q35mm_weight **out, Fill fill) {
    uint8_t *raw = nullptr;
    const size_t raw_bytes = (size_t)rows * cols;
    const int rc = weight_alloc_fill(rows, cols, out, [&](Weight &w, hipStream_t st) -> int {
        if (hipMalloc(&raw, raw_bytes) != hipSuccess) {
            raw = nullptr;
            return set_error(Q35MM_ENOMEM, "hipMalloc(%zu) for staging failed", raw_bytes);
        }
        int r = fill(w, raw, st);
        if (r) return r;
        HIP_TRY(launch_repack(raw, rows, cols, w.nb, w.kb, w.codes, st));
        return Q35MM_OK;
    });
    if (raw) {
        (void)hipStreamSynchronize(g_dev.stream);
        (void)hipFree(raw);
    }
    return rc;
}

int weight_create(const uint8_t *W, const float *scale_f32_rowmajor, uint32_t rows, uint32_t cols,
                  q35mm_weight **out) {
    if (!W || !scale_f32_rowmajor) return set_error(Q35MM_EINVAL, "null argument");
    return weight_build(rows, cols, out, [&](Weight &w, uint8_t *raw, hipStream_t st) -> int {
        HIP_TRY(hipMemcpyAsync(raw, W, (size_t)rows * cols, hipMemcpyHostToDevice, st));
        HIP_TRY(hipMemcpyAsync(w.scale, scale_f32_rowmajor, (size_t)w.nb * w.kb * sizeof(float),
                               hipMemcpyHostToDevice, st));
        return Q35MM_OK;
    });
}

std::vector<float> widen_scales(const uint16_t *sc, uint32_t rows, uint32_t cols) {
    const uint32_t nb = (rows + 127) / 128, kb = (cols + 127) / 128;
    std::vector<float> f((size_t)nb * kb);
    for (size_t i = 0; i < f.size(); i++) {
        uint32_t u = (uint32_t)sc[i] << 16;
        memcpy(&f[i], &u, 4);
    }
    return f;
}

// ---------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------
// What the GEMV stages as activations (kXPlain: X itself; kXRmsNorm: the
// RMSNorm of X with norm_w; kXSwiGLU: silu(X) * x2).
struct GemvInput {
    uint32_t xmode = kXPlain;
    const float *x2 = nullptr;
    const float *norm_w = nullptr;
    float eps = 0.0f;
};

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// SwiGLU costs every down-GEMV workgroup an exp per staged column and token;
// beyond this many tokens the separate kernel (one exp per element) is
// cheaper.
constexpr uint32_t kMlpFusedSwiGLUMaxM = 2;

// Which decode GEMV a weight runs on; fixed by its shape (and the device),
// never by m or by the other weights of a call.
enum GemvKind : uint32_t { kStreamK = 0, kRows = 1 };

uint32_t gemv_kind(const Weight &w) {
    return g_dev.gemv_rows && gemv_rows_shape(w.kb, g_dev.rows_waves) ? kRows : kStreamK;
}

bool uses_gemv_rows(const Weight &w) { return gemv_kind(w) != kStreamK; }

// Launches of at most this many workgroups signal a host-pointer call's
// completion themselves (one counter all of them add to at their end);
// longer ones leave it to the flag kernel, whose cost is small beside them.
constexpr uint32_t kInKernelDoneMaxCtas = 512;

int run_gemv_group(const q35mm_weight *const *w, uint32_t nseg, uint32_t m, const float *dX,
                   float *const *dY, hipStream_t st, const GemvInput &in, float *const *resid, Scratch *scr,
                   bool last_launch = false) {
    GemvParams p{};
    const uint32_t cols = w[0]->w.cols, KB = w[0]->w.kb;
    p.x = dX;
    p.x2 = in.x2;
    p.norm_w = in.norm_w;
    p.eps = in.eps;
    p.xmode = in.xmode;
    p.norm_cols = in.xmode == kXRmsNorm ? gemv_norm_cols(cols) : 0;
    p.ldx = cols;
    p.m = m;
    p.k = cols;
    p.kb = KB;
    p.nseg = nseg;
    p.x_vec = (aligned16(dX) && cols % 8 == 0 && (!in.x2 || aligned16(in.x2)) &&
               (!in.norm_w || aligned16(in.norm_w))) ? 1u : 0u;
    const uint32_t kind = gemv_kind(w[0]->w);
    if (kind != kStreamK) {
        // the callers keep row-split weights on plain activations
        if (in.xmode != kXPlain) return set_error(Q35MM_EINVAL, "row-split GEMV takes plain activations");
        uint32_t cta = 0, rows[4], nct[4];
        for (uint32_t s = 0; s < nseg; s++) rows[s] = w[s]->w.rows;
        gemv_rows_plan(rows, nseg, nct);
        for (uint32_t s = 0; s < nseg; s++) {
            const Weight &ws = w[s]->w;
            GemvSeg &g = p.seg[s];
            g.codes = ws.codes;
            g.scale = ws.scale;
            g.y = dY[s];
            g.resid = resid ? resid[s] : nullptr;
            g.rows = ws.rows;
            g.ldy = ws.rows;
            g.nb = ws.nb;
            g.cta_begin = cta;
            g.nctas = nct[s];
            cta += g.nctas;
        }
        p.nctas = cta;
        if (last_launch && g_dev.done_req.word && cta <= kInKernelDoneMaxCtas) {
            p.done_word = g_dev.done_req.word;
            p.done_cnt = g_dev.done_cnt;
            p.done_value = g_dev.done_req.value;
        }
        HIP_TRY(launch_gemv_rows(p, g_dev.cus, g_dev.rows_waves, g_dev.rows_depth, st));
        if (p.done_word) g_dev.done_req.taken = true;
        return Q35MM_OK;
    }
    uint32_t cta = 0, wsoff = 0, cntoff = 0, max_range = 1;
    for (uint32_t s = 0; s < nseg; s++) {
        const Weight &ws = w[s]->w;
        const uint32_t T = ws.nb * KB;
        const uint32_t P = gemv_ctas(T, g_dev.cus, g_dev.gemv_per_cu);
        GemvSeg &g = p.seg[s];
        g.codes = ws.codes;
        g.scale = ws.scale;
        g.y = dY[s];
        g.resid = resid ? resid[s] : nullptr;
        g.rows = ws.rows;
        g.ldy = ws.rows;
        g.nb = ws.nb;
        g.cta_begin = cta;
        g.nctas = P;
        g.maxc = gemv_max_contrib(T, P, KB);
        g.ws_off = wsoff;
        g.cnt_off = cntoff;
        cta += P;
        wsoff += ws.nb * g.maxc * kGemvMaxM * kBlock;
        cntoff += ws.nb;
        max_range = std::max(max_range, (T + P - 1) / P);
    }
    p.nctas = cta;
    p.max_range = max_range;
    const int rc = scratch_splitk(scr ? *scr : scratch_for(st), (size_t)wsoff * sizeof(float),
                                  (size_t)cntoff * sizeof(uint32_t), &p.ws, &p.cnt);
    if (rc) return rc;
    HIP_TRY(launch_gemv(p, st));
    return Q35MM_OK;
}

// Weights sharing K, in groups of up to 8 tokens; stream-K weights share one
// launch, row-split weights another.
int run_gemv(const q35mm_weight *const *w, uint32_t nseg, uint32_t m, const float *dX,
             float *const *dY, hipStream_t st, const GemvInput &in = GemvInput(),
             float *const *resid = nullptr, Scratch *scr = nullptr) {
    const uint32_t cols = w[0]->w.cols;
    for (uint32_t t0 = 0; t0 < m; t0 += kGemvMaxM) {
        const uint32_t mg = std::min(kGemvMaxM, m - t0);
        GemvInput ig = in;
        if (ig.x2) ig.x2 += (size_t)t0 * cols;
        for (uint32_t kind = kStreamK; kind <= kRows; kind++) {
            const q35mm_weight *wg[4];
            float *ys[4], *rs[4];
            uint32_t n = 0;
            for (uint32_t s = 0; s < nseg; s++) {
                if (gemv_kind(w[s]->w) != kind) continue;
                wg[n] = w[s];
                ys[n] = dY[s] + (size_t)t0 * w[s]->w.rows;
                rs[n] = resid ? resid[s] + (size_t)t0 * w[s]->w.rows : nullptr;
                n++;
            }
            if (!n) continue;
            // the call's last launch: the row-split one of the last token group
            const bool last = t0 + kGemvMaxM >= m && kind == kRows;
            int rc = run_gemv_group(wg, n, mg, dX + (size_t)t0 * cols, ys, st, ig, resid ? rs : nullptr, scr, last);
            if (rc) return rc;
        }
    }
    return Q35MM_OK;
}

// The GEMM kernel addresses both operands with 32-bit byte offsets.
bool gemm_fits(const Weight &w, uint32_t m) {
    if (w.wide_scales) return false;
    const uint64_t mtiles = (m + kGemmTile - 1) / kGemmTile;
    const uint64_t xb_bytes = mtiles * kGemmTile * w.kb * kBlock * sizeof(uint16_t);
    const uint64_t w_bytes = (uint64_t)w.nb * w.kb * kBlockBytes;
    return xb_bytes <= UINT32_MAX && w_bytes <= UINT32_MAX;
}

// Weights sharing K (cols) and x, one launch over all their tiles.  Optional:
// resid[s] (y = resid + product, may alias y) and x2 (the activations are
// silu(x) * x2, formed while rounding them to bf16).
// RMSNorm applied to the GEMM's activations as they are rounded to bf16
// (run_gemm's norm): weight w of the activations' length, epsilon eps.
struct GemmNorm {
    const float *w;
    float eps;
};

// Two weights of one shape (gate and up) run as paired tiles, each holding
// the same rows of both; with a GemmAct the tiles write silu(weight 0) *
// weight 1 straight into the next GEMM's bf16 activations (buf: rows_pad x
// nb*128 of gemm_act_bytes), and done says so (when the weights do not
// pair, they wrote the fp32 outputs).
struct GemmAct {
    uint16_t *buf;
    bool done;
};
size_t gemm_act_bytes(uint32_t m, uint32_t cols) {
    const uint32_t tile_m = m <= kGemmNarrowMaxM && g_dev.gemm_narrow ? kGemmNarrowMaxM : kGemmTile;
    return (size_t)(m + tile_m - 1) / tile_m * tile_m * ((cols + kBlock - 1) / kBlock) * kBlock * sizeof(uint16_t);
}

// xb_ready: the activations already in the GEMM's bf16 layout (a paired
// GEMM's GemmAct output), so no conversion runs and dX is not read.
int run_gemm(const q35mm_weight *const *wt, uint32_t nseg, uint32_t m, const float *dX, float *const *dY,
             hipStream_t st, const float *const *resid = nullptr, const float *x2 = nullptr,
             Scratch *scr = nullptr, const GemmNorm *norm = nullptr, GemmAct *act = nullptr,
             const uint16_t *xb_ready = nullptr) {
    const Weight &w0 = wt[0]->w;
    Scratch &sc = scr ? *scr : scratch_for(st);
    for (uint32_t s = 0; s < nseg; s++) {
        const Weight &w = wt[s]->w;
        if (w.wide_scales)
            return set_error(Q35MM_EINVAL, "block scales of a %ux%u weight span more than 2^64 within a row group: "
                             "beyond the GEMM's accumulator range (q35mm_matmul runs it on the GEMV)", w.rows, w.cols);
        if (!gemm_fits(w, m))
            return set_error(Q35MM_EINVAL, "GEMM operands exceed 4 GiB (m=%u, %ux%u)", m, w.rows, w.cols);
    }
    // Two weights of one shape: paired tiles (the first half of a tile's
    // rows from weight 0, the same rows of weight 1 in the second half).
    const bool pair = nseg == 2 && g_dev.gemm_pair && !resid && !x2 && wt[0]->w.rows == wt[1]->w.rows &&
                      wt[0]->w.nb == wt[1]->w.nb;
    // Up to 128 tokens: tiles of 128 tokens x 512 rows (4 row groups), whose
    // partial round is cut along K -- unless those partials would not fit
    // the fixed scratch of an allocation-free call, which then keeps the
    // 256 x 256 tiles it always took.
    auto plan_for = [&](bool narrow, uint32_t &groups, size_t &xb_bytes) {
        groups = narrow ? kGemmNarrowRows / kBlock : kGemmTile / kBlock;
        uint32_t ntiles = 0;
        if (pair)
            ntiles = (w0.nb + groups / 2 - 1) / (groups / 2);
        else
            for (uint32_t s = 0; s < nseg; s++) ntiles += (wt[s]->w.nb + groups - 1) / groups;
        const GemmPlan pl = gemm_plan(m, ntiles, w0.kb, g_dev.cus, narrow);
        xb_bytes = (size_t)pl.mtiles * (narrow ? kGemmNarrowMaxM : kGemmTile) * w0.kb * kBlock * sizeof(uint16_t);
        return pl;
    };
    bool narrow = m <= kGemmNarrowMaxM && g_dev.gemm_narrow;
    uint32_t groups;
    size_t xb_bytes;
    GemmPlan pl = plan_for(narrow, groups, xb_bytes);
    if (narrow && sc.fixed && ((xb_bytes + 255) & ~(size_t)255) + pl.ws_bytes() > kNoAllocBytes) {
        narrow = false;
        pl = plan_for(false, groups, xb_bytes);
    }
    const uint32_t tile_m = narrow ? kGemmNarrowMaxM : kGemmTile;
    uint16_t *xb = nullptr;
    float *ws = nullptr;
    const int rc = scratch_gemm(sc, xb_ready ? 0 : xb_bytes, pl.ws_bytes(), &xb, &ws);
    if (rc) return rc;
    if (xb_ready) xb = const_cast<uint16_t *>(xb_ready);
    const bool act_out = pair && act && act->buf;
    if (act) act->done = act_out;
    GemmParams p{};
    uint32_t tile0 = 0;
    for (uint32_t s = 0; s < nseg; s++) {
        const Weight &w = wt[s]->w;
        GemmSeg &g = p.seg[s];
        g.codes = w.codes;
        g.scale = w.scale;
        g.y = dY[s];
        g.resid = resid ? resid[s] : nullptr;
        g.rows = w.rows;
        g.ldy = w.rows;
        g.nb = w.nb;
        g.tile0 = pair ? 0 : tile0;
        tile0 += pl.mtiles * ((w.nb + groups - 1) / groups);
    }
    p.pair = pair ? 1u : 0u;
    p.act_out = act_out ? act->buf : nullptr;
    p.act_kb = act_out ? w0.nb : 0u;
    p.nseg = nseg;
    p.xb = xb;
    p.ws = ws;
    p.m = m;
    p.kb = w0.kb;
    p.mtiles = pl.mtiles;
    p.ntiles = pl.ntiles;
    p.split_tile0 = pl.split_tile0;
    p.nslices = pl.nslices;
    p.tail_tile0 = pl.tail_tile0;
    p.narrow = narrow ? 1u : 0u;
    if (xb_ready) {
        // activations written by the previous GEMM
    } else if (norm) {
        HIP_TRY(launch_rmsnorm_bf16(dX, w0.cols, norm->w, m, w0.cols, norm->eps, pl.mtiles * tile_m, w0.kb, xb, st));
    } else {
        HIP_TRY(launch_act_to_bf16(dX, x2, w0.cols, m, w0.cols, pl.mtiles * (tile_m / kSubRows), w0.kb, xb, st));
    }
    HIP_TRY(launch_gemm(p, st));
    return Q35MM_OK;
}

int check_weight(const q35mm_weight *w) {
    if (!w || !w->w.codes) return set_error(Q35MM_EINVAL, "null weight handle");
    return Q35MM_OK;
}

int run_matmul(const q35mm_weight *w, uint32_t m, const float *dX, float *dY, hipStream_t st,
               Scratch *scr = nullptr) {
    if (m == 0) return Q35MM_OK;
    const q35mm_weight *ws[1] = {w};
    float *ys[1] = {dY};
    if (m >= g_dev.gemm_min_m && g_dev.gemm_min_m > 0 && gemm_fits(w->w, m))
        return run_gemm(ws, 1, m, dX, ys, st, nullptr, nullptr, scr);
    return run_gemv(ws, 1, m, dX, ys, st, GemvInput(), nullptr, scr);
}

// ---------------------------------------------------------------------
// Checkpoint (safetensors) -> HBM
// ---------------------------------------------------------------------
constexpr size_t kUpChunk = 16u << 20;   // bytes per pinned chunk
constexpr int kUpBufs = 4;

int upload_ring() {
    for (int i = 0; i < kUpBufs; i++) {
        if (g_dev.up_pin[i]) continue;
        if (hipHostMalloc(&g_dev.up_pin[i], kUpChunk, hipHostMallocDefault) != hipSuccess) {
            g_dev.up_pin[i] = nullptr;
            return set_error(Q35MM_ENOMEM, "hipHostMalloc(%zu) for the upload ring failed", kUpChunk);
        }
        if (hipMalloc(&g_dev.up_dev[i], kUpChunk + kUpChunk / 2) != hipSuccess) {
            g_dev.up_dev[i] = nullptr;
            return set_error(Q35MM_ENOMEM, "hipMalloc for the upload ring failed");
        }
        HIP_TRY(hipEventCreateWithFlags(&g_dev.up_ev[i], hipEventDisableTiming));
    }
    for (int i = 0; i < kUpBufs; i++) HIP_TRY(hipEventSynchronize(g_dev.up_ev[i]));
    return Q35MM_OK;
}

// Streams bytes [0, t.bytes) of tensor t through the ring in pieces of at
// most piece bytes (a multiple of the tensor's row size for the callers
// below): piece i is read from the file into pinned slot i % 4 (reader
// threads), copied to the device slot, and handed to
// consume(i, offset, bytes, device slot) on st; a slot is reused once the
// work queued after it has finished.
template <typename Consume>
int stream_tensor(const st::Archive &a, const st::Tensor &t, uint64_t piece, hipStream_t st, Consume consume) {
    int rc = upload_ring();
    if (rc) return rc;
    size_t i = 0;
    for (uint64_t off = 0; off < t.bytes; off += piece, i++) {
        const int b = (int)(i % kUpBufs);
        if (i >= (size_t)kUpBufs) HIP_TRY(hipEventSynchronize(g_dev.up_ev[b]));
        const uint64_t len = std::min<uint64_t>(piece, t.bytes - off);
        if (!a.read_parallel(t, off, len, g_dev.up_pin[b]))
            return set_error(Q35MM_EIO, "read of %s (%llu bytes at %llu) failed", t.name.c_str(),
                             (unsigned long long)len, (unsigned long long)off);
        HIP_TRY(hipMemcpyAsync(g_dev.up_dev[b], g_dev.up_pin[b], len, hipMemcpyHostToDevice, st));
        rc = consume(i, off, len, static_cast<uint8_t *>(g_dev.up_dev[b]));
        if (rc) return rc;
        HIP_TRY(hipEventRecord(g_dev.up_ev[b], st));
    }
    return Q35MM_OK;
}

// Whole tensor -> device dst (no conversion).
int upload_tensor(const st::Archive &a, const st::Tensor &t, void *dst, hipStream_t st) {
    uint8_t *d = static_cast<uint8_t *>(dst);
    return stream_tensor(a, t, kUpChunk, st, [&](size_t, uint64_t off, uint64_t len, uint8_t *src) -> int {
        HIP_TRY(hipMemcpyAsync(d + off, src, len, hipMemcpyDeviceToDevice, st));
        return Q35MM_OK;
    });
}

// Rows per piece for a tensor of row_bytes bytes per row: whole 128-row
// groups, as many as fit a chunk (0 if one group does not fit).
uint64_t group_rows_per_piece(uint64_t row_bytes) {
    const uint64_t groups = kUpChunk / (128 * row_bytes);
    return groups * 128;
}

// F8_E4M3 [rows][cols] tensor -> the lane-order tiles of w, piece by piece:
// each piece is whole 128-row groups, which are contiguous in the tiles.
int upload_fp8_tiled(const st::Archive &a, const st::Tensor &t, Weight &w, hipStream_t st) {
    const uint64_t prow = group_rows_per_piece(w.cols);
    return stream_tensor(a, t, prow * w.cols, st, [&](size_t, uint64_t off, uint64_t len, uint8_t *src) -> int {
        const uint32_t r0 = (uint32_t)(off / w.cols), n = (uint32_t)(len / w.cols);
        uint8_t *dst = w.codes + (size_t)(r0 / kBlock) * w.kb * kBlockBytes;
        HIP_TRY(launch_repack(src, n, w.cols, (n + kBlock - 1) / kBlock, w.kb, dst, st));
        return Q35MM_OK;
    });
}

// BF16 [rows][cols] tensor -> quantized codes (tiles of w) and fp32 scales,
// piece by piece (whole 128-row groups, which quantize independently).
int upload_bf16_quantized(const st::Archive &a, const st::Tensor &t, Weight &w, hipStream_t st) {
    const uint64_t prow = group_rows_per_piece((uint64_t)w.cols * 2);
    return stream_tensor(a, t, prow * w.cols * 2, st, [&](size_t, uint64_t off, uint64_t len, uint8_t *src) -> int {
        const uint32_t r0 = (uint32_t)(off / ((uint64_t)w.cols * 2)), n = (uint32_t)(len / ((uint64_t)w.cols * 2));
        const uint32_t g0 = r0 / kBlock, ng = (n + kBlock - 1) / kBlock;
        uint8_t *codes = src + kUpChunk;   // the slot's spare half
        HIP_TRY(launch_quantize_bf16(reinterpret_cast<const uint16_t *>(src), n, w.cols, codes, nullptr,
                                     w.scale + (size_t)g0 * w.kb, st));
        HIP_TRY(launch_repack(codes, n, w.cols, ng, w.kb, w.codes + (size_t)g0 * w.kb * kBlockBytes, st));
        return Q35MM_OK;
    });
}

// The reference loader's strict lookup (qwen35-c/src/q35_model.c:225-249):
// present, of dtype dt, with exactly these dims.
int need_tensor(const st::Archive &a, const char *name, int dt, uint32_t ndim, const uint32_t *shape,
                const st::Tensor **out) {
    const st::Tensor *t = a.find(name);
    if (!t) return set_error(Q35MM_ENOTFOUND, "missing tensor: %s", name);
    if (t->dtype != dt)
        return set_error(Q35MM_ESHAPE, "tensor %s: dtype %s, want %s", name, st::dtype_name(t->dtype),
                         st::dtype_name(dt));
    if (t->ndim != ndim) return set_error(Q35MM_ESHAPE, "tensor %s: ndim %u, want %u", name, t->ndim, ndim);
    for (uint32_t i = 0; i < ndim; i++)
        if (t->shape[i] != shape[i])
            return set_error(Q35MM_ESHAPE, "tensor %s: shape[%u]=%u, want %u", name, i, t->shape[i], shape[i]);
    *out = t;
    return Q35MM_OK;
}

// bind_fp8 (qwen35-c/src/q35_model.c:253-273): F8_E4M3 [rows][cols] plus
// BF16 "<name>_scale_inv" [ceil(rows/128)][ceil(cols/128)], uploaded and
// repacked on the device.
int st_load_fp8(const st::Archive &a, const char *name, uint32_t rows, uint32_t cols, q35mm_weight **out) {
    const uint32_t wshape[2] = {rows, cols}, sshape[2] = {(rows + 127) / 128, (cols + 127) / 128};
    const st::Tensor *tw = nullptr, *ts = nullptr;
    int rc = need_tensor(a, name, st::kF8E4M3, 2, wshape, &tw);
    if (rc) return rc;
    const std::string sname = std::string(name) + "_scale_inv";
    rc = need_tensor(a, sname.c_str(), st::kBF16, 2, sshape, &ts);
    if (rc) return rc;
    std::vector<uint16_t> sc((size_t)sshape[0] * sshape[1]);
    if (!a.read(*ts, 0, ts->bytes, sc.data())) return set_error(Q35MM_EIO, "read of %s failed", sname.c_str());
    const std::vector<float> f = widen_scales(sc.data(), rows, cols);
    if (group_rows_per_piece(cols) > 0)
        return weight_alloc_fill(rows, cols, out, [&](Weight &w, hipStream_t st) -> int {
            HIP_TRY(hipMemcpyAsync(w.scale, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice, st));
            return upload_fp8_tiled(a, *tw, w, st);
        });
    return weight_build(rows, cols, out, [&](Weight &w, uint8_t *raw, hipStream_t st) -> int {
        HIP_TRY(hipMemcpyAsync(w.scale, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice, st));
        return upload_tensor(a, *tw, raw, st);
    });
}

// bind_ab (qwen35-c/src/q35_model.c:302-350): an F8_E4M3 tensor binds as
// above; a BF16 [rows][cols] tensor is uploaded and quantized on the device
// (quantize.hip), codes going straight to the repack.
int st_load_ab(const st::Archive &a, const char *name, uint32_t rows, uint32_t cols, q35mm_weight **out) {
    const st::Tensor *t = a.find(name);
    if (!t) return set_error(Q35MM_ENOTFOUND, "missing tensor: %s", name);
    if (t->dtype == st::kF8E4M3) return st_load_fp8(a, name, rows, cols, out);
    if (t->dtype != st::kBF16)
        return set_error(Q35MM_ESHAPE, "tensor %s: dtype %s, want BF16 or F8_E4M3", name, st::dtype_name(t->dtype));
    const uint32_t wshape[2] = {rows, cols};
    int rc = need_tensor(a, name, st::kBF16, 2, wshape, &t);
    if (rc) return rc;
    if (group_rows_per_piece((uint64_t)cols * 2) > 0)
        return weight_alloc_fill(rows, cols, out,
                                 [&](Weight &w, hipStream_t st) { return upload_bf16_quantized(a, *t, w, st); });
    uint16_t *src = nullptr;
    rc = weight_build(rows, cols, out, [&](Weight &w, uint8_t *raw, hipStream_t st) -> int {
        if (hipMalloc(&src, t->bytes) != hipSuccess) {
            src = nullptr;
            return set_error(Q35MM_ENOMEM, "hipMalloc(%llu) for bf16 staging failed", (unsigned long long)t->bytes);
        }
        int r = upload_tensor(a, *t, src, st);
        if (r) return r;
        HIP_TRY(launch_quantize_bf16(src, rows, cols, raw, nullptr, w.scale, st));
        return Q35MM_OK;
    });
    if (src) {
        (void)hipStreamSynchronize(g_dev.stream);
        (void)hipFree(src);
    }
    return rc;
}

// ---------------------------------------------------------------------
// Residency registry for the host-pointer ABI
// ---------------------------------------------------------------------
uint64_t mix64(uint64_t h, uint64_t v) {
    h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
    h *= 0xff51afd7ed558ccdull;
    return h ^ (h >> 33);
}

// Four interleaved lanes: the multiply chains of a single running hash,
// not the memory reads, were the cost (one chain over ~15 KB took ~3.5 us of
// a host-pointer call).
uint64_t hash_bytes(uint64_t h, const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    uint64_t l[4] = {h, h ^ 0x243f6a8885a308d3ull, h ^ 0x13198a2e03707344ull, h ^ 0xa4093822299f31d0ull};
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        uint64_t v[4];
        memcpy(v, b + i, 32);
        for (int j = 0; j < 4; j++) l[j] = mix64(l[j], v[j]);
    }
    for (; i + 8 <= n; i += 8) {
        uint64_t v;
        memcpy(&v, b + i, 8);
        l[0] = mix64(l[0], v);
    }
    uint64_t tail = 0;
    for (; i < n; i++) tail = (tail << 8) | b[i];
    return mix64(mix64(mix64(mix64(l[0], l[1]), l[2]), l[3]), tail ^ n);
}

// Fingerprint of a host weight, checked on every host-pointer call that
// reuses a pointer: all scales, the first and last 4 KiB of the codes and
// kFpWindows evenly spaced 256-byte windows.  A different tensor behind a
// reused pointer differs almost everywhere, so a few windows besides the
// scales and the edges suffice; an in-place edit of a few codes outside
// them is not seen -- such callers call q35mm_release(W) after editing, or
// set Q35MM_VERIFY_WEIGHTS=full, which hashes every byte on every call.
constexpr size_t kFpWindows = 16;
uint64_t fingerprint(const void *W, size_t wbytes, const void *sc, size_t scbytes) {
    uint64_t h = hash_bytes(0x51E5ull, sc, scbytes);
    const uint8_t *b = (const uint8_t *)W;
    if (g_dev.verify_full) return hash_bytes(h, b, wbytes);
    const size_t edge = std::min<size_t>(4096, wbytes);
    h = hash_bytes(h, b, edge);
    h = hash_bytes(h, b + wbytes - edge, edge);
    if (wbytes > 256) {
        for (size_t i = 0; i < kFpWindows; i++) {
            size_t off = (wbytes - 256) / (kFpWindows - 1) * i;
            h = hash_bytes(h, b + off, 256);
        }
    }
    return h;
}

struct Resident {
    q35mm_weight *w = nullptr;
    const void *scale = nullptr;
    uint32_t rows = 0, cols = 0;
    uint64_t fp = 0;
    bool bf16 = false;
    uint16_t *bf16_dev = nullptr;   // q35_mm_bf16 weights (row-major, resident)
};

std::unordered_map<const void *, Resident> g_res;

void drop(Resident &r) {
    if (r.w) q35mm_weight_destroy(r.w);
    if (r.bf16_dev) (void)hipFree(r.bf16_dev);
    r.w = nullptr;
    r.bf16_dev = nullptr;
}

// Resident copy for host W; uploads on first use or when the buffer behind
// the pointer changed (shape, scale pointer or fingerprint).  With hit
// given, a copy found by pointer with the same shape and scale pointer is
// returned without reading W (*hit = true): the caller checks the
// fingerprint with resident_same while the device runs the call, and
// forgets the copy and repeats the call if it differs.
int resident_fp8(const uint8_t *W, const uint16_t *sc, uint32_t rows, uint32_t cols,
                 q35mm_weight **out, bool *hit = nullptr) {
    const size_t wbytes = (size_t)rows * cols;
    const size_t scbytes = (size_t)((rows + 127) / 128) * ((cols + 127) / 128) * 2;
    if (hit) *hit = false;
    auto it = g_res.find(W);
    if (it != g_res.end()) {
        Resident &r = it->second;
        bool same = !r.bf16 && r.rows == rows && r.cols == cols && r.scale == sc;
        if (same && hit) {
            *hit = true;
            *out = r.w;
            return Q35MM_OK;
        }
        if (same && !g_dev.trust_pointers) same = r.fp == fingerprint(W, wbytes, sc, scbytes);
        if (same) {
            *out = r.w;
            return Q35MM_OK;
        }
        drop(r);
        g_res.erase(it);
    }
    std::vector<float> f = widen_scales(sc, rows, cols);
    q35mm_weight *w = nullptr;
    int rc = weight_create(W, f.data(), rows, cols, &w);
    if (rc) return rc;
    Resident r;
    r.w = w;
    r.scale = sc;
    r.rows = rows;
    r.cols = cols;
    r.fp = g_dev.trust_pointers ? 0 : fingerprint(W, wbytes, sc, scbytes);
    g_res[W] = r;
    *out = w;
    return Q35MM_OK;
}

int resident_bf16(const uint16_t *W, uint32_t rows, uint32_t cols, uint16_t **out, bool *hit = nullptr) {
    const size_t wbytes = (size_t)rows * cols * 2;
    if (hit) *hit = false;
    auto it = g_res.find(W);
    if (it != g_res.end()) {
        Resident &r = it->second;
        bool same = r.bf16 && r.rows == rows && r.cols == cols;
        if (same && hit) {
            *hit = true;
            *out = r.bf16_dev;
            return Q35MM_OK;
        }
        if (same && !g_dev.trust_pointers) same = r.fp == fingerprint(W, wbytes, nullptr, 0);
        if (same) {
            *out = r.bf16_dev;
            return Q35MM_OK;
        }
        drop(r);
        g_res.erase(it);
    }
    int rc = ensure_device();
    if (rc) return rc;
    uint16_t *d = nullptr;
    if (hipMalloc(&d, wbytes) != hipSuccess) return set_error(Q35MM_ENOMEM, "hipMalloc(%zu) failed", wbytes);
    if (hipMemcpy(d, W, wbytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return set_error(Q35MM_EHIP, "bf16 weight upload failed");
    }
    Resident r;
    r.bf16 = true;
    r.bf16_dev = d;
    r.rows = rows;
    r.cols = cols;
    r.fp = g_dev.trust_pointers ? 0 : fingerprint(W, wbytes, nullptr, 0);
    g_res[W] = r;
    *out = d;
    return Q35MM_OK;
}

// Whether the bytes behind a resident host pointer are still the ones
// uploaded (fingerprint of the weight and its scales; scbytes 0 for a bf16
// weight).
bool resident_same(const void *W, size_t wbytes, const void *sc, size_t scbytes) {
    if (g_dev.trust_pointers) return true;
    auto it = g_res.find(W);
    return it != g_res.end() && it->second.fp == fingerprint(W, wbytes, sc, scbytes);
}

void forget(const void *W) {
    auto it = g_res.find(W);
    if (it == g_res.end()) return;
    drop(it->second);
    g_res.erase(it);
}

// Pinned completion word of the host-pointer calls.  Fine-grained
// (coherent) host memory: the device's store reaches the host, and no
// device cache holds it.
constexpr uint32_t kWordDone = 0;
constexpr size_t kWordsBytes = 64;

bool host_words() {
    if (g_dev.done) return true;
    if (!g_dev.done_cnt) {
        if (hipMalloc(reinterpret_cast<void **>(&g_dev.done_cnt), 256) != hipSuccess) {
            g_dev.done_cnt = nullptr;
            return false;
        }
        if (hipMemset(g_dev.done_cnt, 0, 256) != hipSuccess) return false;
    }
    if (hipHostMalloc(reinterpret_cast<void **>(&g_dev.done), kWordsBytes, hipHostMallocCoherent) != hipSuccess) {
        g_dev.done = nullptr;
        return false;
    }
    memset(g_dev.done, 0, kWordsBytes);
    return true;
}

uint32_t next_seq(uint32_t &seq) { return ++seq ? seq : ++seq; }   // never 0

// Completion of everything queued on st so far: a flag kernel queued last
// stores a fresh sequence number into the done word and the calling thread
// spins on it (post_done, then wait_done).  Launch + hipStreamSynchronize
// costs ~11.6 us of host round trip on this system, launch + spinning on
// such a flag ~6 us.  Past kSpinLimit (a long call) or if the flag never
// comes (a failed kernel), hipStreamSynchronize takes over and reports any
// error.
hipError_t post_done(hipStream_t st, uint32_t *v) {
    *v = next_seq(g_dev.done_seq);
    return launch_done_flag(g_dev.done + kWordDone, *v, st);
}

hipError_t wait_done(hipStream_t st, uint32_t v) {
    constexpr auto kSpinLimit = std::chrono::microseconds(2000);
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t i = 0;; i++) {
        if (__atomic_load_n(g_dev.done + kWordDone, __ATOMIC_ACQUIRE) == v) return hipSuccess;
        __builtin_ia32_pause();
        if ((i & 255) == 255 && std::chrono::steady_clock::now() - t0 > kSpinLimit) break;
    }
    return hipStreamSynchronize(st);
}

// Host-pointer round trip: X (n*cols floats) in, outputs of nseg segments
// out.  'run' launches on g_dev.stream reading dx and writing dy[s].
// Each queued DMA transfer costs ~8 us of latency (measured: H2D + GEMV +
// D2H + synchronize 32 us against 17 us for the GEMV launch alone), so small
// transfers skip the DMA engines: activations up to kDirectBytes are staged
// in pinned memory, which the matmul kernels read in place, and outputs up
// to kDirectBytes are written by the matmul kernels straight into pinned
// (device-visible) host memory.  (Reading the staged activations in place
// measured 17.6 us per call at 5120 x 5120 against 22.0 us with a copy
// kernel into HBM first: the copy's launch and PCIe round trip cost more
// than the device's cached reads of 20 KB of host memory.)
//
// Order of a call: the activations are staged and the copy, the matmul and
// the completion flag queued; then 'verify' checks the weights behind the
// caller's pointers (their fingerprints) while the device computes.  A
// verify that fails returns kStale once the device has finished: the caller
// forgets those weights and repeats the call.  (Queuing the copy before
// staging the activations, with the copy waiting on a host-written word,
// measured ~2 us slower per call: the device's polls of host memory cost
// more than the launch latency they would hide.)
constexpr size_t kDirectBytes = 256 * 1024;
constexpr int kStale = -1000;   // internal: a resident weight changed behind its pointer
// Larger transfers run in chunks (Q35MM_XFER_CHUNK_KB, default 2048; at
// most kXferChunks) so that the host's copies and the DMA overlap: chunk i
// of the activations is copied into pinned memory while
// chunk i-1 crosses PCIe, and chunk j of the outputs is copied out of
// pinned memory while chunk j+1 crosses.  (Each alone runs at ~55 GB/s over
// PCIe and 32-70 GB/s for the host copy; one after the other they took a
// 512-token 6144 -> 5120 call 1.21 ms.)
constexpr uint32_t kXferChunks = sizeof(Device::xfer_ev) / sizeof(hipEvent_t);

// Host copies of large transfer chunks, split between the calling thread
// and one helper thread (a single host thread copies 32-35 GB/s from memory
// the CPU caches do not hold, below the ~55 GB/s of the DMA it overlaps
// with).  Calls are serialised by the library lock, so there is one job
// slot.  The helper is created on first use and never joined (it waits on
// its condition variable until the process ends; the object is never
// destroyed, so nothing it uses goes away under it); a process forked
// after it started copies on its own thread only.
class CopyHelper {
  public:
    void copy(void *dst, const void *src, size_t n) {
        if (n < kSplitMin || !start()) {
            memcpy(dst, src, n);
            return;
        }
        const size_t h = (n / 2) & ~(size_t)63;
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = (uint8_t *)dst + h;
            src_ = (const uint8_t *)src + h;
            n_ = n - h;
            pending_ = true;
        }
        cv_.notify_one();
        memcpy(dst, src, h);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return !pending_; });
    }

  private:
    static constexpr size_t kSplitMin = 256u << 10;
    bool start() {
        if (started_ && owner_ == getpid()) return true;
        if (started_) return false;   // forked child: the helper did not come along
        try {
            std::thread([this] { run(); }).detach();
        } catch (...) {
            return false;
        }
        started_ = true;
        owner_ = getpid();
        return true;
    }
    void run() {
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return pending_; });
            lk.unlock();
            memcpy(dst_, src_, n_);
            lk.lock();
            pending_ = false;
            done_cv_.notify_one();
        }
    }
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    uint8_t *dst_ = nullptr;
    const uint8_t *src_ = nullptr;
    size_t n_ = 0;
    bool pending_ = false;
    bool started_ = false;
    pid_t owner_ = 0;
};
CopyHelper &copy_helper() {
    static CopyHelper *h = new CopyHelper();   // never destroyed: the helper thread outlives static teardown
    return *h;
}

// Chunk c of n over 'bytes' (16-byte aligned boundaries).
inline void xfer_chunk(size_t bytes, uint32_t n, uint32_t c, size_t *off, size_t *len) {
    const size_t per = ((bytes + n - 1) / n + 15) & ~(size_t)15;
    *off = std::min(bytes, per * c);
    *len = std::min(bytes, *off + per) - *off;
}
inline uint32_t xfer_chunks(size_t bytes) {
    const size_t c = g_dev.xfer_chunk;
    return c ? (uint32_t)std::min<size_t>(kXferChunks, std::max<size_t>(1, (bytes + c - 1) / c)) : 1u;
}

template <class Run, class Verify>
int host_roundtrip(const float *X, size_t xfloats, float *const *Y, const size_t *yfloats,
                   uint32_t nseg, Run run, Verify verify) {
    size_t ytotal = 0;
    for (uint32_t s = 0; s < nseg; s++) ytotal += yfloats[s];
    const bool direct_x = xfloats * sizeof(float) <= kDirectBytes;
    const bool direct_y = ytotal * sizeof(float) <= kDirectBytes;
    int rc = grow(g_dev.dx, xfloats * sizeof(float), false);
    if (!rc && !direct_y) rc = grow(g_dev.dy, ytotal * sizeof(float), false);
    // x and y regions of the pinned buffer each start 256-byte aligned
    const size_t xpad = (xfloats + 63) & ~(size_t)63;
    if (!rc) rc = grow_pinned((xpad + ytotal) * sizeof(float));
    if (rc) return rc;
    if (g_dev.done_spin && !host_words()) g_dev.done_spin = false;
    float *px = (float *)g_dev.pin;
    float *py = px + xpad;
    hipStream_t st = g_dev.stream;
    auto fail = [&](int code) {
        (void)hipStreamSynchronize(st);
        return code;
    };
    hipError_t e = hipSuccess;
    if (direct_x) {
        memcpy(px, X, xfloats * sizeof(float));
    } else {
        const size_t xb = xfloats * sizeof(float);
        const uint32_t nc = xfer_chunks(xb);
        for (uint32_t c = 0; c < nc; c++) {
            size_t o, len;
            xfer_chunk(xb, nc, c, &o, &len);
            copy_helper().copy((uint8_t *)px + o, (const uint8_t *)X + o, len);
            e = hipMemcpyAsync((uint8_t *)g_dev.dx.ptr + o, (uint8_t *)px + o, len, hipMemcpyHostToDevice, st);
            if (e != hipSuccess) return fail(set_error(Q35MM_EHIP, "activation copy: %s", hipGetErrorString(e)));
        }
    }
    float *dys[4];
    size_t off = 0;
    for (uint32_t s = 0; s < nseg; s++) {
        dys[s] = (direct_y ? py : (float *)g_dev.dy.ptr) + off;
        off += yfloats[s];
    }
    // With outputs written straight into pinned memory, the call's last
    // launch, if a row-split GEMV, stores the completion word itself (no
    // flag kernel after it); otherwise the flag kernel is queued last.
    uint32_t v = 0;
    if (g_dev.done_spin && direct_y) {
        v = next_seq(g_dev.done_seq);
        g_dev.done_req.word = g_dev.done + kWordDone;
        g_dev.done_req.value = v;
        g_dev.done_req.taken = false;
    }
    rc = run(direct_x ? (const float *)px : (const float *)g_dev.dx.ptr, dys);
    const bool done_taken = g_dev.done_req.taken;
    g_dev.done_req = Device::DoneReq{};
    if (rc) return fail(rc);
    if (!direct_y) {
        // the outputs in chunks, each followed by an event the host waits
        // for before copying that chunk out
        const size_t yb = ytotal * sizeof(float);
        const uint32_t nc = xfer_chunks(yb);
        for (uint32_t c = 0; c < nc; c++) {
            if (!g_dev.xfer_ev[c]) {
                e = hipEventCreateWithFlags(&g_dev.xfer_ev[c], hipEventDisableTiming);
                if (e != hipSuccess) return fail(set_error(Q35MM_EHIP, "event: %s", hipGetErrorString(e)));
            }
            size_t o, len;
            xfer_chunk(yb, nc, c, &o, &len);
            e = hipMemcpyAsync((uint8_t *)py + o, (uint8_t *)g_dev.dy.ptr + o, len, hipMemcpyDeviceToHost, st);
            if (e == hipSuccess) e = hipEventRecord(g_dev.xfer_ev[c], st);
            if (e != hipSuccess) return fail(set_error(Q35MM_EHIP, "output copy: %s", hipGetErrorString(e)));
        }
        const bool same = verify();
        if (!same) {
            e = hipStreamSynchronize(st);
            return e != hipSuccess ? set_error(Q35MM_EHIP, "host-pointer call: %s", hipGetErrorString(e)) : kStale;
        }
        // output chunk c covers bytes [o, o + len) of the segments laid end
        // to end: copy each segment's part of it
        for (uint32_t c = 0; c < nc; c++) {
            size_t o, len;
            xfer_chunk(yb, nc, c, &o, &len);
            e = hipEventSynchronize(g_dev.xfer_ev[c]);
            if (e != hipSuccess) return fail(set_error(Q35MM_EHIP, "host-pointer call: %s", hipGetErrorString(e)));
            size_t seg0 = 0;
            for (uint32_t s = 0; s < nseg; s++) {
                const size_t sb = yfloats[s] * sizeof(float), a = std::max(o, seg0), b = std::min(o + len, seg0 + sb);
                if (a < b) copy_helper().copy((uint8_t *)Y[s] + (a - seg0), (uint8_t *)py + a, b - a);
                seg0 += sb;
            }
        }
        return Q35MM_OK;
    }
    if (g_dev.done_spin && !done_taken) {
        e = post_done(st, &v);
        if (e != hipSuccess) return fail(set_error(Q35MM_EHIP, "completion flag: %s", hipGetErrorString(e)));
    }
    const bool same = verify();
    e = g_dev.done_spin ? wait_done(st, v) : hipStreamSynchronize(st);
    if (e != hipSuccess) return set_error(Q35MM_EHIP, "host-pointer call: %s", hipGetErrorString(e));
    if (!same) return kStale;
    off = 0;
    for (uint32_t s = 0; s < nseg; s++) {
        memcpy(Y[s], py + off, yfloats[s] * sizeof(float));
        off += yfloats[s];
    }
    return Q35MM_OK;
}

// ---------------------------------------------------------------------
// e4m3 decode table (host)
// ---------------------------------------------------------------------
float e4m3_decode(uint8_t v) {
    const uint32_t sign = (uint32_t)(v >> 7) << 31;
    const uint32_t e = (v >> 3) & 0xF, m = v & 7;
    uint32_t bits;
    if (e == 0) {
        float f = (float)m * 0x1.0p-9f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (e == 15 && m == 7) {
        bits = sign | 0x7FC00000u;
    } else {
        bits = sign | ((e + 120) << 23) | (m << 20);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void fill_lut(float *lut) {
    for (int i = 0; i < 256; i++) lut[i] = e4m3_decode((uint8_t)i);
}

__attribute__((constructor)) void lut_at_load() { fill_lut(q35_mm_fp8_lut); }

}  // namespace

// =====================================================================
// Drop-in ABI (include/q35/q35_mm.h)
// =====================================================================
// The table's initial image is the decoded table itself (computed at compile
// time), so every copy of it is right from the start: a C executable that
// reads the table links it by copy relocation (the executable holds the
// copy, initialised from this image, and the library, linked with
// -Bsymbolic-functions only, binds its own references to that copy).
namespace {
constexpr uint32_t e4m3_const_bits(uint32_t v) {
    const uint32_t sign = (v >> 7) << 31, e = (v >> 3) & 0xF, m = v & 7;
    if (e == 0) return m ? sign | __builtin_bit_cast(uint32_t, (float)m * 0x1.0p-9f) : sign;
    if (e == 15 && m == 7) return sign | 0x7FC00000u;
    return sign | ((e + 120) << 23) | (m << 20);
}
constexpr float e4m3_const(uint32_t v) { return __builtin_bit_cast(float, e4m3_const_bits(v)); }
}  // namespace
#define Q35_LUT4(i) e4m3_const(i), e4m3_const(i + 1), e4m3_const(i + 2), e4m3_const(i + 3)
#define Q35_LUT16(i) Q35_LUT4(i), Q35_LUT4(i + 4), Q35_LUT4(i + 8), Q35_LUT4(i + 12)
#define Q35_LUT64(i) Q35_LUT16(i), Q35_LUT16(i + 16), Q35_LUT16(i + 32), Q35_LUT16(i + 48)

// Braced linkage block: this is the definition of the exported data symbol
// (the single-declaration form extern "C" T x; only declares it).
extern "C" {
__attribute__((visibility("default"))) float q35_mm_fp8_lut[256] = {Q35_LUT64(0), Q35_LUT64(64), Q35_LUT64(128),
                                                                     Q35_LUT64(192)};
}
#undef Q35_LUT4
#undef Q35_LUT16
#undef Q35_LUT64

Q35MM_API void q35_mm_init(void) {
    static std::once_flag once;
    std::call_once(once, [] { fill_lut(q35_mm_fp8_lut); });
}

Q35MM_API float q35_mm_e4m3_to_f32(uint8_t v) { return e4m3_decode(v); }

Q35MM_API float q35_mm_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

Q35MM_API const char *q35_mm_impl_fp8(void) { return "hip-gfx950"; }

Q35MM_API void q35_mm_fp8_batch(const uint8_t *W, const uint16_t *scale_bf16, uint32_t rows,
                                uint32_t cols, uint32_t n, const float *X, float *Y) {
    if (rows == 0 || n == 0) return;
    if (cols == 0) {
        memset(Y, 0, (size_t)n * rows * sizeof(float));
        return;
    }
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    const size_t wbytes = (size_t)rows * cols, scbytes = (size_t)((rows + 127) / 128) * ((cols + 127) / 128) * 2;
    // first with the resident copy checked during the call; if the bytes
    // behind W changed, again on a fresh upload
    for (int attempt = 0; attempt < 2 && !rc; attempt++) {
        q35mm_weight *w = nullptr;
        bool hit = false;
        rc = resident_fp8(W, scale_bf16, rows, cols, &w, attempt == 0 ? &hit : nullptr);
        if (rc) break;
        float *ys[1] = {Y};
        size_t yf[1] = {(size_t)n * rows};
        rc = host_roundtrip(
            X, (size_t)n * cols, ys, yf, 1,
            [&](const float *dx, float **dy) { return run_matmul(w, n, dx, dy[0], g_dev.stream); },
            [&] { return !hit || resident_same(W, wbytes, scale_bf16, scbytes); });
        if (rc != kStale) break;
        forget(W);
        rc = Q35MM_OK;
    }
    if (rc) die("q35_mm_fp8_batch");
}

Q35MM_API void q35_mm_fp8(const uint8_t *W, const uint16_t *scale_bf16, uint32_t rows, uint32_t cols,
                          const float *x, float *y) {
    q35_mm_fp8_batch(W, scale_bf16, rows, cols, 1, x, y);
}

Q35MM_API void q35_mm_fp8_multi4(const uint8_t *W[4], const uint16_t *sc[4], uint32_t rows[4],
                                 uint32_t cols, const float *x, float *y[4]) {
    uint32_t idx[4], nseg = 0;
    for (uint32_t s = 0; s < 4; s++)
        if (rows[s]) idx[nseg++] = s;
    if (nseg == 0) return;
    if (cols == 0) {
        for (uint32_t i = 0; i < nseg; i++) memset(y[idx[i]], 0, (size_t)rows[idx[i]] * sizeof(float));
        return;
    }
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    // A pointer repeated with another row count or scale pointer gets a copy
    // of its own for this call: the registry holds one copy per pointer, and
    // replacing it would free an earlier segment's copy while the launch
    // still needs it.
    q35mm_weight *ws[4], *tmp[4] = {};
    bool hit[4] = {};
    // first with the resident copies checked during the call; if the bytes
    // behind a pointer changed, again on fresh uploads
    for (int attempt = 0; attempt < 2 && !rc; attempt++) {
        for (uint32_t i = 0; i < nseg && !rc; i++) {
            const uint32_t s = idx[i];
            bool clash = false;
            for (uint32_t j = 0; j < i; j++)
                clash |= W[idx[j]] == W[s] && (rows[idx[j]] != rows[s] || sc[idx[j]] != sc[s]);
            hit[i] = false;
            if (clash) {
                if (!tmp[i]) {
                    const std::vector<float> f = widen_scales(sc[s], rows[s], cols);
                    rc = weight_create(W[s], f.data(), rows[s], cols, &tmp[i]);
                }
                ws[i] = tmp[i];
            } else {
                rc = resident_fp8(W[s], sc[s], rows[s], cols, &ws[i], attempt == 0 ? &hit[i] : nullptr);
            }
        }
        if (rc) break;
        float *ys[4];
        size_t yf[4];
        for (uint32_t i = 0; i < nseg; i++) {
            ys[i] = y[idx[i]];
            yf[i] = rows[idx[i]];
        }
        rc = host_roundtrip(
            x, cols, ys, yf, nseg,
            [&](const float *dx, float **dy) { return run_gemv(ws, nseg, 1, dx, dy, g_dev.stream); },
            [&] {
                bool same = true;
                for (uint32_t i = 0; i < nseg; i++) {
                    const uint32_t s = idx[i];
                    if (hit[i])
                        same &= resident_same(W[s], (size_t)rows[s] * cols, sc[s],
                                              (size_t)((rows[s] + 127) / 128) * ((cols + 127) / 128) * 2);
                }
                return same;
            });
        if (rc != kStale) break;
        for (uint32_t i = 0; i < nseg; i++)
            if (hit[i]) forget(W[idx[i]]);
        rc = Q35MM_OK;
    }
    for (uint32_t i = 0; i < nseg; i++)
        if (tmp[i]) q35mm_weight_destroy(tmp[i]);
    if (rc) die("q35_mm_fp8_multi4");
}

Q35MM_API void q35_mm_bf16(const uint16_t *W, uint32_t rows, uint32_t cols, const float *x, float *y) {
    if (rows == 0) return;
    if (cols == 0) {
        memset(y, 0, (size_t)rows * sizeof(float));
        return;
    }
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    for (int attempt = 0; attempt < 2 && !rc; attempt++) {
        uint16_t *dw = nullptr;
        bool hit = false;
        rc = resident_bf16(W, rows, cols, &dw, attempt == 0 ? &hit : nullptr);
        if (rc) break;
        float *ys[1] = {y};
        size_t yf[1] = {rows};
        rc = host_roundtrip(
            x, cols, ys, yf, 1,
            [&](const float *dx, float **dy) -> int {
                HIP_TRY(launch_bf16_gemv(dw, rows, cols, dx, dy[0], g_dev.stream));
                return Q35MM_OK;
            },
            [&] { return !hit || resident_same(W, (size_t)rows * cols * 2, nullptr, 0); });
        if (rc != kStale) break;
        forget(W);
        rc = Q35MM_OK;
    }
    if (rc) die("q35_mm_bf16");
}

// =====================================================================
// Device API (include/q35mm/q35mm.h)
// =====================================================================
Q35MM_API int q35mm_init(int device) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (device >= 0 && g_dev.id < 0) {
        char buf[16];
        snprintf(buf, sizeof buf, "%d", device);
        setenv("Q35MM_DEVICE", buf, 1);
    }
    return ensure_device();
}

Q35MM_API int q35mm_weight_create(const uint8_t *W, const uint16_t *scale_bf16, uint32_t rows,
                                  uint32_t cols, q35mm_weight **out) {
    if (!W || !scale_bf16 || !out) return set_error(Q35MM_EINVAL, "null argument");
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    std::vector<float> f = widen_scales(scale_bf16, rows, cols);
    return weight_create(W, f.data(), rows, cols, out);
}

Q35MM_API int q35mm_weight_create_f32scale(const uint8_t *W, const float *scale_f32, uint32_t rows,
                                           uint32_t cols, q35mm_weight **out) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return weight_create(W, scale_f32, rows, cols, out);
}

Q35MM_API void q35mm_weight_destroy(q35mm_weight *w) {
    if (!w) return;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    (void)hipDeviceSynchronize();
    if (w->w.codes) (void)hipFree(w->w.codes);
    if (w->w.scale) (void)hipFree(w->w.scale);
    delete w;
}

Q35MM_API int q35mm_weight_shape(const q35mm_weight *w, uint32_t *rows, uint32_t *cols) {
    int rc = check_weight(w);
    if (rc) return rc;
    if (rows) *rows = w->w.rows;
    if (cols) *cols = w->w.cols;
    return Q35MM_OK;
}

Q35MM_API size_t q35mm_weight_bytes(const q35mm_weight *w) { return w ? w->bytes : 0; }

Q35MM_API int q35mm_matmul(const q35mm_weight *w, uint32_t m, const float *dX, float *dY, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (!rc) rc = check_weight(w);
    if (rc) return rc;
    if (m && (!dX || !dY)) return set_error(Q35MM_EINVAL, "null activation pointer");
    return run_matmul(w, m, dX, dY, pick_stream(stream));
}

Q35MM_API int q35mm_matmul_noalloc(const q35mm_weight *w, uint32_t m, const float *dX, float *dY, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (g_dev.id < 0)
        return set_error(Q35MM_EINVAL, "q35mm_matmul_noalloc: library not initialised (call q35mm_init first)");
    int rc = check_weight(w);
    if (rc) return rc;
    if (m && (!dX || !dY)) return set_error(Q35MM_EINVAL, "null activation pointer");
    Scratch fixed;
    fixed.fixed = noalloc_scratch(g_dev.id);
    if (!fixed.fixed) return set_error(Q35MM_EINVAL, "q35mm_matmul_noalloc: no scratch on device %d", g_dev.id);
    return run_matmul(w, m, dX, dY, pick_stream(stream), &fixed);
}

Q35MM_API int q35mm_gemv(const q35mm_weight *w, uint32_t m, const float *dX, float *dY, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (!rc) rc = check_weight(w);
    if (rc) return rc;
    if (m == 0) return Q35MM_OK;
    if (!dX || !dY) return set_error(Q35MM_EINVAL, "null activation pointer");
    const q35mm_weight *ws[1] = {w};
    float *ys[1] = {dY};
    return run_gemv(ws, 1, m, dX, ys, pick_stream(stream));
}

Q35MM_API int q35mm_gemm(const q35mm_weight *w, uint32_t m, const float *dX, float *dY, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (!rc) rc = check_weight(w);
    if (rc) return rc;
    if (m == 0) return Q35MM_OK;
    if (!dX || !dY) return set_error(Q35MM_EINVAL, "null activation pointer");
    const q35mm_weight *ws[1] = {w};
    float *ys[1] = {dY};
    return run_gemm(ws, 1, m, dX, ys, pick_stream(stream));
}

Q35MM_API int q35mm_matmul_multi(const q35mm_weight *const *w, uint32_t nseg, uint32_t m,
                                 const float *dX, float *const *dY, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    if (!w || !dY || nseg == 0 || nseg > 4) return set_error(Q35MM_EINVAL, "need 1..4 segments");
    for (uint32_t s = 0; s < nseg; s++) {
        rc = check_weight(w[s]);
        if (rc) return rc;
        if (w[s]->w.cols != w[0]->w.cols) return set_error(Q35MM_EINVAL, "segments differ in cols");
    }
    if (m == 0) return Q35MM_OK;
    hipStream_t st = pick_stream(stream);
    bool gemm = m >= g_dev.gemm_min_m && g_dev.gemm_min_m > 0;
    for (uint32_t s = 0; s < nseg && gemm; s++) gemm = gemm_fits(w[s]->w, m);
    if (gemm) return run_gemm(w, nseg, m, dX, dY, st);   // one launch over all segments' tiles
    return run_gemv(w, nseg, m, dX, dY, st);
}

Q35MM_API int q35mm_dequant_f32(const q35mm_weight *w, float *dOut, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (!rc) rc = check_weight(w);
    if (rc) return rc;
    HIP_TRY(launch_dequant_f32(w->w, dOut, pick_stream(stream)));
    return Q35MM_OK;
}

Q35MM_API int q35mm_decode_bf16(const q35mm_weight *w, uint16_t *dOut, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (!rc) rc = check_weight(w);
    if (rc) return rc;
    HIP_TRY(launch_decode_bf16(w->w, dOut, pick_stream(stream)));
    return Q35MM_OK;
}

Q35MM_API int q35mm_bf16_gemv(const uint16_t *dW, uint32_t rows, uint32_t cols, const float *dx, float *dy,
                              void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    if (rows == 0) return Q35MM_OK;
    if (!dW || !dx || !dy) return set_error(Q35MM_EINVAL, "null pointer");
    HIP_TRY(launch_bf16_gemv(dW, rows, cols, dx, dy, pick_stream(stream)));
    return Q35MM_OK;
}

Q35MM_API int q35mm_rmsnorm(const float *dX, const float *dW, float *dY, uint32_t rows, uint32_t n, float eps,
                            void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    if (rows == 0 || n == 0) return Q35MM_OK;
    if (!dX || !dW || !dY) return set_error(Q35MM_EINVAL, "null pointer");
    HIP_TRY(launch_rmsnorm(dX, n, dW, dY, n, rows, n, eps, pick_stream(stream)));
    return Q35MM_OK;
}

Q35MM_API int q35mm_swiglu(const float *dGate, const float *dUp, float *dY, size_t n, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    if (n == 0) return Q35MM_OK;
    if (!dGate || !dUp || !dY) return set_error(Q35MM_EINVAL, "null pointer");
    HIP_TRY(launch_swiglu(dGate, dUp, dY, n, pick_stream(stream)));
    return Q35MM_OK;
}

// silu(x @ gate^T) * (x @ up^T) for m <= kGemvMaxM tokens of row-split gate
// and up weights in one launch (gemv_rows_kernel, pair mode), on RMSNorm(x)
// when norm_w is given (one token): the bits of rmsnorm, the gate+up GEMV
// and swiglu as separate kernels.
int run_mlp_pair(const q35mm_weight *gate, const q35mm_weight *up, uint32_t m, const float *dX, const float *norm_w,
                 float eps, float *dH, hipStream_t st) {
    const Weight &g = gate->w, &u = up->w;
    GemvParams p{};
    p.x = dX;
    p.norm_w = norm_w;
    p.eps = eps;
    p.xmode = kXPlain;
    p.ldx = g.cols;
    p.m = m;
    p.k = g.cols;
    p.kb = g.kb;
    p.nseg = 2;
    p.x_vec = (aligned16(dX) && g.cols % 8 == 0 && (!norm_w || aligned16(norm_w))) ? 1u : 0u;
    const Weight *ws[2] = {&g, &u};
    for (uint32_t s = 0; s < 2; s++) {
        GemvSeg &sg = p.seg[s];
        sg.codes = ws[s]->codes;
        sg.scale = ws[s]->scale;
        sg.y = dH;
        sg.rows = ws[s]->rows;
        sg.ldy = ws[s]->rows;
        sg.nb = ws[s]->nb;
    }
    HIP_TRY(launch_gemv_pair(p, norm_w != nullptr, g_dev.cus, st));
    return Q35MM_OK;
}

Q35MM_API int q35mm_mlp(const q35mm_weight *gate, const q35mm_weight *up, const q35mm_weight *down,
                        const float *dNormW, float eps, uint32_t m, float *dX, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (!rc) rc = check_weight(gate);
    if (!rc) rc = check_weight(up);
    if (!rc) rc = check_weight(down);
    if (rc) return rc;
    const uint32_t H = gate->w.cols, I = gate->w.rows;
    if (up->w.cols != H || up->w.rows != I || down->w.cols != I || down->w.rows != H)
        return set_error(Q35MM_EINVAL, "MLP shapes disagree: gate %ux%u up %ux%u down %ux%u", gate->w.rows,
                         gate->w.cols, up->w.rows, up->w.cols, down->w.rows, down->w.cols);
    if (m == 0) return Q35MM_OK;
    if (!dX || !dNormW) return set_error(Q35MM_EINVAL, "null pointer");
    // workspace: xn [m][H], g [m][I], u [m][I], y [m][H] (SwiGLU writes g in
    // place), then the down GEMM's bf16 activations when the gate+up GEMM
    // forms them
    const size_t nh = (size_t)m * H, ni = (size_t)m * I;
    hipStream_t st = pick_stream(stream);
    Scratch &scr = scratch_for(st);
    const bool gemm = m >= g_dev.gemm_min_m && g_dev.gemm_min_m > 0 && gemm_fits(gate->w, m) &&
                      gemm_fits(up->w, m) && gemm_fits(down->w, m);
    const size_t act_off = ((2 * nh + 2 * ni) * sizeof(float) + 255) & ~(size_t)255;
    rc = grow(scr.mlp, act_off + (gemm ? gemm_act_bytes(m, I) : 0), false, &scr);
    if (rc) return rc;
    float *xn = (float *)scr.mlp.ptr, *g = xn + nh, *u = g + ni, *y = u + ni;
    if (!gemm) {
        // Decode.  RMSNorm inside the gate+up GEMV when a group's rows fit
        // its registers (each workgroup forms the sums of squares itself),
        // SwiGLU in the down GEMV's staging for groups of up to
        // kMlpFusedSwiGLUMaxM tokens (every workgroup evaluates it for its
        // own K range), the residual add always in the down GEMV's epilogue.
        // Q35MM_MLP_UNFUSED=1 runs the separate kernels instead.
        // A row-split weight takes plain activations: its neighbour runs as
        // the separate kernel, which gives the same bits.
        const uint32_t mg = std::min(m, kGemvMaxM);
        const q35mm_weight *dn[1] = {down};
        float *dy[1] = {dX};
        if (!g_dev.mlp_unfused && g_dev.mlp_pair && uses_gemv_rows(gate->w) && uses_gemv_rows(up->w)) {
            // Row-split gate and up (the model's shapes): one launch per
            // group of up to eight tokens forms silu(gate) * up, with the
            // RMSNorm inside for one token; then the down GEMV with the
            // residual add.
            const bool norm_in = m == 1 && H <= kPairNormMaxCols && g_dev.mlp_pair == 1;
            if (!norm_in) HIP_TRY(launch_rmsnorm(dX, H, dNormW, xn, H, m, H, eps, st));
            for (uint32_t t0 = 0; t0 < m; t0 += kGemvMaxM) {
                const uint32_t mt = std::min(kGemvMaxM, m - t0);
                rc = run_mlp_pair(gate, up, mt, (norm_in ? dX : xn) + (size_t)t0 * H, norm_in ? dNormW : nullptr, eps,
                                  g + (size_t)t0 * I, st);
                if (rc) return rc;
            }
            return run_gemv(dn, 1, m, g, dy, st, GemvInput(), dy);
        }
        const bool fuse_norm = !g_dev.mlp_unfused && gemv_norm_fits(mg, H) && !uses_gemv_rows(gate->w) &&
                               !uses_gemv_rows(up->w);
        const bool fuse_swiglu = !g_dev.mlp_unfused && m <= kMlpFusedSwiGLUMaxM && !uses_gemv_rows(down->w);
        const q35mm_weight *gu[2] = {gate, up};
        float *gy[2] = {g, u};
        GemvInput norm;
        if (fuse_norm) {
            norm.xmode = kXRmsNorm;
            norm.norm_w = dNormW;
            norm.eps = eps;
            rc = run_gemv(gu, 2, m, dX, gy, st, norm);
        } else {
            HIP_TRY(launch_rmsnorm(dX, H, dNormW, xn, H, m, H, eps, st));
            rc = run_gemv(gu, 2, m, xn, gy, st);
        }
        if (rc) return rc;
        GemvInput sw;
        if (fuse_swiglu) {
            sw.xmode = kXSwiGLU;
            sw.x2 = u;
        } else {
            HIP_TRY(launch_swiglu(g, u, g, ni, st));
        }
        if (!g_dev.mlp_unfused) return run_gemv(dn, 1, m, g, dy, st, sw, dy);
        rc = run_gemv(dn, 1, m, g, &y, st, sw);
        if (rc) return rc;
        HIP_TRY(launch_add_inplace(dX, y, nh, st));
        return Q35MM_OK;
    }
    // Prefill: gate and up as one GEMM launch of paired tiles, the RMSNorm
    // written straight into its bf16 activations (a separate RMSNorm kernel
    // and fp32 rows when the row length or alignment does not suit that
    // kernel), the tiles (or their slice sum) forming silu(gate) * up as the
    // down GEMM's bf16 activations (with Q35MM_GEMM_PAIR=0 the down GEMM
    // forms it while rounding its activations), the down GEMM adding the
    // residual in its epilogue -- the bits of the separate calls.
    const q35mm_weight *gu[2] = {gate, up};
    float *gy[2] = {g, u};
    GemmAct act{reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(scr.mlp.ptr) + act_off), false};
    if (rmsnorm_bf16_fits(dX, H, dNormW, H)) {
        const GemmNorm nm{dNormW, eps};
        rc = run_gemm(gu, 2, m, dX, gy, st, nullptr, nullptr, nullptr, &nm, &act);
    } else {
        HIP_TRY(launch_rmsnorm(dX, H, dNormW, xn, H, m, H, eps, st));
        rc = run_gemm(gu, 2, m, xn, gy, st, nullptr, nullptr, nullptr, nullptr, &act);
    }
    if (rc) return rc;
    const q35mm_weight *dn[1] = {down};
    float *dy[1] = {dX};
    const float *res[1] = {dX};
    if (act.done) return run_gemm(dn, 1, m, nullptr, dy, st, res, nullptr, nullptr, nullptr, nullptr, act.buf);
    return run_gemm(dn, 1, m, g, dy, st, res, u);
}

Q35MM_API int q35mm_quantize_f32(const float *dW, uint32_t rows, uint32_t cols, uint8_t *dCodes,
                                 uint16_t *dScale, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    if (rows == 0 || cols == 0) return Q35MM_OK;
    if (!dW || !dCodes || !dScale) return set_error(Q35MM_EINVAL, "null pointer");
    HIP_TRY(launch_quantize_f32(dW, rows, cols, dCodes, dScale, nullptr, pick_stream(stream)));
    return Q35MM_OK;
}

Q35MM_API int q35mm_st_open(const char *path, q35mm_st **out) {
    if (!path || !out) return set_error(Q35MM_EINVAL, "null argument");
    auto *h = new q35mm_st();
    std::string msg;
    const int s = h->a.open(path, msg);
    if (s != st::kOk) {
        delete h;
        *out = nullptr;
        return set_error(s == st::kOpen || s == st::kIo ? Q35MM_EIO : Q35MM_EFORMAT, "%s: %s",
                         st::status_str(s), msg.c_str());
    }
    *out = h;
    return Q35MM_OK;
}

Q35MM_API void q35mm_st_close(q35mm_st *st) { delete st; }

Q35MM_API uint32_t q35mm_st_count(const q35mm_st *st) { return st ? (uint32_t)st->a.tensors.size() : 0u; }

Q35MM_API const char *q35mm_st_name(const q35mm_st *st, uint32_t i) {
    return st && i < st->a.tensors.size() ? st->a.tensors[i].name.c_str() : nullptr;
}

Q35MM_API int q35mm_st_info(const q35mm_st *st, const char *name, const char **dtype, uint32_t *ndim,
                            uint32_t shape[8], uint64_t *nbytes) {
    if (!st || !name) return set_error(Q35MM_EINVAL, "null argument");
    const st::Tensor *t = st->a.find(name);
    if (!t) return set_error(Q35MM_ENOTFOUND, "missing tensor: %s", name);
    if (dtype) *dtype = st::dtype_name(t->dtype);
    if (ndim) *ndim = t->ndim;
    if (shape)
        for (int i = 0; i < 8; i++) shape[i] = t->shape[i];
    if (nbytes) *nbytes = t->bytes;
    return Q35MM_OK;
}

Q35MM_API int q35mm_st_read(const q35mm_st *st, const char *name, void *dst, uint64_t cap) {
    if (!st || !name || !dst) return set_error(Q35MM_EINVAL, "null argument");
    const st::Tensor *t = st->a.find(name);
    if (!t) return set_error(Q35MM_ENOTFOUND, "missing tensor: %s", name);
    if (cap < t->bytes) return set_error(Q35MM_EINVAL, "buffer of %llu bytes for %s (%llu bytes)",
                                         (unsigned long long)cap, name, (unsigned long long)t->bytes);
    if (!st->a.read(*t, 0, t->bytes, dst)) return set_error(Q35MM_EIO, "read of %s failed", name);
    return Q35MM_OK;
}

Q35MM_API int q35mm_st_load_fp8(q35mm_st *st, const char *name, uint32_t rows, uint32_t cols, q35mm_weight **out) {
    if (!st || !name || !out) return set_error(Q35MM_EINVAL, "null argument");
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return st_load_fp8(st->a, name, rows, cols, out);
}

Q35MM_API int q35mm_st_load_ab(q35mm_st *st, const char *name, uint32_t rows, uint32_t cols, q35mm_weight **out) {
    if (!st || !name || !out) return set_error(Q35MM_EINVAL, "null argument");
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return st_load_ab(st->a, name, rows, cols, out);
}

Q35MM_API int q35mm_st_load_bf16(q35mm_st *st, const char *name, uint32_t rows, uint32_t cols, uint16_t **dOut) {
    if (!st || !name || !dOut) return set_error(Q35MM_EINVAL, "null argument");
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    const uint32_t shape[2] = {rows, cols};
    const st::Tensor *t = nullptr;
    rc = need_tensor(st->a, name, st::kBF16, 2, shape, &t);
    if (rc) return rc;
    uint16_t *d = nullptr;
    if (hipMalloc(&d, t->bytes) != hipSuccess)
        return set_error(Q35MM_ENOMEM, "hipMalloc(%llu) failed", (unsigned long long)t->bytes);
    rc = upload_tensor(st->a, *t, d, g_dev.stream);
    if (!rc && hipStreamSynchronize(g_dev.stream) != hipSuccess) rc = set_error(Q35MM_EHIP, "upload failed");
    if (rc) {
        (void)hipStreamSynchronize(g_dev.stream);
        (void)hipFree(d);
        return rc;
    }
    *dOut = d;
    return Q35MM_OK;
}

Q35MM_API void q35mm_free(void *dptr) {
    if (!dptr) return;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    (void)hipDeviceSynchronize();
    (void)hipFree(dptr);
}

Q35MM_API void q35mm_release(const void *W) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto it = g_res.find(W);
    if (it == g_res.end()) return;
    drop(it->second);
    g_res.erase(it);
}

Q35MM_API void q35mm_release_all(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    for (auto &kv : g_res) drop(kv.second);
    g_res.clear();
}

Q35MM_API size_t q35mm_resident_count(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return g_res.size();
}

Q35MM_API void q35mm_shutdown(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    q35mm_release_all();
    if (g_dev.id < 0) return;
    (void)hipDeviceSynchronize();
    for (auto &kv : g_dev.scratch)
        for (DevBuf *b : {&kv.second.ws, &kv.second.cnt, &kv.second.xb, &kv.second.mlp})
            if (b->ptr) (void)hipFree(b->ptr);
    g_dev.scratch.clear();
    g_dev.last_scratch = nullptr;
    for (void *ptr : g_dev.retired) (void)hipFree(ptr);
    g_dev.retired.clear();
    for (DevBuf *b : {&g_dev.dx, &g_dev.dy}) {
        if (b->ptr) (void)hipFree(b->ptr);
        b->ptr = nullptr;
        b->cap = 0;
    }
    if (g_dev.pin) (void)hipHostFree(g_dev.pin);
    g_dev.pin = nullptr;
    g_dev.pin_cap = 0;
    if (g_dev.done) (void)hipHostFree(g_dev.done);
    g_dev.done = nullptr;
    if (g_dev.done_cnt) (void)hipFree(g_dev.done_cnt);
    g_dev.done_cnt = nullptr;
    for (int i = 0; i < 4; i++) {
        if (g_dev.up_pin[i]) (void)hipHostFree(g_dev.up_pin[i]);
        if (g_dev.up_dev[i]) (void)hipFree(g_dev.up_dev[i]);
        if (g_dev.up_ev[i]) (void)hipEventDestroy(g_dev.up_ev[i]);
        g_dev.up_pin[i] = nullptr;
        g_dev.up_dev[i] = nullptr;
        g_dev.up_ev[i] = nullptr;
    }
    for (hipEvent_t &ev : g_dev.xfer_ev) {
        if (ev) (void)hipEventDestroy(ev);
        ev = nullptr;
    }
    if (g_dev.stream) (void)hipStreamDestroy(g_dev.stream);
    g_dev.stream = nullptr;
    g_dev.id = -1;
}

// ---------------------------------------------------------------------
// Chained decode GEMVs
// ---------------------------------------------------------------------
Q35MM_API int q35mm_chain_create(const q35mm_chain_step *steps, uint32_t nsteps, uint32_t m, q35mm_chain **out) {
    if (!steps || !out || nsteps == 0) return set_error(Q35MM_EINVAL, "q35mm_chain_create: need at least one step");
    *out = nullptr;
    if (m == 0 || m > kGemvMaxM) return set_error(Q35MM_EINVAL, "q35mm_chain_create: m=%u (1..%u tokens)", m, kGemvMaxM);
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = ensure_device();
    if (rc) return rc;
    std::vector<ChainStep> tab(nsteps);
    for (uint32_t s = 0; s < nsteps; s++) {
        const q35mm_chain_step &cs = steps[s];
        if (cs.nw == 0 || cs.nw > 4 || !cs.x)
            return set_error(Q35MM_EINVAL, "chain step %u: 1..4 weights and an activation pointer needed", s);
        ChainStep &t = tab[s];
        memset(&t, 0, sizeof t);
        uint32_t item = 0;
        for (uint32_t i = 0; i < cs.nw; i++) {
            rc = check_weight(cs.w[i]);
            if (rc) return rc;
            const Weight &w = cs.w[i]->w;
            if (w.cols != cs.w[0]->w.cols)
                return set_error(Q35MM_EINVAL, "chain step %u: weights differ in cols (%u, %u)", s, cs.w[0]->w.cols,
                                 w.cols);
            if (!gemv_rows_shape(w.kb, 4))
                return set_error(Q35MM_EINVAL, "chain step %u: a %ux%u weight does not run on the row-split GEMV "
                                 "(K of 4..%u blocks of 128)", s, w.rows, w.cols, kGemvRsMaxKb);
            if (!cs.y[i]) return set_error(Q35MM_EINVAL, "chain step %u: null output %u", s, i);
            GemvSeg &g = t.seg[i];
            g.codes = w.codes;
            g.scale = w.scale;
            g.y = cs.y[i];
            g.resid = cs.resid[i];
            g.rows = w.rows;
            g.ldy = w.rows;
            g.nb = w.nb;
            g.cta_begin = item;
            g.nctas = (w.rows + kSubRows - 1) / kSubRows;
            item += g.nctas;
        }
        t.x = cs.x;
        t.ldx = t.k = cs.w[0]->w.cols;
        t.kb = cs.w[0]->w.kb;
        t.nseg = cs.nw;
        t.items = item;
        t.wait = s > 0 ? 1u : 0u;
    }
    // How each step reads x and resid.  Cached loads are safe where no cache
    // of the device can hold a line of those bytes from before their
    // producer's (write-through) stores: no earlier step read them and at
    // most one wrote them (the launch's start invalidates the caches).  The
    // test is made on whole 256-byte spans (cache lines are 128 bytes), so
    // a line shared with other data read earlier counts as read.  A step's
    // outputs must not overlap its own activations (byte ranges).
    struct Span {
        uintptr_t lo, hi;
        bool meets(const Span &o) const { return lo < o.hi && o.lo < hi; }
        Span lines() const { return Span{lo & ~uintptr_t(255), (hi + 255) & ~uintptr_t(255)}; }
    };
    auto span = [&](const void *p, size_t floats) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        return Span{a, a + floats * sizeof(float)};
    };
    std::vector<std::vector<Span>> reads(nsteps), writes(nsteps);
    for (uint32_t s = 0; s < nsteps; s++) {
        const q35mm_chain_step &cs = steps[s];
        const uint32_t k = cs.w[0]->w.cols;
        const Span xs = span(cs.x, (size_t)(m - 1) * k + k);
        reads[s].push_back(xs.lines());
        for (uint32_t i = 0; i < cs.nw; i++) {
            const uint32_t rows = cs.w[i]->w.rows;
            if (cs.resid[i]) reads[s].push_back(span(cs.resid[i], (size_t)m * rows).lines());
            const Span ys = span(cs.y[i], (size_t)m * rows);
            writes[s].push_back(ys.lines());
            if (ys.meets(xs))
                return set_error(Q35MM_EINVAL, "chain step %u: output %u overlaps the step's activations", s, i);
        }
    }
    for (uint32_t s = 0; s < nsteps; s++) {
        bool fresh = true;
        uint32_t writers = 0;
        for (uint32_t t = 0; t < s && fresh; t++) {
            bool w = false;
            for (const Span &r : reads[s]) {
                for (const Span &o : reads[t]) fresh &= !r.meets(o);
                for (const Span &o : writes[t]) w |= r.meets(o);
            }
            writers += w;
        }
        fresh &= writers <= 1;
        tab[s].x_mode = fresh ? kChainXPlain : kChainXCoherent;
        tab[s].count = s + 1 < nsteps ? 1u : 0u;   // every later step waits for all earlier ones
    }
    // One workgroup per CU.  Step s's items are dealt round robin over the
    // workgroups, continuing where step s-1's ended; each workgroup's list is
    // in step order ((step << 16) | item).
    const uint32_t G = g_dev.cus;
    if (nsteps > 0xFFFFu) return set_error(Q35MM_EINVAL, "a chain holds at most 65535 steps");
    std::vector<std::vector<uint32_t>> lists(G);
    uint64_t dealt = 0;
    for (uint32_t s = 0; s < nsteps; s++) {
        if (tab[s].items > 0xFFFFu) return set_error(Q35MM_EINVAL, "chain step %u: more than 65535 sub-tiles", s);
        for (uint32_t j = 0; j < tab[s].items; j++) lists[(dealt + j) % G].push_back((s << 16) | j);
        dealt += tab[s].items;
    }
    std::vector<uint32_t> wg_off(G + 1), wg_items;
    wg_items.reserve(dealt);
    for (uint32_t w = 0; w < G; w++) {
        wg_off[w] = (uint32_t)wg_items.size();
        wg_items.insert(wg_items.end(), lists[w].begin(), lists[w].end());
    }
    wg_off[G] = (uint32_t)wg_items.size();

    auto *c = new q35mm_chain();
    const size_t stride = kChainCtrStride;
    auto up = [](size_t b) { return (b + 4095) & ~(size_t)4095; };
    const size_t tab_bytes = up(nsteps * sizeof(ChainStep));
    const size_t off_bytes = up(wg_off.size() * sizeof(uint32_t));
    const size_t items_bytes = up(std::max<size_t>(1, wg_items.size()) * sizeof(uint32_t));
    const size_t zero_bytes = up(kChainZeroFloats * sizeof(float));
    const size_t ctr_bytes = up((size_t)nsteps * stride);
    const size_t flag_bytes = (size_t)nsteps * kChainFlags * stride;
    const size_t head = tab_bytes + off_bytes + items_bytes;
    const size_t total = head + zero_bytes + ctr_bytes + flag_bytes + 2 * stride;
    if (hipMalloc(&c->mem, total) != hipSuccess) {
        c->mem = nullptr;
        delete c;
        return set_error(Q35MM_ENOMEM, "hipMalloc(%zu) for a chain failed", total);
    }
    uint8_t *base = static_cast<uint8_t *>(c->mem);
    c->p.steps = reinterpret_cast<const ChainStep *>(base);
    c->p.wg_off = reinterpret_cast<const uint32_t *>(base + tab_bytes);
    c->p.wg_items = reinterpret_cast<const uint32_t *>(base + tab_bytes + off_bytes);
    c->p.zero = reinterpret_cast<const float *>(base + head);
    c->p.done = base + head + zero_bytes;
    c->p.ready = c->p.done + ctr_bytes;
    c->p.exit_cnt = reinterpret_cast<uint32_t *>(c->p.ready + flag_bytes);
    c->p.err = reinterpret_cast<uint32_t *>(c->p.ready + flag_bytes + stride);
    c->p.nsteps = nsteps;
    c->p.m = m;
    c->p.nwg = G;
    c->p.spin_limit = env_u32("Q35MM_CHAIN_SPIN_LIMIT", 1u << 20);
    for (uint32_t s = 0; s < nsteps; s++) c->p.coherent |= tab[s].x_mode == kChainXCoherent;
    std::vector<uint8_t> hbuf(head, 0);
    memcpy(hbuf.data(), tab.data(), nsteps * sizeof(ChainStep));
    memcpy(hbuf.data() + tab_bytes, wg_off.data(), wg_off.size() * sizeof(uint32_t));
    if (!wg_items.empty()) memcpy(hbuf.data() + tab_bytes + off_bytes, wg_items.data(), wg_items.size() * 4);
    if (hipMemcpy(base, hbuf.data(), head, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(base + head, 0, total - head) != hipSuccess) {
        (void)hipFree(c->mem);
        delete c;
        return set_error(Q35MM_EHIP, "chain upload failed");
    }
    *out = c;
    return Q35MM_OK;
}

Q35MM_API int q35mm_chain_run(q35mm_chain *c, void *stream) {
    if (!c || !c->mem) return set_error(Q35MM_EINVAL, "null chain");
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    HIP_TRY(launch_chain(c->p, pick_stream(stream)));
    return Q35MM_OK;
}

Q35MM_API int q35mm_chain_status(q35mm_chain *c) {
    if (!c || !c->mem) return set_error(Q35MM_EINVAL, "null chain");
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    HIP_TRY(hipDeviceSynchronize());
    uint32_t err = 0;
    HIP_TRY(hipMemcpy(&err, c->p.err, sizeof err, hipMemcpyDeviceToHost));
    if (err)
        return set_error(Q35MM_EHIP, "a chain launch gave up waiting for an earlier step (another chain launch "
                         "running at the same time can hold the device's workgroup slots)");
    return Q35MM_OK;
}

Q35MM_API uint32_t q35mm_chain_workgroups(const q35mm_chain *c) { return c ? c->p.nwg : 0u; }

Q35MM_API void q35mm_chain_destroy(q35mm_chain *c) {
    if (!c) return;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    (void)hipDeviceSynchronize();
    if (c->mem) (void)hipFree(c->mem);
    delete c;
}

Q35MM_API int q35mm_stream_release(void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (g_dev.id < 0) return Q35MM_OK;
    auto it = g_dev.scratch.find(pick_stream(stream));
    if (it == g_dev.scratch.end()) return Q35MM_OK;
    HIP_TRY(hipDeviceSynchronize());
    Scratch &s = it->second;
    for (DevBuf *b : {&s.ws, &s.cnt, &s.xb, &s.mlp}) {
        if (!b->ptr) continue;
        if (s.captured)
            g_dev.retired.push_back(b->ptr);   // a captured graph may still replay into it
        else
            HIP_TRY(hipFree(b->ptr));
        b->ptr = nullptr;
        b->cap = 0;
    }
    if (g_dev.last_scratch == &s) g_dev.last_scratch = nullptr;
    g_dev.scratch.erase(it);
    return Q35MM_OK;
}

Q35MM_API int q35mm_debug_counters(void *stream, int noalloc, uint64_t *nonzero, uint64_t *words) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (nonzero) *nonzero = 0;
    if (words) *words = 0;
    if (g_dev.id < 0) return Q35MM_OK;
    HIP_TRY(hipDeviceSynchronize());
    const uint32_t *src = nullptr;
    size_t n = 0;
    if (noalloc) {
        src = reinterpret_cast<const uint32_t *>(noalloc_scratch(g_dev.id));
        n = src ? kNoAllocCntBytes / sizeof(uint32_t) : 0;
    } else {
        auto it = g_dev.scratch.find(pick_stream(stream));
        if (it != g_dev.scratch.end() && it->second.cnt.ptr) {
            src = static_cast<const uint32_t *>(it->second.cnt.ptr);
            n = it->second.cnt.cap / sizeof(uint32_t);
        }
    }
    if (!n) return Q35MM_OK;
    std::vector<uint32_t> h(n);
    HIP_TRY(hipMemcpy(h.data(), src, n * sizeof(uint32_t), hipMemcpyDeviceToHost));
    uint64_t nz = 0;
    for (uint32_t v : h) nz += v != 0;
    if (nonzero) *nonzero = nz;
    if (words) *words = n;
    return Q35MM_OK;
}

Q35MM_API const char *q35mm_last_error(void) { return t_last_error.c_str(); }

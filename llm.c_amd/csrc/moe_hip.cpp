// moe_hip.cpp — the C ABI of libmoe_hip: drop-in moe_forward / decode entry
// points over host pointers, the weight residency cache, and the
// device-resident layer API.  All kernels are queued on one HIP stream.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#include "moe_internal.h"
#include "../../include/moe_hip.h"

struct MoeHipLayer {
    int d = 0, F = 0, E = 0, k = 0;
    float *wr = nullptr;     // [d x E]
    float *wrT = nullptr;    // [E x d]
    int wr_nonfinite = 0;    // wr holds an inf or NaN
    float *bias = nullptr;   // [E] or null
    float *wgu = nullptr;    // [E][2F][d]
    float *wdT = nullptr;    // [E][d][F]
};

// Temporaries of the allocation-free forward (moe_hip_forward_dev_noalloc):
// a fixed device array, one copy per GPU the library runs on, held until the
// process ends.  In host code its name is not a device address: host code
// uses the per-device address hipGetSymbolAddress returns (scratch_of).
constexpr size_t kScratchBytes = (size_t)128 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

int g_err = MOE_HIP_OK;
char g_msg[512] = "";
bool g_init = false;
int g_device = 0;
hipStream_t g_stream = nullptr;
bool g_timing = false;
hipEvent_t g_ev[6] = {};
hipEvent_t g_tev[2] = {};
constexpr int kMarks = 64;
hipEvent_t g_marks[kMarks] = {};
bool g_have_times = false;
int g_path = 0;   // 0 auto, 1 grouped GEMMs, 2 decode GEMVs (fused), 3 decode GEMVs (two launches)
int g_rpath = 0;  // 0 auto, 1 token x expert tiles, 2 one token per lane
int g_last_path = 0;   // moe_hip_last_forward_path
// A captured graph keeps the workspace addresses it recorded, so the
// workspace must not be freed and reallocated while one may still run:
// graphs made by moe_hip_graph_end and not yet destroyed, a capture begun by
// moe_hip_graph_begin, or a capture the caller began on its own stream and
// recorded a call into (sticky until moe_hip_shutdown: the library cannot
// see when such a graph is destroyed).
int g_live_graphs = 0;
bool g_api_capture = false;
bool g_ext_capture = false;

int set_err(int code, const char *fmt, ...) {
    g_err = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
    return code;
}

#define HIP_TRY(expr)                                                              \
    do {                                                                           \
        hipError_t e_ = (expr);                                                    \
        if (e_ != hipSuccess)                                                      \
            return set_err(e_ == hipErrorOutOfMemory ? MOE_HIP_ERR_NOMEM : MOE_HIP_ERR_HIP, \
                           "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),  \
                           __FILE__, __LINE__);                                    \
    } while (0)

#define TRY(expr)                        \
    do {                                 \
        int r_ = (expr);                 \
        if (r_ != MOE_HIP_OK) return r_; \
    } while (0)

int ensure_init() {
    if (g_init) return MOE_HIP_OK;
    return moe_hip_init(-1);
}

// The stream a call runs on (NULL: the library stream), for calls that
// record no workspace address (the allocation-free forward, fills, norms).
hipStream_t stream_of(void *s) { return s ? static_cast<hipStream_t>(s) : g_stream; }

// The same for calls whose launches take workspace addresses: notes a
// capture the caller began on the stream (see g_ext_capture).
hipStream_t pick_stream(void *s) {
    hipStream_t st = stream_of(s);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!g_api_capture && hipStreamIsCapturing(st, &cs) == hipSuccess &&
        cs == hipStreamCaptureStatusActive)
        g_ext_capture = true;
    return st;
}

// Grow-only device buffer.  It refuses to grow while a captured graph may
// still use its current address (MOE_HIP_ERR_ARG).
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    int reserve(size_t need) {
        if (need <= bytes) return MOE_HIP_OK;
        if (g_live_graphs > 0 || g_api_capture || g_ext_capture)
            return set_err(MOE_HIP_ERR_ARG,
                           "the workspace would grow to %zu bytes while a captured graph may "
                           "still use it: run the largest call once before capturing, destroy "
                           "the graphs first, or use moe_hip_forward_dev_noalloc", need);
        if (p) {
            hipError_t e = hipFree(p);
            p = nullptr;
            bytes = 0;
            if (e != hipSuccess) return set_err(MOE_HIP_ERR_HIP, "hipFree: %s", hipGetErrorString(e));
        }
        hipError_t e = hipMalloc(&p, need);
        if (e != hipSuccess) {
            p = nullptr;
            return set_err(MOE_HIP_ERR_NOMEM, "hipMalloc(%zu) failed: %s", need, hipGetErrorString(e));
        }
        bytes = need;
        return MOE_HIP_OK;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <class T> T *as() const { return static_cast<T *>(p); }
};

// Workspace shared by every call (calls are serialised by the caller).
struct Workspace {
    DevBuf x, out, probs, ids, gw, counts, offsets, tile_off, tile_expert, perm, h, ys, pieces,
        stage, counters, xn, rmsw, aq, ao, apart, acnt, bw, bwork, xpad, gu_part, wprobs, wide,
        order;
    void release_all() {
        DevBuf *all[] = {&x, &out, &probs, &ids, &gw, &counts, &offsets, &tile_off,
                         &tile_expert, &perm, &h, &ys, &pieces, &stage, &counters, &xn, &rmsw,
                         &aq, &ao, &apart, &acnt, &bw, &bwork, &xpad, &gu_part, &wprobs, &wide,
                         &order};
        for (DevBuf *b : all) b->release();
    }
};
Workspace g_ws;

// Pinned host staging of the host drop-ins (x in; out, probs and ids back).
// The caller's pageable buffers are copied by the CPU into pinned memory and
// moved by the DMA engine from there, so no copy takes the runtime's
// synchronous path for pageable memory; probs and ids go back on a copy
// stream as soon as the routing has run, under the expert products.
constexpr size_t kStageChunk = (size_t)16 << 20;   // half of the pinned area
// Transfers of at most kZeroCopyMax bytes skip the copy engine: a copy
// kernel on the call's stream reads or writes their region of a fine-grained
// (coherent) pinned area of kZeroCopyArea bytes across the bus itself, which
// spares the small decode transfers the copy engine's round trip.
constexpr size_t kZeroCopyMax = (size_t)256 << 10, kZeroCopyArea = (size_t)2 << 20;
struct HostStage {
    char *area = nullptr;         // 2 x kStageChunk bytes, pinned
    char *zc = nullptr;           // kZeroCopyArea bytes, pinned, fine-grained
    hipEvent_t ev[2] = {};        // the last DMA that used each half (chunked transfers)
    hipStream_t copy = nullptr;   // (default priority)
    hipEvent_t routed = nullptr;  // recorded after a drop-in's routing
    bool ready = false;
    void release() {
        if (area) (void)hipHostFree(area);
        if (zc) (void)hipHostFree(zc);
        area = zc = nullptr;
        for (auto &e : ev) {
            if (e) (void)hipEventDestroy(e);
            e = nullptr;
        }
        if (copy) (void)hipStreamDestroy(copy);
        if (routed) (void)hipEventDestroy(routed);
        copy = nullptr;
        routed = nullptr;
        ready = false;
    }
};
HostStage g_hs;
// When set, run_forward records it on its stream right after the routing.
hipEvent_t g_route_mark = nullptr;

// Host copies between pageable and pinned memory split over a few threads
// (one thread copies ~10-20 GB/s, below the link rate).  The workers live
// for the process; a copy is cut into kCopyThreads equal parts, the calling
// thread taking part 0.
class CopyPool {
  public:
    static constexpr int kCopyThreads = 8;
    void copy(void *dst, const void *src, size_t n) {
        if (n < ((size_t)1 << 20)) {
            memcpy(dst, src, n);
            return;
        }
        start();
        {
            std::lock_guard<std::mutex> lk(m_);
            dst_ = static_cast<char *>(dst);
            src_ = static_cast<const char *>(src);
            n_ = n;
            left_ = kCopyThreads - 1;
            ++gen_;
        }
        cv_.notify_all();
        part(0);
        std::unique_lock<std::mutex> lk(m_);
        done_.wait(lk, [&] { return left_ == 0; });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(m_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
    }

  private:
    void start() {
        if (!workers_.empty()) return;
        for (int i = 1; i < kCopyThreads; ++i)
            workers_.emplace_back([this, i] {
                unsigned long seen = 0;
                for (;;) {
                    {
                        std::unique_lock<std::mutex> lk(m_);
                        cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                        if (stop_) return;
                        seen = gen_;
                    }
                    part(i);
                    std::lock_guard<std::mutex> lk(m_);
                    if (--left_ == 0) done_.notify_one();
                }
            });
    }
    void part(int i) {
        const size_t per = (n_ + kCopyThreads - 1) / kCopyThreads;
        const size_t lo = std::min(n_, per * i), hi = std::min(n_, lo + per);
        if (hi > lo) memcpy(dst_ + lo, src_ + lo, hi - lo);
    }
    std::vector<std::thread> workers_;
    std::mutex m_;
    std::condition_variable cv_, done_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0;
    int left_ = 0;
    unsigned long gen_ = 0;
    bool stop_ = false;
};
CopyPool g_copy_pool;

// Device ints that are zero between launches (each launch's last workgroup
// resets what it counted), so they are cleared only when allocated: [0] the
// fused route+dispatch launch's completion counter.
constexpr int kMaxCounters = 64;
int ensure_counters() {
    if (g_ws.counters.bytes >= sizeof(int) * kMaxCounters) return MOE_HIP_OK;
    TRY(g_ws.counters.reserve(sizeof(int) * kMaxCounters));
    HIP_TRY(hipMemsetAsync(g_ws.counters.p, 0, sizeof(int) * kMaxCounters, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

// Each device's address of scratch, resolved once per device with that
// device current (moe_hip_init, or the first allocation-free call there).
constexpr int kMaxDevices = 64;
char *g_scratch[kMaxDevices] = {};

// The current device's scratch; on its first use there the counter block at
// its start (kMaxCounters ints, zero between launches) is cleared on s.
int scratch_of(hipStream_t s, char **out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return set_err(MOE_HIP_ERR_NODEV, "device %d", dev);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        HIP_TRY(moe::launch_zero_ints(static_cast<int *>(p), kMaxCounters, s));
        g_scratch[dev] = static_cast<char *>(p);
    }
    *out = g_scratch[dev];
    return MOE_HIP_OK;
}

int stage_init() {
    if (g_hs.ready) return MOE_HIP_OK;
    if (hipHostMalloc(reinterpret_cast<void **>(&g_hs.area), 2 * kStageChunk,
                      hipHostMallocDefault) != hipSuccess) {
        g_hs.area = nullptr;
        return set_err(MOE_HIP_ERR_NOMEM, "pinned staging of %zu bytes", 2 * kStageChunk);
    }
    if (hipHostMalloc(reinterpret_cast<void **>(&g_hs.zc), kZeroCopyArea, hipHostMallocCoherent) !=
        hipSuccess) {
        g_hs.zc = nullptr;
        return set_err(MOE_HIP_ERR_NOMEM, "pinned staging of %zu bytes", kZeroCopyArea);
    }
    for (auto &e : g_hs.ev) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    HIP_TRY(hipStreamCreateWithFlags(&g_hs.copy, hipStreamNonBlocking));
    HIP_TRY(hipEventCreateWithFlags(&g_hs.routed, hipEventDisableTiming));
    g_hs.ready = true;
    return MOE_HIP_OK;
}

// The staging of one drop-in call (calls are synchronous, so the whole
// pinned area is free when one starts).  An array that fits the area's free
// part takes a region of its own: one CPU copy and one DMA, and for a
// download a copy out in finish(), after one wait per stream.  Larger arrays
// go through the two halves of the area in turn, the CPU copying one while
// the DMA engine moves the other.
class Staging {
  public:
    // host (pageable) -> dev, queued on the library stream.
    int up(void *dev, const void *host, size_t n) {
        TRY(stage_init());
        if (n == 0) return MOE_HIP_OK;
        if (zero_copy(dev, n)) {
            char *pin = g_hs.zc + zoff_;
            zoff_ += align(n);
            memcpy(pin, host, n);
            HIP_TRY(moe::launch_copy16(dev, pin, n, g_stream));
            return MOE_HIP_OK;
        }
        if (fits(n)) {
            if (chunked_up_) {   // (a chunked upload's DMAs may still read the area)
                HIP_TRY(hipStreamSynchronize(g_stream));
                chunked_up_ = false;
            }
            char *pin = g_hs.area + off_;
            off_ += align(n);
            g_copy_pool.copy(pin, host, n);
            HIP_TRY(hipMemcpyAsync(dev, pin, n, hipMemcpyHostToDevice, g_stream));
            return MOE_HIP_OK;
        }
        TRY(drain());
        chunked_up_ = true;
        for (size_t o = 0, i = 0; o < n; o += kStageChunk, ++i) {
            const size_t m = std::min(kStageChunk, n - o);
            char *pin = g_hs.area + (i & 1) * kStageChunk;
            HIP_TRY(hipEventSynchronize(g_hs.ev[i & 1]));   // (the half's last DMA is done)
            g_copy_pool.copy(pin, static_cast<const char *>(host) + o, m);
            HIP_TRY(hipMemcpyAsync(static_cast<char *>(dev) + o, pin, m, hipMemcpyHostToDevice,
                                   g_stream));
            HIP_TRY(hipEventRecord(g_hs.ev[i & 1], g_stream));
        }
        return MOE_HIP_OK;
    }
    // dev -> host (pageable) after the work queued on s; host holds the bytes
    // once finish() has returned.  A download on another stream than the
    // library's must be ordered after the uploads (the drop-ins' copy stream
    // waits for the routing, which follows them on the library stream).
    int down(void *host, const void *dev, size_t n, hipStream_t s) {
        TRY(stage_init());
        if (n == 0) return MOE_HIP_OK;
        if (zero_copy(dev, n)) {
            char *pin = g_hs.zc + zoff_;
            zoff_ += align(n);
            HIP_TRY(moe::launch_copy16(pin, dev, n, s));
            pend_.push_back({host, pin, n, s});
            return MOE_HIP_OK;
        }
        if (fits(n)) {
            char *pin = g_hs.area + off_;
            off_ += align(n);
            HIP_TRY(hipMemcpyAsync(pin, dev, n, hipMemcpyDeviceToHost, s));
            pend_.push_back({host, pin, n, s});
            return MOE_HIP_OK;
        }
        TRY(drain());
        const size_t nch = (n + kStageChunk - 1) / kStageChunk;
        auto issue = [&](size_t i) -> int {
            const size_t o = i * kStageChunk, m = std::min(kStageChunk, n - o);
            HIP_TRY(hipEventSynchronize(g_hs.ev[i & 1]));
            HIP_TRY(hipMemcpyAsync(g_hs.area + (i & 1) * kStageChunk,
                                   static_cast<const char *>(dev) + o, m, hipMemcpyDeviceToHost, s));
            HIP_TRY(hipEventRecord(g_hs.ev[i & 1], s));
            return MOE_HIP_OK;
        };
        TRY(issue(0));
        for (size_t i = 0; i < nch; ++i) {
            if (i + 1 < nch) TRY(issue(i + 1));
            const size_t o = i * kStageChunk, m = std::min(kStageChunk, n - o);
            HIP_TRY(hipEventSynchronize(g_hs.ev[i & 1]));
            g_copy_pool.copy(static_cast<char *>(host) + o, g_hs.area + (i & 1) * kStageChunk, m);
        }
        off_ = 0;   // (every DMA into the area is done)
        return MOE_HIP_OK;
    }
    // A small host array the device updates in place (kernels read and
    // write it across the bus): its region of the fine-grained area, holding
    // the host's values now and copied back by finish().  Null when the
    // array does not qualify; the caller then stages it both ways.
    float *inout(void *host, size_t n) {
        if (stage_init() != MOE_HIP_OK) return nullptr;
        if (n == 0 || n > kZeroCopyMax || n % 16 || zoff_ + n > kZeroCopyArea) return nullptr;
        char *pin = g_hs.zc + zoff_;
        zoff_ += align(n);
        memcpy(pin, host, n);
        pend_.push_back({host, pin, n, g_stream});
        return reinterpret_cast<float *>(pin);
    }
    int finish() {
        TRY(flush());
        HIP_TRY(hipStreamSynchronize(g_stream));
        return MOE_HIP_OK;
    }

  private:
    struct Pending {
        void *host;
        const char *pin;
        size_t n;
        hipStream_t s;
    };
    static size_t align(size_t n) { return (n + 255) & ~(size_t)255; }
    bool fits(size_t n) const { return off_ + n <= 2 * kStageChunk; }
    bool zero_copy(const void *dev, size_t n) const {
        return n <= kZeroCopyMax && n % 16 == 0 && reinterpret_cast<uintptr_t>(dev) % 16 == 0 &&
               zoff_ + n <= kZeroCopyArea;
    }
    // The queued small downloads waited for and copied out.
    int flush() {
        for (const Pending &p : pend_) HIP_TRY(hipStreamSynchronize(p.s));
        for (const Pending &p : pend_) g_copy_pool.copy(p.host, p.pin, p.n);
        pend_.clear();
        return MOE_HIP_OK;
    }
    // Before a chunked transfer: every region handed out is released (the
    // small downloads copied out, the queued DMAs done); after a chunked
    // upload the whole area is handed out afresh.
    int drain() {
        TRY(flush());
        HIP_TRY(hipStreamSynchronize(g_stream));
        off_ = 0;
        return MOE_HIP_OK;
    }
    size_t off_ = 0, zoff_ = 0;
    bool chunked_up_ = false;
    std::vector<Pending> pend_;
};

// Norm: with x_raw set, the rows to route (x, written here) are first
// rms_norm(x_raw; rms_w, eps), by the router where it can.
struct Norm {
    const float *x_raw = nullptr, *rms_w = nullptr;
    float eps = 0.0f;
    // The normalised rows are the caller's output (else only the kernels that
    // read them back need them written).
    bool keep_rows = true;
};

// Residency cache for the drop-in entry points.
// A host drop-in's weights made resident.  d, F: the caller's widths; the
// layer's own are rounded up (padded_dims) when they are not a multiple of
// what the kernels tile.
struct Resident {
    MoeHipLayer *layer = nullptr;
    std::vector<const void *> ptrs;
    int d = 0, F = 0;
};
std::map<const MoEWeights *, Resident> g_resident;

std::vector<const void *> weight_ptrs(const MoEWeights *w) {
    std::vector<const void *> v;
    v.push_back(w->W_router.data);
    for (int e = 0; e < w->n_experts; ++e) {
        v.push_back(w->experts[e].W_gate.data);
        v.push_back(w->experts[e].W_up.data);
        v.push_back(w->experts[e].W_down.data);
    }
    return v;
}

// Shapes a device layer takes (widths = false: the host drop-ins, which pad
// other widths themselves).
int check_shapes(int d, int F, int E, int k, bool widths = true) {
    if (d <= 0 || F <= 0 || E <= 0 || k <= 0)
        return set_err(MOE_HIP_ERR_ARG, "bad MoE shape d=%d F=%d E=%d k=%d", d, F, E, k);
    if (k > E)
        return set_err(MOE_HIP_ERR_ARG, "top_k %d exceeds n_experts %d", k, E);
    // Past the fast routing kernels' tables the general routing kernels take over.
    if ((E > moe::kMaxExperts || k > moe::kMaxTopK) && !moe::route_wide_ok(E, k))
        return set_err(MOE_HIP_ERR_UNSUPPORTED, "n_experts %d / top_k %d above the supported %d / %d",
                       E, k, moe::kWideMaxExperts, moe::kWideMaxTopK);
    if (widths && (d % 64 != 0 || F % 32 != 0))
        return set_err(MOE_HIP_ERR_UNSUPPORTED,
                       "d_model %% 64 and ffn_hidden %% 32 must be 0 (got d=%d F=%d)", d, F);
    return MOE_HIP_OK;
}

// The widths a drop-in's resident layer uses: d_model rounded up to a
// multiple of 64, ffn_hidden to 64 when it is not a multiple of 32.  The
// padding holds zeros in x and in every weight, which leaves the layer
// unchanged: the router's chains add exact zeros (a logit's sign of zero
// aside, which no probability sees), a padded feature has gate = up = 0 and
// so H = silu(0) * 0 = 0, and padded output columns are dropped.
void padded_dims(int d, int F, int *dp, int *Fp) {
    *dp = (d + 63) / 64 * 64;
    *Fp = F % 32 == 0 ? F : (F + 63) / 64 * 64;
}

int validate_weights(const MoEWeights *w, int d, int F) {
    if (!w || !w->experts || !w->W_router.data) return set_err(MOE_HIP_ERR_ARG, "null MoE weights");
    if (w->W_router.rows != d || w->W_router.cols != w->n_experts)
        return set_err(MOE_HIP_ERR_ARG, "W_router is %dx%d, expected %dx%d", w->W_router.rows,
                       w->W_router.cols, d, w->n_experts);
    for (int e = 0; e < w->n_experts; ++e) {
        const FFNWeights &f = w->experts[e];
        if (!f.W_gate.data || !f.W_up.data || !f.W_down.data)
            return set_err(MOE_HIP_ERR_ARG, "expert %d has a null matrix", e);
        if (f.W_gate.rows != d || f.W_gate.cols != F || f.W_up.rows != d || f.W_up.cols != F ||
            f.W_down.rows != F || f.W_down.cols != d)
            return set_err(MOE_HIP_ERR_ARG, "expert %d matrices do not match d=%d F=%d", e, d, F);
    }
    return MOE_HIP_OK;
}

// Router [d x E] from host memory: device copy, its transpose, and the
// non-finite check that selects the zero-skipping router.
int upload_router(MoeHipLayer *L, const float *wr) {
    HIP_TRY(hipMemcpyAsync(L->wr, wr, sizeof(float) * (size_t)L->d * L->E, hipMemcpyHostToDevice,
                           g_stream));
    HIP_TRY(moe::launch_transpose(L->wr, L->wrT, L->d, L->E, g_stream));
    L->wr_nonfinite = 0;
    for (size_t i = 0; i < (size_t)L->d * L->E; ++i)
        if (!std::isfinite(wr[i])) { L->wr_nonfinite = 1; break; }
    return MOE_HIP_OK;
}

// Expert e from host memory (reference layout) into the packed arrays,
// through the device staging buffer (3 d F floats).
int upload_expert(MoeHipLayer *L, int e, const float *wg, const float *wu, const float *wd) {
    const size_t dF = (size_t)L->d * L->F;
    TRY(g_ws.stage.reserve(sizeof(float) * 3 * dF));
    float *st = g_ws.stage.as<float>();
    HIP_TRY(hipMemcpyAsync(st, wg, sizeof(float) * dF, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipMemcpyAsync(st + dF, wu, sizeof(float) * dF, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipMemcpyAsync(st + 2 * dF, wd, sizeof(float) * dF, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(moe::launch_pack_gateup(st, st + dF, L->wgu + 2 * dF * e, L->d, L->F, g_stream));
    HIP_TRY(moe::launch_pack_down(st + 2 * dF, L->wdT + dF * e, L->F, L->d, g_stream));
    return MOE_HIP_OK;
}

// The weights zero-padded to the layer's widths, one expert at a time.
int load_padded(MoeHipLayer *L, const MoEWeights *w, int d, int F) {
    const int dp = L->d, Fp = L->F, E = L->E;
    std::vector<float> wr((size_t)dp * E, 0.0f);
    for (int r = 0; r < d; ++r)
        std::copy_n(w->W_router.data + (size_t)r * E, E, wr.begin() + (size_t)r * E);
    TRY(upload_router(L, wr.data()));
    std::vector<float> g((size_t)dp * Fp, 0.0f), u((size_t)dp * Fp, 0.0f), dn((size_t)Fp * dp, 0.0f);
    for (int e = 0; e < E; ++e) {
        const FFNWeights &f = w->experts[e];
        for (int r = 0; r < d; ++r) {
            std::copy_n(f.W_gate.data + (size_t)r * F, F, g.begin() + (size_t)r * Fp);
            std::copy_n(f.W_up.data + (size_t)r * F, F, u.begin() + (size_t)r * Fp);
        }
        for (int r = 0; r < F; ++r)
            std::copy_n(f.W_down.data + (size_t)r * d, d, dn.begin() + (size_t)r * dp);
        TRY(upload_expert(L, e, g.data(), u.data(), dn.data()));
        HIP_TRY(hipStreamSynchronize(g_stream));   // (the host buffers are reused)
    }
    return MOE_HIP_OK;
}

int resident_layer(const MoEWeights *w, int d, int F, MoeHipLayer **out) {
    TRY(validate_weights(w, d, F));
    std::vector<const void *> ptrs = weight_ptrs(w);
    auto it = g_resident.find(w);
    if (it != g_resident.end()) {
        MoeHipLayer *L = it->second.layer;
        if (it->second.ptrs == ptrs && it->second.d == d && it->second.F == F &&
            L->E == w->n_experts && L->k == w->top_k) {
            *out = L;
            return MOE_HIP_OK;
        }
        moe_hip_layer_destroy(L);
        g_resident.erase(it);
    }
    int dp = d, Fp = F;
    padded_dims(d, F, &dp, &Fp);
    MoeHipLayer *L = nullptr;
    TRY(moe_hip_layer_create(dp, Fp, w->n_experts, w->top_k, &L));
    int rc = dp == d && Fp == F ? moe_hip_layer_load(L, w) : load_padded(L, w, d, F);
    if (rc != MOE_HIP_OK) {
        moe_hip_layer_destroy(L);
        return rc;
    }
    g_resident[w] = Resident{L, ptrs, d, F};
    *out = L;
    return MOE_HIP_OK;
}

// A drop-in's forward of T rows of the caller's width d (x, and out when
// accumulating, in device memory of that width), through a resident layer
// that may be wider: rows are widened with zeros and the output cut back.
int dropin_forward(MoeHipLayer *L, int d, const float *x, int T, float *out, float *probs,
                   int *ids, int accumulate) {
    if (L->d == d) return moe_hip_forward_dev(L, x, T, out, probs, ids, accumulate, g_stream);
    const size_t np = (size_t)T * L->d;
    TRY(g_ws.xpad.reserve(sizeof(float) * 2 * np));
    float *xp = g_ws.xpad.as<float>(), *op = xp + np;
    HIP_TRY(moe::launch_copy_rows(x, T, d, xp, L->d, g_stream));
    if (accumulate) HIP_TRY(moe::launch_copy_rows(out, T, d, op, L->d, g_stream));
    TRY(moe_hip_forward_dev(L, xp, T, op, probs, ids, accumulate, g_stream));
    HIP_TRY(moe::launch_copy_rows(op, T, L->d, out, d, g_stream));
    return MOE_HIP_OK;
}

// A forward of T host rows x [T x d] (the caller's width d, the layer's own
// or narrower) through a resident layer: x goes up through the pinned
// staging, probs and ids (either may be null) come back under the expert
// products, out [T x d] at the end; synchronous at return.
int host_forward(MoeHipLayer *L, int d, const float *x, int T, float *out, float *probs,
                 int *ids) {
    const int E = L->E, k = L->k;
    const size_t xd = (size_t)T * d;
    TRY(g_ws.x.reserve(sizeof(float) * xd));
    TRY(g_ws.out.reserve(sizeof(float) * xd));
    TRY(g_ws.probs.reserve(sizeof(float) * (size_t)T * E));
    TRY(g_ws.ids.reserve(sizeof(int) * (size_t)T * k));
    float *dx = g_ws.x.as<float>(), *dout = g_ws.out.as<float>(), *dprobs = g_ws.probs.as<float>();
    int *dids = g_ws.ids.as<int>();
    Staging st;
    TRY(st.up(dx, x, sizeof(float) * xd));
    g_route_mark = g_hs.routed;
    const int rc = dropin_forward(L, d, dx, T, dout, dprobs, dids, 0);
    g_route_mark = nullptr;
    TRY(rc);
    HIP_TRY(hipStreamWaitEvent(g_hs.copy, g_hs.routed, 0));
    if (probs) TRY(st.down(probs, dprobs, sizeof(float) * (size_t)T * E, g_hs.copy));
    if (ids) TRY(st.down(ids, dids, sizeof(int) * (size_t)T * k, g_hs.copy));
    TRY(st.down(out, dout, sizeof(float) * xd, g_stream));
    return st.finish();
}

void die_on(int rc, const char *what) {
    if (rc == MOE_HIP_OK) return;
    fprintf(stderr, "[libmoe_hip] %s: %s\n", what, g_msg);
    abort();
}

}  // namespace

extern "C" {

int moe_hip_init(int device) {
    if (g_init) return MOE_HIP_OK;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return set_err(MOE_HIP_ERR_NODEV, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0) {
        HIP_TRY(hipGetDevice(&device));
    }
    if (device >= n) return set_err(MOE_HIP_ERR_NODEV, "device %d of %d", device, n);
    HIP_TRY(hipSetDevice(device));
    HIP_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    for (auto &ev : g_ev) HIP_TRY(hipEventCreate(&ev));
    for (auto &ev : g_tev) HIP_TRY(hipEventCreate(&ev));
    for (auto &ev : g_marks) HIP_TRY(hipEventCreate(&ev));
    char *sp = nullptr;
    TRY(scratch_of(g_stream, &sp));
    HIP_TRY(hipStreamSynchronize(g_stream));
    g_device = device;
    g_init = true;
    return MOE_HIP_OK;
}

void moe_hip_shutdown(void) {
    if (!g_init) return;
    (void)hipDeviceSynchronize();
    for (auto &kv : g_resident) moe_hip_layer_destroy(kv.second.layer);
    g_resident.clear();
    g_ws.release_all();
    g_hs.release();
    g_ext_capture = false;
    for (auto &ev : g_ev) (void)hipEventDestroy(ev);
    for (auto &ev : g_tev) (void)hipEventDestroy(ev);
    for (auto &ev : g_marks) (void)hipEventDestroy(ev);
    (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
    g_init = false;
}

int moe_hip_invalidate(const MoEWeights *w) {
    auto it = g_resident.find(w);
    if (it == g_resident.end()) return MOE_HIP_OK;
    (void)hipStreamSynchronize(g_stream);
    moe_hip_layer_destroy(it->second.layer);
    g_resident.erase(it);
    return MOE_HIP_OK;
}

int moe_hip_last_error(void) { return g_err; }
const char *moe_hip_last_error_message(void) { return g_msg; }

const char *moe_hip_error_string(int code) {
    switch (code) {
        case MOE_HIP_OK: return "ok";
        case MOE_HIP_ERR_ARG: return "invalid argument";
        case MOE_HIP_ERR_UNSUPPORTED: return "unsupported shape";
        case MOE_HIP_ERR_HIP: return "HIP runtime error";
        case MOE_HIP_ERR_NOMEM: return "device out of memory";
        case MOE_HIP_ERR_NODEV: return "no GPU";
        default: return "unknown";
    }
}

int moe_hip_layer_create(int d_model, int ffn_hidden, int n_experts, int top_k,
                         MoeHipLayer **layer) {
    if (!layer) return set_err(MOE_HIP_ERR_ARG, "null layer out-pointer");
    *layer = nullptr;
    TRY(check_shapes(d_model, ffn_hidden, n_experts, top_k));
    TRY(ensure_init());
    MoeHipLayer *L = new MoeHipLayer();
    L->d = d_model; L->F = ffn_hidden; L->E = n_experts; L->k = top_k;
    const size_t ne = (size_t)n_experts * d_model * ffn_hidden;
    hipError_t e0 = hipMalloc(&L->wr, sizeof(float) * (size_t)d_model * n_experts);
    hipError_t e1 = e0 == hipSuccess ? hipMalloc(&L->wrT, sizeof(float) * (size_t)d_model * n_experts) : e0;
    hipError_t e2 = e1 == hipSuccess ? hipMalloc(&L->wgu, sizeof(float) * 2 * ne) : e1;
    hipError_t e3 = e2 == hipSuccess ? hipMalloc(&L->wdT, sizeof(float) * ne) : e2;
    if (e3 != hipSuccess) {
        moe_hip_layer_destroy(L);
        return set_err(MOE_HIP_ERR_NOMEM, "layer weights (%zu bytes): %s",
                       sizeof(float) * 3 * ne, hipGetErrorString(e3));
    }
    *layer = L;
    return MOE_HIP_OK;
}

int moe_hip_layer_destroy(MoeHipLayer *L) {
    if (!L) return MOE_HIP_OK;
    if (L->wr) (void)hipFree(L->wr);
    if (L->wrT) (void)hipFree(L->wrT);
    if (L->bias) (void)hipFree(L->bias);
    if (L->wgu) (void)hipFree(L->wgu);
    if (L->wdT) (void)hipFree(L->wdT);
    delete L;
    return MOE_HIP_OK;
}

int moe_hip_layer_load(MoeHipLayer *L, const MoEWeights *w) {
    if (!L) return set_err(MOE_HIP_ERR_ARG, "null layer");
    if (!w || w->n_experts != L->E || w->top_k != L->k)
        return set_err(MOE_HIP_ERR_ARG, "weights do not match the layer (E=%d k=%d)", L->E, L->k);
    TRY(validate_weights(w, L->d, L->F));
    TRY(upload_router(L, w->W_router.data));
    for (int e = 0; e < L->E; ++e) {
        const FFNWeights &f = w->experts[e];
        TRY(upload_expert(L, e, f.W_gate.data, f.W_up.data, f.W_down.data));
    }
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

static int forward_impl(MoeHipLayer *L, const float *x, int T, float *out, float *probs, int *ids,
                        int accumulate, void *stream, Norm nm);

// ---------------------------------------------------------------------------
// Attention of the decode step (src/inference.c:252-308): weights in the
// reference layout, the block's rms_attn scale and the RoPE tables.
struct MoeHipAttn {
    int d = 0, nh = 0, nkv = 0, hd = 0, max_seq = 0;
    float *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
    float *rms = nullptr, *cos_t = nullptr, *sin_t = nullptr;
    // The projections' weights in 16-column tiles (when every width is a
    // multiple of 16): [wq | wk | wv] and wo, for the projection tiles.
    float *wqkv_p = nullptr, *wo_p = nullptr;
};

int moe_hip_attn_destroy(MoeHipAttn *a) {
    if (!a) return MOE_HIP_OK;
    for (float *p : {a->wq, a->wk, a->wv, a->wo, a->rms, a->cos_t, a->sin_t, a->wqkv_p, a->wo_p})
        if (p) (void)hipFree(p);
    delete a;
    return MOE_HIP_OK;
}

int moe_hip_attn_create(int d_model, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                        MoeHipAttn **out) {
    if (!out) return set_err(MOE_HIP_ERR_ARG, "null out-pointer");
    *out = nullptr;
    if (d_model <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_seq_len <= 0 ||
        n_heads % n_kv_heads || head_dim % 8 || head_dim > 64 || n_heads / n_kv_heads > 8 ||
        d_model % 4)
        return set_err(MOE_HIP_ERR_UNSUPPORTED,
                       "decode attention needs head_dim %% 8 == 0, head_dim <= 64, at most 8 "
                       "query heads per kv head and d_model %% 4 == 0");
    TRY(ensure_init());
    auto *a = new MoeHipAttn;
    a->d = d_model; a->nh = n_heads; a->nkv = n_kv_heads; a->hd = head_dim;
    a->max_seq = max_seq_len;
    const size_t qd = (size_t)n_heads * head_dim, kd = (size_t)n_kv_heads * head_dim;
    const size_t tab = (size_t)max_seq_len * (head_dim / 2);
    const size_t sizes[7] = {(size_t)d_model * qd, (size_t)d_model * kd, (size_t)d_model * kd,
                             qd * d_model, (size_t)d_model, tab, tab};
    float **ptrs[7] = {&a->wq, &a->wk, &a->wv, &a->wo, &a->rms, &a->cos_t, &a->sin_t};
    for (int i = 0; i < 7; ++i)
        if (hipMalloc(ptrs[i], sizeof(float) * sizes[i]) != hipSuccess) {
            moe_hip_attn_destroy(a);
            return set_err(MOE_HIP_ERR_NOMEM, "attention weights");
        }
    if (qd % 16 == 0 && kd % 16 == 0 && d_model % 16 == 0 &&
        (hipMalloc(&a->wqkv_p, sizeof(float) * d_model * (qd + 2 * kd)) != hipSuccess ||
         hipMalloc(&a->wo_p, sizeof(float) * qd * d_model) != hipSuccess)) {
        moe_hip_attn_destroy(a);
        return set_err(MOE_HIP_ERR_NOMEM, "attention weights");
    }
    *out = a;
    return MOE_HIP_OK;
}

int moe_hip_attn_load(MoeHipAttn *a, const float *wq, const float *wk, const float *wv,
                      const float *wo, const float *rms_attn) {
    if (!a || !wq || !wk || !wv || !wo || !rms_attn) return set_err(MOE_HIP_ERR_ARG, "null argument");
    const size_t qd = (size_t)a->nh * a->hd, kd = (size_t)a->nkv * a->hd;
    HIP_TRY(hipMemcpy(a->wq, wq, sizeof(float) * a->d * qd, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(a->wk, wk, sizeof(float) * a->d * kd, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(a->wv, wv, sizeof(float) * a->d * kd, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(a->wo, wo, sizeof(float) * qd * a->d, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(a->rms, rms_attn, sizeof(float) * a->d, hipMemcpyHostToDevice));
    if (a->wqkv_p) {
        const int d = a->d, q = (int)qd, kv = (int)kd;
        HIP_TRY(moe::launch_pack_cols16(a->wq, a->wqkv_p, d, q, 0, g_stream));
        HIP_TRY(moe::launch_pack_cols16(a->wk, a->wqkv_p, d, kv, q, g_stream));
        HIP_TRY(moe::launch_pack_cols16(a->wv, a->wqkv_p, d, kv, q + kv, g_stream));
        HIP_TRY(moe::launch_pack_cols16(a->wo, a->wo_p, q, d, 0, g_stream));
        HIP_TRY(hipStreamSynchronize(g_stream));
    }
    return MOE_HIP_OK;
}

int moe_hip_attn_set_rope(MoeHipAttn *a, const float *cos_table, const float *sin_table) {
    if (!a || !cos_table || !sin_table) return set_err(MOE_HIP_ERR_ARG, "null argument");
    const size_t tab = (size_t)a->max_seq * (a->hd / 2);
    HIP_TRY(hipMemcpy(a->cos_t, cos_table, sizeof(float) * tab, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(a->sin_t, sin_table, sizeof(float) * tab, hipMemcpyHostToDevice));
    return MOE_HIP_OK;
}

// The attention sublayer.
static int attn_decode(MoeHipAttn *a, float *x, int B, const int *pos, float *k_cache,
                       float *v_cache, float eps, void *stream) {
    if (!a || B < 0 || (B > 0 && (!x || !pos || !k_cache || !v_cache)))
        return set_err(MOE_HIP_ERR_ARG, "bad attention arguments");
    if (B == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    hipStream_t s = pick_stream(stream);
    const int qd = a->nh * a->hd, kd = a->nkv * a->hd;
    TRY(g_ws.aq.reserve(sizeof(float) * (size_t)B * qd));
    TRY(g_ws.ao.reserve(sizeof(float) * (size_t)B * qd));
    TRY(g_ws.apart.reserve(sizeof(float) * moe::attn_part_floats(B, a->nh, a->hd, a->max_seq)));
    // Merge counters: zero when allocated, reset by the merging workgroup.
    const size_t cnt_bytes = sizeof(int) * (size_t)moe::attn_merge_counters(B, a->nkv);
    if (g_ws.acnt.bytes < cnt_bytes) {
        TRY(g_ws.acnt.reserve(cnt_bytes));
        HIP_TRY(hipMemsetAsync(g_ws.acnt.p, 0, g_ws.acnt.bytes, g_stream));
        HIP_TRY(hipStreamSynchronize(g_stream));
    }
    moe::AttnArgs aa{};
    aa.x = x; aa.rms_w = a->rms; aa.eps = eps;
    aa.wq = a->wq; aa.wk = a->wk; aa.wv = a->wv; aa.wo = a->wo;
    aa.wqkv_p = a->wqkv_p; aa.wo_p = a->wo_p;
    aa.cos_t = a->cos_t; aa.sin_t = a->sin_t; aa.kc = k_cache; aa.vc = v_cache; aa.pos = pos;
    aa.q = g_ws.aq.as<float>(); aa.o = g_ws.ao.as<float>(); aa.part = g_ws.apart.as<float>();
    aa.cnt_merge = g_ws.acnt.as<int>();
    aa.B = B; aa.d = a->d; aa.nh = a->nh; aa.nkv = a->nkv; aa.hd = a->hd; aa.qd = qd; aa.kd = kd;
    aa.max_seq = a->max_seq;
    aa.scale = 1.0f / sqrtf((float)a->hd);
    HIP_TRY(moe::launch_attn_decode(aa, s));
    return MOE_HIP_OK;
}

int moe_hip_attn_decode_dev(MoeHipAttn *a, float *x, int B, const int *pos, float *k_cache,
                            float *v_cache, float eps, void *stream) {
    return attn_decode(a, x, B, pos, k_cache, v_cache, eps, stream);
}

int moe_hip_decode_block_dev(MoeHipAttn *a, MoeHipLayer *L, const float *rms_ffn, float *x, int B,
                             const int *pos, float *k_cache, float *v_cache, float eps,
                             float *x_norm, int *ids, void *stream) {
    if (!a || !L || !rms_ffn || a->d != L->d)
        return set_err(MOE_HIP_ERR_ARG, "block: attention and MoE layer must share d_model");
    if (B < 0) return set_err(MOE_HIP_ERR_ARG, "bad block arguments");
    if (B == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    (void)pick_stream(stream);   // (notes a capture before the workspace is sized)
    float *xn = x_norm;
    if (!xn) {
        TRY(g_ws.xn.reserve(sizeof(float) * (size_t)B * L->d));
        xn = g_ws.xn.as<float>();
    }
    TRY(attn_decode(a, x, B, pos, k_cache, v_cache, eps, stream));
    Norm nm;
    nm.x_raw = x; nm.rms_w = rms_ffn; nm.eps = eps;
    return forward_impl(L, xn, B, x, nullptr, ids, 1, stream, nm);
}

// ---------------------------------------------------------------------------
// Checkpoints written by model_save (src/transformer.c:573-616): uint32
// magic 0x4C4C4D43, ModelConfig, embed [vocab x d], then per block
// rms_attn [d], W_Q [d x nh*hd], W_K, W_V [d x nkv*hd], W_O [nh*hd x d],
// rms_ffn [d] and either W_gate, W_up [d x F], W_down [F x d] (dense) or
// W_router [d x E] and each expert's W_gate, W_up, W_down (n_experts > 1,
// src/transformer.c:437); finally rms_final [d] and lm_head [d x vocab].
// All fp32, row-major, no padding.
struct MoeHipModel {
    ModelConfig cfg{};
    std::vector<MoeHipLayer *> layers;   // null for dense blocks
    std::vector<float *> rms_ffn;        // device [d], every block
};

namespace {

struct CkptFile {
    FILE *f = nullptr;
    ~CkptFile() { if (f) fclose(f); }
    bool skip(size_t floats) { return fseeko(f, (off_t)(floats * sizeof(float)), SEEK_CUR) == 0; }
    bool read(float *dst, size_t floats) { return fread(dst, sizeof(float), floats, f) == floats; }
};

}  // namespace

int moe_hip_model_free(MoeHipModel *m) {
    if (!m) return MOE_HIP_OK;
    for (MoeHipLayer *L : m->layers)
        if (L) moe_hip_layer_destroy(L);
    for (float *p : m->rms_ffn)
        if (p) (void)hipFree(p);
    delete m;
    return MOE_HIP_OK;
}

int moe_hip_model_load(const char *path, MoeHipModel **out) {
    if (!path || !out) return set_err(MOE_HIP_ERR_ARG, "null argument");
    *out = nullptr;
    TRY(ensure_init());
    CkptFile cf;
    cf.f = fopen(path, "rb");
    if (!cf.f) return set_err(MOE_HIP_ERR_ARG, "cannot open %s", path);
    uint32_t magic = 0;
    ModelConfig cfg;
    if (fread(&magic, sizeof(magic), 1, cf.f) != 1 || magic != 0x4C4C4D43u ||
        fread(&cfg, sizeof(cfg), 1, cf.f) != 1)
        return set_err(MOE_HIP_ERR_ARG, "%s: not a model checkpoint (magic/config)", path);
    const int d = cfg.d_model, F = cfg.ffn_hidden, E = cfg.n_experts, k = cfg.top_k_experts;
    if (d <= 0 || F <= 0 || cfg.n_layers < 0 || cfg.vocab_size < 0 || cfg.n_heads <= 0 ||
        cfg.n_kv_heads <= 0 || cfg.head_dim <= 0 || E < 1)
        return set_err(MOE_HIP_ERR_ARG, "%s: implausible config", path);
    const bool moe = E > 1;
    if (moe) TRY(check_shapes(d, F, E, k));
    const size_t qd = (size_t)cfg.n_heads * cfg.head_dim, kd = (size_t)cfg.n_kv_heads * cfg.head_dim;
    const size_t dF = (size_t)d * F;
    // The whole file must be there, as model_load reads it to the end.
    const size_t per_block = (size_t)d + d * qd + 2 * d * kd + qd * d + d +
                             (moe ? (size_t)d * E + (size_t)E * 3 * dF : 3 * dF);
    const size_t floats = (size_t)cfg.vocab_size * d + (size_t)cfg.n_layers * per_block + d +
                          (size_t)d * cfg.vocab_size;
    const off_t header = (off_t)(sizeof(magic) + sizeof(cfg));
    if (fseeko(cf.f, 0, SEEK_END) != 0 || ftello(cf.f) < header + (off_t)(floats * sizeof(float)) ||
        fseeko(cf.f, header, SEEK_SET) != 0)
        return set_err(MOE_HIP_ERR_ARG, "%s: shorter than its config implies (%zu floats)", path,
                       floats);
    auto *m = new MoeHipModel;
    m->cfg = cfg;
    int rc = MOE_HIP_OK;
    std::vector<float> host;
    float *hb = nullptr;   // pinned staging for the expert matrices
    auto fail = [&](int code) {
        if (hb) (void)hipHostFree(hb);
        moe_hip_model_free(m);
        return code;
    };
    auto trunc = [&](int l) {
        return fail(set_err(MOE_HIP_ERR_ARG, "%s: truncated in block %d", path, l));
    };
    if (!cf.skip((size_t)cfg.vocab_size * d)) return trunc(-1);
    if (moe && hipHostMalloc((void **)&hb, sizeof(float) * 3 * dF, hipHostMallocDefault) != hipSuccess) {
        hb = nullptr;
        return fail(set_err(MOE_HIP_ERR_NOMEM, "pinned staging of %zu bytes", sizeof(float) * 3 * dF));
    }
    host.resize(std::max<size_t>((size_t)d * E, d));
    for (int l = 0; l < cfg.n_layers; ++l) {
        if (!cf.skip(d + d * qd + 2 * d * kd + qd * d)) return trunc(l);
        if (!cf.read(host.data(), d)) return trunc(l);
        float *rw = nullptr;
        if (hipMalloc(&rw, sizeof(float) * d) != hipSuccess)
            return fail(set_err(MOE_HIP_ERR_NOMEM, "rms_ffn of block %d", l));
        m->rms_ffn.push_back(rw);
        if (hipMemcpy(rw, host.data(), sizeof(float) * d, hipMemcpyHostToDevice) != hipSuccess)
            return fail(set_err(MOE_HIP_ERR_HIP, "rms_ffn upload"));
        if (!moe) {
            m->layers.push_back(nullptr);
            if (!cf.skip(3 * dF)) return trunc(l);
            continue;
        }
        MoeHipLayer *L = nullptr;
        if ((rc = moe_hip_layer_create(d, F, E, k, &L)) != MOE_HIP_OK) return fail(rc);
        m->layers.push_back(L);
        if (!cf.read(host.data(), (size_t)d * E)) return trunc(l);
        if ((rc = upload_router(L, host.data())) != MOE_HIP_OK) return fail(rc);
        for (int e = 0; e < E; ++e) {
            // (the previous expert's copies out of hb must be done first)
            if (hipStreamSynchronize(g_stream) != hipSuccess)
                return fail(set_err(MOE_HIP_ERR_HIP, "expert upload"));
            if (!cf.read(hb, 3 * dF)) return trunc(l);
            if ((rc = upload_expert(L, e, hb, hb + dF, hb + 2 * dF)) != MOE_HIP_OK) return fail(rc);
        }
    }
    if (hipStreamSynchronize(g_stream) != hipSuccess) return fail(set_err(MOE_HIP_ERR_HIP, "sync"));
    if (hb) (void)hipHostFree(hb);
    *out = m;   // (rms_final and lm_head are not needed here)
    return MOE_HIP_OK;
}

int moe_hip_model_config(const MoeHipModel *m, ModelConfig *cfg) {
    if (!m || !cfg) return set_err(MOE_HIP_ERR_ARG, "null argument");
    *cfg = m->cfg;
    return MOE_HIP_OK;
}

MoeHipLayer *moe_hip_model_layer(MoeHipModel *m, int l) {
    return m && l >= 0 && l < (int)m->layers.size() ? m->layers[l] : nullptr;
}

const float *moe_hip_model_rms_ffn(const MoeHipModel *m, int l) {
    return m && l >= 0 && l < (int)m->rms_ffn.size() ? m->rms_ffn[l] : nullptr;
}

int moe_hip_layer_set_router_bias(MoeHipLayer *L, const float *bias) {
    if (!L) return set_err(MOE_HIP_ERR_ARG, "null layer");
    if (!bias) {
        if (L->bias) {
            HIP_TRY(hipStreamSynchronize(g_stream));
            HIP_TRY(hipFree(L->bias));
        }
        L->bias = nullptr;
        return MOE_HIP_OK;
    }
    if (!L->bias) HIP_TRY(hipMalloc(&L->bias, sizeof(float) * L->E));
    HIP_TRY(hipMemcpyAsync(L->bias, bias, sizeof(float) * L->E, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

int moe_hip_layer_fill_synthetic(MoeHipLayer *L, uint64_t seed, float std_router,
                                 float std_expert) {
    if (!L) return set_err(MOE_HIP_ERR_ARG, "null layer");
    const size_t dF = (size_t)L->d * L->F;
    TRY(g_ws.stage.reserve(sizeof(float) * 3 * dF));
    float *st = g_ws.stage.as<float>();
    HIP_TRY(moe::launch_fill_normal(L->wr, (size_t)L->d * L->E, seed, 1, 0.0f, std_router, g_stream));
    HIP_TRY(moe::launch_transpose(L->wr, L->wrT, L->d, L->E, g_stream));
    L->wr_nonfinite = 0;
    for (int e = 0; e < L->E; ++e) {
        HIP_TRY(moe::launch_fill_normal(st, dF, seed, 16 + 3 * (uint64_t)e, 0.0f, std_expert, g_stream));
        HIP_TRY(moe::launch_fill_normal(st + dF, dF, seed, 17 + 3 * (uint64_t)e, 0.0f, std_expert, g_stream));
        HIP_TRY(moe::launch_fill_normal(st + 2 * dF, dF, seed, 18 + 3 * (uint64_t)e, 0.0f, std_expert, g_stream));
        HIP_TRY(moe::launch_pack_gateup(st, st + dF, L->wgu + 2 * dF * e, L->d, L->F, g_stream));
        HIP_TRY(moe::launch_pack_down(st + 2 * dF, L->wdT + dF * e, L->F, L->d, g_stream));
    }
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

int moe_hip_layer_get_expert(MoeHipLayer *L, int e, float *wg, float *wu, float *wd) {
    if (!L || e < 0 || e >= L->E) return set_err(MOE_HIP_ERR_ARG, "bad layer/expert");
    const size_t dF = (size_t)L->d * L->F;
    TRY(g_ws.stage.reserve(sizeof(float) * 3 * dF));
    float *st = g_ws.stage.as<float>();
    HIP_TRY(moe::launch_unpack_gateup(L->wgu + 2 * dF * e, st, st + dF, L->d, L->F, g_stream));
    HIP_TRY(moe::launch_unpack_down(L->wdT + dF * e, st + 2 * dF, L->F, L->d, g_stream));
    if (wg) HIP_TRY(hipMemcpyAsync(wg, st, sizeof(float) * dF, hipMemcpyDeviceToHost, g_stream));
    if (wu) HIP_TRY(hipMemcpyAsync(wu, st + dF, sizeof(float) * dF, hipMemcpyDeviceToHost, g_stream));
    if (wd) HIP_TRY(hipMemcpyAsync(wd, st + 2 * dF, sizeof(float) * dF, hipMemcpyDeviceToHost, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

int moe_hip_layer_get_router(MoeHipLayer *L, float *wr) {
    if (!L || !wr) return set_err(MOE_HIP_ERR_ARG, "bad layer/pointer");
    HIP_TRY(hipMemcpyAsync(wr, L->wr, sizeof(float) * (size_t)L->d * L->E, hipMemcpyDeviceToHost, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

int moe_hip_fill_normal_dev(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float mean,
                            float std, void *stream) {
    TRY(ensure_init());
    if (!dst && n) return set_err(MOE_HIP_ERR_ARG, "null destination");
    HIP_TRY(moe::launch_fill_normal(dst, n, seed, stream_id, mean, std, stream_of(stream)));
    return MOE_HIP_OK;
}

int moe_hip_link_rate(size_t bytes, float *h2d_gbs, float *d2h_gbs) {
    if (!h2d_gbs || !d2h_gbs || bytes == 0) return set_err(MOE_HIP_ERR_ARG, "bad link-rate arguments");
    TRY(ensure_init());
    void *dev = nullptr, *host = nullptr;
    if (hipMalloc(&dev, bytes) != hipSuccess) return set_err(MOE_HIP_ERR_NOMEM, "link rate: device");
    if (hipHostMalloc(&host, bytes, hipHostMallocDefault) != hipSuccess) {
        (void)hipFree(dev);
        return set_err(MOE_HIP_ERR_NOMEM, "link rate: pinned host");
    }
    memset(host, 0, bytes);
    float ms[2] = {0.0f, 0.0f};
    hipError_t e = hipSuccess;
    for (int rep = 0; rep < 3 && e == hipSuccess; ++rep)   // (the last pass counts)
        for (int dir = 0; dir < 2 && e == hipSuccess; ++dir) {
            e = hipEventRecord(g_tev[0], g_stream);
            if (e == hipSuccess)
                e = dir ? hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, g_stream)
                        : hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, g_stream);
            if (e == hipSuccess) e = hipEventRecord(g_tev[1], g_stream);
            if (e == hipSuccess) e = hipEventSynchronize(g_tev[1]);
            if (e == hipSuccess) e = hipEventElapsedTime(&ms[dir], g_tev[0], g_tev[1]);
        }
    (void)hipHostFree(host);
    (void)hipFree(dev);
    if (e != hipSuccess) return set_err(MOE_HIP_ERR_HIP, "link rate: %s", hipGetErrorString(e));
    *h2d_gbs = (float)(bytes / (ms[0] * 1e-3) / 1e9);
    *d2h_gbs = (float)(bytes / (ms[1] * 1e-3) / 1e9);
    return MOE_HIP_OK;
}

int moe_hip_read_probe(const void *src, size_t bytes, int mode, float *out, void *stream) {
    TRY(ensure_init());
    if (!src || !out || mode < 0 || mode > 2 || bytes == 0 || bytes % ((size_t)32 << 20) != 0)
        return set_err(MOE_HIP_ERR_ARG, "read probe: mode 0-2, bytes a nonzero multiple of 32 MiB");
    HIP_TRY(moe::launch_read_probe(static_cast<const float *>(src), bytes, mode, out,
                                   stream_of(stream)));
    return MOE_HIP_OK;
}

int moe_hip_eval_exp(int which, const float *x, float *y, size_t n, void *stream) {
    TRY(ensure_init());
    if (which != 0 && which != 1) return set_err(MOE_HIP_ERR_ARG, "which must be 0 or 1");
    if (n && (!x || !y)) return set_err(MOE_HIP_ERR_ARG, "null pointer");
    HIP_TRY(moe::launch_eval_exp(which, x, y, n, stream_of(stream)));
    return MOE_HIP_OK;
}

// Layers routed by the general kernels (more experts or a larger top-k than
// the fast routing kernels' tables) need a logits buffer when the caller
// passes no probs, and scratch for their dispatch.
static bool is_wide(int E, int k) { return E > moe::kMaxExperts || k > moe::kMaxTopK; }
struct WideBufs {
    float *probs = nullptr;   // [T x E]
    int *ints = nullptr;      // [moe::wide_dispatch_ints(T k, E)]
};

// Routing (and, with dispatch, the stable counting sort by expert) of T
// rows.  tile_expert: ceil(T k / kGemmBM) + E ints; counter: one device int,
// zero between launches (the fused dispatch's last workgroup resets it).
static int route_impl(MoeHipLayer *L, const float *x, int T, float *probs, int *ids, float *gw,
                      int *counts, int *offsets, int *tile_off, int *perm, int *tile_expert,
                      int *counter, hipStream_t s, bool dispatch = true, Norm nm = Norm{},
                      const WideBufs &wb = WideBufs{}) {
    if (is_wide(L->E, L->k)) {
        // (the general kernels put the logits in probs first)
        if (!probs) probs = wb.probs;
        if (!probs || (dispatch && !wb.ints))
            return set_err(MOE_HIP_ERR_ARG, "wide routing without its buffers");
    }
    moe::RouteArgs ra{x, L->wr, L->bias, T, L->d, L->E, L->k, probs, ids, gw};
    ra.no_dispatch = dispatch ? 0 : 1;
    if (nm.x_raw) {
        ra.x_raw = nm.x_raw; ra.rms_w = nm.rms_w; ra.rms_eps = nm.eps;
        ra.rms_rcp = 1.0f / (float)L->d; ra.xn_out = const_cast<float *>(x);
    }
    if (g_rpath != 1 || L->E > 128) {   // (the tile router takes up to 128 experts)
        ra.wrT = L->wrT;
        ra.wr_nonfinite = L->wr_nonfinite;
    }
    moe::DispatchArgs da{ids, T * L->k, L->E, moe::kGemmBM, counts, offsets, tile_off, perm,
                         counter, tile_expert};
    da.wide = wb.ints;
    if (g_timing) HIP_TRY(hipEventRecord(g_ev[0], s));
    HIP_TRY(moe::launch_route_dispatch(ra, da, s));
    if (g_timing) {
        HIP_TRY(hipEventRecord(g_ev[1], s));
        HIP_TRY(hipEventRecord(g_ev[2], s));
    }
    return MOE_HIP_OK;
}

static size_t max_mtiles_of(size_t n, int E) { return (n + moe::kGemmBM - 1) / moe::kGemmBM + E; }

int moe_hip_route_dev(MoeHipLayer *L, const float *x, int T, float *probs, int *ids, float *gw,
                      int *counts, int *offsets, int *perm, void *stream) {
    if (!L || (!x && T > 0) || T < 0) return set_err(MOE_HIP_ERR_ARG, "bad route arguments");
    if (T == 0) return MOE_HIP_OK;
    hipStream_t s = pick_stream(stream);
    const size_t n = (size_t)T * L->k;
    TRY(g_ws.ids.reserve(sizeof(int) * n));
    TRY(g_ws.gw.reserve(sizeof(float) * n));
    TRY(g_ws.counts.reserve(sizeof(int) * L->E));
    TRY(g_ws.offsets.reserve(sizeof(int) * (L->E + 1)));
    TRY(g_ws.tile_off.reserve(sizeof(int) * (L->E + 1)));
    TRY(g_ws.perm.reserve(sizeof(int) * n));
    TRY(g_ws.tile_expert.reserve(sizeof(int) * max_mtiles_of(n, L->E)));
    TRY(ensure_counters());
    WideBufs wb;
    if (is_wide(L->E, L->k)) {
        TRY(g_ws.wprobs.reserve(sizeof(float) * (size_t)T * L->E));
        TRY(g_ws.wide.reserve(sizeof(int) * moe::wide_dispatch_ints(n, L->E)));
        wb.probs = g_ws.wprobs.as<float>();
        wb.ints = g_ws.wide.as<int>();
    }
    return route_impl(L, x, T, probs, ids ? ids : g_ws.ids.as<int>(), gw ? gw : g_ws.gw.as<float>(),
                      counts ? counts : g_ws.counts.as<int>(),
                      offsets ? offsets : g_ws.offsets.as<int>(), g_ws.tile_off.as<int>(),
                      perm ? perm : g_ws.perm.as<int>(), g_ws.tile_expert.as<int>(),
                      g_ws.counters.as<int>(), s, true, Norm{}, wb);
}

namespace {

// How a forward of T rows runs (expert-product path, partial products per
// slot) and the device memory it takes.
struct FwdPlan {
    size_t n = 0;           // T * k assignments
    int max_mtiles = 0;     // grouped GEMM m-tile bound
    bool use_decode = false, fused = false;
    bool tiny = false;      // a step of at most moe::kTinySlots assignments (decode_tiny.hip)
    int ksplit = 1;         // partial products per slot the combine adds (at most, stream-K)
    int streamk = 0, sk_groups = 0;   // down projection in stream-K form (moe::down_plan)
    size_t h_floats = 0;    // H [n x F] (grouped GEMMs, unfused decode)
    size_t ys_floats = 0;   // per-slot products / split-K partials
    size_t pieces_ints = 0; // stream-K piece counts [n][d / 256]
    int gu_tail = 0;        // gate/up split tail: workgroups per round (moe::gateup_tail_groups)
    size_t gu_part_floats = 0;  // its pieces
    size_t order_ints = 0;  // the down projection's short-first m-tile order (whole tiles, >= 4 rounds)
    size_t wide_probs_floats = 0, wide_ints = 0;   // general routing kernels' buffers (WideBufs)
};

// The device buffers of one forward.
struct FwdBufs {
    int *ids = nullptr;     // [n] (used when the caller passes none)
    float *gw = nullptr;    // [n]
    int *counts = nullptr, *offsets = nullptr, *tile_off = nullptr, *tile_expert = nullptr;
    int *perm = nullptr;    // [n]
    float *h = nullptr, *ys = nullptr;
    int *pieces = nullptr;     // [n][d / 256] (stream-K down projection)
    float *gu_part = nullptr;  // gate/up split-tail pieces
    int *order = nullptr;      // [max_mtiles] m-tile order of the down projection
    int *counters = nullptr;   // kMaxCounters ints, zero between launches
    WideBufs wide;             // (layers routed by the general kernels)
};

// probs_given: the caller takes the router probabilities (the general
// routing kernels then need no logits buffer of their own).
int plan_forward(const MoeHipLayer *L, int T, FwdPlan *p, bool probs_given) {
    const int d = L->d, F = L->F, E = L->E, k = L->k;
    const size_t n = (size_t)T * k;
    if (n > (size_t)0x7fffffff / (size_t)(F > d ? F : d))
        return set_err(MOE_HIP_ERR_UNSUPPORTED, "T*k*max(F,d) exceeds 32-bit indexing");
    p->n = n;
    p->max_mtiles = (int)max_mtiles_of(n, E);
    if (is_wide(E, k)) {
        p->wide_probs_floats = probs_given ? 0 : (size_t)T * E;
        p->wide_ints = moe::wide_dispatch_ints(n, E);
    }
    // Expert products: skinny decode GEMVs (which find their own slots from
    // the expert ids, so routing skips the dispatch) or grouped GEMMs.
    // (the decode kernels address one expert's gate/up block, 2*F*d floats,
    // with 32-bit byte offsets)
    const bool decode_ok = F % 64 == 0 && n <= (size_t)moe::kDecodeMaxSlots &&
                           sizeof(float) * 2 * (size_t)F * d < ((size_t)1 << 31);
    if (g_path >= 2 && !decode_ok)
        return set_err(MOE_HIP_ERR_UNSUPPORTED,
                       "decode kernels need ffn_hidden %% 64 == 0, T*k <= %d and "
                       "8*ffn_hidden*d_model < 2^31", moe::kDecodeMaxSlots);
    p->use_decode = g_path >= 2 || (g_path == 0 && decode_ok && n <= (size_t)16 * E);
    const int fused_splits = F / (16 * moe::decode_fused_waves(d, F));
    const size_t fused_floats = (size_t)fused_splits * n * d;
    p->fused = p->use_decode && g_path != 3 && sizeof(float) * fused_floats <= moe::kFusedPartialBytes;
    // One to a few tokens: their few experts' 16-feature groups spread over
    // the CUs (the items of the fused kernels would leave most of them idle).
    const bool tiny_inside = g_rpath == 0 && L->wrT && !L->wr_nonfinite &&
                             moe::decode_tiny_routed_ok(T, d, F, E, k);
    p->tiny = p->use_decode && g_path == 0 && moe::decode_tiny_ok((int)n, d, F, E) &&
              (tiny_inside || n <= (size_t)moe::kTinyLaunchSlots);
    if (p->tiny) {
        p->fused = false;
        p->ksplit = F / 16;
        p->ys_floats = (size_t)p->ksplit * n * d;
    } else if (p->fused) {
        p->ksplit = fused_splits;
        p->ys_floats = fused_floats;
    } else if (p->use_decode) {
        p->ksplit = moe::decode_ksplit(d, F, E);
        p->h_floats = n * F;
        p->ys_floats = n * d * p->ksplit;
    } else {
        // Small grids split the down projection's reduction (a fixed split,
        // or stream-K pieces); the combine adds the partials in order.
        const moe::DownPlan dp = moe::down_plan(d, F, p->max_mtiles, n);
        p->ksplit = dp.slots;
        p->streamk = dp.streamk;
        p->sk_groups = dp.groups;
        p->pieces_ints = dp.streamk ? n * (size_t)(d / 256) : 0;
        p->gu_tail = moe::gateup_tail_groups(2 * F, d, p->max_mtiles);
        p->gu_part_floats = (size_t)p->gu_tail * moe::kGemmBM * 256;
        if (!dp.streamk && dp.slots == 1 && dp.bn == 256 &&
            (long)p->max_mtiles * (d / 256) >= 4L * moe::device_cus())
            p->order_ints = (size_t)p->max_mtiles;
        p->h_floats = n * F;
        p->ys_floats = (size_t)p->ksplit * n * d;
    }
    return MOE_HIP_OK;
}

// Buffers from the grow-only workspace.
int workspace_bufs(const MoeHipLayer *L, const FwdPlan &p, FwdBufs *b) {
    TRY(g_ws.ids.reserve(sizeof(int) * p.n));
    TRY(g_ws.gw.reserve(sizeof(float) * p.n));
    TRY(g_ws.counts.reserve(sizeof(int) * L->E));
    TRY(g_ws.offsets.reserve(sizeof(int) * (L->E + 1)));
    TRY(g_ws.tile_off.reserve(sizeof(int) * (L->E + 1)));
    TRY(g_ws.tile_expert.reserve(sizeof(int) * p.max_mtiles));
    TRY(g_ws.perm.reserve(sizeof(int) * p.n));
    if (p.h_floats) TRY(g_ws.h.reserve(sizeof(float) * p.h_floats));
    TRY(g_ws.ys.reserve(sizeof(float) * p.ys_floats));
    if (p.pieces_ints) TRY(g_ws.pieces.reserve(sizeof(int) * p.pieces_ints));
    if (p.gu_part_floats) TRY(g_ws.gu_part.reserve(sizeof(float) * p.gu_part_floats));
    if (p.order_ints) TRY(g_ws.order.reserve(sizeof(int) * p.order_ints));
    if (p.wide_probs_floats) TRY(g_ws.wprobs.reserve(sizeof(float) * p.wide_probs_floats));
    if (p.wide_ints) TRY(g_ws.wide.reserve(sizeof(int) * p.wide_ints));
    TRY(ensure_counters());
    b->ids = g_ws.ids.as<int>(); b->gw = g_ws.gw.as<float>();
    b->counts = g_ws.counts.as<int>(); b->offsets = g_ws.offsets.as<int>();
    b->tile_off = g_ws.tile_off.as<int>(); b->tile_expert = g_ws.tile_expert.as<int>();
    b->perm = g_ws.perm.as<int>(); b->h = g_ws.h.as<float>(); b->ys = g_ws.ys.as<float>();
    b->pieces = p.pieces_ints ? g_ws.pieces.as<int>() : nullptr;
    b->gu_part = p.gu_part_floats ? g_ws.gu_part.as<float>() : nullptr;
    b->order = p.order_ints ? g_ws.order.as<int>() : nullptr;
    b->counters = g_ws.counters.as<int>();
    b->wide.probs = p.wide_probs_floats ? g_ws.wprobs.as<float>() : nullptr;
    b->wide.ints = p.wide_ints ? g_ws.wide.as<int>() : nullptr;
    return MOE_HIP_OK;
}

// Buffers carved from one fixed device block of cap bytes at base (the
// allocation-free entry point's scratch array).  Returns the bytes needed in
// *need; the pointers are set only when they fit.
void carve_bufs(const MoeHipLayer *L, const FwdPlan &p, char *base, size_t cap, FwdBufs *b,
                size_t *need) {
    size_t off = 0;
    auto take = [&](size_t bytes) -> void * {
        void *q = base + off;
        off += (bytes + 255) & ~(size_t)255;
        return q;
    };
    FwdBufs c;
    c.counters = static_cast<int *>(take(sizeof(int) * kMaxCounters));   // (first: cleared at set-up)
    c.ids = static_cast<int *>(take(sizeof(int) * p.n));
    c.gw = static_cast<float *>(take(sizeof(float) * p.n));
    c.counts = static_cast<int *>(take(sizeof(int) * L->E));
    c.offsets = static_cast<int *>(take(sizeof(int) * (L->E + 1)));
    c.tile_off = static_cast<int *>(take(sizeof(int) * (L->E + 1)));
    c.tile_expert = static_cast<int *>(take(sizeof(int) * p.max_mtiles));
    c.perm = static_cast<int *>(take(sizeof(int) * p.n));
    c.h = p.h_floats ? static_cast<float *>(take(sizeof(float) * p.h_floats)) : nullptr;
    c.ys = static_cast<float *>(take(sizeof(float) * p.ys_floats));
    c.pieces = p.pieces_ints ? static_cast<int *>(take(sizeof(int) * p.pieces_ints)) : nullptr;
    c.gu_part = p.gu_part_floats ? static_cast<float *>(take(sizeof(float) * p.gu_part_floats)) : nullptr;
    c.order = p.order_ints ? static_cast<int *>(take(sizeof(int) * p.order_ints)) : nullptr;
    c.wide.probs = p.wide_probs_floats ? static_cast<float *>(take(sizeof(float) * p.wide_probs_floats)) : nullptr;
    c.wide.ints = p.wide_ints ? static_cast<int *>(take(sizeof(int) * p.wide_ints)) : nullptr;
    *need = off;
    if (off <= cap) *b = c;
}

}  // namespace

int moe_hip_forward_dev(MoeHipLayer *L, const float *x, int T, float *out, float *probs, int *ids,
                        int accumulate, void *stream) {
    return forward_impl(L, x, T, out, probs, ids, accumulate, stream, Norm{});
}

// The layer on planned buffers.  x: the rows to route and multiply; with
// nm.x_raw set they are written first, as rms_norm(nm.x_raw) (then x must be
// writable device memory).
static int run_forward(MoeHipLayer *L, const float *x, int T, float *out, float *probs, int *ids,
                       int accumulate, hipStream_t s, Norm nm, const FwdPlan &p,
                       const FwdBufs &b) {
    const int d = L->d, F = L->F, E = L->E, k = L->k;
    const size_t n = p.n;
    int *ids_d = ids ? ids : b.ids;
    // Decode steps small enough route inside the fused expert kernel (same
    // routing bits as the row-block router, no routing launch).
    const bool routed = p.fused && g_rpath == 0 && L->wrT && !L->wr_nonfinite &&
                        moe::decode_routed_ok(T, d, F, E, k);
    // Steps of at most 4 assignments route inside the few-row kernel.
    const bool tiny_routed = p.tiny && g_rpath == 0 && L->wrT && !L->wr_nonfinite &&
                             moe::decode_tiny_routed_ok(T, d, F, E, k);
    moe::DecodeArgs tn{};
    tn.x = x; tn.ids = ids_d; tn.topk = k; tn.w = L->wgu; tn.w2 = L->wdT; tn.out = b.ys;
    tn.d = d; tn.F = F; tn.E = E; tn.ksplit = p.ksplit; tn.nslots = (int)n;
    if (routed || tiny_routed) {
        moe::RouteArgs ra{x, L->wr, L->bias, T, d, E, k, probs, ids_d, b.gw};
        ra.wrT = L->wrT;
        ra.no_dispatch = 1;
        if (nm.x_raw) {
            // (the routed kernel keeps the normalised rows in LDS: they go to
            // x only when the caller takes them)
            ra.x_raw = nm.x_raw; ra.rms_w = nm.rms_w; ra.rms_eps = nm.eps;
            ra.rms_rcp = 1.0f / (float)d; ra.xn_out = nm.keep_rows ? const_cast<float *>(x) : nullptr;
        }
        moe::DecodeArgs gu{};
        gu.x = x; gu.ids = ids_d; gu.topk = k; gu.w = L->wgu; gu.w2 = L->wdT; gu.out = b.ys;
        gu.d = d; gu.F = F; gu.E = E; gu.ksplit = 1; gu.nslots = (int)n;
        if (g_timing)
            for (int i = 0; i < 3; ++i) HIP_TRY(hipEventRecord(g_ev[i], s));
        if (tiny_routed) HIP_TRY(moe::launch_decode_tiny(tn, &ra, s));
        else             HIP_TRY(moe::launch_decode_routed(gu, ra, s));
        if (g_route_mark) HIP_TRY(hipEventRecord(g_route_mark, s));
        if (g_timing) {
            HIP_TRY(hipEventRecord(g_ev[3], s));
            HIP_TRY(hipEventRecord(g_ev[4], s));
        }
    } else {
        TRY(route_impl(L, x, T, probs, ids_d, b.gw, b.counts, b.offsets, b.tile_off, b.perm,
                       b.tile_expert, b.counters, s, !p.use_decode, nm, b.wide));
        if (g_route_mark) HIP_TRY(hipEventRecord(g_route_mark, s));
    }
    g_last_path = routed ? 4 : tiny_routed ? 6 : !p.use_decode ? 1 : p.tiny ? 5 : p.fused ? 2 : 3;
    if (routed || tiny_routed) {
        // (the expert products ran with the routing)
    } else if (p.tiny) {
        HIP_TRY(moe::launch_decode_tiny(tn, nullptr, s));
        if (g_timing) {
            HIP_TRY(hipEventRecord(g_ev[3], s));
            HIP_TRY(hipEventRecord(g_ev[4], s));
        }
    } else if (p.use_decode) {
        // Fused gate/up + split-K down while its partials stay small, else
        // gate/up then down.
        moe::DecodeArgs gu{};
        gu.x = x; gu.ids = ids_d; gu.topk = k; gu.w = L->wgu;
        gu.d = d; gu.F = F; gu.E = E; gu.ksplit = 1; gu.nslots = (int)n;
        if (p.fused) {
            gu.out = b.ys;
            gu.w2 = L->wdT;
            HIP_TRY(moe::launch_decode_gateup(gu, s));
            if (g_timing) {
                HIP_TRY(hipEventRecord(g_ev[3], s));
                HIP_TRY(hipEventRecord(g_ev[4], s));
            }
        } else {
            gu.out = b.h;
            HIP_TRY(moe::launch_decode_gateup(gu, s));
            if (g_timing) HIP_TRY(hipEventRecord(g_ev[3], s));
            moe::DecodeArgs dn{};
            dn.x = b.h; dn.ids = ids_d; dn.topk = k; dn.w = L->wdT;
            dn.out = b.ys; dn.d = d; dn.F = F; dn.E = E; dn.ksplit = p.ksplit;
            dn.nslots = (int)n;
            HIP_TRY(moe::launch_decode_down(dn, s));
            if (g_timing) HIP_TRY(hipEventRecord(g_ev[4], s));
        }
    } else {
        moe::GemmArgs gu{x, b.perm, k, L->wgu, b.h, b.offsets, b.tile_off, b.tile_expert, E, d,
                         2 * F, F, p.max_mtiles};
        gu.tail_groups = p.gu_tail;
        gu.tail_part = b.gu_part;
        HIP_TRY(moe::launch_gemm_gateup(gu, s));
        HIP_TRY(moe::launch_gateup_fixup(gu, s));
        if (g_timing) HIP_TRY(hipEventRecord(g_ev[3], s));
        moe::GemmArgs dn{b.h, b.perm, k, L->wdT, b.ys, b.offsets, b.tile_off, b.tile_expert, E, F,
                         d, d, p.max_mtiles};
        dn.ksplit = p.ksplit;
        dn.split_stride = n * (size_t)d;
        dn.streamk = p.streamk;
        dn.sk_groups = p.sk_groups;
        dn.pieces = b.pieces;
        if (b.order) {
            // The experts' short last m-tiles first: a CU that finishes one of
            // them mid-round otherwise idles until the in-order dispatch
            // reaches a workgroup it can take.
            HIP_TRY(moe::launch_short_first_order(b.offsets, b.tile_off, E, b.order, s));
            dn.order = b.order;
        }
        HIP_TRY(moe::launch_gemm_down(dn, s));
        if (g_timing) HIP_TRY(hipEventRecord(g_ev[4], s));
    }
    moe::CombineArgs ca{b.ys, b.gw, out, T, d, k, accumulate, p.ksplit, n * (size_t)d};
    if (p.streamk) {
        ca.pieces = b.pieces;
        ca.pieces_cols = 256;
    }
    HIP_TRY(moe::launch_combine(ca, s));
    if (g_timing) {
        HIP_TRY(hipEventRecord(g_ev[5], s));
        g_have_times = true;
    }
    return MOE_HIP_OK;
}

static int forward_impl(MoeHipLayer *L, const float *x, int T, float *out, float *probs, int *ids,
                        int accumulate, void *stream, Norm nm) {
    if (!L || T < 0 || (T > 0 && (!x || !out))) return set_err(MOE_HIP_ERR_ARG, "bad forward arguments");
    if (T == 0) return MOE_HIP_OK;
    hipStream_t s = pick_stream(stream);
    FwdPlan p;
    TRY(plan_forward(L, T, &p, probs != nullptr));
    FwdBufs b;
    TRY(workspace_bufs(L, p, &b));
    return run_forward(L, x, T, out, probs, ids, accumulate, s, nm, p, b);
}

// moe_hip_forward_dev on the fixed scratch array: no device memory is
// allocated or freed, so callers under graph capture or in serving loops
// can use it.  Every call on a device shares that device's array.
int moe_hip_forward_dev_noalloc(MoeHipLayer *L, const float *x, int T, float *out, float *probs,
                                int *ids, int accumulate, void *stream) {
    if (!L || T < 0 || (T > 0 && (!x || !out))) return set_err(MOE_HIP_ERR_ARG, "bad forward arguments");
    if (!g_init) return set_err(MOE_HIP_ERR_ARG, "the library is not initialised (moe_hip_init)");
    if (T == 0) return MOE_HIP_OK;
    // (its launches take only scratch addresses: a capture of this call
    // leaves the workspace free to grow)
    hipStream_t s = stream_of(stream);
    char *base = nullptr;
    TRY(scratch_of(s, &base));
    FwdPlan p;
    TRY(plan_forward(L, T, &p, probs != nullptr));
    FwdBufs b;
    size_t need = 0;
    carve_bufs(L, p, base, kScratchBytes, &b, &need);
    if (need > kScratchBytes)
        return set_err(MOE_HIP_ERR_UNSUPPORTED,
                       "this forward needs %zu bytes of temporaries, above the fixed %zu-byte "
                       "scratch of the allocation-free entry point", need, kScratchBytes);
    return run_forward(L, x, T, out, probs, ids, accumulate, s, Norm{}, p, b);
}

int moe_hip_set_router_path(int mode) {
    if (mode < 0 || mode > 2) return set_err(MOE_HIP_ERR_ARG, "router path mode %d", mode);
    g_rpath = mode;
    return MOE_HIP_OK;
}

int moe_hip_last_forward_path(void) { return g_last_path; }

int moe_hip_set_expert_path(int mode) {
    if (mode < 0 || mode > 3) return set_err(MOE_HIP_ERR_ARG, "expert path mode %d", mode);
    g_path = mode;
    return MOE_HIP_OK;
}

int moe_hip_timer_start(void) {
    TRY(ensure_init());
    HIP_TRY(hipEventRecord(g_tev[0], g_stream));
    return MOE_HIP_OK;
}

int moe_hip_timer_stop(float *ms) {
    if (!ms) return set_err(MOE_HIP_ERR_ARG, "null output");
    HIP_TRY(hipEventRecord(g_tev[1], g_stream));
    HIP_TRY(hipEventSynchronize(g_tev[1]));
    HIP_TRY(hipEventElapsedTime(ms, g_tev[0], g_tev[1]));
    return MOE_HIP_OK;
}

int moe_hip_timer_mark(int i) {
    TRY(ensure_init());
    if (i < 0 || i >= kMarks) return set_err(MOE_HIP_ERR_ARG, "mark %d outside [0, %d)", i, kMarks);
    HIP_TRY(hipEventRecord(g_marks[i], g_stream));
    return MOE_HIP_OK;
}

int moe_hip_timer_between(int i, int j, float *ms) {
    if (!ms || i < 0 || j < 0 || i >= kMarks || j >= kMarks)
        return set_err(MOE_HIP_ERR_ARG, "bad marks %d, %d", i, j);
    TRY(ensure_init());
    HIP_TRY(hipEventSynchronize(g_marks[j]));
    HIP_TRY(hipEventElapsedTime(ms, g_marks[i], g_marks[j]));
    return MOE_HIP_OK;
}

int moe_hip_set_timing(int on) {
    TRY(ensure_init());
    g_timing = on != 0;
    g_have_times = false;
    return MOE_HIP_OK;
}

int moe_hip_last_timings(float *ms5) {
    if (!ms5) return set_err(MOE_HIP_ERR_ARG, "null output");
    if (!g_have_times) return set_err(MOE_HIP_ERR_ARG, "no timed forward since timing was enabled");
    HIP_TRY(hipEventSynchronize(g_ev[5]));
    for (int i = 0; i < 5; ++i) HIP_TRY(hipEventElapsedTime(&ms5[i], g_ev[i], g_ev[i + 1]));
    return MOE_HIP_OK;
}

int moe_hip_forward(const Matrix *x, const MoEWeights *w, const ModelConfig *cfg,
                    ForwardCache *cache, Matrix *out) {
    if (!x || !w || !cfg || !cache || !out) return set_err(MOE_HIP_ERR_ARG, "null argument");
    const int T = x->rows, d = x->cols, F = cfg->ffn_hidden, E = w->n_experts, k = w->top_k;
    if (out->rows != T || out->cols != d)
        return set_err(MOE_HIP_ERR_ARG, "out is %dx%d, expected %dx%d", out->rows, out->cols, T, d);
    TRY(check_shapes(d, F, E, k, false));
    if (T == 0) return MOE_HIP_OK;
    if (!x->data || !out->data || !cache->router_probs || !cache->expert_ids)
        return set_err(MOE_HIP_ERR_ARG, "null data pointer");
    TRY(ensure_init());
    MoeHipLayer *L = nullptr;
    TRY(resident_layer(w, d, F, &L));
    return host_forward(L, d, x->data, T, out->data, cache->router_probs, cache->expert_ids);
}

int moe_hip_forward_host(MoeHipLayer *L, const float *x, int T, float *out, float *probs,
                         int *ids) {
    if (!L || T < 0 || (T > 0 && (!x || !out))) return set_err(MOE_HIP_ERR_ARG, "bad forward arguments");
    if (T == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    return host_forward(L, L->d, x, T, out, probs, ids);
}

void moe_forward(const Matrix *x, const MoEWeights *w, const ModelConfig *cfg, ForwardCache *cache,
                 Matrix *out) {
    die_on(moe_hip_forward(x, w, cfg, cache, out), "moe_forward");
}

int moe_decode_batch(const MoEWeights *w, const ModelConfig *cfg, const float *x_norm, int n_rows,
                     float *x) {
    if (!w || !cfg || n_rows < 0 || (n_rows > 0 && (!x_norm || !x)))
        return set_err(MOE_HIP_ERR_ARG, "bad decode arguments");
    const int d = cfg->d_model, F = cfg->ffn_hidden;
    TRY(check_shapes(d, F, w->n_experts, w->top_k, false));
    if (n_rows == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    MoeHipLayer *L = nullptr;
    TRY(resident_layer(w, d, F, &L));
    const size_t xd = (size_t)n_rows * d;
    TRY(g_ws.x.reserve(sizeof(float) * xd));
    TRY(g_ws.out.reserve(sizeof(float) * xd));
    float *dxn = g_ws.x.as<float>(), *dx = g_ws.out.as<float>();
    Staging st;
    TRY(st.up(dxn, x_norm, sizeof(float) * xd));
    // x += MoE(x_norm): a small x is updated where it is staged, across the
    // bus, by the combine itself.
    if (float *px = st.inout(x, sizeof(float) * xd)) {
        TRY(dropin_forward(L, d, dxn, n_rows, px, nullptr, nullptr, 1));
    } else {
        TRY(st.up(dx, x, sizeof(float) * xd));
        TRY(dropin_forward(L, d, dxn, n_rows, dx, nullptr, nullptr, 1));
        TRY(st.down(x, dx, sizeof(float) * xd, g_stream));
    }
    TRY(st.finish());
    return MOE_HIP_OK;
}

void moe_decode_step(const MoEWeights *w, const ModelConfig *cfg, const float *x_norm, float *x) {
    die_on(moe_decode_batch(w, cfg, x_norm, 1, x), "moe_decode_step");
}

int moe_hip_rms_norm_dev(const float *x, const float *w, float eps, int rows, int cols, float *y,
                         void *stream) {
    if (rows < 0 || cols <= 0 || (rows > 0 && (!x || !w || !y)))
        return set_err(MOE_HIP_ERR_ARG, "bad rms_norm arguments");
    if (rows == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    HIP_TRY(moe::launch_rms_norm(x, w, eps, rows, cols, y, stream_of(stream)));
    return MOE_HIP_OK;
}

int moe_hip_backward_dev(MoeHipLayer *L, const float *x, int T, const float *dout, float aux_coef,
                         float *dx, float *dw_router, float *dw_gate, float *dw_up, float *dw_down,
                         float *aux_loss, int accumulate, void *stream) {
    if (!L || T < 0 || (T > 0 && (!x || !dout || !dx || !dw_router || !dw_gate || !dw_up || !dw_down)))
        return set_err(MOE_HIP_ERR_ARG, "bad backward arguments");
    if (T == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    const int d = L->d, F = L->F, E = L->E, k = L->k;
    const size_t n = (size_t)T * k;
    if (n * (size_t)(F > d ? F : d) > (size_t)0x7fffffff)
        return set_err(MOE_HIP_ERR_UNSUPPORTED, "T*k*max(F,d) exceeds 32-bit indexing");
    if (is_wide(E, k))
        return set_err(MOE_HIP_ERR_UNSUPPORTED, "backward: n_experts %d / top_k %d above %d / %d",
                       E, k, moe::kMaxExperts, moe::kMaxTopK);
    hipStream_t s = pick_stream(stream);
    // The forward's routing and dispatch (bit-exact with moe_forward).
    TRY(g_ws.probs.reserve(sizeof(float) * (size_t)T * E));
    TRY(g_ws.ids.reserve(sizeof(int) * n));
    TRY(g_ws.gw.reserve(sizeof(float) * n));
    TRY(g_ws.counts.reserve(sizeof(int) * E));
    TRY(g_ws.offsets.reserve(sizeof(int) * (E + 1)));
    TRY(g_ws.tile_off.reserve(sizeof(int) * (E + 1)));
    TRY(g_ws.perm.reserve(sizeof(int) * n));
    TRY(g_ws.tile_expert.reserve(sizeof(int) * max_mtiles_of(n, E)));
    TRY(ensure_counters());
    TRY(route_impl(L, x, T, g_ws.probs.as<float>(), g_ws.ids.as<int>(), g_ws.gw.as<float>(),
                   g_ws.counts.as<int>(), g_ws.offsets.as<int>(), g_ws.tile_off.as<int>(),
                   g_ws.perm.as<int>(), g_ws.tile_expert.as<int>(), g_ws.counters.as<int>(), s,
                   true));
    // Weights: the packed ones and their unit transposes (tile engine), or
    // the reference layout wg, wu [E][d x F], wd [E][F x d].
    const size_t dF = (size_t)d * F;
    const bool engine = moe::backward_engine_ok(d, F);
    const int max_mtiles = (int)((n + moe::kGemmBM - 1) / moe::kGemmBM) + E;
    TRY(g_ws.bw.reserve(sizeof(float) * 3 * E * dF));
    float *w0 = g_ws.bw.as<float>(), *w1 = w0 + E * dF, *w2 = w1 + E * dF;
    if (!engine) HIP_TRY(moe::launch_unpack_experts(L->wgu, L->wdT, w0, w1, w2, E, d, F, s));
    // Workspace: G, U, H [n x F], dH [n x F, at least d E + E: the router
    // gradient's chunk partials reuse it]; Y [splits][n x d], dY [n x d];
    // dgw, inv [n]; dlogits [T x E].
    const size_t nF = n * F, nd = n * d, ndh = moe::backward_dh_floats(n, d, F, E);
    const size_t ysplits = (size_t)moe::backward_slot_splits(d, F, max_mtiles, n);
    const size_t npieces = engine && d % 256 == 0 ? n * (size_t)(d / 256) : 0;
    const size_t ntail = moe::backward_tail_floats(d, F, max_mtiles);
    // (the split-tail pieces last, 256-byte aligned)
    const size_t tail_off = (3 * nF + ndh + (ysplits + 1) * nd + 2 * n + (size_t)T * E + npieces +
                             63) & ~(size_t)63;
    TRY(g_ws.bwork.reserve(sizeof(float) * (tail_off + ntail)));
    float *G = g_ws.bwork.as<float>(), *U = G + nF, *H = U + nF, *dH = H + nF;
    float *Y = dH + ndh, *dY = Y + ysplits * nd, *dgw = dY + nd;
    int *inv = reinterpret_cast<int *>(dgw + n);
    float *dlogits = reinterpret_cast<float *>(inv + n);
    int *pieces = npieces ? reinterpret_cast<int *>(dlogits + (size_t)T * E) : nullptr;
    float *tail = ntail ? G + tail_off : nullptr;
    moe::BackwardArgs b{};
    b.x = x; b.dout = dout; b.wr = L->wr; b.wrT = L->wrT;
    if (engine) {
        b.wgu = L->wgu; b.wdT = L->wdT; b.wguT = w0; b.wdTT = w0 + 2 * E * dF;
    } else {
        b.wg = w0; b.wu = w1; b.wd = w2;
    }
    b.probs = g_ws.probs.as<float>(); b.gw = g_ws.gw.as<float>();
    b.ids = g_ws.ids.as<int>(); b.counts = g_ws.counts.as<int>();
    b.offsets = g_ws.offsets.as<int>(); b.tile_off = g_ws.tile_off.as<int>();
    b.tile_expert = g_ws.tile_expert.as<int>(); b.perm = g_ws.perm.as<int>();
    b.T = T; b.d = d; b.F = F; b.E = E; b.k = k;
    b.max_mtiles = max_mtiles;
    b.aux_coef = aux_coef;
    b.G = G; b.U = U; b.H = H; b.dH = dH; b.Y = Y; b.dY = dY; b.dgw = dgw; b.dlogits = dlogits;
    b.inv = inv;
    b.pieces = pieces;
    b.tail_part = tail;
    b.dx = dx; b.dwr = dw_router; b.dwg = dw_gate; b.dwu = dw_up; b.dwd = dw_down;
    b.aux = aux_loss; b.accumulate = accumulate ? 1 : 0;
    HIP_TRY(moe::launch_moe_backward(b, s));
    return MOE_HIP_OK;
}

int moe_hip_ffn_sublayer_dev(MoeHipLayer *L, float *x, const float *rms_w, float eps, int T,
                             float *x_norm, float *probs, int *ids, void *stream) {
    if (!L || T < 0 || (T > 0 && (!x || !rms_w)))
        return set_err(MOE_HIP_ERR_ARG, "bad sublayer arguments");
    if (T == 0) return MOE_HIP_OK;
    TRY(ensure_init());
    (void)pick_stream(stream);   // (notes a capture before the workspace is sized)
    float *xn = x_norm;
    if (!xn) {
        TRY(g_ws.xn.reserve(sizeof(float) * (size_t)T * L->d));
        xn = g_ws.xn.as<float>();
    }
    Norm nm;
    nm.x_raw = x; nm.rms_w = rms_w; nm.eps = eps;
    nm.keep_rows = x_norm != nullptr;
    return forward_impl(L, xn, T, x, probs, ids, 1, stream, nm);
}

int moe_hip_block_ffn(Matrix *x, const float *rms_ffn, const MoEWeights *w,
                      const ModelConfig *cfg, ForwardCache *cache) {
    if (!x || !rms_ffn || !w || !cfg || !cache) return set_err(MOE_HIP_ERR_ARG, "null argument");
    const int T = x->rows, d = x->cols, F = cfg->ffn_hidden, E = w->n_experts, k = w->top_k;
    if (d != cfg->d_model) return set_err(MOE_HIP_ERR_ARG, "x has %d columns, d_model %d", d, cfg->d_model);
    const Matrix &xn = cache->x_norm_ffn, &fo = cache->ffn_out;
    if (xn.rows != T || xn.cols != d || fo.rows != T || fo.cols != d)
        return set_err(MOE_HIP_ERR_ARG, "cache x_norm_ffn / ffn_out must be %dx%d", T, d);
    TRY(check_shapes(d, F, E, k, false));
    if (T == 0) return MOE_HIP_OK;
    if (!x->data || !xn.data || !fo.data || !cache->router_probs || !cache->expert_ids)
        return set_err(MOE_HIP_ERR_ARG, "null data pointer");
    TRY(ensure_init());
    MoeHipLayer *L = nullptr;
    TRY(resident_layer(w, d, F, &L));
    const size_t xd = (size_t)T * d;
    TRY(g_ws.x.reserve(sizeof(float) * xd));
    TRY(g_ws.xn.reserve(sizeof(float) * xd));
    TRY(g_ws.out.reserve(sizeof(float) * xd));
    TRY(g_ws.rmsw.reserve(sizeof(float) * d));
    TRY(g_ws.probs.reserve(sizeof(float) * (size_t)T * E));
    TRY(g_ws.ids.reserve(sizeof(int) * (size_t)T * k));
    float *dx = g_ws.x.as<float>(), *dxn = g_ws.xn.as<float>(), *dout = g_ws.out.as<float>();
    float *dw = g_ws.rmsw.as<float>(), *dprobs = g_ws.probs.as<float>();
    int *dids = g_ws.ids.as<int>();
    Staging st;
    TRY(st.up(dw, rms_ffn, sizeof(float) * d));
    TRY(st.up(dx, x->data, sizeof(float) * xd));
    HIP_TRY(moe::launch_rms_norm(dx, dw, cfg->rms_norm_eps, T, d, dxn, g_stream));
    g_route_mark = g_hs.routed;
    const int rc = dropin_forward(L, d, dxn, T, dout, dprobs, dids, 0);
    g_route_mark = nullptr;
    TRY(rc);
    // x_norm, probs and ids come back under the expert products, ffn_out at
    // the end
    HIP_TRY(hipStreamWaitEvent(g_hs.copy, g_hs.routed, 0));
    TRY(st.down(xn.data, dxn, sizeof(float) * xd, g_hs.copy));
    TRY(st.down(cache->router_probs, dprobs, sizeof(float) * (size_t)T * E, g_hs.copy));
    TRY(st.down(cache->expert_ids, dids, sizeof(int) * (size_t)T * k, g_hs.copy));
    TRY(st.down(fo.data, dout, sizeof(float) * xd, g_stream));
    TRY(st.finish());
    // Residual 2 (src/transformer.c:767, mat_add_inplace).
    for (size_t i = 0; i < xd; ++i) x->data[i] = x->data[i] + fo.data[i];
    return MOE_HIP_OK;
}

void moe_block_ffn(Matrix *x, const float *rms_ffn, const MoEWeights *w, const ModelConfig *cfg,
                   ForwardCache *cache) {
    die_on(moe_hip_block_ffn(x, rms_ffn, w, cfg, cache), "moe_block_ffn");
}

int moe_hip_dev_alloc(void **ptr, size_t bytes) {
    if (!ptr) return set_err(MOE_HIP_ERR_ARG, "null out-pointer");
    *ptr = nullptr;
    TRY(ensure_init());
    HIP_TRY(hipMalloc(ptr, bytes ? bytes : 1));
    return MOE_HIP_OK;
}

int moe_hip_dev_free(void *ptr) {
    if (!ptr) return MOE_HIP_OK;
    HIP_TRY(hipFree(ptr));
    return MOE_HIP_OK;
}

int moe_hip_memcpy(void *dst, const void *src, size_t bytes, int kind) {
    TRY(ensure_init());
    if (bytes == 0) return MOE_HIP_OK;
    if (!dst || !src) return set_err(MOE_HIP_ERR_ARG, "null pointer");
    hipMemcpyKind k = kind == 1 ? hipMemcpyHostToDevice
                    : kind == 2 ? hipMemcpyDeviceToHost
                    : kind == 3 ? hipMemcpyDeviceToDevice : hipMemcpyDefault;
    if (kind < 1 || kind > 3) return set_err(MOE_HIP_ERR_ARG, "bad copy kind %d", kind);
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, k, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

int moe_hip_memset(void *ptr, int value, size_t bytes) {
    TRY(ensure_init());
    if (bytes == 0) return MOE_HIP_OK;
    if (!ptr) return set_err(MOE_HIP_ERR_ARG, "null pointer");
    HIP_TRY(hipMemsetAsync(ptr, value, bytes, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

int moe_hip_synchronize(void) {
    TRY(ensure_init());
    HIP_TRY(hipStreamSynchronize(g_stream));
    return MOE_HIP_OK;
}

}  // extern "C"

struct MoeHipGraph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int moe_hip_graph_begin(void *stream) {
    TRY(ensure_init());
    hipStream_t s = pick_stream(stream);
    HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    g_api_capture = true;
    return MOE_HIP_OK;
}

int moe_hip_graph_end(void *stream, void **graph) {
    if (!graph) return set_err(MOE_HIP_ERR_ARG, "null graph out-pointer");
    *graph = nullptr;
    MoeHipGraph *G = new MoeHipGraph();
    hipError_t e = hipStreamEndCapture(pick_stream(stream), &G->graph);
    g_api_capture = false;
    if (e == hipSuccess) e = hipGraphInstantiate(&G->exec, G->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (G->graph) (void)hipGraphDestroy(G->graph);
        delete G;
        return set_err(MOE_HIP_ERR_HIP, "graph capture: %s", hipGetErrorString(e));
    }
    ++g_live_graphs;   // (the workspace stays where it is until the graph is destroyed)
    *graph = G;
    return MOE_HIP_OK;
}

int moe_hip_graph_launch(void *graph, void *stream) {
    if (!graph) return set_err(MOE_HIP_ERR_ARG, "null graph");
    HIP_TRY(hipGraphLaunch(static_cast<MoeHipGraph *>(graph)->exec, pick_stream(stream)));
    return MOE_HIP_OK;
}

int moe_hip_graph_destroy(void *graph) {
    if (!graph) return MOE_HIP_OK;
    MoeHipGraph *G = static_cast<MoeHipGraph *>(graph);
    if (G->exec) (void)hipGraphExecDestroy(G->exec);
    if (G->graph) (void)hipGraphDestroy(G->graph);
    delete G;
    if (g_live_graphs > 0) --g_live_graphs;
    return MOE_HIP_OK;
}

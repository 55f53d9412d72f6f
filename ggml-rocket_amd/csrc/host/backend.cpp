// SPDX-License-Identifier: MIT
// The backend instance: the device and its stream, the HBM weight cache, the graph_compute
// node loop and its three op handlers, the per-route circuit breaker, the CPU fallback and the
// counters. The reference's equivalents: context 322-692, graph_compute 7050-7200, MUL_MAT
// 4548-4871 (+ fused groups 4873-5160), FLASH_ATTN_EXT 5444-5691, MUL_MAT_ID 6651-6944, free
// 5172-5326, breaker 263-307 (all ggml-rocket.cpp).
//
// Data flow (the host-buffer contract, ggml-rocket.cpp:7326-7331): tensors live in host memory;
// each claimed op uploads its activations, runs on the device and writes dst back before
// graph_compute returns. Large copies go through pinned staging slots, filled and drained by
// n_threads copy workers while the DMA engine moves the neighbouring chunk. Weights are uploaded once into the HBM weight cache, keyed by
// weight_key (name + content fingerprint), in the layout the kernels read:
//   F16 / Q4_K / Q5_K   the ggml payload as-is;   Q4_0 / Q8_0 / Q6_K / MXFP4   split into aligned planes;
//   F32 / BF16   converted to fp16;        QUANT_RESIDENT=1   quant weights decoded to fp16.

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../../include/mi355x_kernels.h"
#include "host.h"

using namespace mxh;

namespace {

// ---- route health (the contract of ggml-rocket.cpp:263-307) ---------------------------------
// Each route group keeps a failure streak. When the streak reaches kTrip the route "rests": the
// CPU fallback serves the next rest_len() calls without a device attempt, then one call tries
// the device again. Every trip in a row (a failed retry adds one) doubles the rest, from 64
// calls up to a ceiling of 4096; a device success ends the streak and forgets the trips. A
// status that only says the shape or type is not taken (MI355X_E_ARG, MI355X_E_UNSUPPORTED)
// leaves the record as it is.
class RouteHealth {
public:
    static constexpr int kTrip = 3;
    static constexpr int kRestShift0 = 6;     // first rest: 1 << 6 = 64 calls
    static constexpr int kRestShiftMax = 12;  // longest rest: 1 << 12 = 4096 calls

    // false while the route rests (the call is counted as bypassed)
    bool try_device() {
        if (resting_ == 0) return true;
        resting_--;
        bypassed++;
        return false;
    }

    void record(int status, const char * route) {
        if (status == MI355X_OK) {
            streak_ = 0;
            trips_ = 0;
            return;
        }
        if (status == MI355X_E_ARG || status == MI355X_E_UNSUPPORTED) return;
        failures++;
        if (++streak_ < kTrip) return;
        trips_++;
        resting_ = rest_len();
        logw("%s failed on the device %d times running (status %d); the CPU serves its next %ld "
             "calls before the device is tried again\n", route, streak_, status, resting_);
    }

    long attempts = 0, failures = 0, bypassed = 0;
    int inject = 0;   // host-side fault injection for tests: the next `inject` attempts fail

private:
    long rest_len() const {
        const int shift = std::min(kRestShift0 + trips_ - 1, kRestShiftMax);
        return 1L << shift;
    }
    int streak_ = 0;    // device failures since the last success
    int trips_ = 0;     // rests entered since the last success
    long resting_ = 0;  // calls left in the current rest
};

// A grow-only device buffer.
struct DevBuf {
    void * p = nullptr;
    size_t cap = 0;
    int ensure(size_t n) {
        if (n <= cap) return MI355X_OK;
        if (p) {
            (void)hipDeviceSynchronize();   // queued work may still read the old buffer
            (void)hipFree(p);
        }
        p = nullptr;
        cap = 0;
        const size_t want = (n + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
        if (hipMalloc(&p, want) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            return MI355X_E_DEVICE;
        }
        cap = want;
        return MI355X_OK;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

// Host copy workers: one memcpy (or any job over disjoint parts) split across n threads, the
// caller being one of them. Persistent threads, because a copy of one staging chunk takes about
// as long as starting a thread.
class CopyPool {
public:
    explicit CopyPool(int n, size_t min_part) : min_part_(min_part) {
        for (int i = 1; i < n; i++) th_.emplace_back([this] { work(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto & t : th_) t.join();
    }
    int threads() const { return (int)th_.size() + 1; }
    // part(i) for i in [0, parts), spread over the workers and the calling thread
    void run(int parts, const std::function<void(int)> & part) {
        if (th_.empty() || parts <= 1) {
            for (int i = 0; i < parts; i++) part(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            job_ = &part;
            parts_ = parts;
            next_.store(0);
            left_ = parts;
            gen_++;
        }
        cv_.notify_all();
        drain();
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [this] { return left_ == 0; });
        job_ = nullptr;
    }
    void copy(void * dst, const void * src, size_t n) {
        const int parts = (int)std::min<size_t>((size_t)threads(), (n + min_part_ - 1) / min_part_);
        const size_t per = ((n + parts - 1) / parts + 63) & ~(size_t)63;
        run(parts, [&](int i) {
            const size_t o = (size_t)i * per;
            if (o < n) memcpy((char *)dst + o, (const char *)src + o, std::min(per, n - o));
        });
    }

private:
    void drain() {
        for (;;) {
            const int i = next_.fetch_add(1);
            if (i >= parts_) return;
            (*job_)(i);
            std::lock_guard<std::mutex> lk(mu_);
            if (--left_ == 0) done_.notify_all();
        }
    }
    void work() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            drain();
        }
    }
    const size_t min_part_;   // smallest part one worker copies
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    const std::function<void(int)> * job_ = nullptr;
    int parts_ = 0, left_ = 0;
    std::atomic<int> next_{0};
    uint64_t gen_ = 0;
    bool stop_ = false;
};

// Pinned staging for the host <-> device copies of graph_compute. Host tensors are pageable
// (ggml's CPU buffers), and a copy from pageable memory crawls through the runtime's own small
// bounce buffer. A large copy is cut into CHUNK-sized pieces that cycle through NSLOT pinned
// slots: the copy workers fill (or drain) one slot while the DMA engine moves another. Slots are
// reused only after the event of their last DMA has completed, and the ring continues from one
// copy to the next. Measured on the 8B-shape layer's transfers (8-60 MB operands): chunks of 2 to
// 16 MB and 4 to 8 slots perform alike (within 5%); below 2 MB, or with copy parts under 512 KB,
// the per-chunk wake-ups of the copy workers and event waits cost more than the overlap gains.
struct Stager {
    static constexpr int MAX_SLOT = 16;
    size_t CHUNK = (size_t)8 << 20;   // MI355X_STAGE_CHUNK_KB overrides (tuning)
    int NSLOT = 4;                    // MI355X_STAGE_SLOTS overrides (tuning), <= MAX_SLOT
    void * slot[MAX_SLOT] = {};
    hipEvent_t ev[MAX_SLOT] = {};
    bool pending[MAX_SLOT] = {};
    int next = 0;    // the slot the next chunk of an upload takes
    bool ready = false;
    int init() {
        if (ready) return MI355X_OK;
        if (const char * e = getenv("MI355X_STAGE_CHUNK_KB")) {
            const long v = atol(e);
            if (v >= 64 && v <= (64 << 10)) CHUNK = (size_t)v << 10;
        }
        if (const char * e = getenv("MI355X_STAGE_SLOTS")) {
            const int v = atoi(e);
            if (v >= 2 && v <= MAX_SLOT) NSLOT = v;
        }
        for (int i = 0; i < NSLOT; i++) {
            if (hipHostMalloc(&slot[i], CHUNK, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                release();
                return MI355X_E_DEVICE;
            }
        }
        ready = true;
        return MI355X_OK;
    }
    // wait until slot i's last DMA is done
    int settle(int i) {
        if (!pending[i]) return MI355X_OK;
        pending[i] = false;
        return hipEventSynchronize(ev[i]) == hipSuccess ? MI355X_OK : MI355X_E_DEVICE;
    }
    void release() {
        for (int i = 0; i < MAX_SLOT; i++) {
            if (pending[i] && ev[i]) (void)hipEventSynchronize(ev[i]);
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            if (slot[i]) (void)hipHostFree(slot[i]);
            slot[i] = nullptr;
            ev[i] = nullptr;
            pending[i] = false;
        }
        ready = false;
    }
};

struct WEntry {
    void * dev = nullptr;
    size_t bytes = 0;
    int dev_type = 0;   // layout the kernels read: F16, F16_T, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K or MXFP4
    int64_t rows = 0, K = 0;
};

// What the weight cache did with the weights offered to it, per use: the fp16 image of a MUL_MAT
// weight (F16 / F32 / BF16 weights, and quantized ones under QUANT_RESIDENT), its quantized HBM
// layout (decoded in the GEMM on every call), and MUL_MAT_ID expert stacks. Reported at free():
// a run whose cache filled up early reads exactly like one that held everything, except here.
enum WeightUse { USE_F16 = 0, USE_QUANT = 1, USE_MOE = 2, N_USES = 3 };
struct CacheOutcome {
    long hits = 0, fills = 0, per_call = 0, nokey_calls = 0;
    size_t bytes = 0;                             // resident bytes of this use
    std::unordered_set<std::string> streamed;     // keys that ran from per-call scratch
    std::string first_decline;                    // why the first weight was turned away
    size_t used_at_decline = 0;                   // cache bytes at that moment
};

const uint64_t GUID[2] = {0x4d49333535584d49ULL, 0x2d70726566696c6cULL};

}  // namespace

struct mi355x_backend {
    uint64_t guid[2] = {GUID[0], GUID[1]};
    int n_threads = 5;
    bool started = false;
    // The device copy of a FLASH_ATTN_EXT dst written back in this graph_compute call (the fa_o
    // buffer): a MUL_MAT later in the call whose src1 is exactly those host bytes (O reading the
    // attention through a view) reads them from here instead of uploading them again. Cleared
    // at the start of each call and at each FLASH_ATTN_EXT; not used in a call where another
    // node's dst overlaps an attention's dst (mirror_ok).
    bool mirror_ok = false;
    struct {
        const void * host = nullptr;
        size_t bytes = 0;
        const void * dev = nullptr;
    } fa_mirror;
    int quant_resident = -1;   // -1: the QUANT_RESIDENT knob; 0 / 1: this instance's choice

    bool dev_checked = false, dev_ok = false;
    hipStream_t stream = nullptr;

    DevBuf act, a16, scales, out, part, wstage, wconv, fa_q, fa_k, fa_v, fa_m, fa_o, fa_ws, moe_b, moe_ids, moe_o, moe_ws;
    DevBuf wscratch[4], moe_wscratch;   // per-call weights: unnamed, or over the cache budget
    DevBuf w16;                         // the decode-first form's tiled fp16 weights of one call

    std::unordered_map<std::string, WEntry> wcache;
    size_t cache_used = 0, cache_budget = 0;
    CacheOutcome outcome[N_USES];

    std::map<std::string, long> routes;
    long n_cpu_fallbacks = 0;
    long moe_resident = 0, moe_streamed = 0;
    std::unordered_set<std::string> moe_claimed;
    std::unordered_set<std::string> moe_counted;   // stacks whose experts were counted resident
    std::unordered_set<std::string> moe_streamed_experts;   // "<stack key>/e<index>" run from an upload

    RouteHealth brk_gemm, brk_fa, brk_moe;

    Stager stage;                        // pinned slots of the host <-> device copies
    std::unique_ptr<CopyPool> pool;      // n_threads copy workers, started with the device
};

namespace {

using Ctx = mi355x_backend;

bool ensure_device(Ctx * c) {
    if (c->dev_checked) return c->dev_ok;
    c->dev_checked = true;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        logw("no HIP device: every claimed op will run on the CPU fallback\n");
        return false;
    }
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        c->stream = nullptr;
        return false;
    }
    size_t fr = 0, tot = 0;
    (void)hipMemGetInfo(&fr, &tot);
    size_t b = 0;
    const char * e = knob_env("CACHE_MB");
    if (e && parse_mb(e, &b)) c->cache_budget = b ? b : (size_t)-1;
    else c->cache_budget = fr > ((size_t)16 << 30) ? fr - ((size_t)16 << 30) : fr / 2;
    c->dev_ok = true;
    return true;
}

int sync(Ctx * c) {
    return hipStreamSynchronize(c->stream) == hipSuccess ? MI355X_OK : MI355X_E_DEVICE;
}

#define TRY_RC(x) do { const int _r = (x); if (_r != MI355X_OK) return _r; } while (0)

// Copies below STAGE_MIN bytes go straight from pageable memory (the runtime's path is fine
// there); larger ones through the pinned slots.
constexpr size_t STAGE_MIN = (size_t)1 << 20;

bool staging_on(Ctx * c) {
    if (!c->pool) {
        size_t part = (size_t)1 << 20;   // MI355X_COPY_PART_KB overrides (tuning)
        if (const char * e = getenv("MI355X_COPY_PART_KB")) {
            const long v = atol(e);
            if (v >= 16 && v <= (64 << 10)) part = (size_t)v << 10;
        }
        c->pool.reset(new CopyPool(c->n_threads, part));
    }
    return c->stage.init() == MI355X_OK;
}

// host -> device, enqueued on the stream; the host buffer may be reused once this returns
int h2d(Ctx * c, void * dst, const void * src, size_t n) {
    if (!n) return MI355X_OK;
    if (n < STAGE_MIN || !staging_on(c))
        return hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream) == hipSuccess ? MI355X_OK
                                                                                          : MI355X_E_DEVICE;
    Stager & S = c->stage;
    for (size_t o = 0; o < n; o += S.CHUNK) {
        const int k = S.next;
        S.next = (S.next + 1) % S.NSLOT;
        const size_t len = std::min(S.CHUNK, n - o);
        TRY_RC(S.settle(k));
        c->pool->copy(S.slot[k], (const char *)src + o, len);
        if (hipMemcpyAsync((char *)dst + o, S.slot[k], len, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
            hipEventRecord(S.ev[k], c->stream) != hipSuccess)
            return MI355X_E_DEVICE;
        S.pending[k] = true;
    }
    return MI355X_OK;
}

// Rows [0, rows) of a device matrix with row pitch `pitch` bytes, `width` bytes used per row,
// to host memory through the pinned slots, handing each landed block of rows to `take(r0, r1,
// host_rows)` (host_rows = the staged rows, `width` bytes apart). Returns when all rows are in.
int d2h_rows(Ctx * c, const void * src, size_t pitch, size_t width, int64_t rows,
             const std::function<void(int64_t, int64_t, const char *)> & take) {
    Stager & S = c->stage;
    const int64_t per = std::max<int64_t>(1, (int64_t)(S.CHUNK / width));
    const int64_t nchunk = (rows + per - 1) / per;
    auto launch = [&](int64_t i) -> int {
        const int k = (int)(i % S.NSLOT);
        const int64_t r0 = i * per, r1 = std::min(rows, r0 + per);
        const hipError_t e = pitch == width
            ? hipMemcpyAsync(S.slot[k], (const char *)src + r0 * pitch, (size_t)(r1 - r0) * width,
                             hipMemcpyDeviceToHost, c->stream)
            : hipMemcpy2DAsync(S.slot[k], width, (const char *)src + r0 * pitch, pitch, width, (size_t)(r1 - r0),
                               hipMemcpyDeviceToHost, c->stream);
        if (e != hipSuccess || hipEventRecord(S.ev[k], c->stream) != hipSuccess) return MI355X_E_DEVICE;
        S.pending[k] = true;
        return MI355X_OK;
    };
    for (int64_t i = 0; i < std::min<int64_t>(nchunk, S.NSLOT); i++) TRY_RC(launch(i));
    for (int64_t i = 0; i < nchunk; i++) {
        const int k = (int)(i % S.NSLOT);
        TRY_RC(S.settle(k));
        const int64_t r0 = i * per, r1 = std::min(rows, r0 + per);
        take(r0, r1, (const char *)S.slot[k]);
        if (i + S.NSLOT < nchunk) TRY_RC(launch(i + S.NSLOT));
    }
    return MI355X_OK;
}

// device -> host; returns when the bytes are in `dst` (it synchronizes on the copies)
int d2h(Ctx * c, void * dst, const void * src, size_t n) {
    if (!n) return MI355X_OK;
    if (n < STAGE_MIN || !staging_on(c)) {
        if (hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream) != hipSuccess) return MI355X_E_DEVICE;
        return hipStreamSynchronize(c->stream) == hipSuccess ? MI355X_OK : MI355X_E_DEVICE;
    }
    const size_t W = 1 << 16;   // stage as rows of 64 KB (+ one short tail)
    const int64_t full = (int64_t)(n / W);
    TRY_RC(d2h_rows(c, src, W, W, full, [&](int64_t r0, int64_t r1, const char * h) {
        c->pool->copy((char *)dst + r0 * W, h, (size_t)(r1 - r0) * W);
    }));
    if (n % W) {
        if (hipMemcpyAsync((char *)dst + full * W, (const char *)src + full * W, n % W, hipMemcpyDeviceToHost,
                           c->stream) != hipSuccess)
            return MI355X_E_DEVICE;
        return hipStreamSynchronize(c->stream) == hipSuccess ? MI355X_OK : MI355X_E_DEVICE;
    }
    return MI355X_OK;
}

#define TRY(x) do { const int _rc = (x); if (_rc != MI355X_OK) return _rc; } while (0)

// The device layout a weight of ggml type `t` is read in: fp16 for F16 / F32 / BF16 weights, for
// quantized ones when the resident-fp16 form is asked for, and for the types only a registered
// host decoder reads; the quantized HBM layout otherwise. The fp16 form is the tiled one (MI355X_F16_T, the GEMM's fastest input) when the
// caller reads it through mi355x_gemm (`tiled_ok`) and K % 64 == 0; row-major otherwise (the
// expert kernel of MUL_MAT_ID reads rows).
int dev_layout(int t, bool want_f16, bool tiled_ok, int64_t K) {
    if (want_f16 || !device_weight_type(t) || t == MI355X_TYPE_F16 || t == MI355X_TYPE_F32 || t == MI355X_TYPE_BF16)
        return (tiled_ok && K % 64 == 0) ? MI355X_F16_T : MI355X_F16;
    return t;   // Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4
}

// Builds the device form `lay` of `rows` rows of K values of ggml type `t` (host bytes `src`) at
// `dst`. Uses wstage / wconv as staging.
int build_weight(Ctx * c, int t, const void * src, int64_t rows, int64_t K, int lay, void * dst) {
    if (!device_weight_type(t)) {
        // a type only ggml's registered decoder reads: rows to f32 on the host (the copy workers'
        // threads), then the f32 weight's path to fp16
        const mi355x_to_float_fn fn = host_to_float(t);
        const int64_t rb = row_bytes(t, K);
        if (!fn || rb < 0) return MI355X_E_UNSUPPORTED;
        std::vector<float> f((size_t)rows * (size_t)K);
        const int nt = (int)std::max<int64_t>(1, std::min<int64_t>(c->n_threads, rows / 16));
        std::vector<std::thread> th;
        for (int i = 0; i < nt; i++)
            th.emplace_back([&, i] {
                for (int64_t r = i; r < rows; r += nt)
                    fn((const uint8_t *)src + r * rb, f.data() + (size_t)r * (size_t)K, K);
            });
        for (auto & x : th) x.join();
        return build_weight(c, MI355X_TYPE_F32, f.data(), rows, K, lay, dst);
    }
    const size_t raw = (size_t)row_bytes(t, K) * (size_t)rows;
    if ((t == MI355X_TYPE_F16 || t == MI355X_TYPE_Q4_K || t == MI355X_TYPE_Q5_K) && lay == t) return h2d(c, dst, src, raw);
    TRY(c->wstage.ensure(raw));
    TRY(h2d(c, c->wstage.p, src, raw));
    if (t == MI355X_TYPE_F32 || t == MI355X_TYPE_BF16) {
        if (lay == MI355X_F16) return mi355x_convert_f16(t, c->wstage.p, rows * K, (uint16_t *)dst, c->stream);
        TRY(c->wconv.ensure((size_t)rows * K * 2));
        TRY(mi355x_convert_f16(t, c->wstage.p, rows * K, (uint16_t *)c->wconv.p, c->stream));
        return mi355x_weight_f16_tiled(MI355X_F16, c->wconv.p, rows, K, (uint16_t *)dst, c->stream);
    }
    if (lay == MI355X_Q4_K_X) return mi355x_weight_pack(lay, c->wstage.p, rows, K, dst, c->stream);
    if (lay != MI355X_F16 && lay != MI355X_F16_T) return mi355x_weight_pack(t, c->wstage.p, rows, K, dst, c->stream);
    // -> fp16: from the HBM layout, built first when that differs from the ggml one
    const void * q = c->wstage.p;
    if (t == MI355X_TYPE_Q4_0 || t == MI355X_TYPE_Q8_0 || t == MI355X_TYPE_Q6_K || t == MI355X_TYPE_MXFP4) {
        TRY(c->wconv.ensure(raw));
        TRY(mi355x_weight_pack(t, c->wstage.p, rows, K, c->wconv.p, c->stream));
        q = c->wconv.p;
    }
    if (lay == MI355X_F16_T) return mi355x_weight_f16_tiled(t, q, rows, K, (uint16_t *)dst, c->stream);
    return mi355x_weight_dequant_f16(t, q, rows, K, (uint16_t *)dst, c->stream);
}

// A weight in device form: from the cache, or built into it, or (no key / over budget) built
// into per-call scratch. `resident` tells which.
int get_weight(Ctx * c, const mi355x_tensor * a, int64_t rows, int64_t K, bool want_f16, bool tiled_ok,
               int64_t moe_n, DevBuf & scratch, WEntry & out, bool & resident) {
    const bool moe = moe_n > 0;   // an expert stack of experts with moe_n rows each
    int lay = dev_layout(a->type, want_f16, tiled_ok, K);
    // Q4_K experts of whole 32-row groups take the regrouped layout, whose 32-row slabs the
    // expert GEMM loads as contiguous bytes
    if (moe && lay == MI355X_Q4_K && moe_n % 32 == 0) lay = MI355X_Q4_K_X;
    const int64_t dbytes = mi355x_weight_bytes(lay, rows, K);
    if (dbytes < 0) return MI355X_E_ARG;
    CacheOutcome & oc = c->outcome[moe ? USE_MOE : (lay == MI355X_F16 || lay == MI355X_F16_T) ? USE_F16 : USE_QUANT];
    std::string key = weight_key(a);
    if (key.empty()) oc.nokey_calls++;
    if (!key.empty()) {
        key += "|L" + std::to_string(lay);
        auto it = c->wcache.find(key);
        if (it != c->wcache.end() && it->second.rows == rows && it->second.K == K && it->second.dev_type == lay) {
            out = it->second;
            resident = true;
            oc.hits++;
            return MI355X_OK;
        }
        const bool fits = c->cache_used + (size_t)dbytes <= c->cache_budget;
        if (!fits && oc.first_decline.empty()) {
            char why[160];
            snprintf(why, sizeof why, "%.1f MB more would pass the %.0f MB budget", (double)dbytes / (1 << 20),
                     (double)c->cache_budget / (1 << 20));
            oc.first_decline = why;
            oc.used_at_decline = c->cache_used;
        }
        if (fits) {
            void * p = nullptr;
            if (hipMalloc(&p, (size_t)dbytes) != hipSuccess && oc.first_decline.empty()) {
                char why[160];
                snprintf(why, sizeof why, "the device allocation of %.1f MB failed", (double)dbytes / (1 << 20));
                oc.first_decline = why;
                oc.used_at_decline = c->cache_used;
            }
            if (p) {
                const int rc = build_weight(c, a->type, a->data, rows, K, lay, p);
                if (rc != MI355X_OK) {
                    (void)hipFree(p);
                    return rc;
                }
                WEntry e;
                e.dev = p;
                e.bytes = (size_t)dbytes;
                e.dev_type = lay;
                e.rows = rows;
                e.K = K;
                c->wcache[key] = e;
                c->cache_used += e.bytes;
                oc.fills++;
                oc.bytes += e.bytes;
                out = e;
                resident = true;
                return MI355X_OK;
            }
            (void)hipGetLastError();
        }
        oc.streamed.insert(key);
    }
    oc.per_call++;
    TRY(scratch.ensure((size_t)dbytes));
    TRY(build_weight(c, a->type, a->data, rows, K, lay, scratch.p));
    out.dev = scratch.p;
    out.bytes = (size_t)dbytes;
    out.dev_type = lay;
    out.rows = rows;
    out.K = K;
    resident = false;
    return MI355X_OK;
}

// ---- MUL_MAT (one node or a fused group sharing src1) ---------------------------------------
int mul_mat_device(Ctx * c, const std::vector<mi355x_tensor *> & grp, bool want_f16, bool & all_resident) {
    if (!ensure_device(c)) return MI355X_E_DEVICE;
    const mi355x_tensor * b = grp[0]->src[1];
    const int64_t K = b->ne[0], M = b->ne[1] * b->ne[2] * b->ne[3];
    TRY(c->act.ensure((size_t)M * K * 4));
    TRY(c->a16.ensure((size_t)((M + 15) / 16 * 16) * K * 2));
    TRY(c->scales.ensure((size_t)M * 4));
    int64_t ntot = 0;
    for (auto * d : grp) ntot += d->src[0]->ne[1];
    TRY(c->out.ensure((size_t)M * ntot * 4));
    std::vector<WEntry> ws(grp.size());
    all_resident = true;
    mi355x_gemm_out outs[4];
    int64_t col = 0;
    for (size_t i = 0; i < grp.size(); i++) {
        const mi355x_tensor * a = grp[i]->src[0];
        bool res = false;
        TRY(get_weight(c, a, a->ne[1], K, want_f16, true, 0, c->wscratch[i], ws[i], res));
        all_resident = all_resident && res;
        outs[i].w_dev = ws[i].dev;
        outs[i].rows_total = a->ne[1];
        outs[i].row0 = 0;
        outs[i].N = a->ne[1];
        outs[i].c_dev = (float *)c->out.p + col;
        outs[i].ldc = ntot;
        col += a->ne[1];
    }
    // Q8_0 / Q6_K weights at the shapes where one decode pass plus the fp16 GEMM is faster than
    // decoding inside the GEMM: each member decoded into tiled fp16 scratch first
    int gtype = ws[0].dev_type;
    bool same = true;
    for (auto & w : ws) same = same && w.dev_type == gtype;
    if (same && mi355x_mul_mat_decode_first(gtype, M, ntot, K) == 1) {
        std::vector<size_t> off(grp.size() + 1, 0);
        for (size_t i = 0; i < grp.size(); i++)
            off[i + 1] = off[i] + (((size_t)mi355x_weight_bytes(MI355X_F16_T, outs[i].N, K) + 255) & ~(size_t)255);
        TRY(c->w16.ensure(off.back()));
        for (size_t i = 0; i < grp.size(); i++) {
            uint16_t * w16 = (uint16_t *)((char *)c->w16.p + off[i]);
            TRY(mi355x_weight_f16_tiled(gtype, outs[i].w_dev, outs[i].N, K, w16, c->stream));
            outs[i].w_dev = w16;
        }
        gtype = MI355X_F16_T;
    }
    // K-split partials, summed in a fixed order (reproducible results); a two-way split adds
    // into the outputs, which the activation pack then clears in the same launch
    const size_t pbytes = mi355x_gemm_workspace(gtype, M, K, outs, (int)grp.size());
    if (pbytes) TRY(c->part.ensure(pbytes));
    const int acc = mi355x_gemm_accumulates(gtype, M, K, outs, (int)grp.size(), pbytes);
    if (acc < 0) return acc;
    // src1 from the attention this call just computed (same host bytes, row-major F32): its
    // device copy; otherwise uploaded
    const float * act = (const float *)c->act.p;
    const bool dense = b->type == MI355X_TYPE_F32 && b->nb[0] == 4 && b->nb[1] == (size_t)K * 4 &&
                       b->nb[2] == b->nb[1] * (size_t)b->ne[1] && b->nb[3] == b->nb[2] * (size_t)b->ne[2];
    if (dense && c->fa_mirror.dev && b->data == c->fa_mirror.host && (size_t)M * K * 4 <= c->fa_mirror.bytes)
        act = (const float *)c->fa_mirror.dev;
    else
        TRY(h2d(c, c->act.p, b->data, (size_t)M * K * 4));
    const int tiled = gtype == MI355X_F16_T;
    if (acc)   // the outputs are the ntot columns of c->out
        TRY(mi355x_pack_act_clear(tiled, act, K, M, K, (uint16_t *)c->a16.p, (float *)c->scales.p, (float *)c->out.p,
                                  ntot, ntot, c->stream));
    else if (tiled)
        TRY(mi355x_pack_act_tiled(act, K, M, K, (uint16_t *)c->a16.p, (float *)c->scales.p, c->stream));
    else
        TRY(mi355x_pack_act(act, K, M, K, (uint16_t *)c->a16.p, (float *)c->scales.p, c->stream));
    TRY(mi355x_gemm_ws(gtype, (const uint16_t *)c->a16.p, (const float *)c->scales.p, M, K, outs,
                       (int)grp.size(), pbytes ? c->part.p : nullptr, pbytes, acc ? MI355X_GEMM_OUT_ZEROED : 0,
                       c->stream));
    // dst[i] is [N_i, M] contiguous: one member takes the output as is; a group's outputs come
    // back as whole rows of the concatenated [M][ntot] and are split into the members' column
    // blocks on the host
    if (grp.size() == 1) {
        TRY(d2h(c, grp[0]->data, c->out.p, (size_t)M * ntot * 4));
        return sync(c);
    }
    if ((size_t)M * ntot * 4 < STAGE_MIN || !staging_on(c) || (size_t)ntot * 4 > c->stage.CHUNK) {
        col = 0;
        for (auto * d : grp) {
            const int64_t N = d->src[0]->ne[1];
            if (hipMemcpy2DAsync(d->data, (size_t)N * 4, (const float *)c->out.p + col, (size_t)ntot * 4,
                                 (size_t)N * 4, (size_t)M, hipMemcpyDeviceToHost, c->stream) != hipSuccess)
                return MI355X_E_DEVICE;
            col += N;
        }
        return sync(c);
    }
    TRY(d2h_rows(c, c->out.p, (size_t)ntot * 4, (size_t)ntot * 4, M, [&](int64_t r0, int64_t r1, const char * h) {
        const int64_t nr = r1 - r0;
        const int parts = (int)std::min<int64_t>(c->pool->threads(), nr);
        c->pool->run(parts, [&](int pi) {
            for (int64_t r = r0 + nr * pi / parts; r < r0 + nr * (pi + 1) / parts; r++) {
                int64_t cc = 0;
                for (auto * d : grp) {
                    const int64_t N = d->src[0]->ne[1];
                    memcpy((char *)d->data + (size_t)r * N * 4, h + (size_t)(r - r0) * ntot * 4 + (size_t)cc * 4,
                           (size_t)N * 4);
                    cc += N;
                }
            }
        });
    }));
    return sync(c);
}

// ---- FLASH_ATTN_EXT ---------------------------------------------------------------------------
int flash_attn_device(Ctx * c, mi355x_tensor * dst) {
    if (!ensure_device(c)) return MI355X_E_DEVICE;
    const mi355x_tensor * q = dst->src[0];
    const mi355x_tensor * k = dst->src[1];
    const mi355x_tensor * v = dst->src[2];
    const mi355x_tensor * m = dst->src[3];
    const size_t qb = nbytes(q), kb = nbytes(k), vb = nbytes(v), mb = m ? nbytes(m) : 0, ob = nbytes(dst);
    TRY(c->fa_q.ensure(qb));
    TRY(c->fa_k.ensure(kb));
    TRY(c->fa_v.ensure(vb));
    if (m) TRY(c->fa_m.ensure(mb));
    TRY(c->fa_o.ensure(ob));
    TRY(h2d(c, c->fa_q.p, q->data, qb));
    TRY(h2d(c, c->fa_k.p, k->data, kb));
    TRY(h2d(c, c->fa_v.p, v->data, vb));
    if (m) TRY(h2d(c, c->fa_m.p, m->data, mb));
    mi355x_fa_args a;
    memset(&a, 0, sizeof a);
    a.q_dev = (const float *)c->fa_q.p;
    a.q_nb1 = (int64_t)(q->nb[1] / 4);
    a.q_nb2 = (int64_t)(q->nb[2] / 4);
    a.k_dev = (const uint16_t *)c->fa_k.p;
    a.k_nb1 = (int64_t)(k->nb[1] / 2);
    a.k_nb2 = (int64_t)(k->nb[2] / 2);
    a.v_dev = (const uint16_t *)c->fa_v.p;
    a.v_nb1 = (int64_t)(v->nb[1] / 2);
    a.v_nb2 = (int64_t)(v->nb[2] / 2);
    a.mask_dev = m ? (const uint16_t *)c->fa_m.p : nullptr;
    a.mask_nb1 = m ? (int64_t)(m->nb[1] / 2) : 0;
    a.dst_dev = (float *)c->fa_o.p;
    a.dst_nb1 = (int64_t)(dst->nb[1] / 4);
    a.dst_nb2 = (int64_t)(dst->nb[2] / 4);
    a.D = (int)q->ne[0];
    a.DV = (int)v->ne[0];
    a.T = (int)q->ne[1];
    a.H = (int)q->ne[2];
    a.KV = (int)k->ne[1];
    a.HK = (int)k->ne[2];
    memcpy(&a.scale, &dst->op_params[0], 4);
    memcpy(&a.max_bias, &dst->op_params[1], 4);
    memcpy(&a.softcap, &dst->op_params[2], 4);
    const size_t ws = mi355x_flash_attn_workspace(&a, 0);
    if (ws) TRY(c->fa_ws.ensure(ws));
    TRY(mi355x_flash_attn(&a, 0, ws ? c->fa_ws.p : nullptr, ws, c->stream));
    TRY(d2h(c, dst->data, c->fa_o.p, ob));
    TRY(sync(c));
    if (c->mirror_ok) {
        c->fa_mirror.host = dst->data;
        c->fa_mirror.bytes = ob;
        c->fa_mirror.dev = c->fa_o.p;
    }
    return MI355X_OK;
}

// ---- MUL_MAT_ID -------------------------------------------------------------------------------
int mul_mat_id_device(Ctx * c, mi355x_tensor * dst, bool & resident) {
    if (!ensure_device(c)) return MI355X_E_DEVICE;
    const mi355x_tensor * as = dst->src[0];
    const mi355x_tensor * b = dst->src[1];
    const mi355x_tensor * ids = dst->src[2];
    const int64_t K = as->ne[0], N = as->ne[1], E = as->ne[2];
    const int64_t ne11 = b->ne[1], T = ids->ne[1], U = ids->ne[0];
    // the whole stack is one weight panel of E*N rows
    mi355x_tensor panel = *as;
    panel.ne[1] = N * E;
    panel.ne[2] = 1;
    WEntry w;
    TRY(get_weight(c, &panel, N * E, K, false, false, N, c->moe_wscratch, w, resident));
    const size_t bb = (size_t)T * ne11 * K * 4, ib = (size_t)T * U * 4, ob = (size_t)T * U * N * 4;
    TRY(c->moe_b.ensure(bb));
    TRY(c->moe_ids.ensure(ib));
    TRY(c->moe_o.ensure(ob));
    TRY(h2d(c, c->moe_b.p, b->data, bb));
    // ids may be a strided view: pack it to [T][U] on the host side of the copy
    std::vector<int32_t> idh((size_t)T * U);
    for (int64_t t = 0; t < T; t++)
        for (int64_t s = 0; s < U; s++)
            idh[t * U + s] = *(const int32_t *)((const char *)ids->data + t * ids->nb[1] + s * ids->nb[0]);
    TRY(h2d(c, c->moe_ids.p, idh.data(), ib));
    mi355x_moe_args a;
    memset(&a, 0, sizeof a);
    a.wtype = w.dev_type;
    a.as_dev = w.dev;
    a.n_expert = E;
    a.N = N;
    a.K = K;
    a.b_dev = (const float *)c->moe_b.p;
    a.ne11 = ne11;
    a.b_nb1 = K;
    a.b_nb2 = ne11 * K;
    a.ids_dev = (const int32_t *)c->moe_ids.p;
    a.n_used = U;
    a.ids_nb0 = 1;
    a.ids_nb1 = U;
    a.n_tokens = T;
    a.dst_dev = (float *)c->moe_o.p;
    a.dst_nb1 = N;
    a.dst_nb2 = U * N;
    const size_t ws = mi355x_mul_mat_id_workspace(&a);
    TRY(c->moe_ws.ensure(ws));
    TRY(mi355x_mul_mat_id(&a, c->moe_ws.p, ws, nullptr, c->stream));
    TRY(d2h(c, dst->data, c->moe_o.p, ob));
    return sync(c);
}

// Runs a device job under a breaker; on a device failure (or an open breaker) runs `fallback`.
template <class Dev, class Fb>
void guarded(Ctx * c, RouteHealth & brk, const char * route, Dev && dev, Fb && fallback) {
    int rc = MI355X_E_DEVICE;
    if (brk.try_device()) {
        brk.attempts++;
        if (brk.inject > 0) {
            brk.inject--;
            rc = MI355X_E_DEVICE;
        } else {
            rc = dev();
        }
        brk.record(rc, route);
    }
    if (rc != MI355X_OK) {
        fallback();
        c->n_cpu_fallbacks++;
    }
}

bool is_view_op(int op) {
    return op == MI355X_OP_NONE || op == MI355X_OP_RESHAPE || op == MI355X_OP_VIEW ||
           op == MI355X_OP_PERMUTE || op == MI355X_OP_TRANSPOSE;
}

bool fusable(const mi355x_tensor * n) {
    return n->op == MI355X_OP_MUL_MAT && n->src[0] && n->src[1] && n->src[0]->ne[2] == 1 && n->src[0]->ne[3] == 1;
}

}  // namespace

extern "C" {

MI355X_API const char * mi355x_backend_name(void) { return "MI355X"; }

MI355X_API const char * mi355x_backend_description(void) {
    static char desc[160];
    static std::once_flag once;
    std::call_once(once, [] {
        int n = 0, dev = 0, rt = 0;
        hipDeviceProp_t p;
        if (hipGetDeviceCount(&n) == hipSuccess && n > 0 && hipGetDevice(&dev) == hipSuccess &&
            hipGetDeviceProperties(&p, dev) == hipSuccess) {
            (void)hipRuntimeGetVersion(&rt);
            snprintf(desc, sizeof desc, "%s (%d CUs, HIP runtime %d)", p.gcnArchName, p.multiProcessorCount, rt);
        } else {
            (void)hipGetLastError();
            snprintf(desc, sizeof desc, "MI355X backend (no HIP device visible)");
        }
    });
    return desc;
}

MI355X_API void mi355x_backend_get_memory(size_t * fr, size_t * tot) {
    size_t f = 0, t = 0;
    int n = 0;
    if (!(hipGetDeviceCount(&n) == hipSuccess && n > 0 && hipMemGetInfo(&f, &t) == hipSuccess)) {
        (void)hipGetLastError();
        f = t = 0;
    }
    if (fr) *fr = f;
    if (tot) *tot = t;
}

MI355X_API mi355x_backend_t mi355x_backend_init(void) {
    Ctx * c = new Ctx();
    int nt = knob_int("N_THREADS", 5);
    c->n_threads = nt < 1 ? 1 : (nt > 8 ? 8 : nt);
    moe_preflight_open();
    return c;
}

MI355X_API bool mi355x_backend_is(mi355x_backend_t c) {
    return c && c->guid[0] == GUID[0] && c->guid[1] == GUID[1];
}

namespace {

// The teardown report of the weight cache, one block per use that saw any weight (same tags as
// the reference's outcome lines, ggml-rocket.cpp:5185-5303; counts and wording of this cache).
// Weights, not calls, except where a weight has no stable name to count it by.
void report_residency(const Ctx * c) {
    static const char * tag[N_USES] = {"[f16-resident]", "[dq-cache]", "[moe]"};
    static const char * form[N_USES] = {"the fp16 image", "the quantized layout", "the expert stack"};
    for (int u = 0; u < N_USES; u++) {
        const CacheOutcome & o = c->outcome[u];
        const long resident = o.fills, streamed = (long)o.streamed.size();
        if (resident + streamed + o.nokey_calls == 0) continue;
        const double pct = resident + streamed ? 100.0 * resident / (double)(resident + streamed) : 0.0;
        logi("%s %ld weights resident in HBM as %s (%.1f MB), %ld run from per-call uploads: %.0f%% resident; "
             "%ld cached calls, %ld per-call builds\n",
             tag[u], resident, form[u], (double)o.bytes / (1 << 20), streamed, pct, o.hits, o.per_call);
        if (!o.first_decline.empty())
            logi("%s first weight turned away at %.1f MB cached: %s\n", tag[u], (double)o.used_at_decline / (1 << 20),
                 o.first_decline.c_str());
        if (streamed && pct < 80.0)
            logw("%s only %.0f%% resident: every call of a weight outside the cache uploads and converts it again, "
                 "so this run measures the per-call path; raise MI355X_CACHE_MB if HBM allows\n", tag[u], pct);
        if (o.nokey_calls)
            logi("%s %ld calls had a weight with no stable name, which no cache budget can hold\n", tag[u],
                 o.nokey_calls);
    }
}

// The teardown line of the route counters (ops completed per route, CPU fallbacks), so a run
// through a host that cannot call the counter API (llama-bench) still shows where ops ran.
void report_routes(const Ctx * c) {
    long total = 0;
    std::string line;
    for (const auto & kv : c->routes) {
        if (!kv.second) continue;
        total += kv.second;
        line += " " + kv.first + "=" + std::to_string(kv.second);
    }
    if (total || c->n_cpu_fallbacks)
        logi("[routes] %ld ops on the device:%s; %ld recomputed on the CPU after a device failure\n", total,
             line.c_str(), c->n_cpu_fallbacks);
}

}  // namespace

MI355X_API void mi355x_backend_free(mi355x_backend_t c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    c->stage.release();
    c->pool.reset();
    for (auto & kv : c->wcache) (void)hipFree(kv.second.dev);
    report_residency(c);
    report_routes(c);
    c->wcache.clear();
    for (DevBuf * b : {&c->act, &c->a16, &c->scales, &c->out, &c->part, &c->wstage, &c->wconv, &c->fa_q, &c->fa_k, &c->fa_v,
                       &c->fa_m, &c->fa_o, &c->fa_ws, &c->moe_b, &c->moe_ids, &c->moe_o, &c->moe_ws,
                       &c->wscratch[0], &c->wscratch[1], &c->wscratch[2], &c->wscratch[3], &c->moe_wscratch})
        b->release();
    if (c->stream) (void)hipStreamDestroy(c->stream);
    for (const auto & k : c->moe_claimed) moe_preflight_release(k);
    moe_preflight_close();
    c->guid[0] = c->guid[1] = 0;
    delete c;
}

MI355X_API void mi355x_backend_set_n_threads(mi355x_backend_t c, int n) {
    if (!mi355x_backend_is(c)) return;
    if (c->started) {
        logw("set_n_threads(%d) after the first compute changes nothing\n", n);
        return;
    }
    if (n < 1 || n > 8) logw("set_n_threads(%d) clamped to 1..8\n", n);
    c->n_threads = n < 1 ? 1 : (n > 8 ? 8 : n);
}

MI355X_API void mi355x_backend_set_quant_resident(mi355x_backend_t c, int mode) {
    if (mi355x_backend_is(c)) c->quant_resident = mode < 0 ? -1 : (mode > 0 ? 1 : 0);
}

MI355X_API int mi355x_backend_get_n_threads(mi355x_backend_t c) {
    return mi355x_backend_is(c) ? c->n_threads : 0;
}

MI355X_API long mi355x_backend_route_ops(mi355x_backend_t c, const char * route) {
    if (!mi355x_backend_is(c)) return 0;
    if (!route) {
        long s = 0;
        for (const auto & kv : c->routes) s += kv.second;
        return s;
    }
    auto it = c->routes.find(route);
    return it == c->routes.end() ? 0 : it->second;
}

MI355X_API long mi355x_backend_cpu_fallbacks(mi355x_backend_t c) {
    return mi355x_backend_is(c) ? c->n_cpu_fallbacks : 0;
}

MI355X_API void mi355x_backend_moe_stats(mi355x_backend_t c, long * n_resident, long * n_streamed) {
    if (n_resident) *n_resident = mi355x_backend_is(c) ? c->moe_resident : 0;
    if (n_streamed) *n_streamed = mi355x_backend_is(c) ? c->moe_streamed : 0;
}

static RouteHealth * breaker_of(mi355x_backend_t c, const char * g) {
    if (!mi355x_backend_is(c) || !g) return nullptr;
    if (!strcmp(g, "gemm")) return &c->brk_gemm;
    if (!strcmp(g, "fa")) return &c->brk_fa;
    if (!strcmp(g, "moe")) return &c->brk_moe;
    return nullptr;
}

MI355X_API void mi355x_backend_route_stats(mi355x_backend_t c, const char * g, long * attempts,
                                                long * failures, long * bypassed) {
    RouteHealth * b = breaker_of(c, g);
    if (attempts) *attempts = b ? b->attempts : 0;
    if (failures) *failures = b ? b->failures : 0;
    if (bypassed) *bypassed = b ? b->bypassed : 0;
}

MI355X_API void mi355x_backend_inject_faults(mi355x_backend_t c, const char * g, int n) {
    RouteHealth * b = breaker_of(c, g);
    if (b) b->inject = n < 0 ? 0 : n;
}

static int graph_compute_nodes(mi355x_backend_t c, mi355x_tensor * const * nodes, int n_nodes);

// Repacked weights with registered original bytes (ggml-rocket.cpp:7005-7047): for this call,
// each such source descriptor reads the registered bytes (a view at its offset). Only the
// descriptors change, never the host's tensors, so a CPU split running meanwhile still reads its
// repacked copy. A source that needs bytes and has none fails the call before any route reads
// it; a view node reads nothing and does not count as a check of its source.
MI355X_API int mi355x_backend_graph_compute(mi355x_backend_t c, mi355x_tensor * const * nodes, int n_nodes) {
    if (!mi355x_backend_is(c) || (n_nodes > 0 && !nodes)) return MI355X_STATUS_FAILED;
    if (registered_sources() == 0) return graph_compute_nodes(c, nodes, n_nodes);
    struct Saved {
        mi355x_tensor * t;
        void * data;
        int32_t kind;
    };
    std::vector<Saved> swapped;
    std::unordered_set<const mi355x_tensor *> seen;
    auto restore = [&] {
        for (auto it = swapped.rbegin(); it != swapped.rend(); ++it) {
            it->t->data = it->data;
            it->t->buffer_kind = it->kind;
        }
    };
    for (int i = 0; i < n_nodes; i++) {
        mi355x_tensor * node = nodes[i];
        if (!node || node->op == MI355X_OP_NONE || is_view_op(node->op)) continue;
        for (int j = 0; j < MI355X_MAX_SRC; j++) {
            mi355x_tensor * s = node->src[j];
            if (!s || !tensor_needs_source(s) || !seen.insert(s).second) continue;
            const void * p = tensor_source(s);
            if (!p) {
                logw("source %s of %s lives in a buffer this backend cannot read and has no registered "
                     "original bytes\n", s->name, node->name);
                restore();
                return MI355X_STATUS_FAILED;
            }
            swapped.push_back({s, s->data, s->buffer_kind});
            s->data = const_cast<void *>(p);
            s->buffer_kind = MI355X_BUF_HOST;
        }
    }
    const int st = graph_compute_nodes(c, nodes, n_nodes);
    restore();
    return st;
}

static int graph_compute_nodes(mi355x_backend_t c, mi355x_tensor * const * nodes, int n_nodes) {
    c->started = true;
    c->fa_mirror = {};
    // the attention's device copy may stand in for its host bytes only if no other node of the
    // call writes over them
    c->mirror_ok = true;
    for (int i = 0; i < n_nodes && c->mirror_ok; i++) {
        const mi355x_tensor * f = nodes[i];
        if (!f || f->op != MI355X_OP_FLASH_ATTN_EXT || !f->data) continue;
        const char * h = (const char *)f->data;
        const size_t hb = nbytes(f);
        for (int j = 0; j < n_nodes; j++) {
            const mi355x_tensor * o = nodes[j];
            if (!o || j == i || is_view_op(o->op) || o->op == MI355X_OP_NONE || !o->data) continue;
            const char * d = (const char *)o->data;
            if (d < h + hb && h < d + nbytes(o)) {
                c->mirror_ok = false;
                break;
            }
        }
    }
    std::vector<bool> done((size_t)(n_nodes > 0 ? n_nodes : 0), false);
    for (int i = 0; i < n_nodes; i++) {
        if (done[i]) continue;
        mi355x_tensor * node = nodes[i];
        if (!node) continue;
        if (is_view_op(node->op)) continue;
        switch (node->op) {
            case MI355X_OP_MUL_MAT: {
                std::vector<mi355x_tensor *> grp{node};
                if (fusion_on() && fusable(node)) {
                    for (int j = i + 1; j < n_nodes && grp.size() < 4; j++) {
                        mi355x_tensor * o = nodes[j];
                        if (!o || done[j] || !fusable(o)) continue;
                        if (o->src[1] == node->src[1] && o->src[0]->type == node->src[0]->type &&
                            o->src[0]->ne[0] == node->src[0]->ne[0]) {
                            grp.push_back(o);
                            done[j] = true;
                        }
                    }
                }
                const bool quant = type_is_quantized(node->src[0]->type);
                const bool qres = c->quant_resident < 0 ? quant_resident_on() : c->quant_resident > 0;
                // a type only the host decodes is always an fp16 image
                const bool want_f16 = quant && (qres || !device_weight_type(node->src[0]->type));
                bool resident = false;
                guarded(c, c->brk_gemm, "MUL_MAT",
                        [&] { return mul_mat_device(c, grp, want_f16, resident); },
                        [&] { for (auto * d : grp) cpu_mul_mat(d); });
                const char * label;
                if (grp.size() > 1) label = (resident && (!quant || want_f16)) ? "fused-resident" : "fused";
                else if (!resident) label = "mt";
                else label = quant ? (want_f16 ? "prepacked-q" : "mt") : "prepacked";
                c->routes[label] += (long)grp.size();
                break;
            }
            case MI355X_OP_FLASH_ATTN_EXT: {
                c->fa_mirror = {};
                guarded(c, c->brk_fa, "FLASH_ATTN_EXT", [&] { return flash_attn_device(c, node); },
                        [&] { cpu_flash_attn(node); });
                c->routes["fa"]++;
                break;
            }
            case MI355X_OP_MUL_MAT_ID: {
                const mi355x_tensor * as = node->src[0];
                const mi355x_tensor * ids = node->src[2];
                // an id outside [0, n_expert) is a malformed graph (ggml-rocket.cpp:6719)
                std::vector<bool> routed((size_t)as->ne[2], false);
                for (int64_t t = 0; t < ids->ne[1]; t++)
                    for (int64_t s = 0; s < ids->ne[0]; s++) {
                        const int32_t e = *(const int32_t *)((const char *)ids->data + t * ids->nb[1] + s * ids->nb[0]);
                        if (e < 0 || e >= as->ne[2]) return MI355X_STATUS_FAILED;
                        routed[(size_t)e] = true;
                    }
                const std::string key = weight_key(as);
                if (!key.empty() && !c->moe_claimed.count(key) && moe_preflight_claim(key) == MOE_CLAIMED)
                    c->moe_claimed.insert(key);
                bool resident = false;
                bool ok = true;
                bool on_device = false;
                guarded(c, c->brk_moe, "MUL_MAT_ID",
                        [&] {
                            const int rc = mul_mat_id_device(c, node, resident);
                            on_device = rc == MI355X_OK;
                            return rc;
                        },
                        [&] { ok = cpu_mul_mat_id(node); });
                if (!ok) return MI355X_STATUS_FAILED;
                // distinct experts over the backend's life (ggml-rocket.h:39-57), device runs only:
                // a resident stack is ingested whole, so all its experts count once; a streamed
                // named stack counts each expert the ids routed to (an unnamed one has no identity)
                if (on_device && resident) {
                    if (c->moe_counted.insert(key).second) c->moe_resident += as->ne[2];
                } else if (on_device && !key.empty()) {
                    for (size_t e = 0; e < routed.size(); e++)
                        if (routed[e]) c->moe_streamed_experts.insert(key + "/e" + std::to_string(e));
                    c->moe_streamed = (long)c->moe_streamed_experts.size();
                }
                c->routes["moe"]++;
                break;
            }
            default:
                return MI355X_STATUS_FAILED;
        }
    }
    return MI355X_STATUS_SUCCESS;
}

}  // extern "C"

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

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
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

// A grow-only device buffer of one backend, allocated and freed in the order of that backend's
// stream (the device's stream-ordered pool): a buffer that grows releases its old bytes after
// the work already queued on the stream has read them, and neither waits for nor holds up
// other streams or other backends (hipFree would synchronize the whole device first).
struct DevBuf {
    void * p = nullptr;
    size_t cap = 0;
    hipStream_t owner = nullptr;   // the stream p was allocated on
    int ensure(size_t n, hipStream_t s) {
        if (n <= cap) return MI355X_OK;
        if (p) (void)hipFreeAsync(p, owner);
        p = nullptr;
        cap = 0;
        const size_t want = (n + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
        if (hipMallocAsync(&p, want, s) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            return MI355X_E_DEVICE;
        }
        owner = s;
        cap = want;
        return MI355X_OK;
    }
    // after the owner stream has been synchronized
    void release() {
        if (p) (void)hipFreeAsync(p, owner);
        p = nullptr;
        cap = 0;
    }
};

// n bytes from src to dst with non-temporal (streaming) 32-byte stores: the destination lines
// are written whole without being read first, as a plain memcpy of cache-sized parts does, and
// go to DRAM, where the DMA engine (a staging slot) or the host's next reader (a tensor larger
// than the caches) takes them from anyway. That is a third less memory traffic per copied byte.
__attribute__((target("avx2"))) void stream_copy_avx2(void * dst, const void * src, size_t n) {
    char * d = (char *)dst;
    const char * s = (const char *)src;
    size_t head = (32 - ((uintptr_t)d & 31)) & 31;
    if (head > n) head = n;
    memcpy(d, s, head);
    d += head;
    s += head;
    n -= head;
    const size_t body = n & ~(size_t)127;
    for (size_t i = 0; i < body; i += 128) {
        const __m256i x0 = _mm256_loadu_si256((const __m256i *)(s + i));
        const __m256i x1 = _mm256_loadu_si256((const __m256i *)(s + i + 32));
        const __m256i x2 = _mm256_loadu_si256((const __m256i *)(s + i + 64));
        const __m256i x3 = _mm256_loadu_si256((const __m256i *)(s + i + 96));
        _mm256_stream_si256((__m256i *)(d + i), x0);
        _mm256_stream_si256((__m256i *)(d + i + 32), x1);
        _mm256_stream_si256((__m256i *)(d + i + 64), x2);
        _mm256_stream_si256((__m256i *)(d + i + 96), x3);
    }
    _mm_sfence();   // the streamed lines are visible before anyone is told the copy is done
    memcpy(d + body, s + body, n - body);
}

bool stream_copy_ok() {
    static const bool ok = [] {
        if (const char * e = getenv("MI355X_COPY_NT"))
            if (atoi(e) == 0) return false;
        return __builtin_cpu_supports("avx2") != 0;
    }();
    return ok;
}

void copy_bytes(void * dst, const void * src, size_t n) {
    if (n >= 4096 && stream_copy_ok()) stream_copy_avx2(dst, src, n);
    else memcpy(dst, src, n);
}

// Host copy workers: one copy (or any job over disjoint parts) split across n threads, the
// caller being one of them. Persistent threads, because a copy of one staging piece takes about
// as long as starting a thread; after a job a worker keeps polling for the next one for
// `spin_us` before it sleeps, since during a graph_compute call the next piece comes within
// tens of microseconds and waking a sleeping thread costs about as long.
class CopyPool {
public:
    CopyPool(int n, size_t min_part, int spin_us) : min_part_(min_part), spin_us_(spin_us) {
        for (int i = 1; i < n; i++) th_.emplace_back([this] { work(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_.store(true);
        }
        cv_.notify_all();
        for (auto & t : th_) t.join();
    }
    int threads() const { return (int)th_.size() + 1; }
    size_t min_part() const { return min_part_; }
    // part(i) for i in [0, parts), spread over the workers and the calling thread
    void run(int parts, const std::function<void(int)> & part) {
        if (th_.empty() || parts <= 1) {
            for (int i = 0; i < parts; i++) part(i);
            return;
        }
        Job j;
        j.fn = &part;
        j.parts = parts;
        j.left.store(parts);
        j.gen = ++published_;
        cur_.store(&j);
        gen_.store(j.gen);
        if (sleepers_.load() > 0) {
            { std::lock_guard<std::mutex> lk(mu_); }
            cv_.notify_all();
        }
        drain(&j);
        while (j.left.load() > 0) __builtin_ia32_pause();
        cur_.store(nullptr);
        while (busy_.load() > 0) __builtin_ia32_pause();   // no worker still holds &j
    }
    void copy(void * dst, const void * src, size_t n) {
        const int parts = (int)std::max<size_t>(1, std::min<size_t>((size_t)threads(), n / min_part_));
        const size_t per = ((n + parts - 1) / parts + 127) & ~(size_t)127;
        run(parts, [&](int i) {
            const size_t o = (size_t)i * per;
            if (o < n) copy_bytes((char *)dst + o, (const char *)src + o, std::min(per, n - o));
        });
    }

private:
    struct Job {
        const std::function<void(int)> * fn = nullptr;
        int parts = 0;
        uint64_t gen = 0;
        std::atomic<int> next{0};
        std::atomic<int> left{0};
    };
    static void drain(Job * j) {
        for (;;) {
            const int i = j->next.fetch_add(1);
            if (i >= j->parts) return;
            (*j->fn)(i);
            j->left.fetch_sub(1);
        }
    }
    void work() {
        uint64_t seen = 0;
        for (;;) {
            const auto t0 = std::chrono::steady_clock::now();
            int polls = 0;
            while (gen_.load() == seen && !stop_.load()) {
                __builtin_ia32_pause();
                if (++polls < 256) continue;
                polls = 0;
                if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(spin_us_)) {
                    std::unique_lock<std::mutex> lk(mu_);
                    sleepers_.fetch_add(1);
                    cv_.wait(lk, [&] { return stop_.load() || gen_.load() != seen; });
                    sleepers_.fetch_sub(1);
                }
            }
            if (stop_.load()) return;
            busy_.fetch_add(1);
            seen = gen_.load();
            Job * j = cur_.load();
            if (j && j->gen == seen) drain(j);
            busy_.fetch_sub(1);
        }
    }
    const size_t min_part_;   // smallest part one worker copies
    const int spin_us_;
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_;
    std::atomic<Job *> cur_{nullptr};
    std::atomic<uint64_t> gen_{0};
    std::atomic<int> busy_{0}, sleepers_{0};
    std::atomic<bool> stop_{false};
    uint64_t published_ = 0;
};

// Pinned staging of one copy direction. Host tensors are pageable (ggml's CPU buffers), and a
// copy from pageable memory crawls through the runtime's own small bounce buffer, so every copy
// passes through `nslot` pinned slots of `chunk` bytes: the copy workers fill (or drain) one slot
// while the DMA engine moves another. A slot is reused only after the event of its last DMA has
// completed. Uploads and downloads have a ring each, so neither waits for the other's slots.
struct Ring {
    static constexpr int MAX_SLOT = 16;
    size_t chunk = 0;
    int nslot = 0;
    void * slot[MAX_SLOT] = {};
    hipEvent_t ev[MAX_SLOT] = {};
    bool pending[MAX_SLOT] = {};
    int init(size_t ch, int n) {
        chunk = ch;
        nslot = n;
        for (int i = 0; i < n; i++) {
            if (hipHostMalloc(&slot[i], ch, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                release();
                return MI355X_E_DEVICE;
            }
        }
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
        nslot = 0;
    }
};

// Rows of a device matrix to be copied into contiguous host rows once the compute-stream event
// `after` has passed. `buf` is the device buffer the rows are in, `op` the queued op they belong
// to.
struct DlItem {
    const char * dev;
    size_t pitch;       // bytes between device rows
    char * host;        // host rows
    size_t hpitch;      // bytes between host rows
    size_t width;       // bytes copied per row
    int64_t rows;
    const void * buf;
    hipEvent_t after;
    int op;
};
struct DlPiece {
    int item;
    int64_t r0, r1;
};
// An op whose outputs are queued: the first of its pieces, and how to compute it on the CPU if
// the device cannot deliver them.
struct DlOp {
    size_t first_piece;
    std::function<void()> redo;
    RouteHealth * brk;
    const char * route;
};

// Host-side accounting of the copies (mi355x_backend_host_stats).
struct HostStats {
    long calls = 0, fa_mirror_hits = 0, redone = 0, pieces_up = 0, pieces_down = 0;
    double bytes_up = 0, bytes_down = 0;
    double wall_s = 0, up_copy_s = 0, up_wait_s = 0, down_copy_s = 0, down_wait_s = 0;
    double copy_api_s = 0;   // enqueueing the copies (hipMemcpy*Async, event records and waits)
    double weight_s = 0;     // finding (or building) the weights in the HBM cache
};

double now_s() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

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
    size_t w16_peak = 0;                // its largest size (outside the cache budget)

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

    // Host <-> device copies. Uploads run on `stream`, in order before the kernels that read
    // them; downloads on `dstream`, queued by the ops (dl_*) and drained while later ops of the
    // call upload and compute, and entirely before graph_compute returns.
    hipStream_t dstream = nullptr;
    hipStream_t ustream = nullptr;       // a row-chunked MUL_MAT's activation uploads
    int row_chunk = -1;                  // rows per chunk of such a MUL_MAT (-1: by link bytes, 0: one)
    Ring up, down;                       // pinned slots of each direction
    bool staging_ready = false;
    int up_next = 0;                     // the upload slot the next piece takes
    size_t up_piece = 0;                 // size of the next upload piece (grows within an op)
    size_t first_piece = 0, last_piece = 0;
    std::vector<DlItem> dl_items;
    std::vector<DlPiece> dl_pieces;
    std::vector<DlOp> dl_ops;
    size_t dl_issued = 0, dl_drained = 0;
    int dl_waited_item = -1;             // the item whose event dstream last waited on
    bool dl_broken = false;              // a piece failed while polled (dl_drain then recomputes)
    std::vector<hipEvent_t> evpool;      // compute-stream events of queued outputs
    size_t ev_used = 0;
    int inject_drain = 0;                // test hook: the next n drained pieces report a failure
    HostStats hs;
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

#define TRY_RC(x) do { const int _r = (x); if (_r != MI355X_OK) return _r; } while (0)

// The copy pipeline's shape: `nslot` slots of `chunk` bytes per direction; an op's uploads start
// with a piece of `first_piece` bytes that doubles up to the slot size, so its first DMA starts
// after a short host copy rather than a whole slot's; each queued output ends with pieces that
// halve down to `last_piece`, so the host copy left after its last DMA lands is short. Host copies
// of POOL_MIN bytes or more are split over the copy workers (parts of at least COPY_PART);
// smaller ones run on the calling thread.
constexpr size_t POOL_MIN = (size_t)512 << 10;
constexpr int64_t CHUNK_LINK_BYTES = (int64_t)8 << 20;
constexpr size_t COPY_PART = (size_t)256 << 10;

size_t env_kb(const char * name, size_t dflt, size_t lo, size_t hi) {
    if (const char * e = getenv(name)) {
        const long v = atol(e);
        if (v >= (long)(lo >> 10) && v <= (long)(hi >> 10)) return (size_t)v << 10;
    }
    return dflt;
}

// The staging slots, the copy workers and the download stream, made on first use. Without them
// no device op runs (the op falls back to the CPU).
bool staging_on(Ctx * c) {
    if (c->staging_ready) return true;
    if (!c->pool) {
        int spin = 300;   // microseconds a copy worker polls for the next job before it sleeps
        if (const char * e = getenv("MI355X_COPY_SPIN_US")) spin = std::max(0, std::min(atoi(e), 100000));
        c->pool.reset(new CopyPool(c->n_threads, env_kb("MI355X_COPY_PART_KB", COPY_PART, 16 << 10, 64 << 20), spin));
    }
    // rows per chunk of a MUL_MAT whose activations are uploaded: -1 sizes chunks by their link
    // bytes, 0 runs one chunk, n > 0 forces n rows (a multiple of 16)
    c->row_chunk = -1;
    if (const char * e = getenv("MI355X_ROW_CHUNK")) c->row_chunk = std::max(0, atoi(e)) / 16 * 16;
    const size_t chunk = env_kb("MI355X_STAGE_CHUNK_KB", (size_t)8 << 20, 64 << 10, (size_t)64 << 20);
    int nslot = 4;
    if (const char * e = getenv("MI355X_STAGE_SLOTS")) {
        const int v = atoi(e);
        if (v >= 2 && v <= Ring::MAX_SLOT) nslot = v;
    }
    c->first_piece = env_kb("MI355X_FIRST_PIECE_KB", (size_t)1 << 20, 64 << 10, chunk);
    c->last_piece = env_kb("MI355X_LAST_PIECE_KB", (size_t)1 << 20, 64 << 10, chunk);
    if (!c->dstream && hipStreamCreateWithFlags(&c->dstream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        c->dstream = nullptr;
        return false;
    }
    if (!c->ustream && hipStreamCreateWithFlags(&c->ustream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        c->ustream = nullptr;
        return false;
    }
    if (c->up.init(chunk, nslot) != MI355X_OK) return false;
    if (c->down.init(chunk, nslot) != MI355X_OK) {
        c->up.release();
        return false;
    }
    c->up_piece = c->first_piece;
    c->staging_ready = true;
    return true;
}

void host_copy(Ctx * c, void * dst, const void * src, size_t n) {
    if (n >= POOL_MIN) c->pool->copy(dst, src, n);
    else copy_bytes(dst, src, n);
}

// whether an event has passed, without waiting (a not-ready answer leaves no error behind for
// the next launch's error check)
bool passed(hipEvent_t e) {
    const hipError_t r = hipEventQuery(e);
    if (r == hipErrorNotReady) {
        (void)hipGetLastError();
        return false;
    }
    return true;
}

// ---- the download queue -------------------------------------------------------------------
// An op queues the rows of its outputs with the compute-stream event after which they are final,
// and returns; the pieces are copied into the download slots on `dstream` and out of them by the
// host while later ops of the call upload and compute. Everything queued is delivered before
// graph_compute returns, before the host reads bytes a queued piece has yet to write, and before
// an op writes or regrows a device buffer a queued piece still reads.

// An event recorded on stream `st` now (reused once the queue has been drained).
hipEvent_t mark_event_on(Ctx * c, hipStream_t st) {
    if (c->ev_used == c->evpool.size()) {
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        c->evpool.push_back(e);
    }
    hipEvent_t e = c->evpool[c->ev_used];
    if (hipEventRecord(e, st) != hipSuccess) return nullptr;
    c->ev_used++;
    return e;
}

hipEvent_t mark_event(Ctx * c) { return mark_event_on(c, c->stream); }

int dl_op(Ctx * c, std::function<void()> redo, RouteHealth * brk, const char * route) {
    c->dl_ops.push_back({c->dl_pieces.size(), std::move(redo), brk, route});
    return (int)c->dl_ops.size() - 1;
}

// `rows` rows of `width` bytes, `pitch` apart at `dev` (inside device buffer `buf`), to host rows
// `hpitch` apart at `host`, once `after` has passed.
void dl_rows(Ctx * c, int op, const void * dev, size_t pitch, void * host, size_t hpitch, size_t width, int64_t rows,
             const void * buf, hipEvent_t after, bool shrink = true) {
    if (rows <= 0 || !width) return;
    const size_t chunk = c->down.chunk;
    if (width > chunk) {   // rows wider than a slot: column slices of at most a slot
        for (size_t o = 0; o < width; o += chunk)
            dl_rows(c, op, (const char *)dev + o, pitch, (char *)host + o, hpitch, std::min(chunk, width - o), rows,
                    buf, after, shrink);
        return;
    }
    if (pitch == width && hpitch == width && rows > 1 && width < ((size_t)64 << 10)) {
        // contiguous on both sides: copied as 64 KB rows, so pieces can be cut finely
        const size_t n = (size_t)rows * width, W = (size_t)1 << 16;
        const int64_t full = (int64_t)(n / W);
        dl_rows(c, op, dev, W, host, W, W, full, buf, after, shrink && n % W == 0);
        if (n % W)
            dl_rows(c, op, (const char *)dev + full * W, n % W, (char *)host + full * W, n % W, n % W, 1, buf, after,
                    shrink);
        return;
    }
    const int item = (int)c->dl_items.size();
    c->dl_items.push_back({(const char *)dev, pitch, (char *)host, hpitch, width, rows, buf, after, op});
    // piece sizes from the end: last_piece, doubling up to the slot size (or whole slots)
    const size_t first = c->dl_pieces.size();
    size_t target = shrink ? c->last_piece : chunk;
    for (int64_t r1 = rows; r1 > 0;) {
        const int64_t per = std::max<int64_t>(1, (int64_t)(std::min(target, chunk) / width));
        const int64_t r0 = std::max<int64_t>(0, r1 - per);
        c->dl_pieces.push_back({item, r0, r1});
        r1 = r0;
        target = std::min(target * 2, chunk);
    }
    std::reverse(c->dl_pieces.begin() + (ptrdiff_t)first, c->dl_pieces.end());
    c->hs.bytes_down += (double)width * (double)rows;
}

// n contiguous bytes, as rows of 64 KB and a short last row
void dl_bytes(Ctx * c, int op, const void * dev, void * host, size_t n, const void * buf, hipEvent_t after) {
    const size_t W = (size_t)1 << 16;
    const int64_t full = (int64_t)(n / W);
    dl_rows(c, op, dev, W, host, W, W, full, buf, after, n % W == 0);
    if (n % W) dl_rows(c, op, (const char *)dev + full * W, n % W, (char *)host + full * W, n % W, n % W, 1, buf, after);
}

// Starts the DMAs of queued pieces into free download slots.
int dl_issue(Ctx * c) {
    Ring & R = c->down;
    const double t0 = now_s();
    struct Account {
        Ctx * c;
        double t0;
        ~Account() { c->hs.copy_api_s += now_s() - t0; }
    } account{c, t0};
    while (c->dl_issued < c->dl_pieces.size() && c->dl_issued < c->dl_drained + (size_t)R.nslot) {
        const DlPiece & p = c->dl_pieces[c->dl_issued];
        const DlItem & it = c->dl_items[(size_t)p.item];
        const int k = (int)(c->dl_issued % (size_t)R.nslot);   // its previous piece has been drained
        if (p.item != c->dl_waited_item) {
            if (it.after && hipStreamWaitEvent(c->dstream, it.after, 0) != hipSuccess) return MI355X_E_DEVICE;
            c->dl_waited_item = p.item;
        }
        const size_t rows = (size_t)(p.r1 - p.r0);
        const char * src = it.dev + (size_t)p.r0 * it.pitch;
        const hipError_t e =
            it.pitch == it.width
                ? hipMemcpyAsync(R.slot[k], src, rows * it.width, hipMemcpyDeviceToHost, c->dstream)
                : hipMemcpy2DAsync(R.slot[k], it.width, src, it.pitch, it.width, rows, hipMemcpyDeviceToHost, c->dstream);
        if (e != hipSuccess || hipEventRecord(R.ev[k], c->dstream) != hipSuccess) return MI355X_E_DEVICE;
        R.pending[k] = true;
        c->dl_issued++;
        c->hs.pieces_down++;
    }
    return MI355X_OK;
}

// Copies the oldest issued piece out of its slot once its DMA has landed.
int dl_drain_one(Ctx * c) {
    Ring & R = c->down;
    const DlPiece & p = c->dl_pieces[c->dl_drained];
    const DlItem & it = c->dl_items[(size_t)p.item];
    const int k = (int)(c->dl_drained % (size_t)R.nslot);
    const double t0 = now_s();
    const int rc = R.settle(k);
    const double t1 = now_s();
    c->hs.down_wait_s += t1 - t0;
    if (rc != MI355X_OK) return rc;
    if (c->inject_drain > 0) {
        c->inject_drain--;
        return MI355X_E_DEVICE;
    }
    const int64_t rows = p.r1 - p.r0;
    char * h = it.host + (size_t)p.r0 * it.hpitch;
    const char * s = (const char *)R.slot[k];
    if (it.hpitch == it.width) {
        host_copy(c, h, s, (size_t)rows * it.width);
    } else {
        const int parts = (int)std::min<int64_t>(c->pool->threads(),
                                                 std::max<int64_t>(1, (int64_t)((size_t)rows * it.width / COPY_PART)));
        c->pool->run(parts, [&](int pi) {
            for (int64_t r = rows * pi / parts; r < rows * (pi + 1) / parts; r++)
                memcpy(h + (size_t)r * it.hpitch, s + (size_t)r * it.width, it.width);
        });
    }
    c->hs.down_copy_s += now_s() - t1;
    c->dl_drained++;
    return MI355X_OK;
}

// Copies out the issued pieces whose DMA has landed, without waiting for the others. A piece
// that fails here marks the queue broken, which the next dl_drain handles.
void dl_poll(Ctx * c) {
    while (!c->dl_broken && c->dl_drained < c->dl_issued) {
        const int k = (int)(c->dl_drained % (size_t)c->down.nslot);
        if (c->down.pending[k] && !passed(c->down.ev[k])) break;
        if (dl_drain_one(c) != MI355X_OK || dl_issue(c) != MI355X_OK) c->dl_broken = true;
    }
}

void dl_reset(Ctx * c) {
    c->dl_broken = false;
    c->dl_items.clear();
    c->dl_pieces.clear();
    c->dl_ops.clear();
    c->dl_issued = c->dl_drained = 0;
    c->dl_waited_item = -1;
    c->ev_used = 0;
}

// Delivers everything queued. The op whose piece the device could not deliver is computed again
// on the CPU (a device failure on its route), and so is every op queued after it, since those
// may have read its device result.
void dl_drain(Ctx * c) {
    int rc = c->dl_broken ? MI355X_E_DEVICE : MI355X_OK;
    while (rc == MI355X_OK && c->dl_drained < c->dl_pieces.size()) {
        rc = dl_issue(c);
        if (rc == MI355X_OK) rc = dl_drain_one(c);
    }
    if (rc != MI355X_OK && c->dl_drained < c->dl_pieces.size()) {
        const size_t bad = (size_t)c->dl_items[(size_t)c->dl_pieces[c->dl_drained].item].op;
        for (int i = 0; i < Ring::MAX_SLOT; i++)
            if (c->down.pending[i]) {
                (void)hipEventSynchronize(c->down.ev[i]);
                c->down.pending[i] = false;
            }
        (void)hipGetLastError();
        for (size_t o = bad; o < c->dl_ops.size(); o++) {
            DlOp & op = c->dl_ops[o];
            logw("%s: its device result could not be copied back; computed on the CPU\n", op.route);
            op.brk->failures++;
            op.redo();
            c->n_cpu_fallbacks++;
            c->hs.redone++;
        }
    }
    dl_reset(c);
}

// whether a queued piece has yet to write host bytes in [p, p + n)
bool dl_writes_host(const Ctx * c, const void * p, size_t n) {
    if (c->dl_drained == c->dl_pieces.size() || !p || !n) return false;
    const char * a = (const char *)p;
    for (size_t i = (size_t)c->dl_pieces[c->dl_drained].item; i < c->dl_items.size(); i++) {
        const DlItem & it = c->dl_items[i];
        const char * h = it.host;
        const char * e = h + (size_t)(it.rows - 1) * it.hpitch + it.width;
        if (a < e && h < a + n) return true;
    }
    return false;
}

// whether a queued piece still reads device buffer `buf`
bool dl_reads_buf(const Ctx * c, const void * buf) {
    if (c->dl_drained == c->dl_pieces.size() || !buf) return false;
    for (size_t i = (size_t)c->dl_pieces[c->dl_drained].item; i < c->dl_items.size(); i++)
        if (c->dl_items[i].buf == buf) return true;
    return false;
}

// host -> device on stream `st`, through the upload slots; the host bytes may be reused once
// this returns
int upload_on(Ctx * c, hipStream_t st, void * dst, const void * src, size_t n) {
    if (!n) return MI355X_OK;
    if (!staging_on(c)) return MI355X_E_DEVICE;
    if (dl_writes_host(c, src, n)) dl_drain(c);
    Ring & R = c->up;
    for (size_t o = 0; o < n;) {
        const size_t len = std::min(std::min(c->up_piece, R.chunk), n - o);
        const int k = c->up_next;
        c->up_next = (k + 1) % R.nslot;
        const double t0 = now_s();
        TRY_RC(R.settle(k));
        const double t1 = now_s();
        host_copy(c, R.slot[k], (const char *)src + o, len);
        const double t2 = now_s();
        c->hs.up_wait_s += t1 - t0;
        c->hs.up_copy_s += t2 - t1;
        if (hipMemcpyAsync((char *)dst + o, R.slot[k], len, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipEventRecord(R.ev[k], st) != hipSuccess)
            return MI355X_E_DEVICE;
        c->hs.copy_api_s += now_s() - t2;
        c->hs.pieces_up++;
        R.pending[k] = true;
        o += len;
        c->up_piece = std::min(c->up_piece * 2, R.chunk);
        if (c->dl_issued > c->dl_drained) dl_poll(c);   // results that landed meanwhile
    }
    c->hs.bytes_up += (double)n;
    return MI355X_OK;
}

// host -> device on the compute stream, ahead of the kernels that read it
int upload(Ctx * c, void * dst, const void * src, size_t n) { return upload_on(c, c->stream, dst, src, n); }

// the start of a device op: its uploads begin with a short piece again
void begin_op(Ctx * c) { c->up_piece = c->first_piece; }

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
    if ((t == MI355X_TYPE_F16 || t == MI355X_TYPE_Q4_K || t == MI355X_TYPE_Q5_K) && lay == t) return upload(c, dst, src, raw);
    TRY(c->wstage.ensure(raw, c->stream));
    TRY(upload(c, c->wstage.p, src, raw));
    if (t == MI355X_TYPE_F32 || t == MI355X_TYPE_BF16) {
        if (lay == MI355X_F16) return mi355x_convert_f16(t, c->wstage.p, rows * K, (uint16_t *)dst, c->stream);
        TRY(c->wconv.ensure((size_t)rows * K * 2, c->stream));
        TRY(mi355x_convert_f16(t, c->wstage.p, rows * K, (uint16_t *)c->wconv.p, c->stream));
        return mi355x_weight_f16_tiled(MI355X_F16, c->wconv.p, rows, K, (uint16_t *)dst, c->stream);
    }
    if (lay == MI355X_Q4_K_X || lay == MI355X_Q8_0_X || lay == MI355X_Q6_K_X || lay == MI355X_MXFP4_X)
        return mi355x_weight_pack(lay, c->wstage.p, rows, K, dst, c->stream);
    if (lay != MI355X_F16 && lay != MI355X_F16_T) return mi355x_weight_pack(t, c->wstage.p, rows, K, dst, c->stream);
    // -> fp16: from the HBM layout, built first when that differs from the ggml one
    const void * q = c->wstage.p;
    if (t == MI355X_TYPE_Q4_0 || t == MI355X_TYPE_Q8_0 || t == MI355X_TYPE_Q6_K || t == MI355X_TYPE_MXFP4) {
        TRY(c->wconv.ensure(raw, c->stream));
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
    // Q4_K, Q8_0, Q6_K and MXFP4 experts of whole 32-row groups take the regrouped layouts,
    // whose 32-row slabs the expert GEMM loads as contiguous bytes
    if (moe && moe_n % 32 == 0) {
        if (lay == MI355X_Q4_K) lay = MI355X_Q4_K_X;
        else if (lay == MI355X_Q8_0) lay = MI355X_Q8_0_X;
        else if (lay == MI355X_Q6_K) lay = MI355X_Q6_K_X;
        else if (lay == MI355X_MXFP4) lay = MI355X_MXFP4_X;
    }
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
    TRY(scratch.ensure((size_t)dbytes, c->stream));
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
    if (!ensure_device(c) || !staging_on(c)) return MI355X_E_DEVICE;
    begin_op(c);
    if (dl_reads_buf(c, c->out.p)) dl_drain(c);   // out is rewritten (and may regrow) below
    const mi355x_tensor * b = grp[0]->src[1];
    const int64_t K = b->ne[0], M = b->ne[1] * b->ne[2] * b->ne[3];
    TRY(c->act.ensure((size_t)M * K * 4, c->stream));
    TRY(c->a16.ensure((size_t)((M + 15) / 16 * 16) * K * 2, c->stream));
    TRY(c->scales.ensure((size_t)M * 4, c->stream));
    int64_t ntot = 0;
    for (auto * d : grp) ntot += d->src[0]->ne[1];
    TRY(c->out.ensure((size_t)M * ntot * 4, c->stream));
    std::vector<WEntry> ws(grp.size());
    all_resident = true;
    mi355x_gemm_out outs[4];
    int64_t col = 0;
    for (size_t i = 0; i < grp.size(); i++) {
        const mi355x_tensor * a = grp[i]->src[0];
        bool res = false;
        const double tw = now_s();
        TRY(get_weight(c, a, a->ne[1], K, want_f16, true, 0, c->wscratch[i], ws[i], res));
        c->hs.weight_s += now_s() - tw;
        all_resident = all_resident && res;
        outs[i].w_dev = ws[i].dev;
        outs[i].rows_total = a->ne[1];
        outs[i].row0 = 0;
        outs[i].N = a->ne[1];
        outs[i].c_dev = (float *)c->out.p + M * col;   // member i's [M][N_i], so it comes back in one run
        outs[i].ldc = a->ne[1];
        col += a->ne[1];
    }
    // Quantized weights (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4) at the shapes where one decode
    // pass plus the fp16 GEMM is faster than decoding inside the GEMM
    // (mi355x_mul_mat_decode_first): each member decoded into tiled fp16 scratch first. That
    // scratch lives outside the weight cache's budget; its peak size is in the teardown report.
    int gtype = ws[0].dev_type;
    bool same = true;
    for (auto & w : ws) same = same && w.dev_type == gtype;
    if (same && mi355x_mul_mat_decode_first(gtype, M, ntot, K) == 1) {
        std::vector<size_t> off(grp.size() + 1, 0);
        for (size_t i = 0; i < grp.size(); i++)
            off[i + 1] = off[i] + (((size_t)mi355x_weight_bytes(MI355X_F16_T, outs[i].N, K) + 255) & ~(size_t)255);
        TRY(c->w16.ensure(off.back(), c->stream));
        c->w16_peak = std::max(c->w16_peak, c->w16.cap);
        for (size_t i = 0; i < grp.size(); i++) {
            uint16_t * w16 = (uint16_t *)((char *)c->w16.p + off[i]);
            TRY(mi355x_weight_f16_tiled(gtype, outs[i].w_dev, outs[i].N, K, w16, c->stream));
            outs[i].w_dev = w16;
        }
        gtype = MI355X_F16_T;
    }
    // src1 from the attention this call just computed (same host bytes, row-major F32): its
    // device copy; otherwise uploaded
    const float * act = (const float *)c->act.p;
    const bool dense = b->type == MI355X_TYPE_F32 && b->nb[0] == 4 && b->nb[1] == (size_t)K * 4 &&
                       b->nb[2] == b->nb[1] * (size_t)b->ne[1] && b->nb[3] == b->nb[2] * (size_t)b->ne[2];
    const bool mirrored = dense && c->fa_mirror.dev && b->data == c->fa_mirror.host &&
                          (size_t)M * K * 4 <= c->fa_mirror.bytes;
    if (mirrored) {
        act = (const float *)c->fa_mirror.dev;
        c->hs.fa_mirror_hits++;
    }
    // Uploaded activations run in chunks of row_chunk rows: chunk j's rows go up on the upload
    // stream while chunk j-1 is packed and multiplied on the compute stream and the result rows of
    // earlier chunks come back, so the link, the kernels and the host copies overlap. The upload
    // stream first waits for the compute stream's earlier readers of the activation buffer.
    // By default a chunk carries about CHUNK_LINK_BYTES over the link (its activations up, its
    // results down), in 128-row steps: measured on the 8B-shape layer's calls at M 512, that is
    // 256-row chunks for Q/K/V (40 KB a row; 128-row chunks made its narrow GEMMs slower than the
    // overlap gained), 128 for gate/up (128 KB a row) and down (73 KB a row).
    int64_t R = M;
    if (!mirrored && c->row_chunk > 0) {
        R = c->row_chunk;
    } else if (!mirrored && c->row_chunk < 0) {
        const int64_t per_row = K * 4 + ntot * 4;
        R = std::max<int64_t>(128, (CHUNK_LINK_BYTES / per_row + 127) / 128 * 128);
    }
    if (M < 2 * R) R = M;
    const int n_out = (int)grp.size();
    auto chunk_outs = [&](int64_t r0, mi355x_gemm_out * o) {
        for (int i = 0; i < n_out; i++) {
            o[i] = outs[i];
            o[i].c_dev = outs[i].c_dev + r0 * outs[i].ldc;
        }
    };
    // K-split partials, summed in a fixed order (reproducible results), sized for the largest
    // chunk; a two-way split adds into the outputs, which the activation pack then clears in the
    // same launch
    size_t pmax = 0;
    for (const int64_t m : {R, M % R}) {
        if (!m) continue;
        mi355x_gemm_out o[4];
        chunk_outs(0, o);
        pmax = std::max(pmax, mi355x_gemm_workspace(gtype, m, K, o, n_out));
    }
    if (pmax) TRY(c->part.ensure(pmax, c->stream));
    if (R < M) {
        hipEvent_t ready = mark_event(c);
        if (!ready || hipStreamWaitEvent(c->ustream, ready, 0) != hipSuccess) return MI355X_E_DEVICE;
    }
    const int tiled = gtype == MI355X_F16_T;
    const int op = dl_op(c, [grp] { for (auto * d : grp) cpu_mul_mat(d); }, &c->brk_gemm, "MUL_MAT");
    for (int64_t r0 = 0; r0 < M; r0 += R) {
        const int64_t m = std::min(R, M - r0);
        mi355x_gemm_out o[4];
        chunk_outs(r0, o);
        const size_t pbytes = mi355x_gemm_workspace(gtype, m, K, o, n_out);
        const int acc = mi355x_gemm_accumulates(gtype, m, K, o, n_out, pbytes);
        if (acc < 0) return acc;
        if (!mirrored) {
            const size_t xb = (size_t)m * K * 4;
            float * x = (float *)c->act.p + r0 * K;
            if (R < M) {
                TRY(upload_on(c, c->ustream, x, (const char *)b->data + (size_t)r0 * K * 4, xb));
                hipEvent_t up = mark_event_on(c, c->ustream);
                if (!up || hipStreamWaitEvent(c->stream, up, 0) != hipSuccess) return MI355X_E_DEVICE;
            } else {
                TRY(upload(c, x, b->data, xb));
            }
        }
        const float * x = act + r0 * K;
        uint16_t * a16 = (uint16_t *)c->a16.p + r0 * K;   // row r0 (a multiple of 16) of either layout
        float * sc = (float *)c->scales.p + r0;
        if (acc && n_out == 1) {   // the pack clears the output rows the split adds into
            TRY(mi355x_pack_act_clear(tiled, x, K, m, K, a16, sc, o[0].c_dev, o[0].ldc, o[0].N, c->stream));
        } else {
            for (int i = 0; acc && i < n_out; i++)   // a group's outputs are separate blocks
                if (hipMemsetAsync(o[i].c_dev, 0, (size_t)m * (size_t)o[i].N * 4, c->stream) != hipSuccess)
                    return MI355X_E_DEVICE;
            if (tiled) TRY(mi355x_pack_act_tiled(x, K, m, K, a16, sc, c->stream));
            else TRY(mi355x_pack_act(x, K, m, K, a16, sc, c->stream));
        }
        TRY(mi355x_gemm_ws(gtype, a16, sc, m, K, o, n_out, pbytes ? c->part.p : nullptr, pbytes,
                           acc ? MI355X_GEMM_OUT_ZEROED : 0, c->stream));
        // dst[i] is [N_i, M] contiguous, as member i's output block: these rows are queued for
        // download behind the GEMM, ending in short pieces after the op's last chunk only
        hipEvent_t done = mark_event(c);
        if (!done) return MI355X_E_DEVICE;
        const bool last = r0 + m == M;
        for (int i = 0; i < n_out; i++) {
            const size_t w = (size_t)o[i].N * 4;
            dl_rows(c, op, o[i].c_dev, w, (float *)grp[(size_t)i]->data + r0 * o[i].N, w, w, m, c->out.p, done,
                    last && i == n_out - 1);
        }
        TRY(dl_issue(c));
        if (R < M) dl_poll(c);
    }
    return MI355X_OK;
}

// ---- FLASH_ATTN_EXT ---------------------------------------------------------------------------
int flash_attn_device(Ctx * c, mi355x_tensor * dst) {
    if (!ensure_device(c) || !staging_on(c)) return MI355X_E_DEVICE;
    begin_op(c);
    if (dl_reads_buf(c, c->fa_o.p)) dl_drain(c);   // fa_o is rewritten (and may regrow) below
    const mi355x_tensor * q = dst->src[0];
    const mi355x_tensor * k = dst->src[1];
    const mi355x_tensor * v = dst->src[2];
    const mi355x_tensor * m = dst->src[3];
    const size_t qb = nbytes(q), kb = nbytes(k), vb = nbytes(v), mb = m ? nbytes(m) : 0, ob = nbytes(dst);
    TRY(c->fa_q.ensure(qb, c->stream));
    TRY(c->fa_k.ensure(kb, c->stream));
    TRY(c->fa_v.ensure(vb, c->stream));
    if (m) TRY(c->fa_m.ensure(mb, c->stream));
    TRY(c->fa_o.ensure(ob, c->stream));
    TRY(upload(c, c->fa_q.p, q->data, qb));
    TRY(upload(c, c->fa_k.p, k->data, kb));
    TRY(upload(c, c->fa_v.p, v->data, vb));
    if (m) TRY(upload(c, c->fa_m.p, m->data, mb));
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
    if (ws) TRY(c->fa_ws.ensure(ws, c->stream));
    TRY(mi355x_flash_attn(&a, 0, ws ? c->fa_ws.p : nullptr, ws, c->stream));
    hipEvent_t done = mark_event(c);
    if (!done) return MI355X_E_DEVICE;
    const int op = dl_op(c, [dst] { cpu_flash_attn(dst); }, &c->brk_fa, "FLASH_ATTN_EXT");
    dl_bytes(c, op, c->fa_o.p, dst->data, ob, c->fa_o.p, done);
    if (c->mirror_ok) {
        c->fa_mirror.host = dst->data;
        c->fa_mirror.bytes = ob;
        c->fa_mirror.dev = c->fa_o.p;
    }
    return dl_issue(c);
}

// ---- MUL_MAT_ID -------------------------------------------------------------------------------
int mul_mat_id_device(Ctx * c, mi355x_tensor * dst, bool & resident) {
    if (!ensure_device(c) || !staging_on(c)) return MI355X_E_DEVICE;
    begin_op(c);
    if (dl_reads_buf(c, c->moe_o.p)) dl_drain(c);   // moe_o is rewritten (and may regrow) below
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
    TRY(c->moe_b.ensure(bb, c->stream));
    TRY(c->moe_ids.ensure(ib, c->stream));
    TRY(c->moe_o.ensure(ob, c->stream));
    TRY(upload(c, c->moe_b.p, b->data, bb));
    // ids may be a strided view: pack it to [T][U] on the host side of the copy
    std::vector<int32_t> idh((size_t)T * U);
    for (int64_t t = 0; t < T; t++)
        for (int64_t s = 0; s < U; s++)
            idh[t * U + s] = *(const int32_t *)((const char *)ids->data + t * ids->nb[1] + s * ids->nb[0]);
    TRY(upload(c, c->moe_ids.p, idh.data(), ib));
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
    TRY(c->moe_ws.ensure(ws, c->stream));
    TRY(mi355x_mul_mat_id(&a, c->moe_ws.p, ws, nullptr, c->stream));
    hipEvent_t done = mark_event(c);
    if (!done) return MI355X_E_DEVICE;
    const int op = dl_op(c, [dst] { cpu_mul_mat_id(dst); }, &c->brk_moe, "MUL_MAT_ID");
    dl_bytes(c, op, c->moe_o.p, dst->data, ob, c->moe_o.p, done);
    return dl_issue(c);
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
        dl_drain(c);   // the CPU reads host bytes that queued outputs may still have to write
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

MI355X_API void mi355x_backend_get_host_memory(size_t * fr, size_t * tot) {
    size_t total = 0, avail = 0;
    if (FILE * f = fopen("/proc/meminfo", "r")) {
        char line[256];
        int found = 0;
        while (found < 2 && fgets(line, sizeof line, f)) {
            unsigned long long kb = 0;
            if (sscanf(line, "MemTotal: %llu kB", &kb) == 1) {
                total = (size_t)kb << 10;
                found++;
            } else if (sscanf(line, "MemAvailable: %llu kB", &kb) == 1) {
                avail = (size_t)kb << 10;
                found++;
            }
        }
        fclose(f);
    }
    if (fr) *fr = std::min(avail, total);
    if (tot) *tot = total;
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

// The decode-first scratch: per-call HBM beside the cache budget, so a run near that budget
// can see where the rest went.
void report_scratch(const Ctx * c) {
    if (c->w16_peak)
        logi("[dq-scratch] per-call fp16 decode of quantized weights peaked at %.1f MB of HBM, outside the "
             "%.0f MB cache budget\n", (double)c->w16_peak / (1 << 20), (double)c->cache_budget / (1 << 20));
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
    if (c->dstream) (void)hipStreamSynchronize(c->dstream);
    c->up.release();
    c->down.release();
    for (hipEvent_t e : c->evpool) (void)hipEventDestroy(e);
    c->evpool.clear();
    if (c->dstream) (void)hipStreamDestroy(c->dstream);
    if (c->ustream) {
        (void)hipStreamSynchronize(c->ustream);
        (void)hipStreamDestroy(c->ustream);
    }
    c->pool.reset();
    for (auto & kv : c->wcache) (void)hipFree(kv.second.dev);
    report_residency(c);
    report_scratch(c);
    report_routes(c);
    c->wcache.clear();
    for (DevBuf * b : {&c->act, &c->a16, &c->scales, &c->out, &c->part, &c->wstage, &c->wconv, &c->fa_q, &c->fa_k, &c->fa_v,
                       &c->fa_m, &c->fa_o, &c->fa_ws, &c->moe_b, &c->moe_ids, &c->moe_o, &c->moe_ws,
                       &c->wscratch[0], &c->wscratch[1], &c->wscratch[2], &c->wscratch[3], &c->moe_wscratch, &c->w16})
        b->release();
    if (c->stream) {
        (void)hipStreamSynchronize(c->stream);   // the stream-ordered frees above
        (void)hipStreamDestroy(c->stream);
        // hand the freed bytes back to the device rather than keeping them in its pool
        int dev = 0;
        hipMemPool_t mp = nullptr;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetDefaultMemPool(&mp, dev) == hipSuccess && mp)
            (void)hipMemPoolTrimTo(mp, 0);
        (void)hipGetLastError();
    }
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
    if (mi355x_backend_is(c) && g && !strcmp(g, "copyback")) {
        c->inject_drain = n < 0 ? 0 : n;
        return;
    }
    RouteHealth * b = breaker_of(c, g);
    if (b) b->inject = n < 0 ? 0 : n;
}

MI355X_API void mi355x_backend_host_stats(mi355x_backend_t c, mi355x_host_stats * out) {
    if (!out) return;
    memset(out, 0, sizeof *out);
    if (!mi355x_backend_is(c)) return;
    const HostStats & h = c->hs;
    out->calls = h.calls;
    out->fa_mirror_hits = h.fa_mirror_hits;
    out->copyback_redone = h.redone;
    out->bytes_up = h.bytes_up;
    out->bytes_down = h.bytes_down;
    out->wall_s = h.wall_s;
    out->up_copy_s = h.up_copy_s;
    out->up_wait_s = h.up_wait_s;
    out->down_copy_s = h.down_copy_s;
    out->down_wait_s = h.down_wait_s;
    out->copy_api_s = h.copy_api_s;
    out->weight_s = h.weight_s;
    out->pieces_up = h.pieces_up;
    out->pieces_down = h.pieces_down;
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

static int graph_compute_queued(mi355x_backend_t c, mi355x_tensor * const * nodes, int n_nodes);

// Runs the nodes, then delivers every output still queued for download: each dst is written
// when this returns, whatever the status.
static int graph_compute_nodes(mi355x_backend_t c, mi355x_tensor * const * nodes, int n_nodes) {
    const double t0 = now_s();
    const int st = graph_compute_queued(c, nodes, n_nodes);
    dl_drain(c);
    c->hs.calls++;
    c->hs.wall_s += now_s() - t0;
    return st;
}

static int graph_compute_queued(mi355x_backend_t c, mi355x_tensor * const * nodes, int n_nodes) {
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
                if (dl_writes_host(c, ids->data, nbytes(ids))) dl_drain(c);   // the ids are read here
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

// runtime.hip -- device context, status reporting, counters, the pooled HBM
// arena and host/device copies.
//
// Replaces the reference's runtime (src/cuda/runtime.cu:65-152 context and
// peaks, 216-225 counters, 352-418 allocation and copies) and the host buffer
// pool of src/storage.cpp:44-128. One device (device 0), one engine stream.

#include "common.hpp"

#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace ehip {

thread_local hipStream_t t_capture = nullptr;

namespace {

thread_local std::string g_error;
thread_local uint64_t t_capture_graph = 0;  // serial of the graph this thread captures

struct Context {
    bool ok = false;
    int status = EHIP_ENODEV;
    std::string why;
    hipDeviceProp_t prop{};
};

std::once_flag g_init_once;
Context g_ctx;
std::atomic<int> g_enabled{1};
std::atomic<uint64_t> g_launched{0};
std::atomic<uint64_t> g_failed{0};
std::atomic<uint64_t> g_launch_serial{0};
int64_t g_fail_launch_at = 0;  // ENGINE_HIP_FAIL_LAUNCH
bool g_sync_each = false;      // ENGINE_HIP_SYNC

std::mutex g_stats_mu;
ehip_transfer_stats_t g_stats{};

void init_once() {
    const char* on = std::getenv("ENGINE_HIP");
    if (on != nullptr && std::strcmp(on, "0") == 0) g_enabled = 0;
    const char* fl = std::getenv("ENGINE_HIP_FAIL_LAUNCH");
    if (fl != nullptr) g_fail_launch_at = std::atoll(fl);
    const char* sy = std::getenv("ENGINE_HIP_SYNC");
    g_sync_each = sy != nullptr && std::strcmp(sy, "1") == 0;

    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) {
        g_ctx.why = std::string("no HIP device: ") +
                    (e != hipSuccess ? hipGetErrorString(e) : "device count is 0");
        return;
    }
    e = hipSetDevice(0);
    if (e == hipSuccess) e = hipGetDeviceProperties(&g_ctx.prop, 0);
    if (e != hipSuccess) {
        g_ctx.why = std::string("device 0: ") + hipGetErrorString(e);
        return;
    }
    if (std::strncmp(g_ctx.prop.gcnArchName, "gfx950", 6) != 0) {
        g_ctx.why = std::string("device 0 is ") + g_ctx.prop.gcnArchName +
                    ", this library is built for gfx950 only";
        return;
    }
    g_ctx.ok = true;
    g_ctx.status = EHIP_OK;
}

std::mutex& occupancy_mu() {
    static std::mutex mu;
    return mu;
}

std::vector<OccupancyKernel>& occupancy_kernels() {
    static std::vector<OccupancyKernel> all;
    return all;
}

}  // namespace

void register_occupancy(const OccupancyKernel* kernels, int count) {
    std::lock_guard<std::mutex> lock(occupancy_mu());
    occupancy_kernels().insert(occupancy_kernels().end(), kernels, kernels + count);
}

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int ready() {
    std::call_once(g_init_once, init_once);
    if (!g_ctx.ok) return fail(g_ctx.status, "%s", g_ctx.why.c_str());
    if (!g_enabled.load(std::memory_order_relaxed))
        return fail(EHIP_EDISABLED, "the HIP backend is switched off");
    return EHIP_OK;
}

int before_launch(const char* name) {
    const uint64_t serial = ++g_launch_serial;
    if (g_fail_launch_at > 0 && serial == static_cast<uint64_t>(g_fail_launch_at)) {
        ++g_failed;
        return fail(EHIP_ELAUNCH, "%s: launch %llu refused by ENGINE_HIP_FAIL_LAUNCH", name,
                    static_cast<unsigned long long>(serial));
    }
    return EHIP_OK;
}

int after_launch(const char* name, hipStream_t stream) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && g_sync_each && !capturing()) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        ++g_failed;
        return fail(EHIP_ELAUNCH, "%s: %s", name, hipGetErrorString(e));
    }
    ++g_launched;
    return EHIP_OK;
}

// ------------------------------------------------------------------ arena

namespace {

// The blocks a captured graph may touch: every block live when its capture
// began and every block handed out while it ran. Such a block, once freed, is
// held for the graph (replays still write or read it) instead of going back to
// the cache, until the graph is destroyed; allocations made during the capture
// itself reuse the graph's held blocks first.
struct GraphPool {
    std::unordered_set<void*> touched;
    std::unordered_map<size_t, std::vector<void*>> held;  // class size -> freed blocks
};

struct Arena {
    std::mutex mu;
    std::unordered_map<size_t, std::vector<void*>> cache;  // class size -> free blocks
    std::unordered_map<void*, size_t> live;                // block -> class size
    std::unordered_map<uint64_t, GraphPool> graphs;        // graph serial -> its blocks
    ehip_arena_stats_t stats{};
};

Arena& arena() {
    static Arena* a = new Arena();  // never destroyed: blocks outlive static teardown
    return *a;
}

// 256-byte granules up to 4 KiB, then four classes per power of two.
size_t size_class(size_t bytes) {
    size_t n = bytes < 256 ? 256 : (bytes + 255) & ~size_t(255);
    if (n <= 4096) return n;
    int e = 63 - __builtin_clzll(n);
    size_t step = (size_t(1) << e) / 4;
    return (n + step - 1) / step * step;
}

// Frees every cached block. Caller holds the lock.
void release_cache(Arena& a) {
    (void)hipDeviceSynchronize();
    for (auto& kv : a.cache) {
        for (void* p : kv.second) {
            (void)hipFree(p);
            a.stats.bytes_cached -= kv.first;
            a.stats.bytes_reserved -= kv.first;
        }
        kv.second.clear();
    }
}

}  // namespace

void* scratch(size_t bytes, int slot) {
    static std::mutex mu;
    static void* buf[kScratchSlots] = {};
    static size_t cap[kScratchSlots] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (bytes <= cap[slot]) return buf[slot];
    const size_t want = cap[slot] * 2 > bytes ? cap[slot] * 2 : bytes;
    void* p = nullptr;
    if (ehip_arena_alloc(want, &p) != EHIP_OK) return nullptr;
    if (buf[slot] != nullptr) ehip_arena_free(buf[slot]);
    buf[slot] = p;
    cap[slot] = want;
    return p;
}

}  // namespace ehip

using namespace ehip;

extern "C" {

const char* ehip_last_error(void) { return g_error.c_str(); }

int ehip_init(void) {
    std::call_once(g_init_once, init_once);
    if (!g_ctx.ok) return fail(g_ctx.status, "%s", g_ctx.why.c_str());
    return EHIP_OK;
}

int ehip_available(void) { return ehip_init() == EHIP_OK ? 1 : 0; }

int ehip_enabled(void) { return g_enabled.load(); }

void ehip_set_enabled(int on) {
    std::call_once(g_init_once, init_once);
    g_enabled = on ? 1 : 0;
}

int ehip_version_info(int* compiled, int* runtime, int* driver) {
    if (!compiled || !runtime || !driver) return fail(EHIP_EINVAL, "ehip_version_info: null output");
    *compiled = HIP_VERSION;
    *runtime = 0;
    *driver = 0;
    hipError_t e = hipRuntimeGetVersion(runtime);
    if (e != hipSuccess)
        return fail(EHIP_ENODEV, "hipRuntimeGetVersion: %s", hipGetErrorString(e));
    e = hipDriverGetVersion(driver);
    if (e != hipSuccess)
        return fail(EHIP_ENODEV, "hipDriverGetVersion: %s", hipGetErrorString(e));
    return EHIP_OK;
}

int ehip_kernel_occupancy(ehip_kernel_occupancy_t* out, int capacity, int* count) {
    if (count == nullptr || (capacity > 0 && out == nullptr))
        return fail(EHIP_EINVAL, "ehip_kernel_occupancy: null output");
    if (int rc = ehip_init()) return rc;
    const hipDeviceProp_t& p = g_ctx.prop;
    const int max_waves = p.maxThreadsPerMultiProcessor / 64;  // per CU
    const int64_t lds_cu = int64_t(p.maxSharedMemoryPerMultiProcessor);
    std::lock_guard<std::mutex> lock(occupancy_mu());
    const std::vector<OccupancyKernel>& all = occupancy_kernels();
    *count = int(all.size());
    for (int i = 0; i < int(all.size()) && i < capacity; ++i) {
        const OccupancyKernel& k = all[i];
        ehip_kernel_occupancy_t& o = out[i];
        std::memset(&o, 0, sizeof(o));
        std::snprintf(o.name, sizeof(o.name), "%s", k.name);
        o.block_threads = k.block_threads;
        hipFuncAttributes fa{};
        hipError_t e = hipFuncGetAttributes(&fa, k.func);
        if (e != hipSuccess)
            return fail(EHIP_ENODEV, "hipFuncGetAttributes(%s): %s", k.name, hipGetErrorString(e));
        int blocks = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, k.func, k.block_threads, 0);
        if (e != hipSuccess)
            return fail(EHIP_ENODEV, "hipOccupancyMaxActiveBlocksPerMultiprocessor(%s): %s",
                        k.name, hipGetErrorString(e));
        o.registers = fa.numRegs;
        o.lds_bytes = int64_t(fa.sharedSizeBytes);
        o.blocks_per_cu = blocks;
        const int waves = (k.block_threads + 63) / 64;
        o.occupancy = max_waves > 0 ? double(blocks * waves) / max_waves : 0.0;
        // What runs out first: LDS when one more block would not fit in it,
        // waves when one more block's waves would exceed the CU's, registers
        // otherwise.
        const char* lim = "registers";
        if (o.lds_bytes > 0 && (blocks + 1) * o.lds_bytes > lds_cu)
            lim = "lds";
        else if ((blocks + 1) * waves > max_waves)
            lim = "waves";
        std::snprintf(o.limiter, sizeof(o.limiter), "%s", lim);
    }
    return EHIP_OK;
}

int ehip_device_info(ehip_device_info_t* out) {
    if (out == nullptr) return fail(EHIP_EINVAL, "ehip_device_info: null output");
    if (int rc = ehip_init()) return rc;
    const hipDeviceProp_t& p = g_ctx.prop;
    std::memset(out, 0, sizeof *out);
    std::snprintf(out->name, sizeof out->name, "%s", p.name);
    std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width_bits = p.memoryBusWidth;
    out->total_memory = p.totalGlobalMem;
    out->lds_per_block = p.sharedMemPerBlock;
    out->l2_bytes = p.l2CacheSize;
    // fp32 MFMA retires 256 FLOP per clock per CU on CDNA4.
    out->peak_fp32_mfma_gflops = double(p.multiProcessorCount) * 256.0 * double(p.clockRate) * 1e-6;
    out->peak_hbm_gbs = 2.0 * double(p.memoryClockRate) * 1e3 * double(p.memoryBusWidth) / 8.0 * 1e-9;
    return EHIP_OK;
}

int ehip_synchronize(void) {
    if (int rc = ehip_init()) return rc;
    if (capturing()) return fail(EHIP_EINVAL, "synchronize: not allowed during a graph capture");
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(EHIP_ELAUNCH, "synchronize: %s", hipGetErrorString(e));
    return EHIP_OK;
}

int ehip_stream_synchronize(void* stream) {
    if (int rc = ehip_init()) return rc;
    if (stream == nullptr && capturing())
        return fail(EHIP_EINVAL, "stream synchronize: not allowed during a graph capture");
    hipError_t e = hipStreamSynchronize(as_stream(stream));
    if (e != hipSuccess) return fail(EHIP_ELAUNCH, "stream synchronize: %s", hipGetErrorString(e));
    return EHIP_OK;
}

uint64_t ehip_kernels_launched(void) { return g_launched.load(); }
uint64_t ehip_kernels_failed(void) { return g_failed.load(); }
void ehip_reset_counters(void) {
    g_launched = 0;
    g_failed = 0;
}

void ehip_fail_launch_after(int64_t n) {
    g_fail_launch_at = n > 0 ? int64_t(g_launch_serial.load()) + n : 0;
}

void ehip_transfer_stats(ehip_transfer_stats_t* out) {
    if (out == nullptr) return;
    std::lock_guard<std::mutex> lock(g_stats_mu);
    *out = g_stats;
}

void ehip_reset_transfer_stats(void) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_stats = ehip_transfer_stats_t{};
}

int ehip_arena_alloc(size_t bytes, void** out) {
    if (out == nullptr) return fail(EHIP_EINVAL, "ehip_arena_alloc: null output");
    *out = nullptr;
    if (int rc = ehip_init()) return rc;
    const size_t cls = size_class(bytes);
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    ++a.stats.allocations;
    GraphPool* pool = nullptr;
    if (t_capture_graph != 0) {
        auto g = a.graphs.find(t_capture_graph);
        if (g != a.graphs.end()) pool = &g->second;
    }
    if (pool != nullptr) {
        auto h = pool->held.find(cls);
        if (h != pool->held.end() && !h->second.empty()) {
            void* p = h->second.back();
            h->second.pop_back();
            a.live[p] = cls;
            a.stats.bytes_cached -= cls;
            a.stats.bytes_graph_held -= cls;
            a.stats.bytes_in_use += cls;
            *out = p;
            return EHIP_OK;
        }
    }
    auto it = a.cache.find(cls);
    if (it != a.cache.end() && !it->second.empty()) {
        void* p = it->second.back();
        it->second.pop_back();
        a.live[p] = cls;
        a.stats.bytes_cached -= cls;
        a.stats.bytes_in_use += cls;
        if (pool != nullptr) pool->touched.insert(p);
        *out = p;
        return EHIP_OK;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, cls);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        release_cache(a);
        e = hipMalloc(&p, cls);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(EHIP_ENOMEM, "hipMalloc(%zu): %s", cls, hipGetErrorString(e));
    }
    ++a.stats.driver_allocations;
    a.stats.bytes_reserved += cls;
    a.stats.bytes_in_use += cls;
    a.live[p] = cls;
    if (pool != nullptr) pool->touched.insert(p);
    *out = p;
    return EHIP_OK;
}

void ehip_arena_free(void* ptr) {
    if (ptr == nullptr) return;
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    auto it = a.live.find(ptr);
    if (it == a.live.end()) {
        std::fprintf(stderr, "ehip_arena_free: %p was not allocated by the arena\n", ptr);
        return;
    }
    const size_t cls = it->second;
    a.live.erase(it);
    a.stats.bytes_in_use -= cls;
    a.stats.bytes_cached += cls;
    // Held for the newest graph that may touch the block, if any.
    GraphPool* keep = nullptr;
    uint64_t newest = 0;
    for (auto& g : a.graphs)
        if (g.first > newest && g.second.touched.count(ptr) != 0) {
            newest = g.first;
            keep = &g.second;
        }
    if (keep != nullptr) {
        keep->held[cls].push_back(ptr);
        a.stats.bytes_graph_held += cls;
        return;
    }
    a.cache[cls].push_back(ptr);
}

int ehip_arena_trim(void) {
    if (int rc = ehip_init()) return rc;
    if (capturing()) return fail(EHIP_EINVAL, "ehip_arena_trim: not allowed during a graph capture");
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    release_cache(a);
    return EHIP_OK;
}

void ehip_arena_stats(ehip_arena_stats_t* out) {
    if (out == nullptr) return;
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    *out = a.stats;
}

}  // extern "C"

namespace {

// Host-to-device uploads up to a quarter of the ring go through a pinned
// staging ring: the bytes are copied into it on the host and the device copy
// is enqueued asynchronously, so an upload in the middle of a training step
// (labels, gather indices) neither waits for the queued kernels nor for the
// transfer. A ring region is reused only after the event recorded behind its
// copy has completed.
struct Staging {
    std::mutex mu;
    char* base = nullptr;
    size_t cap = size_t(64) << 20;
    size_t head = 0;
    struct Pending {
        size_t begin, end;
        hipEvent_t done;
    };
    std::vector<Pending> inflight;
};

Staging& staging() {
    static Staging* s = new Staging();
    return *s;
}

// Returns hipSuccess and sets *used when the upload went through the ring.
hipError_t staged_upload(void* dst, const void* src, size_t bytes, hipStream_t s, bool* used) {
    *used = false;
    Staging& st = staging();
    if (bytes > st.cap / 4) return hipSuccess;
    std::lock_guard<std::mutex> lock(st.mu);
    if (st.base == nullptr) {
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&st.base), st.cap, 0);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            st.base = nullptr;
            return hipSuccess;  // no pinned memory: the caller copies synchronously
        }
    }
    const size_t len = (bytes + 255) & ~size_t(255);
    if (st.head + len > st.cap) st.head = 0;
    const size_t b = st.head, e_ = st.head + len;
    for (auto it = st.inflight.begin(); it != st.inflight.end();) {
        const bool overlaps = it->begin < e_ && b < it->end;
        if (overlaps || hipEventQuery(it->done) == hipSuccess) {
            if (overlaps) {
                hipError_t e = hipEventSynchronize(it->done);
                if (e != hipSuccess) return e;
            }
            (void)hipEventDestroy(it->done);
            it = st.inflight.erase(it);
        } else {
            ++it;
        }
    }
    std::memcpy(st.base + b, src, bytes);
    hipError_t e = hipMemcpyAsync(dst, st.base + b, bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return e;
    hipEvent_t done;
    e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(done, s);
    if (e != hipSuccess) return e;
    st.inflight.push_back({b, e_, done});
    st.head = e_;
    *used = true;
    return hipSuccess;
}

int copy(void* dst, const void* src, size_t bytes, void* stream, hipMemcpyKind kind) {
    if (int rc = ehip_init()) return rc;
    if (bytes == 0) return EHIP_OK;
    if (dst == nullptr || src == nullptr) return fail(EHIP_EINVAL, "memcpy: null pointer");
    const auto t0 = std::chrono::steady_clock::now();
    hipStream_t s = as_stream(stream);
    if (capturing() && s == t_capture && kind != hipMemcpyDeviceToDevice)
        return fail(EHIP_EINVAL, "memcpy: a host transfer cannot be recorded into a graph");
    bool staged = false;
    hipError_t e = hipSuccess;
    if (kind == hipMemcpyHostToDevice) e = staged_upload(dst, src, bytes, s, &staged);
    if (e == hipSuccess && !staged) {
        e = hipMemcpyAsync(dst, src, bytes, kind, s);
        if (e == hipSuccess && kind != hipMemcpyDeviceToDevice) e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) return fail(EHIP_ELAUNCH, "memcpy: %s", hipGetErrorString(e));
    const double sec =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    std::lock_guard<std::mutex> lock(g_stats_mu);
    if (kind == hipMemcpyHostToDevice) {
        g_stats.to_device_bytes += bytes;
        ++g_stats.to_device_count;
        g_stats.to_device_seconds += sec;
    } else if (kind == hipMemcpyDeviceToHost) {
        g_stats.to_host_bytes += bytes;
        ++g_stats.to_host_count;
        g_stats.to_host_seconds += sec;
    } else {
        g_stats.device_to_device_bytes += bytes;
        ++g_stats.device_to_device_count;
    }
    return EHIP_OK;
}

}  // namespace

extern "C" {

int ehip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return copy(dst, src, bytes, stream, hipMemcpyHostToDevice);
}
int ehip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return copy(dst, src, bytes, stream, hipMemcpyDeviceToHost);
}
int ehip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return copy(dst, src, bytes, stream, hipMemcpyDeviceToDevice);
}

}  // extern "C"

// ------------------------------------------------------------------ graphs

namespace {

std::atomic<uint64_t> g_graph_serial{0};
thread_local hipStream_t t_capture_owned = nullptr;  // the stream this thread captures on

struct Graph {
    hipGraphExec_t exec = nullptr;
    uint64_t serial = 0;
};

// Hands a graph's held blocks to the next graph that may touch them, or back
// to the cache, and forgets the graph. Caller holds no lock.
void release_pool(uint64_t serial) {
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    auto it = a.graphs.find(serial);
    if (it == a.graphs.end()) return;
    GraphPool pool = std::move(it->second);
    a.graphs.erase(it);
    for (auto& kv : pool.held)
        for (void* p : kv.second) {
            GraphPool* next = nullptr;
            uint64_t newest = 0;
            for (auto& g : a.graphs)
                if (g.first > newest && g.second.touched.count(p) != 0) {
                    newest = g.first;
                    next = &g.second;
                }
            if (next != nullptr) {
                next->held[kv.first].push_back(p);
            } else {
                a.cache[kv.first].push_back(p);
                a.stats.bytes_graph_held -= kv.first;
            }
        }
}

void end_capture_state() {
    t_capture = nullptr;
    t_capture_graph = 0;
    if (t_capture_owned != nullptr) (void)hipStreamDestroy(t_capture_owned);
    t_capture_owned = nullptr;
}

}  // namespace

extern "C" {

int ehip_graph_begin(void) {
    EHIP_READY();
    if (capturing()) return fail(EHIP_EINVAL, "ehip_graph_begin: this thread is already capturing");
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(EHIP_ELAUNCH, "ehip_graph_begin: %s", hipGetErrorString(e));
    const uint64_t serial = ++g_graph_serial;
    {
        Arena& a = arena();
        std::lock_guard<std::mutex> lock(a.mu);
        GraphPool& pool = a.graphs[serial];
        pool.touched.reserve(a.live.size() * 2 + 64);
        for (const auto& kv : a.live) pool.touched.insert(kv.first);
    }
    e = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(s);
        release_pool(serial);
        return fail(EHIP_ELAUNCH, "ehip_graph_begin: %s", hipGetErrorString(e));
    }
    t_capture = s;
    t_capture_owned = s;
    t_capture_graph = serial;
    return EHIP_OK;
}

int ehip_graph_end(void** graph) {
    if (graph != nullptr) *graph = nullptr;
    if (!capturing()) return fail(EHIP_EINVAL, "ehip_graph_end: no capture in progress");
    const uint64_t serial = t_capture_graph;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(t_capture, &g);
    end_capture_state();
    hipGraphExec_t exec = nullptr;
    if (e == hipSuccess && graph == nullptr) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (g != nullptr) (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        release_pool(serial);
        return fail(EHIP_ELAUNCH, "ehip_graph_end: %s", hipGetErrorString(e));
    }
    *graph = new Graph{exec, serial};
    return EHIP_OK;
}

int ehip_graph_abort(void) {
    if (!capturing()) return EHIP_OK;
    const uint64_t serial = t_capture_graph;
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(t_capture, &g);
    (void)hipGetLastError();
    end_capture_state();
    if (g != nullptr) (void)hipGraphDestroy(g);
    release_pool(serial);
    return EHIP_OK;
}

int ehip_capturing(void) { return capturing() ? 1 : 0; }

int ehip_graph_launch(void* graph, void* stream) {
    EHIP_READY();
    if (graph == nullptr) return fail(EHIP_EINVAL, "ehip_graph_launch: null graph");
    if (capturing()) return fail(EHIP_EINVAL, "ehip_graph_launch: not allowed during a capture");
    if (int rc = before_launch("graph")) return rc;
    hipError_t e = hipGraphLaunch(static_cast<Graph*>(graph)->exec, as_stream(stream));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        ++g_failed;
        return fail(EHIP_ELAUNCH, "ehip_graph_launch: %s", hipGetErrorString(e));
    }
    ++g_launched;
    if (g_sync_each) {
        e = hipStreamSynchronize(as_stream(stream));
        if (e != hipSuccess) return fail(EHIP_ELAUNCH, "graph: %s", hipGetErrorString(e));
    }
    return EHIP_OK;
}

int ehip_graph_destroy(void* graph) {
    if (graph == nullptr) return EHIP_OK;
    if (capturing()) return fail(EHIP_EINVAL, "ehip_graph_destroy: not allowed during a capture");
    Graph* g = static_cast<Graph*>(graph);
    hipError_t e = hipDeviceSynchronize();  // the last replay has finished with the blocks
    if (g->exec != nullptr) (void)hipGraphExecDestroy(g->exec);
    release_pool(g->serial);
    delete g;
    if (e != hipSuccess) return fail(EHIP_ELAUNCH, "ehip_graph_destroy: %s", hipGetErrorString(e));
    return EHIP_OK;
}

}  // extern "C"

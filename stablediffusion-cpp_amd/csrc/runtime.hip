// runtime.hip - backend_hip runtime: device selection, the single stream, the
// device memory arena, pinned staging for host transfers, pointer-range
// validation, per-call scratch, timers and the C-ABI memory entry points.
//
// Counterparts in the reference: the lazy State (backend_cuda.cu:50-89), the
// caching allocator (:111-166) and upload/download/copy/zero (:168-175).
// Design differences:
//   * The arena reserves large segments with hipMalloc and carves blocks out
//     of them (best fit, coalescing on free), so op outputs never hit the HIP
//     allocator; blocks are 256-byte aligned and not zero-filled.
//   * Host transfers go through two pinned staging buffers with
//     hipMemcpyAsync on the library stream, double-buffered.
//   * Every op argument is checked against the live blocks before launch, so
//     a stale or host pointer is an SDH_ERR_INVALID, not a GPU fault.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "sdh_internal.hpp"

namespace sdh {

namespace {

thread_local std::string t_last_error;

constexpr size_t kAlign = 256;
constexpr size_t kStageBytes = 8u << 20;  // per staging buffer
constexpr int kTimerSlots = 16;
constexpr size_t kUncachedWords = 64u << 10;  // 256 KiB

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t env_mb(const char* name, size_t dflt) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    unsigned long long v = std::strtoull(e, &end, 10);
    return (end && *end == 0) ? (size_t)v << 20 : dflt;
}

// Arena: segments of device memory; free ranges indexed by address (for
// coalescing) and by size (for best fit). Blocks never span segments.
struct Arena {
    struct Seg {
        uintptr_t base;
        size_t bytes;
    };
    std::vector<Seg> segs;
    std::map<uintptr_t, size_t> free_by_addr;          // addr -> size
    std::multimap<size_t, uintptr_t> free_by_size;     // size -> addr
    std::map<uintptr_t, size_t> live;                  // addr -> rounded size
    std::map<uintptr_t, size_t> requested;             // addr -> bytes asked for
    size_t reserved = 0, in_use = 0, limit = 0;        // limit 0 = none

    int seg_of(uintptr_t a) const {
        for (size_t i = 0; i < segs.size(); ++i)
            if (a >= segs[i].base && a < segs[i].base + segs[i].bytes) return (int)i;
        return -1;
    }
    void erase_free(uintptr_t a, size_t sz) {
        free_by_addr.erase(a);
        auto r = free_by_size.equal_range(sz);
        for (auto it = r.first; it != r.second; ++it)
            if (it->second == a) {
                free_by_size.erase(it);
                return;
            }
    }
    void insert_free(uintptr_t a, size_t sz) {
        // coalesce with neighbours inside the same segment
        const int s = seg_of(a);
        auto next = free_by_addr.lower_bound(a);
        if (next != free_by_addr.end() && next->first == a + sz && seg_of(next->first) == s) {
            const uintptr_t na = next->first;
            const size_t nsz = next->second;
            erase_free(na, nsz);
            sz += nsz;
        }
        auto prev = free_by_addr.lower_bound(a);
        if (prev != free_by_addr.begin()) {
            --prev;
            if (prev->first + prev->second == a && seg_of(prev->first) == s) {
                const uintptr_t pa = prev->first;
                const size_t psz = prev->second;
                erase_free(pa, psz);
                a = pa;
                sz += psz;
            }
        }
        free_by_addr[a] = sz;
        free_by_size.emplace(sz, a);
    }
    bool grow(size_t need) {
        size_t bytes = round_up(std::max(need, (size_t)256 << 20), (size_t)2 << 20);
        if (limit && reserved + bytes > limit) {
            if (reserved + round_up(need, (size_t)2 << 20) > limit) return false;
            bytes = round_up(need, (size_t)2 << 20);
        }
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess || !p) {
            (void)hipGetLastError();
            return false;
        }
        segs.push_back({(uintptr_t)p, bytes});
        reserved += bytes;
        insert_free((uintptr_t)p, bytes);
        return true;
    }
    void* alloc(size_t bytes) {
        const size_t sz = round_up(bytes, kAlign);
        auto it = free_by_size.lower_bound(sz);
        if (it == free_by_size.end()) {
            if (!grow(sz)) return nullptr;
            it = free_by_size.lower_bound(sz);
            if (it == free_by_size.end()) return nullptr;
        }
        const uintptr_t a = it->second;
        const size_t fsz = it->first;
        erase_free(a, fsz);
        if (fsz > sz) insert_free(a + sz, fsz - sz);
        live[a] = sz;
        requested[a] = bytes;
        in_use += sz;
        return (void*)a;
    }
    bool release(void* p) {
        auto it = live.find((uintptr_t)p);
        if (it == live.end()) return false;
        const size_t sz = it->second;
        live.erase(it);
        requested.erase((uintptr_t)p);
        in_use -= sz;
        insert_free((uintptr_t)p, sz);
        return true;
    }
    void clear() {
        for (auto& s : segs) (void)hipFree((void*)s.base);
        segs.clear();
        free_by_addr.clear();
        free_by_size.clear();
        live.clear();
        requested.clear();
        reserved = in_use = 0;
    }
};

struct Runtime {
    std::mutex mu;
    bool inited = false;
    bool probed = false;
    bool present = false;
    char name[256] = {0};
    size_t total_mem = 0;
    int cus = 0;
    hipStream_t stream = nullptr;
    Arena arena;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
    hipEvent_t timers[kTimerSlots] = {};
    std::map<uintptr_t, size_t> external;
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    unsigned* counters = nullptr;
    size_t counter_count = 0;
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    // Words that kernels set when a bounded wait expired (see
    // arm_device_check): one per scratch area that such a launch used since
    // the last synchronisation, so a second area armed before the host reads
    // the first does not hide the first's failure.
    struct ArmedCheck {
        unsigned* word;
        const char* what;
        void (*failure)();
    };
    std::vector<ArmedCheck> armed;
    // Set between sdh_capture_begin and sdh_capture_end: the stream is being
    // recorded into a graph, so nothing may wait on it or grow a buffer
    // that queued work could still be reading.
    bool capturing = false;
    // Incremented by every sdh_capture_begin (capture_generation).
    unsigned capture_gen = 0;
    // Uncached device words for cross-workgroup exchange polled through the
    // scalar path (uncached_words): allocated once, never freed, because
    // memory of this kind that a kernel has read must outlive the process's
    // later allocations.
    unsigned* uncached = nullptr;
    size_t uncached_count = 0;
    // A vector of 1.0f for kernels that take a missing column vector as ones
    // (ones_vector).
    float* ones = nullptr;
    size_t ones_count = 0;
};

Runtime& rt() {
    static Runtime r;
    return r;
}

}  // namespace

std::recursive_mutex& op_mutex() {
    static std::recursive_mutex m;
    return m;
}

namespace {

void probe_locked(Runtime& r) {
    if (r.probed) return;
    r.probed = true;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        (void)hipGetLastError();
        return;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    r.present = true;
    std::snprintf(r.name, sizeof r.name, "%s (%s)", prop.name, prop.gcnArchName);
    r.total_mem = prop.totalGlobalMem;
    r.cus = prop.multiProcessorCount;
}

void init_locked(Runtime& r, size_t arena_bytes) {
    if (r.inited) return;
    probe_locked(r);
    if (!r.present) fail(SDH_ERR_UNAVAILABLE, "backend_hip: no HIP device available");
    hip_check(hipSetDevice(0), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking), "hipStreamCreate");
    for (int i = 0; i < 2; ++i) {
        hip_check(hipHostMalloc(&r.stage[i], kStageBytes, hipHostMallocDefault), "hipHostMalloc(staging)");
        hip_check(hipEventCreateWithFlags(&r.stage_ev[i], hipEventDisableTiming), "hipEventCreate");
    }
    for (int i = 0; i < kTimerSlots; ++i) hip_check(hipEventCreate(&r.timers[i]), "hipEventCreate(timer)");
    r.arena.limit = env_mb("SDH_ARENA_LIMIT_MB", 0);
    const size_t first = arena_bytes ? arena_bytes : env_mb("SDH_ARENA_MB", (size_t)1024 << 20);
    if (first && !r.arena.grow(first))
        fail(SDH_ERR_OOM, "backend_hip: cannot reserve the initial arena segment of " + std::to_string(first) + " bytes");
    gn_fixed_scratch_setup();
    if (!r.uncached) {
        // kept across sdh_shutdown and re-initialisation (see Runtime::uncached);
        // without it the kernels that would poll it poll ordinary memory instead
        void* p = nullptr;
        if (hipExtMallocWithFlags(&p, kUncachedWords * sizeof(unsigned), hipDeviceMallocUncached) == hipSuccess && p) {
            zero_device(p, kUncachedWords * sizeof(unsigned));
            r.uncached = (unsigned*)p;
            r.uncached_count = kUncachedWords;
        } else {
            (void)hipGetLastError();
        }
    }
    r.inited = true;
}

void range_check_locked(Runtime& r, const void* p, size_t bytes, const char* op, const char* what) {
    const uintptr_t a = (uintptr_t)p;
    if (!p) fail(SDH_ERR_INVALID, std::string(op) + ": " + what + " is NULL");
    auto inside = [&](const std::map<uintptr_t, size_t>& m) {
        auto it = m.upper_bound(a);
        if (it == m.begin()) return false;
        --it;
        return a >= it->first && a - it->first <= it->second && bytes <= it->second - (a - it->first);
    };
    // exact extents: the bytes the caller asked for, not the rounded block
    if (inside(r.arena.requested) || inside(r.external)) return;
    fail(SDH_ERR_INVALID, std::string(op) + ": " + what + " (" + std::to_string(bytes) +
                              " bytes) is not inside a live backend_hip allocation");
}

// Refuses what would wait on the stream (or replace a buffer that queued
// work may read) while the stream is being recorded into a graph.
void not_capturing_locked(const Runtime& r, const char* what) {
    if (r.capturing)
        fail(SDH_ERR_INVALID, std::string(what) +
                                  ": not allowed while the library stream is being captured (sdh_capture_begin); "
                                  "run the op once before capturing so its scratch is sized");
}

// Reads and clears every word registered by arm_device_check since the
// last check; the stream must be synchronised. Reports the first that was
// set, after clearing them all and running every failed op's callback.
void device_check_locked(Runtime& r) {
    if (r.armed.empty()) return;
    std::vector<Runtime::ArmedCheck> armed;
    armed.swap(r.armed);
    const char* failed = nullptr;
    for (const auto& a : armed) {
        unsigned v = 0;
        hip_check(hipMemcpyAsync(&v, a.word, sizeof v, hipMemcpyDeviceToHost, r.stream), "hipMemcpyAsync(device check)");
        hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
        if (!v) continue;
        const unsigned z = 0;
        hip_check(hipMemcpyAsync(a.word, &z, sizeof z, hipMemcpyHostToDevice, r.stream), "hipMemcpyAsync(device check)");
        hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
        if (a.failure) a.failure();
        if (!failed) failed = a.what;
    }
    if (failed)
        fail(SDH_ERR_HIP, std::string(failed) +
                              ": a bounded wait inside the kernel expired; the affected outputs hold NaN (and, for "
                              "a call made in place, the same parts of its input)");
}

}  // namespace

// ---------------------------------------------------------------------------
// internal API
// ---------------------------------------------------------------------------
void set_last_error(const char* msg) { t_last_error = msg; }

void fail(int status, const std::string& msg) { throw Error(status, msg); }

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(SDH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    }
}

int64_t launch_items() {
    static const int64_t v = [] {
        const char* e = std::getenv("SDH_LAUNCH_ITEMS");
        if (!e || !*e) return kMaxGridItems;
        char* end = nullptr;
        const long long n = std::strtoll(e, &end, 10);
        if (!end || *end != 0 || n <= 0) return kMaxGridItems;
        return std::max<int64_t>(1024, std::min<int64_t>(n, kMaxGridItems));
    }();
    return v;
}

void launched(const char* op) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) fail(SDH_ERR_HIP, std::string(op) + ": kernel launch failed: " + hipGetErrorString(e));
}

void ensure_init() {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    init_locked(r, 0);
}

bool initialized() {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    return r.inited;
}

hipStream_t stream() { return rt().stream; }
bool capturing() {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    return r.capturing;
}
unsigned capture_generation() {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    return r.capture_gen;
}
int num_cus() { return rt().cus > 0 ? rt().cus : 256; }

void check_range(const void* p, size_t bytes, const char* op, const char* what) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    range_check_locked(r, p, bytes, op, what);
}

void* scratch(size_t bytes) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    if (bytes > r.scratch_bytes) {
        not_capturing_locked(r, "backend_hip scratch");
        if (r.scratch) {
            // Work queued earlier may still read the old scratch.
            hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
            r.arena.release(r.scratch);
        }
        r.scratch_bytes = round_up(std::max(bytes, (size_t)1 << 20), kAlign);
        r.scratch = r.arena.alloc(r.scratch_bytes);
        if (!r.scratch) {
            r.scratch_bytes = 0;
            fail(SDH_ERR_OOM, "backend_hip: arena exhausted allocating scratch");
        }
    }
    return r.scratch;
}

void* workspace(size_t bytes) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    if (bytes > r.workspace_bytes) {
        not_capturing_locked(r, "backend_hip GEMM workspace");
        if (r.workspace) {
            hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
            r.arena.release(r.workspace);
        }
        r.workspace_bytes = round_up(bytes, kAlign);
        r.workspace = r.arena.alloc(r.workspace_bytes);
        if (!r.workspace) {
            r.workspace_bytes = 0;
            fail(SDH_ERR_OOM, "backend_hip: arena exhausted allocating the GEMM workspace");
        }
    }
    return r.workspace;
}

void arm_device_check(unsigned* word, const char* what, void (*on_failure)()) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    for (auto& a : r.armed)
        if (a.word == word) {  // the same area again: the word still holds both launches' outcome
            if (!a.failure) a.failure = on_failure;
            return;
        }
    r.armed.push_back({word, what, on_failure});
}

__global__ void k_fill_ones(float* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 1.0f;
}

const float* ones_vector(size_t n) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    if (n > r.ones_count) {
        not_capturing_locked(r, "backend_hip ones vector");
        if (r.ones) {
            hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
            r.arena.release(r.ones);
        }
        const size_t cnt = round_up(std::max(n, (size_t)4096), 64);
        r.ones = (float*)r.arena.alloc(cnt * sizeof(float));
        if (!r.ones) {
            r.ones_count = 0;
            fail(SDH_ERR_OOM, "backend_hip: arena exhausted allocating the ones vector");
        }
        k_fill_ones<<<(unsigned)std::min<size_t>((cnt + 255) / 256, 1024), 256, 0, r.stream>>>(r.ones, cnt);
        hip_check(hipGetLastError(), "k_fill_ones");
        r.ones_count = cnt;
    }
    return r.ones;
}

unsigned* uncached_words(size_t count) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    if (!r.uncached || count > r.uncached_count) return nullptr;
    return r.uncached;
}

unsigned* counters(size_t count) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    if (count > r.counter_count) {
        not_capturing_locked(r, "backend_hip counters");
        if (r.counters) {
            hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
            device_check_locked(r);  // the registered word may live in the old block
            r.arena.release(r.counters);
        }
        const size_t n = std::max(count, (size_t)4096);
        r.counters = (unsigned*)r.arena.alloc(n * sizeof(unsigned));
        if (!r.counters) {
            r.counter_count = 0;
            fail(SDH_ERR_OOM, "backend_hip: arena exhausted allocating counters");
        }
        zero_device(r.counters, n * sizeof(unsigned));
        r.counter_count = n;
    }
    return r.counters;
}

}  // namespace sdh

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace sdh;

extern "C" {

const char* sdh_last_error(void) { return t_last_error.c_str(); }

int sdh_available(void) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    probe_locked(r);
    return r.present ? 1 : 0;
}

const char* sdh_device_name(void) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    probe_locked(r);
    return r.present ? r.name : "";
}

size_t sdh_device_memory(void) {
    Runtime& r = rt();
    std::lock_guard<std::mutex> lk(r.mu);
    probe_locked(r);
    return r.present ? r.total_mem : 0;
}

int sdh_init(size_t arena_bytes) {
    return guarded([&] {
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        init_locked(r, arena_bytes);
    });
}

int sdh_shutdown(void) {
    return guarded([&] {
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (!r.inited) return;
        not_capturing_locked(r, "sdh_shutdown");
        hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
        r.arena.clear();
        r.external.clear();
        r.scratch = nullptr;
        r.scratch_bytes = 0;
        r.counters = nullptr;
        r.counter_count = 0;
        r.ones = nullptr;
        r.ones_count = 0;
        r.armed.clear();
        r.workspace = nullptr;
        r.workspace_bytes = 0;
        for (int i = 0; i < 2; ++i) {
            (void)hipHostFree(r.stage[i]);
            (void)hipEventDestroy(r.stage_ev[i]);
            r.stage[i] = nullptr;
        }
        for (int i = 0; i < kTimerSlots; ++i) (void)hipEventDestroy(r.timers[i]);
        (void)hipStreamDestroy(r.stream);
        r.stream = nullptr;
        r.inited = false;
    });
}

int sdh_malloc(size_t bytes, void** out) {
    return guarded([&] {
        if (!out) fail(SDH_ERR_INVALID, "sdh_malloc: out is NULL");
        *out = nullptr;
        if (bytes == 0) return;
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        void* p = r.arena.alloc(bytes);
        if (!p)
            fail(SDH_ERR_OOM, "sdh_malloc: arena exhausted (" + std::to_string(bytes) + " bytes requested, " +
                                  std::to_string(r.arena.in_use) + " in use, " + std::to_string(r.arena.reserved) +
                                  " reserved)");
        *out = p;
    });
}

int sdh_free(void* p) {
    return guarded([&] {
        if (!p) return;
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (!r.inited) fail(SDH_ERR_INVALID, "sdh_free: backend not initialised");
        // Kernels queued earlier may still use the block; a later op reusing
        // it is ordered after them on the same stream, so no wait is needed.
        if (!r.arena.release(p)) fail(SDH_ERR_INVALID, "sdh_free: pointer is not a live backend_hip block");
    });
}

int sdh_upload(void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        if (bytes == 0) return;
        if (!src) fail(SDH_ERR_INVALID, "sdh_upload: src is NULL");
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        not_capturing_locked(r, "sdh_upload");
        range_check_locked(r, dst, bytes, "sdh_upload", "dst");
        size_t off = 0;
        int b = 0;
        while (off < bytes) {
            const size_t n = std::min(kStageBytes, bytes - off);
            hip_check(hipEventSynchronize(r.stage_ev[b]), "hipEventSynchronize(staging)");
            std::memcpy(r.stage[b], (const char*)src + off, n);
            hip_check(hipMemcpyAsync((char*)dst + off, r.stage[b], n, hipMemcpyHostToDevice, r.stream),
                      "hipMemcpyAsync(upload)");
            hip_check(hipEventRecord(r.stage_ev[b], r.stream), "hipEventRecord(staging)");
            off += n;
            b ^= 1;
        }
    });
}

int sdh_download(void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        if (bytes == 0) return;
        if (!dst) fail(SDH_ERR_INVALID, "sdh_download: dst is NULL");
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        not_capturing_locked(r, "sdh_download");
        range_check_locked(r, src, bytes, "sdh_download", "src");
        // Pipeline: copy chunk i into staging buffer i%2 while the host drains
        // chunk i-1 from the other buffer.
        size_t off = 0, prev_off = 0, prev_n = 0;
        int b = 0;
        while (off < bytes) {
            const size_t n = std::min(kStageBytes, bytes - off);
            hip_check(hipEventSynchronize(r.stage_ev[b]), "hipEventSynchronize(staging)");
            hip_check(hipMemcpyAsync(r.stage[b], (const char*)src + off, n, hipMemcpyDeviceToHost, r.stream),
                      "hipMemcpyAsync(download)");
            hip_check(hipEventRecord(r.stage_ev[b], r.stream), "hipEventRecord(staging)");
            if (prev_n) {
                hip_check(hipEventSynchronize(r.stage_ev[b ^ 1]), "hipEventSynchronize(staging)");
                std::memcpy((char*)dst + prev_off, r.stage[b ^ 1], prev_n);
            }
            prev_off = off;
            prev_n = n;
            off += n;
            b ^= 1;
        }
        hip_check(hipEventSynchronize(r.stage_ev[b ^ 1]), "hipEventSynchronize(staging)");
        std::memcpy((char*)dst + prev_off, r.stage[b ^ 1], prev_n);
        hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
        device_check_locked(r);
    });
}

int sdh_copy(void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        if (bytes == 0) return;
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        range_check_locked(r, dst, bytes, "sdh_copy", "dst");
        range_check_locked(r, src, bytes, "sdh_copy", "src");
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, r.stream), "hipMemcpyAsync(copy)");
    });
}

int sdh_synchronize(void) {
    return guarded([&] {
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (!r.inited) return;
        not_capturing_locked(r, "sdh_synchronize");
        hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
        device_check_locked(r);
    });
}

int sdh_register_external(void* p, size_t bytes) {
    return guarded([&] {
        if (!p || bytes == 0) fail(SDH_ERR_INVALID, "sdh_register_external: empty range");
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        r.external[(uintptr_t)p] = bytes;
    });
}

int sdh_unregister_external(void* p) {
    return guarded([&] {
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (!r.external.erase((uintptr_t)p)) fail(SDH_ERR_INVALID, "sdh_unregister_external: range not registered");
    });
}

int sdh_memory_stats(size_t* reserved, size_t* in_use) {
    return guarded([&] {
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (reserved) *reserved = r.arena.reserved;
        if (in_use) *in_use = r.arena.in_use;
    });
}

int sdh_timer_record(int slot) {
    return guarded([&] {
        if (slot < 0 || slot >= kTimerSlots) fail(SDH_ERR_INVALID, "sdh_timer_record: slot out of range");
        ensure_init();
        Runtime& r = rt();
        hip_check(hipEventRecord(r.timers[slot], r.stream), "hipEventRecord(timer)");
    });
}

int sdh_timer_elapsed(int a, int b, float* ms) {
    return guarded([&] {
        if (a < 0 || a >= kTimerSlots || b < 0 || b >= kTimerSlots || !ms)
            fail(SDH_ERR_INVALID, "sdh_timer_elapsed: bad slot or NULL output");
        ensure_init();
        Runtime& r = rt();
        {
            std::lock_guard<std::mutex> lk(r.mu);
            not_capturing_locked(r, "sdh_timer_elapsed");
        }
        hip_check(hipEventSynchronize(r.timers[b]), "hipEventSynchronize(timer)");
        hip_check(hipEventElapsedTime(ms, r.timers[a], r.timers[b]), "hipEventElapsedTime");
    });
}

// Graph capture of the library stream: the launches of the ops called
// between begin and end are recorded, not run, and replay as one graph with
// no host work between them. Ops whose scratch would have to grow, and
// everything that waits on the stream, are refused while capturing.
int sdh_capture_begin(void) {
    return guarded([&] {
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (r.capturing) fail(SDH_ERR_INVALID, "sdh_capture_begin: a capture is already open");
        hip_check(hipStreamBeginCapture(r.stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
        r.capturing = true;
        ++r.capture_gen;
    });
}

int sdh_capture_end(void** graph) {
    return guarded([&] {
        if (!graph) fail(SDH_ERR_INVALID, "sdh_capture_end: graph is NULL");
        *graph = nullptr;
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        if (!r.capturing) fail(SDH_ERR_INVALID, "sdh_capture_end: no capture is open");
        r.capturing = false;
        hipGraph_t g = nullptr;
        hip_check(hipStreamEndCapture(r.stream, &g), "hipStreamEndCapture");
        if (!g) fail(SDH_ERR_HIP, "sdh_capture_end: the capture produced no graph");
        hipGraphExec_t e = nullptr;
        const hipError_t ie = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        hip_check(ie, "hipGraphInstantiate");
        *graph = (void*)e;
    });
}

int sdh_graph_launch(void* graph) {
    return guarded([&] {
        if (!graph) fail(SDH_ERR_INVALID, "sdh_graph_launch: graph is NULL");
        ensure_init();
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        not_capturing_locked(r, "sdh_graph_launch");
        hip_check(hipGraphLaunch((hipGraphExec_t)graph, r.stream), "hipGraphLaunch");
    });
}

int sdh_graph_destroy(void* graph) {
    return guarded([&] {
        if (!graph) return;
        Runtime& r = rt();
        std::lock_guard<std::mutex> lk(r.mu);
        not_capturing_locked(r, "sdh_graph_destroy");
        // a launch of it may still be queued
        hip_check(hipStreamSynchronize(r.stream), "hipStreamSynchronize");
        hip_check(hipGraphExecDestroy((hipGraphExec_t)graph), "hipGraphExecDestroy");
    });
}

}  // extern "C"

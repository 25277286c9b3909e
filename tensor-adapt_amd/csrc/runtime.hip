// runtime.hip — status reporting and the per-device scratch pool behind the
// C-ABI.
//
// Scratch: ops that need temporary device memory (reduction partials) take
// it from grow-only buffers kept per (device, stream).  Work on one stream
// is ordered, so reusing a stream's buffers across its calls is safe, and
// ops on two streams of one device never share one; growing a buffer
// synchronises its stream before freeing the old one.  This replaces the
// reference's per-call cudaMalloc/cudaFree inside sdpa_* (ops.cu:595-680,
// 727-869), which synchronised the device on every attention call.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ta_internal.hpp"

namespace ta {

static thread_local std::string g_err;

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(-3, "%s: launch failed: %s", what, hipGetErrorString(e));
    return 0;
}

struct Scratch {
    void* ptr = nullptr;
    size_t bytes = 0;
};
static std::mutex g_scratch_mu;
constexpr int kSlots = 4;  // 0: reduction partials, 1: operand staging, 2-3: spare
struct ScratchSet {
    Scratch slot[kSlots];
};
static std::map<std::pair<int, hipStream_t>, ScratchSet> g_scratch;

// Slot `slot` of the pool of (current device, stream s), at least `bytes`
// long.  Two buffers an op needs at once must come from different slots.
void* scratch_get(size_t bytes, hipStream_t s, int slot) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
    if (slot < 0 || slot >= kSlots) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch& sc = g_scratch[{dev, s}].slot[slot];
    if (sc.bytes >= bytes && sc.ptr) return sc.ptr;
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    want = (want + 255) & ~(size_t)255;
    if (sc.ptr) {
        // earlier launches on this stream may still read the old buffer
        if (hipStreamSynchronize(s) != hipSuccess) return nullptr;
        (void)hipFree(sc.ptr);
        sc.ptr = nullptr;
        sc.bytes = 0;
    }
    if (hipMalloc(&sc.ptr, want) != hipSuccess) {
        sc.ptr = nullptr;
        return nullptr;
    }
    sc.bytes = want;
    return sc.ptr;
}

// Caching allocator behind the host API's Tensor (ta_mem_alloc/free).
// Sizes round up to a power of two below 2 MiB and to a multiple of 2 MiB
// above; a freed block goes back to its device's bin and is handed out again
// without hipFree/hipMalloc.  Reuse is ordered by the device's one stream:
// the caller frees a block only after the work that reads it is enqueued on
// that stream (what the Tensor destructor does).
struct MemPool {
    std::map<size_t, std::vector<void*>> bins;  // size class -> free blocks
    std::unordered_map<void*, size_t> live;     // block -> size class
    size_t cached = 0, in_use = 0;
};
static std::mutex g_mem_mu;
static MemPool g_mem[64];

static size_t mem_class(size_t bytes) {
    const size_t two_mib = (size_t)2 << 20;
    if (bytes <= 256) return 256;
    if (bytes >= two_mib) return (bytes + two_mib - 1) / two_mib * two_mib;
    size_t c = 512;
    while (c < bytes) c <<= 1;
    return c;
}

// Kernel-level timing (measurement only).  When kernel id `sel` is
// selected, every launch of that kernel carries a pair of events in its own
// dispatch (tlaunch), with the algorithmic flops and HBM bytes of the launch;
// ta_kprof_read() waits for the events and sums.
struct KProf {
    std::atomic<int> sel{-1};
    std::atomic<bool> paused{false};  // selected, but launches are not timed for now
    std::vector<hipEvent_t> ev;
    std::vector<double> flops, bytes;
    std::vector<char> valid;  // the slot's launch carried its events
    size_t used = 0;          // slots reserved since the last read
    const char* name[KP_COUNT] = {};
};
static std::mutex g_kp_mu;
static KProf g_kp;
static thread_local KpArm t_kp_arm;

KpArm& kprof_arm() { return t_kp_arm; }

bool kprof_pool_pair(hipEvent_t* start, hipEvent_t* stop) {
    KpArm& k = t_kp_arm;
    if (!k.pool || !k.npairs) return false;
    const size_t i = *k.npairs;
    while (k.pool->size() < 2 * (i + 1)) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return false;
        k.pool->push_back(e);
    }
    *start = (*k.pool)[2 * i];
    *stop = (*k.pool)[2 * i + 1];
    *k.npairs = i + 1;
    return true;
}

// Each timed call reserves its own slot (event pair) here, so calls on
// several threads never share one; kprof_end marks whether the launch
// carried the events.
bool kprof_begin(int kid, hipStream_t s) {
    (void)s;
    t_kp_arm.start = t_kp_arm.stop = nullptr;
    t_kp_arm.used = false;
    if (g_kp.sel.load() != kid || g_kp.paused.load()) return false;
    std::lock_guard<std::mutex> lk(g_kp_mu);
    const size_t i = g_kp.used;
    while (g_kp.ev.size() < 2 * (i + 1)) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return false;
        g_kp.ev.push_back(e);
    }
    if (g_kp.flops.size() <= i) {
        g_kp.flops.resize(i + 1);
        g_kp.bytes.resize(i + 1);
        g_kp.valid.resize(i + 1);
    }
    g_kp.valid[i] = 0;
    g_kp.used = i + 1;
    t_kp_arm.start = g_kp.ev[2 * i];
    t_kp_arm.stop = g_kp.ev[2 * i + 1];
    t_kp_arm.slot = i;
    return true;
}

void kprof_end(int kid, hipStream_t s, double flops, double bytes, const char* name) {
    (void)s;
    const bool armed = t_kp_arm.stop != nullptr, used = t_kp_arm.used;
    const size_t i = t_kp_arm.slot;
    t_kp_arm.start = t_kp_arm.stop = nullptr;
    t_kp_arm.used = false;
    if (!armed) return;
    std::lock_guard<std::mutex> lk(g_kp_mu);
    if (i >= g_kp.used) return;  // a selection since kprof_begin dropped the slot
    g_kp.flops[i] = flops;
    g_kp.bytes[i] = bytes;
    g_kp.valid[i] = used ? 1 : 0;
    if (used) g_kp.name[kid] = name;
}

}  // namespace ta

extern "C" {

int ta_kprof_select(int kid) {
    TA_REQUIRE(kid >= -1 && kid < ta::KP_COUNT, "kprof_select: bad kernel id %d", kid);
    std::lock_guard<std::mutex> lk(ta::g_kp_mu);
    ta::g_kp.sel = kid;
    ta::g_kp.used = 0;
    ta::g_kp.paused = false;
    return 0;
}

int ta_kprof_pause(int paused) {
    std::lock_guard<std::mutex> lk(ta::g_kp_mu);
    ta::g_kp.paused = paused != 0;
    return 0;
}

int ta_kprof_read(double* ms, int64_t* launches, double* flops, double* bytes) {
    std::lock_guard<std::mutex> lk(ta::g_kp_mu);
    double tms = 0, tf = 0, tb = 0;
    int64_t n = 0;
    for (size_t i = 0; i < ta::g_kp.used; i++) {
        if (!ta::g_kp.valid[i]) continue;
        n++;
        TA_HIP(hipEventSynchronize(ta::g_kp.ev[2 * i + 1]));
        float x = 0.f;
        TA_HIP(hipEventElapsedTime(&x, ta::g_kp.ev[2 * i], ta::g_kp.ev[2 * i + 1]));
        tms += x;
        tf += ta::g_kp.flops[i];
        tb += ta::g_kp.bytes[i];
    }
    if (ms) *ms = tms;
    if (launches) *launches = n;
    if (flops) *flops = tf;
    if (bytes) *bytes = tb;
    ta::g_kp.used = 0;
    return 0;
}

int ta_mem_alloc(void** ptr, int64_t bytes, int device) {
    TA_REQUIRE(ptr && bytes >= 0 && device >= 0 && device < 64, "mem_alloc: bad argument");
    *ptr = nullptr;
    if (bytes == 0) return 0;
    TA_HIP(hipSetDevice(device));
    size_t c = ta::mem_class((size_t)bytes);
    std::lock_guard<std::mutex> lk(ta::g_mem_mu);
    ta::MemPool& mp = ta::g_mem[device];
    auto it = mp.bins.find(c);
    if (it != mp.bins.end() && !it->second.empty()) {
        *ptr = it->second.back();
        it->second.pop_back();
        mp.cached -= c;
    } else {
        hipError_t e = hipMalloc(ptr, c);
        if (e != hipSuccess) {
            // give the cached blocks back and try once more
            (void)hipDeviceSynchronize();
            for (auto& kv : mp.bins)
                for (void* q : kv.second) (void)hipFree(q);
            mp.bins.clear();
            mp.cached = 0;
            (void)hipGetLastError();
            e = hipMalloc(ptr, c);
        }
        if (e != hipSuccess) {
            *ptr = nullptr;
            return ta::set_error(-2, "mem_alloc: %lld bytes on device %d: %s", (long long)bytes,
                                 device, hipGetErrorString(e));
        }
    }
    mp.live[*ptr] = c;
    mp.in_use += c;
    return 0;
}

int ta_mem_free(void* ptr, int device) {
    if (!ptr) return 0;
    TA_REQUIRE(device >= 0 && device < 64, "mem_free: bad device %d", device);
    std::lock_guard<std::mutex> lk(ta::g_mem_mu);
    ta::MemPool& mp = ta::g_mem[device];
    auto it = mp.live.find(ptr);
    TA_REQUIRE(it != mp.live.end(), "mem_free: %p was not allocated by ta_mem_alloc on device %d",
               ptr, device);
    size_t c = it->second;
    mp.live.erase(it);
    mp.in_use -= c;
    mp.bins[c].push_back(ptr);
    mp.cached += c;
    return 0;
}

int ta_mem_stats(int device, int64_t* in_use, int64_t* cached) {
    TA_REQUIRE(device >= 0 && device < 64, "mem_stats: bad device %d", device);
    std::lock_guard<std::mutex> lk(ta::g_mem_mu);
    if (in_use) *in_use = (int64_t)ta::g_mem[device].in_use;
    if (cached) *cached = (int64_t)ta::g_mem[device].cached;
    return 0;
}

int ta_mem_trim(int device) {
    TA_REQUIRE(device >= 0 && device < 64, "mem_trim: bad device %d", device);
    TA_HIP(hipSetDevice(device));
    TA_HIP(hipDeviceSynchronize());
    std::lock_guard<std::mutex> lk(ta::g_mem_mu);
    ta::MemPool& mp = ta::g_mem[device];
    for (auto& kv : mp.bins)
        for (void* q : kv.second) (void)hipFree(q);
    mp.bins.clear();
    mp.cached = 0;
    return 0;
}

int ta_scratch_release(void* stream) {
    hipStream_t s = (hipStream_t)stream;
    int dev = 0;
    TA_HIP(hipGetDevice(&dev));
    TA_HIP(hipStreamSynchronize(s));
    std::lock_guard<std::mutex> lk(ta::g_scratch_mu);
    auto it = ta::g_scratch.find({dev, s});
    if (it == ta::g_scratch.end()) return 0;
    for (auto& sc : it->second.slot)
        if (sc.ptr) (void)hipFree(sc.ptr);
    ta::g_scratch.erase(it);
    return 0;
}

const char* ta_kprof_name(int kid) {
    if (kid < 0 || kid >= ta::KP_COUNT) return "";
    const char* n = ta::g_kp.name[kid];
    return n ? n : "";
}

const char* ta_last_error(void) { return ta::g_err.c_str(); }

const char* ta_version(void) { return "tensor-adapt-amd gfx950 " __DATE__ " " __TIME__; }

}  // extern "C"

// runtime.hip — status reporting and the per-device scratch pool behind the
// C-ABI.
//
// Scratch: ops that need temporary device memory (reduction partials) take
// it from one grow-only buffer per device.  Work on one stream is ordered,
// so reusing the buffer across calls on the same stream is safe; growing it
// synchronises the device before freeing the old buffer.  This replaces the
// reference's per-call cudaMalloc/cudaFree inside sdpa_* (ops.cu:595-680,
// 727-869), which synchronised the device on every attention call.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>
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
static Scratch g_scratch[64][kSlots];

// Slot `slot` of the current device's pool, at least `bytes` long.  Two
// buffers an op needs at once must come from different slots.
void* scratch_get(size_t bytes, hipStream_t s, int slot) {
    (void)s;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (slot < 0 || slot >= kSlots) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch& sc = g_scratch[dev][slot];
    if (sc.bytes >= bytes && sc.ptr) return sc.ptr;
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    want = (want + 255) & ~(size_t)255;
    if (sc.ptr) {
        // earlier launches on any stream may still read the old buffer
        if (hipDeviceSynchronize() != hipSuccess) return nullptr;
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

// Kernel-level timing (measurement only).  When kernel id `sel` is
// selected, every launch of that kernel is bracketed with a pair of events
// recorded on the stream it is launched on, with the algorithmic flops and
// HBM bytes of the launch; ta_kprof_read() waits for the events and sums.
struct KProf {
    int sel = -1;
    std::vector<hipEvent_t> ev;
    std::vector<double> flops, bytes;
    size_t used = 0;
    const char* name[KP_COUNT] = {};
};
static std::mutex g_kp_mu;
static KProf g_kp;

bool kprof_begin(int kid, hipStream_t s) {
    if (g_kp.sel != kid) return false;
    std::lock_guard<std::mutex> lk(g_kp_mu);
    size_t i = g_kp.used;
    while (g_kp.ev.size() < 2 * (i + 1)) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return false;
        g_kp.ev.push_back(e);
    }
    return hipEventRecord(g_kp.ev[2 * i], s) == hipSuccess;
}

void kprof_end(int kid, hipStream_t s, double flops, double bytes, const char* name) {
    if (g_kp.sel != kid) return;
    std::lock_guard<std::mutex> lk(g_kp_mu);
    size_t i = g_kp.used;
    if (g_kp.ev.size() < 2 * (i + 1) || hipEventRecord(g_kp.ev[2 * i + 1], s) != hipSuccess)
        return;
    if (g_kp.flops.size() <= i) {
        g_kp.flops.resize(i + 1);
        g_kp.bytes.resize(i + 1);
    }
    g_kp.flops[i] = flops;
    g_kp.bytes[i] = bytes;
    g_kp.name[kid] = name;
    g_kp.used = i + 1;
}

}  // namespace ta

extern "C" {

int ta_kprof_select(int kid) {
    TA_REQUIRE(kid >= -1 && kid < ta::KP_COUNT, "kprof_select: bad kernel id %d", kid);
    std::lock_guard<std::mutex> lk(ta::g_kp_mu);
    ta::g_kp.sel = kid;
    ta::g_kp.used = 0;
    return 0;
}

int ta_kprof_read(double* ms, int64_t* launches, double* flops, double* bytes) {
    std::lock_guard<std::mutex> lk(ta::g_kp_mu);
    double tms = 0, tf = 0, tb = 0;
    for (size_t i = 0; i < ta::g_kp.used; i++) {
        TA_HIP(hipEventSynchronize(ta::g_kp.ev[2 * i + 1]));
        float x = 0.f;
        TA_HIP(hipEventElapsedTime(&x, ta::g_kp.ev[2 * i], ta::g_kp.ev[2 * i + 1]));
        tms += x;
        tf += ta::g_kp.flops[i];
        tb += ta::g_kp.bytes[i];
    }
    if (ms) *ms = tms;
    if (launches) *launches = (int64_t)ta::g_kp.used;
    if (flops) *flops = tf;
    if (bytes) *bytes = tb;
    ta::g_kp.used = 0;
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

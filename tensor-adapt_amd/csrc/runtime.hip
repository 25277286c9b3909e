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

#include "ta_common.hpp"

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

}  // namespace ta

extern "C" {

const char* ta_last_error(void) { return ta::g_err.c_str(); }

const char* ta_version(void) { return "tensor-adapt-amd gfx950 " __DATE__ " " __TIME__; }

}  // extern "C"

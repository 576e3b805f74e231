// Host plumbing of libtenzo_hip.so: error reporting, library-owned scratch,
// version and device queries.
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace tz {

namespace {
thread_local std::string g_error;

struct Region {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_scratch_mu;
std::vector<std::vector<Region>> g_scratch;  // [device][slot]
}  // namespace

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
}

int hip_fail(hipError_t e, const char* what) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? TENZO_ERROR_OUT_OF_MEMORY : TENZO_ERROR_UNSUPPORTED;
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return TENZO_SUCCESS;
}

void* Scratch::get(int slot, size_t bytes, hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error("scratch: hipGetDevice failed");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1);
    auto& regions = g_scratch[dev];
    if (regions.empty()) regions.resize(kScratchSlots);
    Region& r = regions[slot];
    if (r.bytes >= bytes && r.ptr) return r.ptr;
    size_t want = bytes < 4096 ? 4096 : bytes;
    want = (want + 4095) & ~size_t(4095);
    if (r.ptr) {
        // Earlier work on this stream may still use the old region.
        if (hipStreamSynchronize(stream) != hipSuccess || hipFree(r.ptr) != hipSuccess) {
            set_error("scratch: releasing the previous region failed");
            return nullptr;
        }
        r.ptr = nullptr;
        r.bytes = 0;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        hip_fail(e, "scratch hipMalloc");
        return nullptr;
    }
    e = hipMemset(p, 0, want);
    if (e != hipSuccess) {
        (void)hipFree(p);
        hip_fail(e, "scratch hipMemset");
        return nullptr;
    }
    r.ptr = p;
    r.bytes = want;
    return p;
}

}  // namespace tz

extern "C" {

TENZO_HIP_API const char* tenzo_hip_version(void) { return TENZO_VERSION_STRING " gfx950"; }

TENZO_HIP_API const char* tenzo_hip_last_error(void) { return tz::g_error.c_str(); }

TENZO_HIP_API int tenzo_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

TENZO_HIP_API int tenzo_hip_release_scratch(void) {
    int dev = 0;
    TZ_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(tz::g_scratch_mu);
    if ((int)tz::g_scratch.size() <= dev) return TENZO_SUCCESS;
    TZ_HIP(hipDeviceSynchronize());
    for (auto& r : tz::g_scratch[dev]) {
        if (r.ptr) TZ_HIP(hipFree(r.ptr));
        r.ptr = nullptr;
        r.bytes = 0;
    }
    return TENZO_SUCCESS;
}

}  // extern "C"

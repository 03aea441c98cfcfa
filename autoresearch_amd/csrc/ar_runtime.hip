// ar_runtime.hip -- error reporting and the library-owned workspace.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "ar_common.hpp"

namespace ar {

static thread_local char g_err[512] = "";

int32_t set_error(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int32_t check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(AR_EHIP, "%s: %s", what, hipGetErrorString(e));
    return AR_OK;
}

namespace {
struct Workspace {
    std::mutex mu;
    void* ptr[64] = {};
    size_t bytes[64] = {};
};
Workspace g_ws;
}  // namespace

void* workspace(size_t bytes, int32_t* status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        *status = set_error(AR_EHIP, "workspace: hipGetDevice failed");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_ws.mu);
    if (g_ws.bytes[dev] >= bytes && g_ws.ptr[dev]) {
        *status = AR_OK;
        return g_ws.ptr[dev];
    }
    if (g_ws.ptr[dev]) {
        // Work queued on any stream may still use the old buffer.
        if (hipDeviceSynchronize() != hipSuccess || hipFree(g_ws.ptr[dev]) != hipSuccess) {
            *status = set_error(AR_EHIP, "workspace: releasing old buffer failed");
            return nullptr;
        }
        g_ws.ptr[dev] = nullptr;
        g_ws.bytes[dev] = 0;
    }
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    want = (want + 4095) & ~size_t(4095);
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        *status = set_error(AR_ENOMEM, "workspace: hipMalloc(%zu) failed", want);
        return nullptr;
    }
    g_ws.ptr[dev] = p;
    g_ws.bytes[dev] = want;
    *status = AR_OK;
    return p;
}

}  // namespace ar

extern "C" const char* ar_last_error(void) { return ar::g_err; }
extern "C" int32_t ar_version(void) { return 1; }

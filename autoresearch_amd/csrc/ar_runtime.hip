// ar_runtime.hip -- error reporting and the caller-created workspaces.
//
// A workspace is device scratch for the entry points that need some (split-K
// partials, the in-place linear_bwd_dx copy, the embedding scatter's sort and
// chunk sums, reduction partials, Muon temporaries, bf16 operand copies).
// The caller creates it once and binds it to a stream; an entry point called
// on that stream takes its scratch from the bound workspace and never
// allocates, frees or synchronises.  The reference's kernels never allocate
// either: their host code owns every DeviceBuffer (model.mojo:263-335).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "ar_common.hpp"

struct ar_workspace {
    void* ptr;
    size_t bytes;
    int device;
};

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
struct Binding {
    hipStream_t stream;
    int device;
    ar_workspace* ws;
};
std::mutex g_mu;
std::vector<Binding> g_bind;  // a handful of entries: linear search
}  // namespace

void* workspace(hipStream_t st, size_t bytes, int32_t* status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        *status = set_error(AR_EHIP, "workspace: hipGetDevice failed");
        return nullptr;
    }
    ar_workspace* ws = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (const Binding& b : g_bind)
            if (b.stream == st && b.device == dev) ws = b.ws;
    }
    if (!ws) {
        *status = set_error(AR_ENOMEM,
                            "no workspace bound to this stream (needs %zu bytes): ar_workspace_create, then "
                            "ar_workspace_bind",
                            bytes);
        return nullptr;
    }
    if (ws->bytes < bytes) {
        *status = set_error(AR_ENOMEM, "the stream's workspace holds %zu bytes, this call needs %zu", ws->bytes,
                            bytes);
        return nullptr;
    }
    *status = AR_OK;
    return ws->ptr;
}

}  // namespace ar

using namespace ar;

extern "C" const char* ar_last_error(void) { return ar::g_err; }
extern "C" int32_t ar_version(void) { return 2; }

extern "C" int32_t ar_workspace_create(ar_workspace** out, size_t bytes) {
    AR_CHECK_ARG(out != nullptr, "workspace_create: null pointer");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(AR_EHIP, "workspace_create: hipGetDevice failed");
    const size_t want = ((bytes < 4096 ? 4096 : bytes) + 4095) & ~size_t(4095);
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) return set_error(AR_ENOMEM, "workspace_create: hipMalloc(%zu) failed", want);
    *out = new ar_workspace{p, want, dev};
    return AR_OK;
}

extern "C" int32_t ar_workspace_bind(ar_stream_t stream, ar_workspace* ws) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(AR_EHIP, "workspace_bind: hipGetDevice failed");
    AR_CHECK_ARG(ws == nullptr || ws->device == dev, "workspace_bind: the workspace lives on device %d, not %d",
                 ws ? ws->device : -1, dev);
    const hipStream_t st = S(stream);
    std::lock_guard<std::mutex> lk(g_mu);
    for (size_t i = 0; i < g_bind.size(); ++i)
        if (g_bind[i].stream == st && g_bind[i].device == dev) {
            if (ws) g_bind[i].ws = ws;
            else g_bind.erase(g_bind.begin() + i);
            return AR_OK;
        }
    if (ws) g_bind.push_back(Binding{st, dev, ws});
    return AR_OK;
}

extern "C" int32_t ar_workspace_destroy(ar_workspace* ws) {
    if (!ws) return AR_OK;
    int32_t r = AR_OK;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (size_t i = 0; i < g_bind.size();) {
            if (g_bind[i].ws == ws) g_bind.erase(g_bind.begin() + i);
            else ++i;
        }
    }
    // Work queued on the streams it served may still use it.  Those stream
    // handles may already be destroyed, so wait for the workspace's whole
    // device instead of each recorded stream.
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return set_error(AR_EHIP, "workspace_destroy: hipGetDevice failed");
    if (cur != ws->device && hipSetDevice(ws->device) != hipSuccess)
        return set_error(AR_EHIP, "workspace_destroy: hipSetDevice(%d) failed", ws->device);
    if (hipDeviceSynchronize() != hipSuccess) r = set_error(AR_EHIP, "workspace_destroy: device sync failed");
    if (hipFree(ws->ptr) != hipSuccess) r = set_error(AR_EHIP, "workspace_destroy: hipFree failed");
    if (cur != ws->device) (void)hipSetDevice(cur);
    delete ws;
    return r;
}

extern "C" size_t ar_workspace_bytes(const ar_workspace* ws) { return ws ? ws->bytes : 0; }

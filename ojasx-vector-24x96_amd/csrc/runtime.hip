// runtime.hip -- error reporting, device buffers and engine metadata.
//
// Metadata entry points mirror split_manifold_lut_experiment/native/src/
// ojasx_lut_c_api.cpp:17-31 (version and backend strings); the strings name
// this engine instead of the reference's CPU backends.
#include <cstdarg>

#include "common.h"

namespace ojx {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char *what) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? OJASX_ERR_OOM : OJASX_ERR_HIP;
}

int DevBuf::ensure(size_t n) {
    if (n <= bytes && ptr) return OJASX_OK;
    release();
    if (n == 0) return OJASX_OK;
    hipError_t e = hipMalloc(&ptr, n);
    if (e != hipSuccess) {
        ptr = nullptr;
        return hip_fail(e, "hipMalloc");
    }
    bytes = n;
    return OJASX_OK;
}

void DevBuf::release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

int upload(DevBuf &buf, const void *host, size_t n) {
    int rc = buf.ensure(n);
    if (rc) return rc;
    if (n) OJX_HIP(hipMemcpy(buf.ptr, host, n, hipMemcpyHostToDevice));
    return OJASX_OK;
}

}  // namespace ojx

extern "C" {

OJASX_API const char *ojasx_get_version(void) { return "OjasX-LUT-Engine-v1.0.0-MI355X-HIP"; }

OJASX_API const char *ojasx_get_backend_name(void) { return "AMD_MI355X_HIP_gfx950"; }

OJASX_API const char *ojasx_get_last_error(void) { return ojx::g_err; }

}  // extern "C"

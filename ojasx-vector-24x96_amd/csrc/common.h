// common.h -- shared helpers of the gfx950 LUT engine (host + device).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "ojasx_lut_c_api.h"

namespace ojx {

// Thread-local message of the last failing C-ABI call.
void set_error(const char *fmt, ...);

// Map a HIP status to the C-ABI codes, recording a message.
int hip_fail(hipError_t e, const char *what);

#define OJX_HIP(call)                                           \
    do {                                                        \
        hipError_t _e = (call);                                 \
        if (_e != hipSuccess) return ::ojx::hip_fail(_e, #call); \
    } while (0)

// Device buffer owned by a handle.  Grows on request; never shrinks.
struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
    int ensure(size_t n);  // 0 or an error code
    void release();
    template <typename T> T *as() const { return static_cast<T *>(ptr); }
};

int upload(DevBuf &buf, const void *host, size_t n);  // ensure + memcpy

inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// ---- device helpers ------------------------------------------------------
__device__ __forceinline__ float load_act(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float load_act(const __hip_bfloat16 *p, size_t i) {
    return __bfloat162float(p[i]);
}
__device__ __forceinline__ void store_act(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store_act(__hip_bfloat16 *p, size_t i, float v) {
    p[i] = __float2bfloat16(v);
}

// Exclusive prefix sum over the 64 lanes of a wave of a value < 256.
__device__ __forceinline__ int wave_excl_scan_u8(int v) {
    const uint64_t lt = (uint64_t(1) << (threadIdx.x & 63)) - 1;
    int r = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint64_t m = __ballot(v & (1 << b));
        r += __popcll(m & lt) << b;
    }
    return r;
}

}  // namespace ojx

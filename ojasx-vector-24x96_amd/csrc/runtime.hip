// runtime.hip -- error reporting, device buffers and engine metadata.
//
// Metadata entry points mirror split_manifold_lut_experiment/native/src/
// ojasx_lut_c_api.cpp:17-31 (version and backend strings); the strings name
// this engine instead of the reference's CPU backends.
#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <map>
#include <string>
#include <vector>

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

namespace {
// fp32 -> bf16, round to nearest even (finite values; NaN stays NaN)
uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float bf16_to_f(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
}  // namespace

void split_codebook_bf16x3(const float *cb, uint16_t *out) {
    for (int c = 0; c < 256; ++c)
        for (int h = 0; h < 2; ++h)
            for (int i = 0; i < 8; ++i) {
                const float v = cb[c * 16 + 8 * h + i];
                const uint16_t h1 = bf16_rne(v);
                const float r1 = v - bf16_to_f(h1);
                const uint16_t h2 = bf16_rne(r1);
                const uint16_t h3 = bf16_rne(r1 - bf16_to_f(h2));
                uint16_t *o = out + ((c * 2 + h) * 3) * 8 + i;
                o[0] = h1;
                o[8] = h2;
                o[16] = h3;
            }
}

int HostIO::reserve(size_t bytes) {
    if (!st) OJX_HIP(hipStreamCreate(&st));   // blocking: ordered after null-stream work
    if (bytes <= cap) return OJASX_OK;
    if (pin) (void)hipHostFree(pin);
    pin = nullptr;
    cap = 0;
    const size_t n = round_up(std::max<size_t>(bytes, 64 << 10), 4096);
    OJX_HIP(hipHostMalloc(reinterpret_cast<void **>(&pin), n, hipHostMallocDefault));
    cap = n;
    return OJASX_OK;
}

HostIO::~HostIO() {
    if (pin) (void)hipHostFree(pin);
    if (st) (void)hipStreamDestroy(st);
}

HostIO &host_io() {
    static thread_local HostIO io;
    return io;
}

int StagingRing::reserve(size_t bytes) {
    if (bytes <= cap) return OJASX_OK;
    for (hipEvent_t &e : ev)
        if (e) OJX_HIP(hipEventSynchronize(e));
    if (pinned) (void)hipHostFree(pinned);
    pinned = nullptr;
    cap = 0;
    for (size_t &b : bytes_of) b = 0;
    const size_t n = round_up(std::max<size_t>(bytes, 64 << 10), 256);
    OJX_HIP(hipHostMalloc(reinterpret_cast<void **>(&pinned), n * kSlots, hipHostMallocDefault));
    const int rc = dev.ensure(n * kSlots);
    if (rc) return rc;
    for (hipEvent_t &e : ev)
        if (!e) OJX_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    cap = n;
    return OJASX_OK;
}

int StagingRing::stage(const void *host, size_t bytes, bool reuse, hipStream_t st, void **dev_out) {
    int rc = reserve(bytes);
    if (rc) return rc;
    int k = -1;
    if (reuse) {
        // the newest matching slot first (the one before next)
        for (int i = 1; i <= kSlots && k < 0; ++i) {
            const int s = (next - i + kSlots) % kSlots;
            if (bytes_of[s] != bytes || memcmp(pinned + (size_t)s * cap, host, bytes) != 0) continue;
            if (stream_of[s] == st) k = s;   // its upload precedes this call on st
        }
    }
    if (k < 0) {
        k = next;
        next = (k + 1) % kSlots;
        OJX_HIP(hipEventSynchronize(ev[k]));             // slot k's last launch is done
        memcpy(pinned + (size_t)k * cap, host, bytes);
        OJX_HIP(hipMemcpyAsync(dev.as<unsigned char>() + (size_t)k * cap, pinned + (size_t)k * cap,
                               bytes, hipMemcpyHostToDevice, st));
        bytes_of[k] = bytes;
        stream_of[k] = st;
    }
    cur = k;
    *dev_out = dev.as<unsigned char>() + (size_t)k * cap;
    return OJASX_OK;
}

int StagingRing::launched(hipStream_t st) {
    if (cur >= 0) OJX_HIP(hipEventRecord(ev[cur], st));
    return OJASX_OK;
}

StagingRing::~StagingRing() {
    dev.release();
    if (pinned) (void)hipHostFree(pinned);
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
}

// ---- kernel timing -------------------------------------------------------
namespace {
struct TimingRecord {
    std::string name;
    hipEvent_t start, stop;
};
constexpr size_t kMaxTimed = 1 << 16;  // event pairs kept between reports
bool g_timing = false;
std::vector<TimingRecord> g_records;   // used entries
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_pool;
size_t g_dropped = 0;
}  // namespace

bool timing_on() { return g_timing; }

void timing_events(const char *name, hipEvent_t *start, hipEvent_t *stop) {
    *start = *stop = nullptr;
    if (g_records.size() >= kMaxTimed) {
        ++g_dropped;
        return;
    }
    if (g_pool.size() <= g_records.size()) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess) return;
        if (hipEventCreate(&b) != hipSuccess) {
            (void)hipEventDestroy(a);
            return;
        }
        g_pool.emplace_back(a, b);
    }
    auto &pr = g_pool[g_records.size()];
    // "(ns::kernel<...>)" -> "kernel<...>"
    std::string n(name);
    if (!n.empty() && n.front() == '(') n = n.substr(1, n.size() - 2);
    g_records.push_back({n, pr.first, pr.second});
    *start = pr.first;
    *stop = pr.second;
}

}  // namespace ojx

extern "C" {

OJASX_API int ojasx_kernel_timing_enable(int enable) {
    ojx::g_timing = enable != 0;
    ojx::g_records.clear();
    ojx::g_dropped = 0;
    return OJASX_OK;
}

OJASX_API int ojasx_kernel_timing_report(char *buf, size_t buf_size) {
    using namespace ojx;
    OJX_HIP(hipDeviceSynchronize());
    std::map<std::string, std::pair<double, long>> agg;   // name -> (total ms, count)
    for (const auto &r : g_records) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) continue;
        auto &a = agg[r.name];
        a.first += ms;
        a.second += 1;
    }
    std::string out = "{";
    bool first = true;
    for (const auto &kv : agg) {
        char item[512];
        snprintf(item, sizeof(item), "%s\"%s\": {\"calls\": %ld, \"avg_us\": %.4f}", first ? "" : ", ",
                 kv.first.c_str(), kv.second.second, 1e3 * kv.second.first / kv.second.second);
        out += item;
        first = false;
    }
    char tail[64];
    snprintf(tail, sizeof(tail), "%s\"_dropped\": %zu}", first ? "" : ", ", g_dropped);
    out += tail;
    if (buf && buf_size) {
        strncpy(buf, out.c_str(), buf_size - 1);
        buf[buf_size - 1] = '\0';
    }
    g_records.clear();
    g_dropped = 0;
    return (int)out.size() + 1;
}

OJASX_API const char *ojasx_get_version(void) { return "OjasX-LUT-Engine-v1.0.0-MI355X-HIP"; }

OJASX_API const char *ojasx_get_backend_name(void) { return "AMD_MI355X_HIP_gfx950"; }

OJASX_API const char *ojasx_get_last_error(void) { return ojx::g_err; }

}  // extern "C"

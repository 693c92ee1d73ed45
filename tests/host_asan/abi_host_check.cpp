// Host-side memory and undefined-behaviour check of the C-ABI, built with
// AddressSanitizer and UBSan on the host code only (tests/host_asan/build.py:
// every csrc/*.hip with -Xarch_host -fsanitize=address,undefined, GPU code
// untouched).  It drives the reference-facing entry points of
// include/ojasx_lut_c_api.h through their argument validation, and, when a
// GPU is visible, through create / outliers / forward / destroy of a linear
// (block 16 and 24), the MoE and the KV cache, plus the kernel-timing report
// with a short buffer.  Numbers are checked against direct fp64 restatements
// of the reference's formulas (ojasx_lut_cpu.cpp:92-184, 213-365) written
// here, so a silent corruption also fails.  Any sanitizer report aborts with
// a non-zero status; the last line is "HOST_CHECK_OK" on success.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "ojasx_lut_c_api.h"

static int g_fail = 0;
#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);             \
            std::fprintf(stderr, "\n");                    \
            ++g_fail;                                      \
        }                                                  \
    } while (0)

static double rel_err(const std::vector<float> &y, const std::vector<double> &ref) {
    double num = 0, den = 0;
    for (size_t i = 0; i < y.size(); ++i) {
        num = std::max(num, std::fabs((double)y[i] - ref[i]));
        den = std::max(den, std::fabs(ref[i]));
    }
    return num / (den > 0 ? den : 1.0);
}

// ---- argument validation: no device work is reached ----------------------
static void check_validation() {
    CHECK(ojasx_get_version() && std::strlen(ojasx_get_version()) > 0, "version");
    CHECK(ojasx_get_backend_name() && std::strlen(ojasx_get_backend_name()) > 0, "backend");
    float cb[16] = {0};
    uint8_t codes[4] = {0};
    CHECK(!ojasx_create_linear(0, 4, 16, 1, cb, codes, nullptr, nullptr), "zero in_features");
    CHECK(!ojasx_create_linear(32, 4, 24, 1, cb, codes, nullptr, nullptr), "block not dividing");
    CHECK(!ojasx_create_linear(32, 4, 16, 257, cb, codes, nullptr, nullptr), "codebook > 256");
    CHECK(!ojasx_create_linear(32, -1, 16, 1, cb, codes, nullptr, nullptr), "negative out");
    CHECK(std::strlen(ojasx_get_last_error()) > 0, "last error set");
    int rp[2] = {0, 0};
    CHECK(ojasx_set_linear_outliers(nullptr, 0, rp, nullptr, nullptr) != 0, "outliers null");
    float x[4] = {0}, y[4] = {0};
    CHECK(ojasx_linear_forward(nullptr, x, y, 1, 1) != 0, "forward null handle");
    CHECK(ojasx_linear_forward_device(nullptr, x, y, 1, 0, nullptr) != 0, "device forward null");
    CHECK(!ojasx_create_moe(0, 32, 32, 2, 16, cb, cb, codes, cb, codes, cb), "moe zero experts");
    CHECK(!ojasx_create_moe(4, 33, 32, 2, 16, cb, cb, codes, cb, codes, cb), "moe block");
    CHECK(!ojasx_create_kv_cache(0, 32, 8, 16), "kv zero heads");
    CHECK(!ojasx_create_kv_cache(2, 30, 8, 16), "kv block");
    CHECK(ojasx_kv_cache_append(nullptr, 0, x, x) != 0, "kv append null");
    CHECK(ojasx_moe_forward(nullptr, x, nullptr, nullptr, y, 1) != 0, "moe forward null");
    ojasx_destroy_linear(nullptr);
    ojasx_destroy_moe(nullptr);
    ojasx_destroy_kv_cache(nullptr);
    CHECK(ojasx_get_compressed_size(nullptr) == 0, "size of null");
}

// ---- one linear, host pointers --------------------------------------------
static void check_linear(int K, int M, int D, int B, unsigned seed) {
    std::mt19937 r(seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    const int G = K / D, Kcb = 256;
    std::vector<float> cb((size_t)Kcb * D), sc(M), bias(M), x((size_t)B * K);
    std::vector<uint8_t> codes((size_t)M * G);
    for (auto &v : cb) v = 0.02f * nd(r);
    for (auto &v : sc) v = 0.5f + 0.01f * (float)(r() % 100);
    for (auto &v : bias) v = 0.1f * nd(r);
    for (auto &v : x) v = nd(r);
    for (auto &c : codes) c = (uint8_t)(r() & 255);
    // CSR: a few outliers per row, columns unsorted within a row
    std::vector<int> rp(M + 1, 0), col;
    std::vector<float> val;
    for (int m = 0; m < M; ++m) {
        const int n = (int)(r() % 3);
        for (int i = 0; i < n; ++i) {
            col.push_back((int)(r() % K));
            val.push_back(2.0f * nd(r));
        }
        rp[m + 1] = (int)col.size();
    }
    OjasxLinearHandle h = ojasx_create_linear(K, M, D, Kcb, cb.data(), codes.data(), sc.data(),
                                              bias.data());
    CHECK(h, "create_linear K=%d M=%d D=%d: %s", K, M, D, ojasx_get_last_error());
    if (!h) return;
    // invalid CSR: -3, then a valid one
    std::vector<int> bad = rp;
    if (M > 1) bad[1] = rp[M] + 5;
    if (!col.empty()) {
        CHECK(ojasx_set_linear_outliers(h, rp[M], bad.data(), col.data(), val.data()) == -3,
              "non-monotone row_ptrs");
        std::vector<int> badc = col;
        badc[0] = K;
        CHECK(ojasx_set_linear_outliers(h, rp[M], rp.data(), badc.data(), val.data()) == -3,
              "column out of range");
    }
    CHECK(ojasx_set_linear_outliers(h, rp[M], rp.data(), col.data(), val.data()) == 0,
          "set outliers: %s", ojasx_get_last_error());
    std::vector<float> y((size_t)B * M, -7.f);
    CHECK(ojasx_linear_forward(h, x.data(), y.data(), B, 4) == 0, "forward: %s",
          ojasx_get_last_error());
    // y = s_m * sum_g <x_g, C[code]> + bias, then + outliers (ojasx_lut_cpu.cpp:160-184)
    std::vector<double> ref((size_t)B * M);
    for (int b = 0; b < B; ++b)
        for (int m = 0; m < M; ++m) {
            double acc = 0;
            for (int g = 0; g < G; ++g) {
                const float *c = &cb[(size_t)codes[(size_t)m * G + g] * D];
                for (int d = 0; d < D; ++d) acc += (double)x[(size_t)b * K + g * D + d] * c[d];
            }
            double o = 0;
            for (int j = rp[m]; j < rp[m + 1]; ++j) o += (double)val[j] * x[(size_t)b * K + col[j]];
            ref[(size_t)b * M + m] = sc[m] * acc + bias[m] + o;
        }
    const double e = rel_err(y, ref);
    CHECK(e < 1e-5, "linear K=%d M=%d D=%d B=%d rel err %.3g", K, M, D, B, e);
    CHECK(ojasx_get_compressed_size(h) > 0 && ojasx_get_dense_size(h) == (size_t)K * M * 4,
          "sizes");
    ojasx_destroy_linear(h);
    std::printf("linear K=%d M=%d D=%d B=%d rel %.2e\n", K, M, D, B, e);
}

// ---- MoE, one token per call, host pointers --------------------------------
static void check_moe(unsigned seed) {
    const int E = 6, H = 64, I = 48, k = 3, D = 16, Gi = H / D, Gd = I / D;
    std::mt19937 r(seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<float> cbi(256 * D), cbd(256 * D), gus((size_t)E * 2 * I), dns((size_t)E * H);
    std::vector<uint8_t> guc((size_t)E * 2 * I * Gi), dnc((size_t)E * H * Gd);
    for (auto &v : cbi) v = 0.05f * nd(r);
    for (auto &v : cbd) v = 0.05f * nd(r);
    for (auto &v : gus) v = 0.5f + 0.01f * (float)(r() % 100);
    for (auto &v : dns) v = 0.5f + 0.01f * (float)(r() % 100);
    for (auto &c : guc) c = (uint8_t)(r() & 255);
    for (auto &c : dnc) c = (uint8_t)(r() & 255);
    OjasxMoEHandle h = ojasx_create_moe(E, H, I, k, D, cbi.data(), cbd.data(), guc.data(),
                                        gus.data(), dnc.data(), dns.data());
    CHECK(h, "create_moe: %s", ojasx_get_last_error());
    if (!h) return;
    std::vector<float> x(H), y(H, -3.f);
    for (auto &v : x) v = nd(r);
    const int idx[k] = {4, 1, E + 2};               // the last is out of range: skipped
    const float w[k] = {0.6f, 0.3f, 0.1f};
    CHECK(ojasx_moe_forward(h, x.data(), idx, w, y.data(), k) == 0, "moe forward: %s",
          ojasx_get_last_error());
    // gate/up rows, silu(gate) * up, down rows, sum_j w_j down_j (ojasx_lut_cpu.cpp:213-365)
    std::vector<double> ref(H, 0.0);
    for (int j = 0; j < k; ++j) {
        const int e = idx[j];
        if (e < 0 || e >= E || std::fabs(w[j]) < 1e-8f) continue;
        std::vector<double> gu(2 * I), inter(I);
        for (int rr = 0; rr < 2 * I; ++rr) {
            double a = 0;
            for (int g = 0; g < Gi; ++g) {
                const float *c = &cbi[(size_t)guc[((size_t)e * 2 * I + rr) * Gi + g] * D];
                for (int d = 0; d < D; ++d) a += (double)x[g * D + d] * c[d];
            }
            gu[rr] = gus[(size_t)e * 2 * I + rr] * a;
        }
        for (int i = 0; i < I; ++i) inter[i] = gu[i] / (1.0 + std::exp(-gu[i])) * gu[I + i];
        for (int hh = 0; hh < H; ++hh) {
            double a = 0;
            for (int g = 0; g < Gd; ++g) {
                const float *c = &cbd[(size_t)dnc[((size_t)e * H + hh) * Gd + g] * D];
                for (int d = 0; d < D; ++d) a += inter[g * D + d] * c[d];
            }
            ref[hh] += w[j] * dns[(size_t)e * H + hh] * a;
        }
    }
    const double e = rel_err(y, ref);
    CHECK(e < 1e-5, "moe rel err %.3g", e);
    std::vector<float> y2(H, 5.f);
    CHECK(ojasx_moe_forward(h, x.data(), idx, w, y2.data(), 0) == 0 && y2[0] == 5.f,
          "k_active 0 leaves y untouched");
    CHECK(ojasx_moe_get_compressed_size(h) > 0, "moe size");
    ojasx_destroy_moe(h);
    std::printf("moe rel %.2e\n", e);
}

// ---- KV cache: append, attention against fp64 attention on the inputs -----
static void check_kv(unsigned seed) {
    const int heads = 2, hd = 32, T = 7;
    std::mt19937 r(seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    OjasxKVHandle h = ojasx_create_kv_cache(heads, hd, 16, 16);
    CHECK(h, "create_kv_cache: %s", ojasx_get_last_error());
    if (!h) return;
    std::vector<float> K((size_t)T * hd), V((size_t)T * hd), q(hd), out(hd, 9.f);
    for (auto &v : K) v = nd(r);
    for (auto &v : V) v = nd(r);
    for (auto &v : q) v = nd(r);
    CHECK(ojasx_kv_cache_attention(h, 1, q.data(), out.data(), 0.f) == 0 && out[0] == 9.f,
          "empty head leaves the output untouched");
    for (int t = 0; t < T; ++t)
        CHECK(ojasx_kv_cache_append(h, 1, &K[(size_t)t * hd], &V[(size_t)t * hd]) == 0,
              "append %d: %s", t, ojasx_get_last_error());
    CHECK(ojasx_kv_cache_append(h, heads, K.data(), V.data()) != 0, "head out of range");
    CHECK(ojasx_kv_cache_attention(h, 1, q.data(), out.data(), 0.f) == 0, "attention: %s",
          ojasx_get_last_error());
    // the reference's scalar quantiser (ojasx_lut_kv_cache.cpp:16-65): per token
    // scale = max(|x|, 1e-8) / 127, one code per block from its first
    // coordinate, round half away from zero; attention over the dequantised
    // keys and values (ojasx_lut_kv_cache.cpp:67-132)
    auto quant = [&](const float *row, std::vector<double> &deq) {
        float mxv = 1e-8f;
        for (int d = 0; d < hd; ++d) mxv = std::max(mxv, std::fabs(row[d]));
        const float sc = mxv / 127.0f;
        deq.assign(hd, 0.0);
        for (int g = 0; g < hd / 16; ++g) {
            int qv = (int)std::round(row[g * 16] / sc);
            qv = std::max(-128, std::min(127, qv));
            deq[g * 16] = (double)qv * sc;
        }
    };
    std::vector<double> s(T), ref(hd, 0.0), kd, vd;
    double mx = -1e300, sum = 0;
    for (int t = 0; t < T; ++t) {
        quant(&K[(size_t)t * hd], kd);
        double a = 0;
        for (int d = 0; d < hd; ++d) a += (double)q[d] * kd[d];
        s[t] = a / std::sqrt((double)hd);
        mx = std::max(mx, s[t]);
    }
    for (int t = 0; t < T; ++t) sum += std::exp(s[t] - mx);
    for (int t = 0; t < T; ++t) {
        quant(&V[(size_t)t * hd], vd);
        for (int d = 0; d < hd; ++d) ref[d] += std::exp(s[t] - mx) / sum * vd[d];
    }
    const double e = rel_err(out, ref);
    CHECK(e < 1e-5, "kv attention rel err %.3g", e);
    CHECK(ojasx_kv_cache_get_memory_size(h) > 0, "kv size");
    ojasx_destroy_kv_cache(h);
    std::printf("kv rel %.2e\n", e);
}

// ---- kernel-timing report into short and long buffers ---------------------
static void check_timing() {
    CHECK(ojasx_kernel_timing_enable(1) == 0, "timing enable");
    check_linear(64, 40, 16, 1, 99);
    char small[8];
    std::memset(small, 'x', sizeof small);
    const int need = ojasx_kernel_timing_report(small, sizeof small);
    CHECK(need > (int)sizeof small && small[sizeof small - 1] == 0, "truncated report (%d)", need);
    CHECK(ojasx_kernel_timing_enable(1) == 0, "timing enable");
    check_linear(64, 40, 16, 1, 98);
    std::vector<char> big(1 << 16);
    const int n = ojasx_kernel_timing_report(big.data(), big.size());
    CHECK(n > 0 && n <= (int)big.size() && std::strstr(big.data(), "calls"), "report");
    CHECK(ojasx_kernel_timing_enable(0) == 0, "timing disable");
}

int main() {
    check_validation();
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess) ndev = 0;
    std::printf("devices %d\n", ndev);
    if (ndev > 0) {
        check_linear(64, 40, 16, 3, 1);
        check_linear(2560, 300, 16, 2, 2);
        check_linear(96, 33, 24, 2, 3);
        check_linear(128, 17, 64, 1, 4);
        check_moe(5);
        check_kv(6);
        check_timing();
    }
    if (g_fail) {
        std::printf("HOST_CHECK_FAILED %d\n", g_fail);
        return 1;
    }
    std::printf("HOST_CHECK_OK\n");
    return 0;
}

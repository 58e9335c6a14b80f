// Device set-up, the registration known-answer test and error reporting for
// the C ABI.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "zest_common.h"

namespace zest {

static thread_local std::string g_last_error;

int fail(int status, const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int check_launch(const char * what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ZEST_E_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return ZEST_OK;
}

} // namespace zest

namespace {

// Frees device memory on scope exit.
struct dev_buf {
    void * p = nullptr;
    ~dev_buf() {
        if (p) (void) hipFree(p);
    }
};

#define HIP_OR_FAIL(call)                                                                            \
    do {                                                                                             \
        const hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

} // namespace

extern "C" {

const char * zest_last_error(void) { return zest::g_last_error.c_str(); }

int zest_init(int device) {
    int n = 0;
    HIP_OR_FAIL(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return zest::fail(ZEST_E_ARG, "zest_init: device %d of %d", device, n);
    HIP_OR_FAIL(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_OR_FAIL(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return zest::fail(ZEST_E_UNSUPPORTED, "zest_init: device %d is %s; the kernels are built for gfx950", device,
                          prop.gcnArchName);
    return zest::scratch_setup(device);
}

// npu_self_test (src/xdna-npu.cpp:142-184): small whole numbers, which the
// 8-bit blocks hold exactly and fp32 sums add exactly, so every output must
// equal the integer dot product under any summation order.
int zest_self_test(void) {
    constexpr int64_t M = 512, K = 128, N = 512;
    std::vector<int8_t> ai((size_t) (M * K)), wi((size_t) (N * K));
    uint32_t seed = 1;
    auto next = [&](int span) {
        seed = seed * 1664525u + 1013904223u;
        return (int8_t) ((int) (seed >> 24) % span - span / 2);
    };
    for (int8_t & v : ai) v = next(5);
    for (int8_t & v : wi) v = next(7);
    std::vector<float> a(ai.begin(), ai.end()), w(wi.begin(), wi.end());

    dev_buf da, dw, pa, pw, dc;
    HIP_OR_FAIL(hipMalloc(&da.p, a.size() * 4));
    HIP_OR_FAIL(hipMalloc(&dw.p, w.size() * 4));
    HIP_OR_FAIL(hipMalloc(&pa.p, zest_act_bytes(M, K)));
    HIP_OR_FAIL(hipMalloc(&pw.p, zest_bfp16_bytes(N, K)));
    HIP_OR_FAIL(hipMalloc(&dc.p, (size_t) (M * N) * 4));
    HIP_OR_FAIL(hipMemcpy(da.p, a.data(), a.size() * 4, hipMemcpyHostToDevice));
    HIP_OR_FAIL(hipMemcpy(dw.p, w.data(), w.size() * 4, hipMemcpyHostToDevice));
    int st = zest_pack_act_x((const float *) da.p, M, K, K, pa.p, nullptr);
    if (st == ZEST_OK) st = zest_convert_weight(ZEST_TYPE_F32, dw.p, N, K, pw.p, nullptr);
    if (st == ZEST_OK) st = zest_gemm(pa.p, M, pw.p, N, K, (float *) dc.p, N, nullptr, nullptr);
    if (st != ZEST_OK) return st;
    std::vector<float> c((size_t) (M * N));
    HIP_OR_FAIL(hipMemcpy(c.data(), dc.p, c.size() * 4, hipMemcpyDeviceToHost));
    for (int64_t r = 0; r < M; r++)
        for (int64_t n = 0; n < N; n++) {
            int want = 0;
            for (int64_t k = 0; k < K; k++) want += ai[r * K + k] * wi[n * K + k];
            if (c[r * N + n] != (float) want)
                return zest::fail(ZEST_E_SELF_TEST, "self-test multiply wrong at row %lld, column %lld: %g instead of %d",
                                  (long long) r, (long long) n, c[r * N + n], want);
        }
    return ZEST_OK;
}

} // extern "C"

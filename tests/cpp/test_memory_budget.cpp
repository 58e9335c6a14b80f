// The weight cache is held to a memory limit, decided through supports_op
// like the rest of the policy (the reference's tests/test-memory-budget.cpp).
// Run with GGML_XDNA_MAX_COPY_GB=0.05 (51.2 MiB) and the other settings at
// their defaults, on the GPU or under GGML_XDNA_PLAN_ONLY=1.
//
// A 2048 x 2048 weight's cache entry is 4.5 MiB, so a layer of four is 18 MiB:
// layers 0 and 1 fit (36 MiB), layer 2's fourth weight would pass the limit.
#include <cstdio>
#include <cstdlib>
#include <string>

#include "mini_ggml.h"

int main() {
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "XDNA0 not registered - is GGML_BACKEND_PATH set?\n");
        return 2;
    }
    const char * po = getenv("GGML_XDNA_PLAN_ONLY");
    const bool plan_only = po && *po && po[0] != '0';

    // weights as llama.cpp loads them: named by layer, in a buffer marked as
    // weights (device memory; host memory when planning only)
    ggml_init_params wp = {ggml_tensor_overhead() * 32, nullptr, true};
    ggml_context * wctx = ggml_init(wp);
    ggml_tensor * w[3][4] = {};
    for (int l = 0; l < 3; l++)
        for (int i = 0; i < 4; i++) {
            w[l][i] = ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, 2048, 2048);
            ggml_set_name(w[l][i], ("blk." + std::to_string(l) + ".w" + std::to_string(i) + ".weight").c_str());
        }
    ggml_tensor * small = ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, 2048, 512);  // 1.1 MiB
    ggml_set_name(small, "blk.3.w0.weight");
    ggml_backend_buffer_type_t buft = plan_only
                                          ? ggml_backend_dev_buffer_type(ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU))
                                          : ggml_backend_dev_buffer_type(dev);
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors_from_buft(wctx, buft);
    if (!buf) {
        fprintf(stderr, "cannot allocate the weights\n");
        return 2;
    }
    ggml_backend_buffer_set_usage(buf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);

    ggml_init_params ip = {ggml_tensor_overhead() * 256, nullptr, true};
    ggml_context * ctx = ggml_init(ip);
    auto claimed = [&](ggml_tensor * weight) {
        ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, weight->ne[0], 1024);
        return ggml_backend_dev_supports_op(dev, ggml_mul_mat(ctx, weight, x));
    };

    test_check(claimed(small), "with no context started, the limit doesn't apply (llama.cpp's load-time checks)");

    ggml_backend_t be = ggml_backend_dev_init(dev, nullptr);
    if (!be) {
        fprintf(stderr, "cannot start the XDNA0 backend\n");
        return 2;
    }

    // a 72 MiB weight with no data, as in llama.cpp's memory-fitting trial
    ggml_tensor * trial = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_K, 2048, 32768);
    ggml_set_name(trial, "blk.0.trial.weight");
    test_check(claimed(trial), "a weight with no data is claimed, and doesn't count against the limit");

    bool all = true;
    for (int l = 0; l < 2; l++)
        for (int i = 0; i < 4; i++) all &= claimed(w[l][i]);
    test_check(all, "layers 0 and 1 fit (36 MiB of 51.2) and are claimed");
    test_check(claimed(w[2][0]) && claimed(w[2][1]) && claimed(w[2][2]), "layer 2's first three weights fit when asked");
    test_check(!claimed(w[2][3]), "layer 2's fourth weight would pass the limit: not claimed");
    test_check(!claimed(w[2][0]) && !claimed(w[2][1]) && !claimed(w[2][2]),
               "layer 2's first three then stay off the GPU path too (no layer is split)");
    test_check(!claimed(small), "a weight that would still fit is not claimed once the limit is reached");
    test_check(claimed(w[0][0]) && claimed(w[1][3]), "what was taken stays taken");

    ggml_backend_free(be);
    be = ggml_backend_dev_init(dev, nullptr);
    test_check(claimed(small) && claimed(w[2][3]), "after the context is freed, the next one starts with nothing counted");
    ggml_backend_free(be);

    ggml_free(ctx);
    ggml_backend_buffer_free(buf);
    ggml_free(wctx);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

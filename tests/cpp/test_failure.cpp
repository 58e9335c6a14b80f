// Failure semantics (the reference's mul-mat-npu-nan / -fail ctest cases,
// CMakeLists.txt:216-220, and src/ggml-zest.cpp:123-130): with
// GGML_XDNA_FAIL_AFTER=0 every GEMM submission fails; with
// GGML_XDNA_NAN_AFTER=0 every GEMM result comes back as NaN and the non-finite
// check must catch it. Either way graph_compute returns GGML_STATUS_FAILED and
// from then on the backend claims nothing, so the scheduler keeps the work on
// other devices. Both are forced from the host: every kernel runs normally.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "mini_ggml.h"

int main() {
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "XDNA device not registered - is GGML_BACKEND_PATH set?\n");
        return 2;
    }
    const bool fail = getenv("GGML_XDNA_FAIL_AFTER") != nullptr, nan = getenv("GGML_XDNA_NAN_AFTER") != nullptr;
    if (fail == nan) {
        fprintf(stderr, "set exactly one of GGML_XDNA_FAIL_AFTER and GGML_XDNA_NAN_AFTER\n");
        return 2;
    }
    ggml_backend_t be = ggml_backend_dev_init(dev, nullptr);
    ggml_init_params ip = {ggml_tensor_overhead() * 8 + ggml_graph_overhead(), nullptr, true};
    ggml_context * ctx = ggml_init(ip);
    const int64_t K = 1024, N = 1024, M = 1024;
    ggml_tensor * w = ggml_new_tensor_2d(ctx, GGML_TYPE_Q8_0, K, N);
    ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, M);
    ggml_tensor * y = ggml_mul_mat(ctx, w, x);
    test_check(ggml_backend_dev_supports_op(dev, y), "before the failure, a prompt-sized matmul is claimed");
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
    std::vector<uint8_t> wb(ggml_nbytes(w));
    std::vector<float> wf((size_t) (K * N)), xf((size_t) (K * M));
    test_rng rng(3);
    for (float & v : wf) v = rng.normal(0, 1);
    for (float & v : xf) v = rng.normal(0, 1);
    ggml_quantize_chunk(GGML_TYPE_Q8_0, wf.data(), wb.data(), 0, N, K, nullptr);
    ggml_backend_tensor_set(w, wb.data(), 0, wb.size());
    ggml_backend_tensor_set(x, xf.data(), 0, xf.size() * 4);
    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, y);
    const ggml_status st = ggml_backend_graph_compute(be, gf);
    test_check(st == GGML_STATUS_FAILED, "graph_compute reports the %s (status %d)",
               fail ? "injected submission failure" : "NaN results", (int) st);
    test_check(!ggml_backend_dev_supports_op(dev, y), "afterwards the backend claims nothing");
    test_check(ggml_backend_graph_compute(be, gf) == GGML_STATUS_FAILED, "and refuses further graphs");
    ggml_backend_buffer_free(buf);
    ggml_free(ctx);
    ggml_backend_free(be);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

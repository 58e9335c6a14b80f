// Process-wide state under concurrency: the weight budget and the reader
// tracking are shared by every backend context and are reached from several
// threads (the reference guards them with g_budget.mu and g_read_mu,
// src/ggml-zest.cpp:467 and :1086, and fixed a race in its own thread pool,
// src/npu/thread_pool.h:42-48). Built with ThreadSanitizer and with
// AddressSanitizer (tests/cpp/Makefile, target `sanitize`) and run under
// GGML_XDNA_PLAN_ONLY=1 with GGML_XDNA_MAX_COPY_GB=0.05, so it needs no GPU.
//
// Two contexts are started on two threads at once; four threads then ask
// about every weight of a five-layer model, each in model order (as llama.cpp
// asks, layer by layer) but interleaved with the others at random, while
// asking about small ops next to the matmuls (which records readers). Every
// weight is first asked about in model order whatever the interleaving (the
// thread furthest ahead has asked about everything before it), so the
// budget's answers must come out as they would from one thread: the weights
// taken form whole layers and fit the limit, and every thread's last answers
// are the settled ones. Freeing both contexts on two threads at once must
// reset the count.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "mini_ggml.h"

namespace {

constexpr int LAYERS = 5, PER_LAYER = 4, THREADS = 4;
constexpr int64_t K = 2048, N = 2048;  // a 4.5 MiB cache entry each

double entry_bytes() { return (double) N * K * 9.0 / 8.0; }

}  // namespace

int main() {
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    const char * lim = getenv("GGML_XDNA_MAX_COPY_GB");
    if (!dev || !lim) {
        fprintf(stderr, "needs GGML_BACKEND_PATH and GGML_XDNA_MAX_COPY_GB\n");
        return 2;
    }
    const double limit = atof(lim) * 1073741824.0;

    ggml_init_params wp = {ggml_tensor_overhead() * (LAYERS * PER_LAYER + 4), nullptr, true};
    ggml_context * wctx = ggml_init(wp);
    std::vector<ggml_tensor *> w;
    for (int l = 0; l < LAYERS; l++)
        for (int i = 0; i < PER_LAYER; i++) {
            ggml_tensor * t = ggml_new_tensor_2d(wctx, GGML_TYPE_Q8_0, K, N);
            ggml_set_name(t, ("blk." + std::to_string(l) + ".w" + std::to_string(i) + ".weight").c_str());
            w.push_back(t);
        }
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors_from_buft(
        wctx, ggml_backend_dev_buffer_type(ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU)));
    ggml_backend_buffer_set_usage(buf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);

    // 1. two contexts started at once
    ggml_backend_t be[2] = {};
    {
        std::thread a([&] { be[0] = ggml_backend_dev_init(dev, nullptr); });
        std::thread b([&] { be[1] = ggml_backend_dev_init(dev, nullptr); });
        a.join();
        b.join();
    }
    test_check(be[0] && be[1], "two contexts start on two threads at once");

    // 2. four threads ask about every weight in model order, at their own pace, with
    // small ops on the matmuls in between; each thread builds in its own ggml context
    std::vector<std::vector<int>> seen(THREADS, std::vector<int>(w.size(), -1));
    std::atomic<int> go{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < THREADS; t++)
        pool.emplace_back([&, t] {
            ggml_init_params ip = {ggml_tensor_overhead() * 4096, nullptr, true};
            ggml_context * ctx = ggml_init(ip);
            std::mt19937 pace(1234 + t);
            go.fetch_add(1);
            while (go.load() < THREADS) std::this_thread::yield();
            for (int round = 0; round < 3; round++)
                for (int i = 0; i < (int) w.size(); i++) {
                    for (unsigned y = pace() % 4; y; y--) std::this_thread::yield();
                    ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, 2048);
                    ggml_tensor * mm = ggml_mul_mat(ctx, w[i], x);
                    const bool took = ggml_backend_dev_supports_op(dev, mm);
                    (void) ggml_backend_dev_supports_op(dev, ggml_scale(ctx, mm, 0.5f));
                    (void) ggml_backend_dev_supports_op(dev, ggml_rms_norm(ctx, mm, 1e-6f));
                    if (round == 2) seen[t][i] = took;
                }
            ggml_free(ctx);
        });
    for (std::thread & th : pool) th.join();

    // the settled answers, asked once more from this thread
    ggml_init_params qp = {ggml_tensor_overhead() * 256, nullptr, true};
    ggml_context * qctx = ggml_init(qp);
    auto asks = [&](ggml_tensor * weight) {
        return ggml_backend_dev_supports_op(dev, ggml_mul_mat(qctx, weight, ggml_new_tensor_2d(qctx, GGML_TYPE_F32, K, 2048)));
    };
    std::vector<int> final_(w.size());
    double taken = 0;
    int first_refused_layer = LAYERS;
    for (size_t i = 0; i < w.size(); i++) {
        final_[i] = asks(w[i]);
        if (final_[i]) taken += entry_bytes();
        else first_refused_layer = std::min(first_refused_layer, (int) i / PER_LAYER);
    }
    bool whole = true;
    for (int l = 0; l < LAYERS; l++)
        for (int i = 0; i < PER_LAYER; i++) whole &= final_[l * PER_LAYER + i] == final_[l * PER_LAYER];
    test_check(whole, "the weights taken form whole layers");
    test_check(taken <= limit, "they fit the limit (%.1f of %.1f MiB)", taken / 1048576.0, limit / 1048576.0);
    test_check(taken + PER_LAYER * entry_bytes() > limit, "and no further whole layer would have fit");
    bool agree = true;
    for (int t = 0; t < THREADS; t++)
        for (size_t i = 0; i < w.size(); i++) agree &= seen[t][i] == final_[i];
    test_check(agree, "every thread's last answers agree with the settled ones");
    test_check(first_refused_layer < LAYERS, "the limit was reached (layer %d refused)", first_refused_layer);

    // 3. both contexts freed at once: the count starts again
    {
        std::thread a([&] { ggml_backend_free(be[0]); });
        std::thread b([&] { ggml_backend_free(be[1]); });
        a.join();
        b.join();
    }
    ggml_backend_t again = ggml_backend_dev_init(dev, nullptr);
    bool fresh = again != nullptr;
    double now = 0;
    for (size_t i = 0; i < w.size() && now + entry_bytes() <= limit; i++, now += entry_bytes()) fresh &= asks(w[i]);
    test_check(fresh, "after both are freed, a new context takes weights from nothing again");
    if (again) ggml_backend_free(again);

    ggml_free(qctx);
    ggml_backend_buffer_free(buf);
    ggml_free(wctx);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

// The weight-cache budget, as the scheduler sees it through supports_op.
//
// Contract (reference: src/ggml-zest.cpp:429-552, the budget; its
// acceptance criteria are the XDNA-MEMORY-BUDGET section of
// specs/xdna-backend/spec.md):
//   * a weight's cache entry costs rows_pad(N) * k_pad(K) * 9/8 bytes;
//   * weights are taken in the order they are asked about while the entries
//     taken so far plus this one fit the limit (GGML_XDNA_MAX_COPY_GB);
//   * the first weight that does not fit stops all new takes, and the weights
//     already taken from its layer ("blk.N.") are given back, so no layer is
//     split; every answer is then fixed while a context lives;
//   * questions asked with no context alive, weights with no data and tensors
//     outside a weights buffer are answered but not counted;
//   * when the last context is freed, counting starts again from nothing.
//
// The model here is a small decoder with seven weights a layer of mixed
// shapes (q, k, v, o, gate, up, down at hidden 1024, FFN 2816), so the cut
// falls inside a layer at a place this program works out from the byte
// formula and the limit, rather than at a position written into it.
// Run with GGML_XDNA_MAX_COPY_GB=0.05, on the GPU or under
// GGML_XDNA_PLAN_ONLY=1.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "mini_ggml.h"

namespace {

struct shape {
    const char * name;
    int64_t n, k;  // output rows and K of the weight (ggml ne1, ne0)
};

const shape LAYER[] = {{"attn_q", 2048, 1024}, {"attn_k", 512, 1024},   {"attn_v", 512, 1024},
                       {"attn_output", 1024, 2048}, {"ffn_gate", 2816, 1024}, {"ffn_up", 2816, 1024},
                       {"ffn_down", 1024, 2816}};
constexpr int PER_LAYER = sizeof(LAYER) / sizeof(LAYER[0]);
constexpr int LAYERS = 5;

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// the cache entry's bytes: rows padded to 256, K to 64, 9 bytes per 8 values
double entry_bytes(int64_t n, int64_t k) { return (double) round_up(n, 256) * (double) round_up(k, 64) * 9.0 / 8.0; }

}  // namespace

int main() {
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "no XDNA0 device: set GGML_BACKEND_PATH to libggml-zest.so\n");
        return 2;
    }
    const char * lim_env = getenv("GGML_XDNA_MAX_COPY_GB");
    if (!lim_env) {
        fprintf(stderr, "run with GGML_XDNA_MAX_COPY_GB set (0.05)\n");
        return 2;
    }
    const double limit = atof(lim_env) * 1024.0 * 1024.0 * 1024.0;
    const char * po = getenv("GGML_XDNA_PLAN_ONLY");
    const bool planning = po && *po && po[0] != '0';

    // the model's weights in a buffer marked as weights, named as llama.cpp names them
    ggml_init_params wparams = {ggml_tensor_overhead() * (LAYERS * PER_LAYER + 8), nullptr, true};
    ggml_context * wctx = ggml_init(wparams);
    std::vector<ggml_tensor *> weights;  // model order: layer by layer
    std::vector<int> layer_of;
    for (int l = 0; l < LAYERS; l++)
        for (const shape & s : LAYER) {
            ggml_tensor * t = ggml_new_tensor_2d(wctx, GGML_TYPE_Q8_0, s.k, s.n);
            ggml_set_name(t, ("blk." + std::to_string(l) + "." + s.name + ".weight").c_str());
            weights.push_back(t);
            layer_of.push_back(l);
        }
    ggml_backend_buffer_type_t buft = planning
        ? ggml_backend_dev_buffer_type(ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU))
        : ggml_backend_dev_buffer_type(dev);
    ggml_backend_buffer_t wbuf = ggml_backend_alloc_ctx_tensors_from_buft(wctx, buft);
    if (!wbuf) {
        fprintf(stderr, "weight buffer allocation failed\n");
        return 2;
    }
    ggml_backend_buffer_set_usage(wbuf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);

    // a tensor of weight shape in an ordinary (compute) buffer: not a weight for the budget
    ggml_init_params oparams = {ggml_tensor_overhead() * 4, nullptr, true};
    ggml_context * octx = ggml_init(oparams);
    ggml_tensor * scratch_w = ggml_new_tensor_2d(octx, GGML_TYPE_Q8_0, 8192, 4096);  // 36 MiB if it counted
    ggml_set_name(scratch_w, "blk.0.scratch.weight");
    ggml_backend_buffer_t obuf = ggml_backend_alloc_ctx_tensors_from_buft(octx, buft);

    // the questions: a matmul of the weight at batch 2048
    ggml_init_params qparams = {ggml_tensor_overhead() * 512, nullptr, true};
    ggml_context * qctx = ggml_init(qparams);
    auto asks = [&](ggml_tensor * w) {
        ggml_tensor * x = ggml_new_tensor_2d(qctx, GGML_TYPE_F32, w->ne[0], 2048);
        return ggml_backend_dev_supports_op(dev, ggml_mul_mat(qctx, w, x));
    };

    // where the contract puts the cut: the first weight whose entry does not fit
    int cut = -1;
    double sum = 0;
    for (size_t i = 0; i < weights.size(); i++) {
        const double b = entry_bytes(weights[i]->ne[1], weights[i]->ne[0]);
        if (sum + b > limit) {
            cut = (int) i;
            break;
        }
        sum += b;
    }
    if (cut < 0 || cut % PER_LAYER == 0) {
        fprintf(stderr, "the scenario must cut inside a layer (limit %.1f MiB, cut at %d)\n", limit / 1048576.0, cut);
        return 2;
    }
    const int cut_layer = layer_of[cut];
    printf("limit %.1f MiB: weights 0..%d fit (%.1f MiB); weight %d (%s) does not\n", limit / 1048576.0, cut - 1,
           sum / 1048576.0, cut, weights[cut]->name);

    // 1. no context alive: every weight is answered and none counts
    bool all = true;
    for (ggml_tensor * w : weights) all &= asks(w);
    test_check(all, "before any context exists every weight is claimed (load-time questions do not count)");

    ggml_backend_t ctx1 = ggml_backend_dev_init(dev, nullptr);
    if (!ctx1) {
        fprintf(stderr, "backend init failed\n");
        return 2;
    }

    // 2. things that are answered but not counted while a context lives
    ggml_tensor * no_data = ggml_new_tensor_2d(qctx, GGML_TYPE_Q8_0, 4096, 16384);  // 72 MiB: more than the limit
    ggml_set_name(no_data, "blk.0.fit_trial.weight");
    test_check(asks(no_data), "a weight without data (the memory-fitting trial) is claimed");
    test_check(asks(scratch_w), "a weight-shaped tensor outside a weights buffer is claimed");

    // 3. the model in order: everything before the cut is taken, the cut is not
    std::vector<int> first(weights.size());
    for (size_t i = 0; i < weights.size(); i++) first[i] = asks(weights[i]);
    bool before = true;
    for (int i = 0; i < cut; i++) before &= first[i] == 1;
    test_check(before, "the %d weights before the cut fit and were claimed as asked (neither the trial weight nor the "
                       "compute-buffer tensor used up the limit)", cut);
    test_check(first[cut] == 0, "the weight that passes the limit (%s) is refused", weights[cut]->name);
    bool after = true;
    for (size_t i = cut + 1; i < weights.size(); i++) after &= first[i] == 0;
    test_check(after, "every later weight is refused, even those small enough to fit what is left");

    // 4. the decisions are fixed, and the cut layer is handed back whole
    std::vector<int> second(weights.size());
    for (size_t i = 0; i < weights.size(); i++) second[i] = asks(weights[i]);
    bool whole_layers = true, fixed = true;
    for (size_t i = 0; i < weights.size(); i++) {
        const bool want = layer_of[i] < cut_layer;
        whole_layers &= second[i] == (int) want;
        if (layer_of[i] != cut_layer) fixed &= second[i] == first[i];
    }
    test_check(whole_layers, "asked again: layers 0..%d are claimed and layer %d is refused whole", cut_layer - 1,
               cut_layer);
    test_check(fixed, "no answer outside the cut layer changed");

    // 5. a second context while the first lives shares the process budget
    ggml_backend_t ctx2 = ggml_backend_dev_init(dev, nullptr);
    test_check(ctx2 && !asks(weights[cut]) && asks(weights[0]), "a second context sees the same decisions");
    if (ctx2) ggml_backend_free(ctx2);
    test_check(!asks(weights[cut]), "freeing one of two contexts keeps the decisions");

    // 6. the last context goes: the count starts again
    ggml_backend_free(ctx1);
    ggml_backend_t ctx3 = ggml_backend_dev_init(dev, nullptr);
    test_check(ctx3 && asks(weights[cut]) && asks(weights.back()),
               "after the last context is freed, a new one takes the cut weight and the last layer's");
    if (ctx3) ggml_backend_free(ctx3);

    ggml_free(qctx);
    ggml_backend_buffer_free(obuf);
    ggml_free(octx);
    ggml_backend_buffer_free(wbuf);
    ggml_free(wctx);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

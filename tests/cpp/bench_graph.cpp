// The qwen3-4b layer stack (36 layers, hidden 2560, q 4096, k/v 1024, FFN
// 9728; Q4_K q/k/v/gate/up, Q8_0 o/down; an 8192-token prompt in 2048-token
// chunks) through the add-on surface: ggml graphs of RMS_NORM, MUL, MUL_MAT,
// ADD and GLU nodes handed to the backend's graph_compute, as
// ggml_backend_sched hands llama.cpp's prompt graphs over (the reference's
// graph_compute is src/ggml-zest.cpp:768-926). The work is the C-ABI stack's
// (ggml_xdna_amd/stack.py, Stack.run_prompt), node for node: attention is
// left out, the output projection reading q where attention's result would
// be, so the two figures compare the same GEMMs and host ops.
//
// Two ways of cutting the prompt into graphs:
//   chunk  one graph per chunk holding all 36 layers (a model whose every
//          node runs on this backend);
//   layer  one graph per layer, cut where attention would run on another
//          backend (q/k/v in one graph, then o, the FFN and the next layer's
//          q/k/v in the next), as the scheduler splits a model whose
//          attention stays on the CPU: 37 graph_compute calls per chunk,
//          each ending in a stream synchronize.
// Weights are N(0, 0.02) values quantised to Q4_K / Q8_0, as the C-ABI
// stack's: one set of GGUF bytes per weight shape, shared by the layers,
// each layer still its own tensor and cache entry. They are converted into
// the weight cache at load (graph_optimize); the input rows are resident on
// the GPU before the clock starts.
//
// Prints one JSON line per mode: tokens per second and the MUL_MAT TFLOP/s
// of the whole prompt, host time per graph_compute included. With
// GGML_XDNA_TRACE=2 the backend also prints, per graph, its node and launch
// counts and the host time spent planning it (fusions, residual adds and the
// reader index), issuing its launches and waiting for the GPU.
//
// usage: bench_graph [--mode chunk|layer|both] [--layers L] [--steps S] [--warmup W]
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "mini_ggml.h"

namespace {

constexpr int64_t HIDDEN = 2560, QDIM = 4096, KVDIM = 1024, FFN = 9728, TOKENS = 8192, CHUNK = 2048;

struct layer_w {
    ggml_tensor * q, * k, * v, * o, * gate, * up, * down, * attn_norm, * ffn_norm;
};

ggml_tensor * new_weight(ggml_context * c, ggml_type t, int64_t k, int64_t n, int layer, const char * name) {
    ggml_tensor * w = ggml_new_tensor_2d(c, t, k, n);
    ggml_set_name(w, ("blk." + std::to_string(layer) + "." + name).c_str());
    return w;
}

// RMS_NORM -> MUL by the layer's scale row
ggml_tensor * norm(ggml_context * c, ggml_tensor * h, ggml_tensor * w) { return ggml_mul(c, ggml_rms_norm(c, h, 1e-6f), w); }

// The layer's nodes from its q projection's consumer on: o (reading `a`,
// attention's stand-in), the residual add onto h, the FFN block and its
// residual add. Returns the new h.
ggml_tensor * layer_rest(ggml_context * c, const layer_w & L, ggml_tensor * a, ggml_tensor * h) {
    h = ggml_add(c, ggml_mul_mat(c, L.o, a), h);
    ggml_tensor * n2 = norm(c, h, L.ffn_norm);
    ggml_tensor * s = ggml_swiglu_split(c, ggml_mul_mat(c, L.gate, n2), ggml_mul_mat(c, L.up, n2));
    return ggml_add(c, ggml_mul_mat(c, L.down, s), h);
}

// q, k, v of a layer on h; k and v are outputs (the cache), appended to
// `kv` for the caller to add to its graph; q feeds o
ggml_tensor * layer_qkv(ggml_context * c, const layer_w & L, ggml_tensor * h, std::vector<ggml_tensor *> & kv) {
    ggml_tensor * n1 = norm(c, h, L.attn_norm);
    ggml_tensor * q = ggml_mul_mat(c, L.q, n1);
    for (ggml_tensor * w : {L.k, L.v}) {
        kv.push_back(ggml_mul_mat(c, w, n1));
        ggml_set_output(kv.back());
    }
    return q;
}

double flops_per_token(int layers) {
    return 2.0 * layers * (double) (HIDDEN * (QDIM + 2 * KVDIM) + QDIM * HIDDEN + 2 * HIDDEN * FFN + FFN * HIDDEN);
}

}  // namespace

int main(int argc, char ** argv) {
    std::string mode = "both";
    int layers = 36, steps = 3, warmup = 1;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string a = argv[i];
        if (a == "--mode") mode = argv[i + 1];
        else if (a == "--layers") layers = atoi(argv[i + 1]);
        else if (a == "--steps") steps = atoi(argv[i + 1]);
        else if (a == "--warmup") warmup = atoi(argv[i + 1]);
        else {
            fprintf(stderr, "usage: bench_graph [--mode chunk|layer|both] [--layers L] [--steps S] [--warmup W]\n");
            return 2;
        }
    }
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "no XDNA0 device: set GGML_BACKEND_PATH to libggml-zest.so\n");
        return 2;
    }
    ggml_backend_t be = ggml_backend_dev_init(dev, nullptr);
    if (!be) {
        fprintf(stderr, "backend init failed\n");
        return 2;
    }

    // ---- weights: one set per layer, in a weights buffer on the device ----
    ggml_init_params wp = {ggml_tensor_overhead() * (size_t) (layers * 9 + 4), nullptr, true};
    ggml_context * wctx = ggml_init(wp);
    std::vector<layer_w> L((size_t) layers);
    for (int l = 0; l < layers; l++) {
        layer_w & w = L[(size_t) l];
        w.q = new_weight(wctx, GGML_TYPE_Q4_K, HIDDEN, QDIM, l, "attn_q.weight");
        w.k = new_weight(wctx, GGML_TYPE_Q4_K, HIDDEN, KVDIM, l, "attn_k.weight");
        w.v = new_weight(wctx, GGML_TYPE_Q4_K, HIDDEN, KVDIM, l, "attn_v.weight");
        w.o = new_weight(wctx, GGML_TYPE_Q8_0, QDIM, HIDDEN, l, "attn_output.weight");
        w.gate = new_weight(wctx, GGML_TYPE_Q4_K, HIDDEN, FFN, l, "ffn_gate.weight");
        w.up = new_weight(wctx, GGML_TYPE_Q4_K, HIDDEN, FFN, l, "ffn_up.weight");
        w.down = new_weight(wctx, GGML_TYPE_Q8_0, FFN, HIDDEN, l, "ffn_down.weight");
        w.attn_norm = ggml_new_tensor_1d(wctx, GGML_TYPE_F32, HIDDEN);
        w.ffn_norm = ggml_new_tensor_1d(wctx, GGML_TYPE_F32, HIDDEN);
        ggml_set_name(w.attn_norm, ("blk." + std::to_string(l) + ".attn_norm.weight").c_str());
        ggml_set_name(w.ffn_norm, ("blk." + std::to_string(l) + ".ffn_norm.weight").c_str());
    }
    ggml_backend_buffer_t wbuf = ggml_backend_alloc_ctx_tensors(wctx, be);
    if (!wbuf) {
        fprintf(stderr, "weight allocation failed\n");
        return 2;
    }
    ggml_backend_buffer_set_usage(wbuf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    {
        // the GGUF bytes of each weight shape: N(0, 0.02) rows quantised
        std::vector<std::vector<uint8_t>> src;
        test_rng wrng(7);
        for (ggml_tensor * t : {L[0].q, L[0].k, L[0].v, L[0].o, L[0].gate, L[0].up, L[0].down}) {
            std::vector<float> wf((size_t) (t->ne[0] * t->ne[1]));
            for (float & f : wf) f = wrng.normal(0.0f, 0.02f);
            src.emplace_back(ggml_nbytes(t));
            ggml_quantize_chunk(t->type, wf.data(), src.back().data(), 0, t->ne[1], t->ne[0], nullptr);
        }
        std::vector<float> row((size_t) HIDDEN);
        test_rng rng(11);
        for (int l = 0; l < layers; l++) {
            const layer_w & w = L[(size_t) l];
            size_t i = 0;
            for (ggml_tensor * t : {w.q, w.k, w.v, w.o, w.gate, w.up, w.down}) {
                ggml_backend_tensor_set(t, src[i].data(), 0, src[i].size());
                i++;
            }
            for (ggml_tensor * t : {w.attn_norm, w.ffn_norm}) {
                for (float & f : row) f = 1.0f + 0.1f * rng.normal(0.0f, 1.0f);
                ggml_backend_tensor_set(t, row.data(), 0, row.size() * sizeof(float));
            }
        }
    }
    std::vector<float> xv((size_t) (HIDDEN * CHUNK));
    {
        test_rng rng(5);
        for (float & f : xv) f = rng.normal(0.0f, 1.0f);
    }
    const double flops_chunk = flops_per_token(layers) * CHUNK;
    const int chunks = (int) (TOKENS / CHUNK);

    auto report = [&](const char * m, int graphs_per_chunk, double secs) {
        const double tokens = (double) steps * chunks * CHUNK;
        printf("{\"mode\": \"%s\", \"layers\": %d, \"tokens\": %lld, \"chunk\": %lld, \"graphs_per_chunk\": %d, "
               "\"steps\": %d, \"ms_per_step\": %.3f, \"tok_per_s\": %.1f, \"tflops\": %.2f}\n",
               m, layers, (long long) TOKENS, (long long) CHUNK, graphs_per_chunk, steps, secs * 1e3 / steps,
               tokens / secs, flops_chunk * steps * chunks / secs / 1e12);
        fflush(stdout);
    };
    using clock = std::chrono::steady_clock;
    int status = 0;
    std::vector<std::pair<ggml_context *, ggml_backend_buffer_t>> keep;

    // ---- one graph per chunk ----
    if (mode == "chunk" || mode == "both") {
        ggml_init_params ip = {ggml_tensor_overhead() * (size_t) (layers * 32 + 8) + ggml_graph_overhead(), nullptr, true};
        ggml_context * ctx = ggml_init(ip);
        ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, HIDDEN, CHUNK);
        ggml_set_input(x);
        ggml_tensor * h = x;
        ggml_cgraph * gf = ggml_new_graph(ctx);
        for (int l = 0; l < layers; l++) {
            std::vector<ggml_tensor *> kv;
            ggml_tensor * q = layer_qkv(ctx, L[(size_t) l], h, kv);
            for (ggml_tensor * t : kv) ggml_build_forward_expand(gf, t);
            h = layer_rest(ctx, L[(size_t) l], q, h);
        }
        ggml_set_output(h);
        ggml_build_forward_expand(gf, h);
        ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
        if (!buf) {
            fprintf(stderr, "chunk graph: allocation failed\n");
            return 2;
        }
        ggml_backend_tensor_set(x, xv.data(), 0, ggml_nbytes(x));
        ggml_backend_plan_graph(be, gf);
        bool ok = true;
        for (int i = 0; i < warmup * chunks && ok; i++) ok = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
        const auto t0 = clock::now();
        for (int i = 0; i < steps * chunks && ok; i++) ok = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
        const double secs = std::chrono::duration<double>(clock::now() - t0).count();
        if (ok) report("chunk", 1, secs);
        else {
            fprintf(stderr, "chunk graph: graph_compute failed\n");
            status = 1;
        }
        // kept until the end: a tensor of the next graphs allocated where one
        // of these was would inherit its recorded readers (the backend keeps
        // readers by address, as the reference does)
        keep.push_back({ctx, buf});
    }

    // ---- one graph per layer, cut where attention would run ----
    if (status == 0 && (mode == "layer" || mode == "both")) {
        ggml_init_params ip = {ggml_tensor_overhead() * (size_t) (layers * 32 + 8) + ggml_graph_overhead() * (size_t) (layers + 2),
                               nullptr, true};
        ggml_context * ctx = ggml_init(ip);   // every node, allocated
        ggml_context * lctx = ggml_init(ip);  // each graph's inputs: leaves sharing an earlier graph's result
        ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, HIDDEN, CHUNK);
        ggml_set_input(x);
        struct link {
            ggml_tensor * leaf, * from;
        };
        std::vector<link> links;
        auto leaf_of = [&](ggml_tensor * from) {
            ggml_tensor * t = ggml_new_tensor_2d(lctx, GGML_TYPE_F32, from->ne[0], from->ne[1]);
            links.push_back({t, from});
            return t;
        };
        std::vector<ggml_cgraph *> graphs;
        // graph 0: layer 0's q, k, v
        std::vector<ggml_tensor *> kv;
        ggml_tensor * q = layer_qkv(ctx, L[0], x, kv);
        ggml_set_output(q);
        graphs.push_back(ggml_new_graph(ctx));
        for (ggml_tensor * t : kv) ggml_build_forward_expand(graphs.back(), t);
        ggml_build_forward_expand(graphs.back(), q);
        ggml_tensor * h = x;
        for (int l = 0; l < layers; l++) {
            // graph l+1: layer l's o, FFN, and layer l+1's q, k, v, on the
            // previous graph's results (q standing in for attention's)
            ggml_tensor * hin = l == 0 ? x : leaf_of(h);
            h = layer_rest(ctx, L[(size_t) l], leaf_of(q), hin);
            ggml_set_output(h);
            graphs.push_back(ggml_new_graph(ctx));
            ggml_build_forward_expand(graphs.back(), h);
            if (l + 1 < layers) {
                kv.clear();
                q = layer_qkv(ctx, L[(size_t) l + 1], h, kv);
                ggml_set_output(q);
                for (ggml_tensor * t : kv) ggml_build_forward_expand(graphs.back(), t);
                ggml_build_forward_expand(graphs.back(), q);
            }
        }
        ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
        if (!buf) {
            fprintf(stderr, "layer graphs: allocation failed\n");
            return 2;
        }
        for (const link & k : links) {
            k.leaf->buffer = k.from->buffer;
            k.leaf->data = k.from->data;
        }
        ggml_backend_tensor_set(x, xv.data(), 0, ggml_nbytes(x));
        for (ggml_cgraph * g : graphs) ggml_backend_plan_graph(be, g);
        bool ok = true;
        auto chunk_pass = [&] {
            for (ggml_cgraph * g : graphs)
                if (ok) ok = ggml_backend_graph_compute(be, g) == GGML_STATUS_SUCCESS;
        };
        for (int i = 0; i < warmup * chunks && ok; i++) chunk_pass();
        const auto t0 = clock::now();
        for (int i = 0; i < steps * chunks && ok; i++) chunk_pass();
        const double secs = std::chrono::duration<double>(clock::now() - t0).count();
        if (ok) report("layer", (int) graphs.size(), secs);
        else {
            fprintf(stderr, "layer graphs: graph_compute failed\n");
            status = 1;
        }
        keep.push_back({ctx, buf});
        keep.push_back({lctx, nullptr});
    }

    for (auto & k : keep) {
        ggml_backend_buffer_free(k.second);
        ggml_free(k.first);
    }
    ggml_backend_buffer_free(wbuf);
    ggml_free(wctx);
    ggml_backend_free(be);
    return status;
}

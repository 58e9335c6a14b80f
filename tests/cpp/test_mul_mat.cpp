// The backend's MUL_MAT through graph_compute, on the GPU, at the shapes of
// the reference's tests/test-mul-mat.cpp (its types this path converts).
//
// Two bars. (1) The rigorous one: against an fp64 product of the SAME operands
// the GPU multiplies (activations through the oracle's bfp16 encode/decode,
// weights through the oracle's GGUF dequantiser and then bfp16), every output within
// 2*K*2^-24*sum|a_k w_k| (bf16 products are exact in fp32, so only the fp32
// summation order may differ; no relative slack). (2) The reference's own style: against the
// fp64 product of the raw operands, nrmse <= 1e-2 and cosine > 0.9999 (bfp16
// activations carry 8-bit mantissas).
//
// Weights in a weight buffer exercise the load-time conversion
// (graph_optimize, then the cache); host-memory activations and weights
// exercise the upload path.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "mini_ggml.h"
#include "zest_oracle.h"

struct case_spec {
    const char * name;
    ggml_type wtype;
    int64_t k, n, m;
    bool weights;     // in a weight buffer, converted at load
    bool host_input;  // activations in host memory
    bool host_weight; // weights in host memory
};

struct result {
    bool ok_bound;
    double worst, nrmse, cos;
};

static std::vector<float> run_on(ggml_backend_t be, const case_spec & c, const std::vector<uint8_t> & wdata,
                                 const std::vector<float> & xdata) {
    ggml_init_params ip = {ggml_tensor_overhead() * 8 + ggml_graph_overhead(), nullptr, true};
    ggml_context * wctx = ggml_init(ip), * ictx = ggml_init(ip), * ctx = ggml_init(ip);
    ggml_backend_buffer_type_t host = ggml_backend_dev_buffer_type(ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU));
    ggml_backend_buffer_type_t dev = ggml_backend_get_default_buffer_type(be);

    ggml_tensor * a = ggml_new_tensor_2d(wctx, c.wtype, c.k, c.n);
    ggml_set_name(a, "blk.0.ffn_up.weight");
    ggml_tensor * b = ggml_new_tensor_2d(ictx, GGML_TYPE_F32, c.k, c.m);
    ggml_set_input(b);
    ggml_tensor * d = ggml_mul_mat(ctx, a, b);
    ggml_set_output(d);

    ggml_backend_buffer_t wbuf = ggml_backend_alloc_ctx_tensors_from_buft(wctx, c.host_weight ? host : dev);
    ggml_backend_buffer_t ibuf = ggml_backend_alloc_ctx_tensors_from_buft(ictx, c.host_input ? host : dev);
    ggml_backend_buffer_t obuf = ggml_backend_alloc_ctx_tensors_from_buft(ctx, dev);
    std::vector<float> out;
    if (!wbuf || !ibuf || !obuf) {
        fprintf(stderr, "  alloc failed\n");
    } else {
        if (c.weights) ggml_backend_buffer_set_usage(wbuf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
        ggml_backend_tensor_set(a, wdata.data(), 0, ggml_nbytes(a));
        ggml_backend_tensor_set(b, xdata.data(), 0, ggml_nbytes(b));
        ggml_cgraph * gf = ggml_new_graph(ctx);
        ggml_build_forward_expand(gf, d);
        ggml_backend_plan_graph(be, gf);
        const ggml_status st = ggml_backend_graph_compute(be, gf);
        if (st != GGML_STATUS_SUCCESS) {
            fprintf(stderr, "  compute failed: %d\n", (int) st);
        } else {
            out.resize((size_t) (c.n * c.m));
            ggml_backend_tensor_get(d, out.data(), 0, out.size() * sizeof(float));
        }
    }
    ggml_backend_buffer_free(obuf);
    ggml_backend_buffer_free(ibuf);
    ggml_backend_buffer_free(wbuf);
    ggml_free(ctx);
    ggml_free(ictx);
    ggml_free(wctx);
    return out;
}

static result judge(const case_spec & c, const std::vector<float> & got, const std::vector<uint8_t> & wdata,
                    const std::vector<float> & x) {
    // the operands the GPU multiplies
    std::vector<float> w((size_t) (c.n * c.k)), xq(x.size());
    const size_t rb = ggml_row_size(c.wtype, c.k);
    for (int64_t i = 0; i < c.n; i++) ggml_dequantize_row(c.wtype, wdata.data() + i * rb, w.data() + i * c.k, c.k);
    // both operands go through bfp16: the activations when packed, the
    // dequantised weights when their cache entry is built
    std::vector<float> wq(w.size());
    std::vector<uint8_t> enc((size_t) (std::max(c.m, c.n) * c.k / 8 * 9));
    orc_bfp16_encode_rows(x.data(), c.m, c.k, enc.data());
    orc_bfp16_decode_rows(enc.data(), c.m, c.k, xq.data());
    orc_bfp16_encode_rows(w.data(), c.n, c.k, enc.data());
    orc_bfp16_decode_rows(enc.data(), c.n, c.k, wq.data());
    std::vector<double> r((size_t) (c.m * c.n)), absdot(r.size()), raw(r.size());
    orc_mul_mat_f64(wq.data(), c.n, c.k, xq.data(), c.m, r.data(), absdot.data(), 8);
    orc_mul_mat_f64(w.data(), c.n, c.k, x.data(), c.m, raw.data(), nullptr, 8);

    result res{true, 0, 0, 0};
    double se = 0, ss = 0, dot = 0, ng = 0;
    for (size_t i = 0; i < r.size(); i++) {
        const double g = got[i];
        // fp32 summation order of exact bf16 products is the only allowed
        // difference: no relative slack, so a systematic error shows
        const double bound = 2.0 * (double) c.k * 0x1p-24 * absdot[i];
        const double e = std::fabs(g - r[i]);
        if (!(e <= bound)) res.ok_bound = false;
        res.worst = std::max(res.worst, bound > 0 ? e / bound : (e > 0 ? INFINITY : 0));
        se += (g - raw[i]) * (g - raw[i]);
        ss += raw[i] * raw[i];
        dot += g * raw[i];
        ng += g * g;
    }
    res.nrmse = std::sqrt(se / std::max(ss, 1e-300));
    res.cos = dot / std::max(std::sqrt(ng * ss), 1e-300);
    return res;
}

int main() {
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "XDNA device not registered - is GGML_BACKEND_PATH set?\n");
        return 2;
    }
    ggml_backend_t be = ggml_backend_dev_init(dev, nullptr);
    if (!be) {
        fprintf(stderr, "cannot start the backend\n");
        return 2;
    }

    const case_spec cases[] = {
        {"f32   256x128 x 64", GGML_TYPE_F32, 256, 128, 64, false, false, false},
        {"f16   256x128 x 64", GGML_TYPE_F16, 256, 128, 64, false, false, false},
        {"q8_0  512x256 x 64", GGML_TYPE_Q8_0, 512, 256, 64, false, false, false},
        {"q4_0  512x256 x 64", GGML_TYPE_Q4_0, 512, 256, 64, false, false, false},
        {"q4_K  512x256 x 64", GGML_TYPE_Q4_K, 512, 256, 64, false, false, false},
        {"q4_K 2048x512 x 512", GGML_TYPE_Q4_K, 2048, 512, 512, false, false, false},
        {"q6_K  512x256 x 64", GGML_TYPE_Q6_K, 512, 256, 64, false, false, false},
        // the other GGUF types the converter takes
        {"bf16  256x128 x 64", GGML_TYPE_BF16, 256, 128, 64, false, false, false},
        {"q4_1  512x256 x 64", GGML_TYPE_Q4_1, 512, 256, 64, false, false, false},
        {"q5_0  512x256 x 64", GGML_TYPE_Q5_0, 512, 256, 64, false, false, false},
        {"q5_1  512x256 x 64", GGML_TYPE_Q5_1, 512, 256, 64, false, false, false},
        {"q2_K  512x256 x 64", GGML_TYPE_Q2_K, 512, 256, 64, false, false, false},
        {"q3_K  512x256 x 64", GGML_TYPE_Q3_K, 512, 256, 64, false, false, false},
        {"q5_K  512x256 x 64", GGML_TYPE_Q5_K, 512, 256, 64, false, false, false},
        {"iq4_nl 512x256 x 64", GGML_TYPE_IQ4_NL, 512, 256, 64, false, false, false},
        {"iq4_xs 512x256 x 64", GGML_TYPE_IQ4_XS, 512, 256, 64, false, false, false},
        // held in a weight buffer, as llama.cpp loads a model; one weight type
        // each: the cache is keyed by where a weight lives, and a freed
        // buffer's address comes back
        {"q4_0 2048x1024 x 512 w", GGML_TYPE_Q4_0, 2048, 1024, 512, true, false, false},
        {"q4_K 2048x1024 x 600 w", GGML_TYPE_Q4_K, 2048, 1024, 600, true, false, false},
        // a Q4_K_M model's Q6_K down projection (Qwen3-4B: 9728 -> 2560)
        {"q6_K 9728x2560 x 256 w", GGML_TYPE_Q6_K, 9728, 2560, 256, true, false, false},
        // widths that are not multiples of the 256-row tile
        {"q4_0 1536x896 x 512 w", GGML_TYPE_Q4_0, 1536, 896, 512, true, false, false},
        {"q8_0 1536x256 x 512 w", GGML_TYPE_Q8_0, 1536, 256, 512, true, false, false},
        {"q4_K 1536x8960 x 520 w", GGML_TYPE_Q4_K, 1536, 8960, 520, true, false, false},
        // K not a multiple of 64 (padded chunk), odd batch
        {"f32   200x300 x 77", GGML_TYPE_F32, 200, 300, 77, false, false, false},
        // memory on the host side
        {"q4_K 2560x2560 x 1024 host x", GGML_TYPE_Q4_K, 2560, 2560, 1024, true, true, false},
        {"q8_0 2560x1024 x 1024 host w", GGML_TYPE_Q8_0, 2560, 1024, 1024, true, false, true},
        // the headline correctness shape: 1024 tokens x 2560 x 2560, Q8_0
        {"q8_0 2560x2560 x 1024 w", GGML_TYPE_Q8_0, 2560, 2560, 1024, true, false, false},
    };

    test_rng rng(1234);
    for (const case_spec & c : cases) {
        std::vector<float> wf((size_t) (c.k * c.n));
        for (float & v : wf) v = rng.normal(0.0f, 1.0f);
        std::vector<uint8_t> wdata(ggml_row_size(c.wtype, c.k) * (size_t) c.n);
        ggml_quantize_chunk(c.wtype, wf.data(), wdata.data(), 0, c.n, c.k, nullptr);
        std::vector<float> x((size_t) (c.k * c.m));
        for (float & v : x) v = rng.normal(0.0f, 1.0f);

        const std::vector<float> got = run_on(be, c, wdata, x);
        if (got.size() != (size_t) (c.n * c.m)) {
            test_check(false, "%-28s could not compute", c.name);
            continue;
        }
        const result r = judge(c, got, wdata, x);
        test_check(r.ok_bound && r.nrmse <= 1e-2 && r.cos > 0.9999,
                   "%-28s bound use %.2e, nrmse vs raw %.2e, cos %.6f", c.name, r.worst, r.nrmse, r.cos);
    }

    ggml_backend_free(be);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

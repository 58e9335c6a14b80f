// The small ops between the matmuls, through the backend's graph_compute on
// the GPU, against the oracle's CPU restatement of the reference's host passes
// (src/xdna-exec.cpp:253-346): the 21 cases of the reference's
// tests/test-host-ops.cpp, nrmse <= 1e-5 each (GELUs are computed, not read
// from a table, on both sides). Inputs as there: normal(0, 1.5), rope factors
// uniform in [1, 4), positions 5000 + 300 i.
//
// Then whole pieces as the scheduler hands them over (supports_op asked first,
// so the reader tracking knows the graph): RMS_NORM+MUL fused with the pack
// for the q/k/v matmuls, and an FFN block whose SwiGLU writes packed
// activations for the down projection, checked end to end against fp64.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <vector>

#include "mini_ggml.h"
#include "zest_oracle.h"

using fvec = std::vector<float>;
using ivec = std::vector<int32_t>;

// The inputs of one case, each made together with how its values are drawn:
// activations and scale rows normal(0, 1.5), rope frequency factors uniform
// in [1, 4), positions 5000 + 300 i (past a short context). Values are drawn
// in the order the inputs are made, so a case makes them in separate
// statements (the order in which a call's arguments are evaluated is not
// specified).
class case_inputs {
public:
    enum class draw { normal, factor, position };
    explicit case_inputs(ggml_context * ctx) : ctx_(ctx) {}

    ggml_tensor * rows(int64_t width, int64_t n, int64_t planes = 1) {
        return add(ggml_new_tensor_3d(ctx_, GGML_TYPE_F32, width, n, planes), draw::normal);
    }
    ggml_tensor * row(int64_t width) { return add(ggml_new_tensor_1d(ctx_, GGML_TYPE_F32, width), draw::normal); }
    ggml_tensor * factors(int64_t n) { return add(ggml_new_tensor_1d(ctx_, GGML_TYPE_F32, n), draw::factor); }
    ggml_tensor * positions(int64_t n) { return add(ggml_new_tensor_1d(ctx_, GGML_TYPE_I32, n), draw::position); }
    ggml_context * ctx() const { return ctx_; }

    // Draws every input's values (in creation order, from one seeded
    // stream), uploads them, and returns them for the oracle: the float
    // inputs in order, and the position inputs in order.
    void upload(uint64_t seed, std::vector<fvec> & floats, std::vector<ivec> & pos) const {
        test_rng rng(seed);
        for (const auto & [t, how] : made_) {
            const size_t n = (size_t) ggml_nelements(t);
            if (how == draw::position) {
                ivec v(n);
                for (size_t i = 0; i < n; i++) v[i] = 5000 + 300 * (int32_t) i;
                ggml_backend_tensor_set(t, v.data(), 0, ggml_nbytes(t));
                pos.push_back(std::move(v));
                continue;
            }
            fvec v(n);
            for (float & x : v) x = how == draw::factor ? (float) (1.0 + 3.0 * rng.uniform()) : rng.normal(0.0f, 1.5f);
            ggml_backend_tensor_set(t, v.data(), 0, ggml_nbytes(t));
            floats.push_back(std::move(v));
        }
    }

private:
    ggml_tensor * add(ggml_tensor * t, draw how) {
        made_.emplace_back(t, how);
        return t;
    }
    ggml_context * ctx_;
    std::vector<std::pair<ggml_tensor *, draw>> made_;
};

struct op_case {
    const char * name;
    std::function<ggml_tensor *(case_inputs &)> build;
    // the oracle's answer from the inputs' values (floats, positions)
    std::function<fvec(const std::vector<fvec> &, const std::vector<ivec> &)> cpu;
};

static double nrmse(const fvec & got, const fvec & want) {
    double se = 0, ss = 0;
    for (size_t i = 0; i < got.size(); i++) {
        se += ((double) got[i] - want[i]) * ((double) got[i] - want[i]);
        ss += (double) want[i] * want[i];
    }
    return std::sqrt(se / std::max(ss, 1e-300));
}

// One case: its graph on the backend, its inputs drawn with seed 42, its
// result against the oracle's.
static bool run_case(ggml_backend_t be, const op_case & c) {
    ggml_init_params ip = {ggml_tensor_overhead() * 16 + ggml_graph_overhead(), nullptr, true};
    ggml_context * ctx = ggml_init(ip);
    case_inputs in(ctx);
    ggml_tensor * out = c.build(in);
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
    if (!buf) {
        ggml_free(ctx);
        return test_check(false, "%-32s could not allocate", c.name);
    }
    std::vector<fvec> floats;
    std::vector<ivec> pos;
    in.upload(42, floats, pos);
    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, out);
    const bool ran = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
    fvec got(ran ? (size_t) ggml_nelements(out) : 0);
    if (ran) ggml_backend_tensor_get(out, got.data(), 0, ggml_nbytes(out));
    ggml_backend_buffer_free(buf);
    ggml_free(ctx);
    const fvec want = c.cpu(floats, pos);
    if (!ran || got.size() != want.size()) return test_check(false, "%-32s could not compute", c.name);
    const double e = nrmse(got, want);
    return test_check(std::isfinite(e) && e <= 1e-5, "%-32s nrmse %.2e (allowed 1e-05)", c.name, e);
}

// ---- whole pieces ------------------------------------------------------------------

struct weight {
    ggml_tensor * t;
    std::vector<uint8_t> bytes;
    fvec deq;  // what the GPU multiplies
};

// rows of k floats through the bfp16 encoder and back (what packing does)
static fvec bfp16(const fvec & x, int64_t rows, int64_t k) {
    std::vector<uint8_t> enc((size_t) (rows * k / 8 * 9));
    fvec y(x.size());
    orc_bfp16_encode_rows(x.data(), rows, k, enc.data());
    orc_bfp16_decode_rows(enc.data(), rows, k, y.data());
    return y;
}

static void make_weight(weight & w, test_rng & rng, float sd) {
    const int64_t k = w.t->ne[0], n = w.t->ne[1];
    fvec f((size_t) (k * n));
    for (float & v : f) v = rng.normal(0.0f, sd);
    w.bytes.resize(ggml_row_size(w.t->type, k) * (size_t) n);
    ggml_quantize_chunk(w.t->type, f.data(), w.bytes.data(), 0, n, k, nullptr);
    w.deq.resize(f.size());
    const size_t rb = ggml_row_size(w.t->type, k);
    for (int64_t i = 0; i < n; i++) ggml_dequantize_row(w.t->type, w.bytes.data() + i * rb, w.deq.data() + i * k, k);
    w.deq = bfp16(w.deq, n, k);  // the weight cache holds bfp16
}

static fvec matmul64(const fvec & w, int64_t n, int64_t k, const fvec & x, int64_t m) {
    std::vector<double> y((size_t) (m * n));
    orc_mul_mat_f64(w.data(), n, k, x.data(), m, y.data(), nullptr, 8);
    return fvec(y.begin(), y.end());
}

static void cos_nrmse(const fvec & got, const fvec & want, double & e, double & cs) {
    double se = 0, ss = 0, dot = 0, gg = 0;
    for (size_t i = 0; i < got.size(); i++) {
        se += ((double) got[i] - want[i]) * ((double) got[i] - want[i]);
        ss += (double) want[i] * want[i];
        dot += (double) got[i] * want[i];
        gg += (double) got[i] * got[i];
    }
    e = std::sqrt(se / std::max(ss, 1e-300));
    cs = dot / std::max(std::sqrt(ss * gg), 1e-300);
}

// x -> RMS_NORM -> MUL(scale row) -> q, k, v projections (Q4_K); then an FFN block:
// x -> RMS_NORM -> MUL -> gate, up (Q4_K) -> SwiGLU -> down (Q8_0) -> ADD x.
static void piece_tests(ggml_backend_t be) {
    const int64_t T = 1024, D = 1024, F = 2816, DQ = 1024, DKV = 256;
    test_rng rng(7);
    ggml_init_params ip = {ggml_tensor_overhead() * 64 + ggml_graph_overhead(), nullptr, true};
    ggml_context * wctx = ggml_init(ip), * ctx = ggml_init(ip);
    weight wq{ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, D, DQ), {}, {}}, wk{ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, D, DKV), {}, {}},
        wv{ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, D, DKV), {}, {}}, wg{ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, D, F), {}, {}},
        wu{ggml_new_tensor_2d(wctx, GGML_TYPE_Q4_K, D, F), {}, {}}, wd{ggml_new_tensor_2d(wctx, GGML_TYPE_Q8_0, F, D), {}, {}};
    ggml_set_name(wq.t, "blk.0.attn_q.weight");
    ggml_set_name(wk.t, "blk.0.attn_k.weight");
    ggml_set_name(wv.t, "blk.0.attn_v.weight");
    ggml_set_name(wg.t, "blk.0.ffn_gate.weight");
    ggml_set_name(wu.t, "blk.0.ffn_up.weight");
    ggml_set_name(wd.t, "blk.0.ffn_down.weight");
    ggml_tensor * n1 = ggml_new_tensor_1d(wctx, GGML_TYPE_F32, D), * n2 = ggml_new_tensor_1d(wctx, GGML_TYPE_F32, D);
    ggml_set_name(n1, "blk.0.attn_norm.weight");
    ggml_set_name(n2, "blk.0.ffn_norm.weight");

    ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, D, T);
    ggml_set_input(x);
    ggml_tensor * h1 = ggml_mul(ctx, ggml_rms_norm(ctx, x, 1e-6f), n1);
    ggml_tensor * q = ggml_mul_mat(ctx, wq.t, h1), * k = ggml_mul_mat(ctx, wk.t, h1), * v = ggml_mul_mat(ctx, wv.t, h1);
    ggml_tensor * h2 = ggml_mul(ctx, ggml_rms_norm(ctx, x, 1e-6f), n2);
    ggml_tensor * g = ggml_mul_mat(ctx, wg.t, h2), * u = ggml_mul_mat(ctx, wu.t, h2);
    ggml_tensor * s = ggml_swiglu_split(ctx, g, u);
    ggml_tensor * o = ggml_add(ctx, ggml_mul_mat(ctx, wd.t, s), x);
    // h2 is also read outside (a graph output): its fp32 values are written
    // beside the packed copy; h1 and the SwiGLU result exist only packed
    for (ggml_tensor * t : {q, k, v, o, h2}) ggml_set_output(t);

    ggml_backend_buffer_t wbuf = ggml_backend_alloc_ctx_tensors(wctx, be);
    ggml_backend_buffer_t abuf = ggml_backend_alloc_ctx_tensors(ctx, be);
    if (!wbuf || !abuf) {
        test_check(false, "pieces: could not allocate");
        return;
    }
    ggml_backend_buffer_set_usage(wbuf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    for (weight * w : {&wq, &wk, &wv, &wg, &wu, &wd}) {
        make_weight(*w, rng, 0.05f);
        ggml_backend_tensor_set(w->t, w->bytes.data(), 0, w->bytes.size());
    }
    fvec xv((size_t) (D * T)), n1v((size_t) D), n2v((size_t) D);
    for (float & f : xv) f = rng.normal(0.0f, 1.0f);
    for (float & f : n1v) f = 1.0f + 0.1f * rng.normal(0.0f, 1.0f);
    for (float & f : n2v) f = 1.0f + 0.1f * rng.normal(0.0f, 1.0f);
    ggml_backend_tensor_set(x, xv.data(), 0, ggml_nbytes(x));
    ggml_backend_tensor_set(n1, n1v.data(), 0, ggml_nbytes(n1));
    ggml_backend_tensor_set(n2, n2v.data(), 0, ggml_nbytes(n2));

    ggml_cgraph * gf = ggml_new_graph(ctx);
    for (ggml_tensor * t : {q, k, v, o, h2}) ggml_build_forward_expand(gf, t);
    ggml_backend_plan_graph(be, gf);
    const bool ok = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
    test_check(ok, "pieces: an attention-input and FFN block run as one graph");
    if (ok) {
        // the same chain on the CPU: fp32 host ops, bfp16 packing where the
        // GPU packs, fp64 products; only fp32 rounding (and the rare packed
        // value it moves across a rounding boundary) can differ
        fvec r1((size_t) (D * T)), h1v((size_t) (D * T)), r2((size_t) (D * T)), h2v((size_t) (D * T));
        orc_rms_norm(xv.data(), T, D, 1e-6f, r1.data());
        orc_mul_row(r1.data(), T, D, n1v.data(), h1v.data());
        orc_rms_norm(xv.data(), T, D, 1e-6f, r2.data());
        orc_mul_row(r2.data(), T, D, n2v.data(), h2v.data());
        const fvec h1p = bfp16(h1v, T, D), h2p = bfp16(h2v, T, D);
        const fvec qw = matmul64(wq.deq, DQ, D, h1p, T), kw = matmul64(wk.deq, DKV, D, h1p, T),
                   vw = matmul64(wv.deq, DKV, D, h1p, T);
        const fvec gw = matmul64(wg.deq, F, D, h2p, T), uw = matmul64(wu.deq, F, D, h2p, T);
        fvec sw((size_t) (F * T));
        orc_glu(ORC_GLU_SWIGLU, gw.data(), F, uw.data(), F, T, F, sw.data());
        fvec ow = matmul64(wd.deq, D, F, bfp16(sw, T, F), T);
        for (size_t i = 0; i < ow.size(); i++) ow[i] += xv[i];
        struct {
            const char * name;
            ggml_tensor * t;
            const fvec * want;
            double tol;
        } outs[] = {{"q", q, &qw, 1e-3}, {"k", k, &kw, 1e-3}, {"v", v, &vw, 1e-3}, {"ffn out + residual", o, &ow, 1e-3},
                    {"ffn norm (fp32 out)", h2, &h2v, 1e-5}};
        for (auto & e : outs) {
            fvec got((size_t) ggml_nelements(e.t));
            ggml_backend_tensor_get(e.t, got.data(), 0, ggml_nbytes(e.t));
            double err, cs;
            cos_nrmse(got, *e.want, err, cs);
            test_check(err <= e.tol, "pieces: %-20s nrmse %.2e (allowed %.0e) cos %.7f vs the CPU chain", e.name, err,
                       e.tol, cs);
        }

        // The same graph again: the backend reuses what it worked out about it,
        // and the results are the same bits.
        auto read = [](ggml_tensor * t) {
            fvec v((size_t) ggml_nelements(t));
            ggml_backend_tensor_get(t, v.data(), 0, ggml_nbytes(t));
            return v;
        };
        const fvec q1 = read(q), o1 = read(o);
        bool again = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
        test_check(again && read(q) == q1 && read(o) == o1, "pieces: computed again, the same results bit for bit");

        // The gate's result made a graph output: it is now read outside the
        // piece, so gate and up may no longer run fused (the fused GEMM never
        // writes them). A plan kept from before would leave g unwritten.
        ggml_set_output(g);
        std::vector<float> poison((size_t) ggml_nelements(g), -12345.0f);
        ggml_backend_tensor_set(g, poison.data(), 0, ggml_nbytes(g));
        again = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
        if (again) {
            double eg, cg, eo, co;
            cos_nrmse(read(g), gw, eg, cg);
            cos_nrmse(read(o), ow, eo, co);
            test_check(eg <= 1e-3 && eo <= 1e-3,
                       "pieces: with the gate an output, planned again: gate nrmse %.2e, ffn out nrmse %.2e", eg, eo);
        } else {
            test_check(false, "pieces: compute with the gate an output");
        }
    }
    ggml_backend_buffer_free(abuf);
    ggml_backend_buffer_free(wbuf);
    ggml_free(ctx);
    ggml_free(wctx);
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

    const int64_t D = 256, T = 8, HD = 64, H = 4;
    using vin = std::vector<fvec>;
    using pin = std::vector<ivec>;
    // the oracle's answer of `rows` x `width` floats, filled by `f`
    auto answer = [](int64_t n, auto f) {
        fvec y((size_t) n);
        f(y.data());
        return y;
    };
    auto glu_split = [&](const char * name, ggml_glu_op op, int kind) {
        return op_case{name,
                       [=](case_inputs & in) {
                           ggml_tensor * g = in.rows(D, T);  // made first: its values are drawn first
                           ggml_tensor * u = in.rows(D, T);
                           return ggml_glu_split(in.ctx(), g, u, op);
                       },
                       [=](const vin & v, const pin &) {
                           return answer(D * T, [&](float * y) { orc_glu(kind, v[0].data(), D, v[1].data(), D, T, D, y); });
                       }};
    };
    auto glu_one = [&](const char * name, ggml_glu_op op, int kind, bool swapped) {
        return op_case{name, [=](case_inputs & in) { return ggml_glu(in.ctx(), in.rows(2 * D, T), op, swapped); },
                       [=](const vin & v, const pin &) {
                           const float * gate = v[0].data() + (swapped ? D : 0), * up = v[0].data() + (swapped ? 0 : D);
                           return answer(D * T, [&](float * y) { orc_glu(kind, gate, 2 * D, up, 2 * D, T, D, y); });
                       }};
    };
    // ROPE over T tokens of H heads of HD, rotating the first n_dims of each
    // head, base 10000, beta_fast 32, beta_slow 1
    auto rope = [&](const char * name, int n_dims, int mode, int n_ctx_orig, float freq_scale, float ext_factor,
                    bool factors) {
        return op_case{name,
                       [=](case_inputs & in) {
                           ggml_tensor * x = in.rows(HD, H, T);
                           ggml_tensor * p = in.positions(T);
                           ggml_tensor * ff = factors ? in.factors(n_dims / 2) : nullptr;
                           return ggml_rope_ext(in.ctx(), x, p, ff, n_dims, mode, n_ctx_orig, 10000.0f, freq_scale,
                                                ext_factor, 1.0f, 32.0f, 1.0f);
                       },
                       [=](const vin & v, const pin & p) {
                           return answer(HD * H * T, [&](float * y) {
                               orc_rope(v[0].data(), T, H, HD, p[0].data(), factors ? v[1].data() : nullptr, n_dims,
                                        mode, n_ctx_orig, 10000.0f, freq_scale, ext_factor, 1.0f, 32.0f, 1.0f, y);
                           });
                       }};
    };

    const op_case cases[] = {
        {"rms_norm", [&](case_inputs & in) { return ggml_rms_norm(in.ctx(), in.rows(D, T), 1e-6f); },
         [&](const vin & v, const pin &) {
             return answer(D * T, [&](float * y) { orc_rms_norm(v[0].data(), T, D, 1e-6f, y); });
         }},
        {"mul by a scale row",
         [&](case_inputs & in) {
             ggml_tensor * x = in.rows(D, T);
             return ggml_mul(in.ctx(), x, in.row(D));
         },
         [&](const vin & v, const pin &) {
             return answer(D * T, [&](float * y) { orc_mul_row(v[0].data(), T, D, v[1].data(), y); });
         }},
        {"add",
         [&](case_inputs & in) {
             ggml_tensor * a = in.rows(D, T);
             return ggml_add(in.ctx(), a, in.rows(D, T));
         },
         [&](const vin & v, const pin &) {
             return answer(D * T, [&](float * y) { orc_add(v[0].data(), v[1].data(), D * T, y); });
         }},
        {"add a bias row",
         [&](case_inputs & in) {
             ggml_tensor * x = in.rows(D, T);
             return ggml_add(in.ctx(), x, in.row(D));
         },
         [&](const vin & v, const pin &) {
             return answer(D * T, [&](float * y) { orc_add_row(v[0].data(), T, D, v[1].data(), y); });
         }},
        {"scale and bias", [&](case_inputs & in) { return ggml_scale_bias(in.ctx(), in.rows(D, T), 0.37f, 0.25f); },
         [&](const vin & v, const pin &) {
             return answer(D * T, [&](float * y) { orc_scale(v[0].data(), D * T, 0.37f, 0.25f, y); });
         }},
        glu_split("swiglu, split", GGML_GLU_OP_SWIGLU, ORC_GLU_SWIGLU),
        glu_split("geglu, split", GGML_GLU_OP_GEGLU, ORC_GLU_GEGLU),
        glu_split("geglu_erf, split", GGML_GLU_OP_GEGLU_ERF, ORC_GLU_GEGLU_ERF),
        glu_split("geglu_quick, split", GGML_GLU_OP_GEGLU_QUICK, ORC_GLU_GEGLU_QUICK),
        glu_split("reglu, split", GGML_GLU_OP_REGLU, ORC_GLU_REGLU),
        glu_one("swiglu, one tensor", GGML_GLU_OP_SWIGLU, ORC_GLU_SWIGLU, false),
        glu_one("swiglu, one tensor, swapped", GGML_GLU_OP_SWIGLU, ORC_GLU_SWIGLU, true),
        glu_one("geglu, one tensor", GGML_GLU_OP_GEGLU, ORC_GLU_GEGLU, false),
        glu_one("geglu_erf, one tensor", GGML_GLU_OP_GEGLU_ERF, ORC_GLU_GEGLU_ERF, false),
        rope("rope, normal", HD, GGML_ROPE_TYPE_NORMAL, 0, 1.0f, 0.0f, false),
        rope("rope, neox", HD, GGML_ROPE_TYPE_NEOX, 0, 1.0f, 0.0f, false),
        rope("rope, normal, half the head", HD / 2, GGML_ROPE_TYPE_NORMAL, 0, 1.0f, 0.0f, false),
        rope("rope, neox, three quarters", HD * 3 / 4, GGML_ROPE_TYPE_NEOX, 0, 1.0f, 0.0f, false),
        rope("rope, neox, yarn", HD, GGML_ROPE_TYPE_NEOX, 4096, 0.25f, 1.0f, false),
        rope("rope, neox, frequency factors", HD, GGML_ROPE_TYPE_NEOX, 4096, 1.0f, 0.0f, true),
        rope("rope, normal, yarn and factors", HD, GGML_ROPE_TYPE_NORMAL, 4096, 0.25f, 1.0f, true),
    };
    for (const op_case & c : cases) run_case(be, c);

    piece_tests(be);

    ggml_backend_free(be);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

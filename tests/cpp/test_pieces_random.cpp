// Seeded random pieces through graph_compute on the GPU: chains of the ops a
// transformer block hands this backend, at random token counts, widths and
// weight types. Each case draws one or two blocks of
//   a norm (RMS_NORM with its scale row, RMS_NORM alone, the scale row
//   multiplied in place, or none) -> one to three matmuls on its result (a
//   group), sometimes through a reshape, sometimes a bias row added to one,
//   sometimes a residual ADD of the first with the matmul on either side,
//   sometimes one of them taken as
//   heads through ROPE (normal or NeoX, partial, YaRN, frequency factors),
//   sometimes a matmul over a range of rows, sometimes the norm's result
//   scaled in place and multiplied again ->
//   a second norm -> gate/up as two matmuls or as one of 2F rows (either half
//   first) under a random GLU kind -> the down projection, added to the
//   block's input on either side or in place -> sometimes a SCALE, in place
//   or not,
// with random intermediate results made graph outputs (which undoes the
// fusions that would skip writing them), and the block's input in host memory
// or the GPU's. Every output is checked against the same chain run on the CPU
// in node order: the oracle's host ops in fp32, every matmul input through
// the bfp16 encoder as the GPU packs it, fp64 products of the dequantised
// weights as the weight cache holds them (bfp16), in-place results written
// into the memory they share. The graph is then computed again (the backend
// reuses its plan of it): the same bits; and once more after one of its
// weights is rewritten with new values (its cache entries must go).
//
// Every sixth case is model-sized: config 3's shapes (2048 or 1537 tokens,
// hidden 2560, projections of 4096, 1024 and 2560 rows, an FFN of 9728) in
// one block. Every op here is row-local, so for those the CPU chain runs on 16
// sampled token rows (the first, the last and 14 others) and the outputs are
// compared on those rows.
//
// Bars: nrmse <= 5e-3 over each output and <= 5e-2 over each of its rows.
// Only fp32 rounding differs between the two chains, but every matmul input
// is packed again to 8-bit mantissas, so a rounding difference that moves a
// value across a bfp16 rounding boundary changes it by a whole mantissa step
// of its block, and the next matmuls carry that on. The CPU chain itself,
// with every product perturbed by a relative 2^-20 (the size of an fp32
// summation's error at these widths), moves by up to 2.2e-3 over an output
// and 1.6e-2 over a row on the first 24 seeds. A stale packed copy, a row
// read from the wrong place or a missing write moved whole outputs by 7e-2
// to 1 when this test was written.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <deque>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "mini_ggml.h"
#include "zest_oracle.h"

using fvec = std::vector<float>;

namespace {

struct weight {
    ggml_tensor * t;
    std::vector<uint8_t> bytes;
    fvec deq;  // what the GPU multiplies: dequantised, then through bfp16
};

fvec bfp16(const fvec & x, int64_t rows, int64_t k) {
    std::vector<uint8_t> enc((size_t) (rows * k / 8 * 9));
    fvec y(x.size());
    orc_bfp16_encode_rows(x.data(), rows, k, enc.data());
    orc_bfp16_decode_rows(enc.data(), rows, k, y.data());
    return y;
}

const ggml_tensor * root(const ggml_tensor * t) {
    while (t->view_src) t = t->view_src;
    return t;
}

const ggml_type k_types[] = {GGML_TYPE_Q4_K, GGML_TYPE_Q6_K, GGML_TYPE_Q8_0, GGML_TYPE_Q4_0, GGML_TYPE_Q5_1,
                             GGML_TYPE_F16,  GGML_TYPE_BF16, GGML_TYPE_IQ4_XS, GGML_TYPE_Q3_K, GGML_TYPE_Q5_0};
bool super_blocks(ggml_type t) {
    return t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q6_K || t == GGML_TYPE_IQ4_XS || t == GGML_TYPE_Q3_K;
}

// One case: its graph, the values of its leaves, and what it expects.
class random_piece {
public:
    random_piece(uint64_t seed, bool big = false) : rng_(seed), big_(big) {
        ggml_init_params ip = {ggml_tensor_overhead() * 256 + ggml_graph_overhead(), nullptr, true};
        wctx_ = ggml_init(ip);
        ictx_ = ggml_init(ip);
        ctx_ = ggml_init(ip);
    }
    ~random_piece() {
        ggml_backend_buffer_free(abuf_);
        ggml_backend_buffer_free(ibuf_);
        ggml_backend_buffer_free(wbuf_);
        ggml_free(ctx_);
        ggml_free(ictx_);
        ggml_free(wctx_);
    }

    std::string describe;

    void build() {
        static const int64_t tokens[] = {1, 3, 17, 64, 100, 255, 256, 257, 513, 1000, 1024, 1100, 1500};
        T_ = big_ ? (pick(2) ? 2048 : 1537) : tokens[pick(13)];
        D_ = big_ ? 2560 : pick(2) ? 512 : 256;
        host_input_ = coin(0.3);
        if (big_) {
            std::vector<int64_t> rows{0, T_ - 1};
            while (rows.size() < 16) {
                const int64_t r = 1 + pick((int) T_ - 2);
                if (std::find(rows.begin(), rows.end(), r) == rows.end()) rows.push_back(r);
            }
            std::sort(rows.begin(), rows.end());
            sample_ = rows;
        }
        char buf[96];
        snprintf(buf, sizeof(buf), "T=%lld D=%lld%s%s", (long long) T_, (long long) D_, host_input_ ? " x on host" : "",
                 big_ ? " (model-sized, 16 rows checked)" : "");
        describe = buf;
        ggml_tensor * cur = ggml_new_tensor_2d(ictx_, GGML_TYPE_F32, D_, T_);
        ggml_set_name(cur, "x");
        ggml_set_input(cur);
        leaf(cur, 1.0f, 0.0f);
        const int blocks = big_ ? 1 : 1 + pick(2);
        for (int b = 0; b < blocks; b++) cur = block(b, cur);
        output(cur);
    }

    bool run(ggml_backend_t be) {
        ggml_backend_buffer_type_t host = ggml_backend_dev_buffer_type(ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU));
        wbuf_ = ggml_backend_alloc_ctx_tensors(wctx_, be);
        ibuf_ = host_input_ ? ggml_backend_alloc_ctx_tensors_from_buft(ictx_, host) : ggml_backend_alloc_ctx_tensors(ictx_, be);
        abuf_ = ggml_backend_alloc_ctx_tensors(ctx_, be);
        if (!wbuf_ || !ibuf_ || !abuf_) return test_check(false, "%s: could not allocate", describe.c_str());
        ggml_backend_buffer_set_usage(wbuf_, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
        for (weight & w : weights_) ggml_backend_tensor_set(w.t, w.bytes.data(), 0, w.bytes.size());
        for (auto & [t, v] : leaves_) ggml_backend_tensor_set(t, v.data(), 0, ggml_nbytes(t));
        for (auto & [t, v] : positions_) ggml_backend_tensor_set(t, v.data(), 0, ggml_nbytes(t));
        ggml_cgraph * gf = ggml_new_graph(ctx_);
        for (ggml_tensor * t : outputs_) ggml_build_forward_expand(gf, t);
        ggml_backend_plan_graph(be, gf);
        if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS)
            return test_check(false, "%s: graph_compute failed", describe.c_str());
        std::vector<fvec> first;
        bool ok = check(gf, "", &first);
        // again: no in-place op here writes a leaf, so the results repeat
        bool same = ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS;
        for (size_t i = 0; same && i < outputs_.size(); i++) {
            fvec got(first[i].size());
            ggml_backend_tensor_get(outputs_[i], got.data(), 0, ggml_nbytes(outputs_[i]));
            same = memcmp(got.data(), first[i].data(), got.size() * sizeof(float)) == 0;
        }
        ok &= test_check(same, "%s: computed again, the same bits", describe.c_str());
        // one weight given new values in place
        weight & w = weights_[(size_t) pick((int) weights_.size())];
        quantize(w);
        ggml_backend_tensor_set(w.t, w.bytes.data(), 0, w.bytes.size());
        if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS)
            return test_check(false, "%s: graph_compute failed after %s was rewritten", describe.c_str(), w.t->name);
        char after[96];
        snprintf(after, sizeof(after), " (%s rewritten)", w.t->name);
        return check(gf, after, nullptr) && ok;
    }

    // The CPU chain on every row, then on four token rows (cases without a
    // row-range view, whose offsets the sampled chain does not follow): the
    // same values on those rows. Tensors in host memory, nothing computed on
    // a device.
    bool self_check(ggml_backend_buffer_type_t host, int & checked) {
        if (T_ < 8) return true;
        wbuf_ = ggml_backend_alloc_ctx_tensors_from_buft(wctx_, host);
        ibuf_ = ggml_backend_alloc_ctx_tensors_from_buft(ictx_, host);
        abuf_ = ggml_backend_alloc_ctx_tensors_from_buft(ctx_, host);
        ggml_cgraph * gf = ggml_new_graph(ctx_);
        for (ggml_tensor * t : outputs_) ggml_build_forward_expand(gf, t);
        for (int i = 0; i < gf->n_nodes; i++)
            if (gf->nodes[i]->op == GGML_OP_VIEW) return true;
        mem_.clear();
        cpu_chain(gf);
        const std::unordered_map<const ggml_tensor *, fvec> full = mem_;
        sample_ = {0, 2, 5, T_ - 1};
        mem_.clear();
        cpu_chain(gf);
        for (ggml_tensor * t : outputs_) {
            const fvec & a = full.at(root(t)), & b = mem_.at(root(t));
            const int64_t w = t->ne[0], per = ggml_nrows(t) / T_;
            for (int64_t r = 0; r < rows_of(t); r++) {
                const int64_t g = sample_[(size_t) (r / per)] * per + r % per;
                if (memcmp(&a[(size_t) (g * w)], &b[(size_t) (r * w)], (size_t) w * sizeof(float)) != 0)
                    return test_check(false, "%s: %s row %lld of the sampled chain differs", describe.c_str(), t->name,
                                      (long long) r);
            }
            checked++;
        }
        return true;
    }

    // every output against the CPU chain; the GPU's values kept in `got_all`
    bool check(const ggml_cgraph * gf, const char * when, std::vector<fvec> * got_all) {
        mem_.clear();
        cpu_chain(gf);
        bool ok = true;
        for (ggml_tensor * t : outputs_) {
            fvec got((size_t) ggml_nelements(t));
            ggml_backend_tensor_get(t, got.data(), 0, ggml_nbytes(t));
            if (got_all) got_all->push_back(got);
            const fvec & want = mem_.at(root(t));
            double se = 0, ss = 0, worst_row = 0;
            const int64_t w = t->ne[0], per_token = ggml_nrows(t) / T_;
            for (int64_t r = 0; r < rows_of(t); r++) {
                // row r of the chain's rows: its token's row in the GPU's output
                const int64_t g = sample_.empty() ? r : sample_[(size_t) (r / per_token)] * per_token + r % per_token;
                double rse = 0, rss = 0;
                for (int64_t c = 0; c < w; c++) {
                    const double d = (double) got[g * w + c] - want[r * w + c];
                    rse += d * d;
                    rss += (double) want[r * w + c] * want[r * w + c];
                }
                se += rse;
                ss += rss;
                worst_row = std::max(worst_row, std::sqrt(rse / std::max(rss, 1e-30)));
            }
            const double e = std::sqrt(se / std::max(ss, 1e-30));
            ok &= test_check(std::isfinite(e) && e <= 5e-3 && worst_row <= 5e-2,
                             "%s%s: %-28s nrmse %.2e, worst row %.2e", describe.c_str(), when, t->name, e, worst_row);
        }
        return ok;
    }

private:
    test_rng rng_;
    ggml_context * wctx_, * ictx_, * ctx_;  // weights, the block's input, the rest
    ggml_backend_buffer_t wbuf_ = nullptr, ibuf_ = nullptr, abuf_ = nullptr;
    int64_t T_ = 0, D_ = 0;
    bool host_input_ = false;
    bool big_ = false;
    std::vector<int64_t> sample_;  // model-sized cases: the token rows the CPU chain computes

    // rows of t the CPU chain holds: all, or its rows of the sampled tokens
    int64_t rows_of(const ggml_tensor * t) const {
        return sample_.empty() ? ggml_nrows(t) : ggml_nrows(t) / T_ * (int64_t) sample_.size();
    }
    // a leaf's values on the sampled tokens: per = values per token (the
    // width of [w x T] rows, 1 for ROPE's positions); parameters stay whole
    template <class V>
    V sampled(const V & v, int64_t per) const {
        if (sample_.empty() || per == 0) return v;
        V out;
        for (int64_t tok : sample_) out.insert(out.end(), v.begin() + tok * per, v.begin() + (tok + 1) * per);
        return out;
    }
    int n_weights_ = 0;
    std::deque<weight> weights_;
    std::unordered_map<const ggml_tensor *, const weight *> weight_of_;
    std::vector<std::pair<ggml_tensor *, fvec>> leaves_;
    std::vector<std::pair<ggml_tensor *, std::vector<int32_t>>> positions_;  // ROPE's token positions
    std::vector<ggml_tensor *> outputs_;
    std::unordered_map<const ggml_tensor *, fvec> mem_;  // the CPU chain: root tensor -> its memory

    int pick(int n) { return std::min(n - 1, (int) (rng_.uniform() * n)); }
    bool coin(double p) { return rng_.uniform() < p; }

    void output(ggml_tensor * t) {
        if (std::find(outputs_.begin(), outputs_.end(), t) != outputs_.end()) return;
        ggml_set_output(t);
        outputs_.push_back(t);
    }
    void name(ggml_tensor * t, const char * fmt, int b) {
        char s[64];
        snprintf(s, sizeof(s), fmt, b);
        ggml_set_name(t, s);
    }
    // a leaf of random values: mean + sd * normal
    void leaf(ggml_tensor * t, float sd, float mean) {
        fvec v((size_t) ggml_nelements(t));
        for (float & x : v) x = mean + sd * rng_.normal(0.0f, 1.0f);
        leaves_.emplace_back(t, std::move(v));
    }
    // a K x N weight of type ty (quantised from normal(0, 0.05) values)
    ggml_tensor * new_weight(int64_t k, int64_t n, ggml_type ty, int b) {
        weights_.push_back({ggml_new_tensor_2d(wctx_, ty, k, n), {}, {}});
        weight & w = weights_.back();
        char s[64];
        snprintf(s, sizeof(s), "blk.%d.w%d.weight", b, n_weights_++);
        ggml_set_name(w.t, s);
        quantize(w);
        weight_of_[w.t] = &w;
        return w.t;
    }
    // new values for w: its GGUF bytes and what the GPU multiplies
    void quantize(weight & w) {
        const int64_t k = w.t->ne[0], n = w.t->ne[1];
        const ggml_type ty = w.t->type;
        fvec f((size_t) (k * n));
        for (float & x : f) x = rng_.normal(0.0f, 0.05f);
        const size_t rb = ggml_row_size(ty, k);
        w.bytes.resize(rb * (size_t) n);
        ggml_quantize_chunk(ty, f.data(), w.bytes.data(), 0, n, k, nullptr);
        w.deq.resize(f.size());
        for (int64_t i = 0; i < n; i++) ggml_dequantize_row(ty, w.bytes.data() + i * rb, w.deq.data() + i * k, k);
        w.deq = bfp16(w.deq, n, k);
    }
    ggml_type any_type() { return k_types[pick(10)]; }

    ggml_tensor * last_proj_ = nullptr;
    // p's rows as heads of 64 (or 32) through ROPE with random settings
    void rope_heads(ggml_tensor * p, int b) {
        const int64_t hd = p->ne[0] % 64 == 0 ? 64 : 32, heads = p->ne[0] / hd;
        const int n_dims = (int) (coin(0.5) ? hd : hd / 2), mode = coin(0.5) ? GGML_ROPE_TYPE_NEOX : GGML_ROPE_TYPE_NORMAL;
        const bool yarn = coin(0.5);
        ggml_tensor * pos = ggml_new_tensor_1d(ctx_, GGML_TYPE_I32, T_);
        name(pos, "pos%d", b);
        std::vector<int32_t> pv((size_t) T_);
        const int32_t p0 = (int32_t) pick(40000);
        for (int64_t i = 0; i < T_; i++) pv[(size_t) i] = p0 + (int32_t) i;
        positions_.emplace_back(pos, std::move(pv));
        ggml_tensor * ff = nullptr;
        if (coin(0.4)) {
            ff = ggml_new_tensor_1d(ctx_, GGML_TYPE_F32, n_dims / 2);
            name(ff, "freq_factors%d", b);
            fvec v((size_t) (n_dims / 2));
            for (float & f : v) f = (float) (1.0 + 3.0 * rng_.uniform());
            leaves_.emplace_back(ff, std::move(v));
        }
        ggml_tensor * q3 = ggml_reshape_3d(ctx_, p, hd, heads, T_);
        ggml_tensor * r = ggml_rope_ext(ctx_, q3, pos, ff, n_dims, mode, yarn ? 4096 : 0, 10000.0f, yarn ? 0.25f : 1.0f,
                                        yarn ? 1.0f : 0.0f, 1.0f, 32.0f, 1.0f);
        name(r, "rope%d", b);
        output(r);
    }
    ggml_type type_for(int64_t k) {
        for (;;) {
            const ggml_type t = any_type();
            if (!super_blocks(t) || k % 256 == 0) return t;
        }
    }

    // a norm over x, in one of four forms
    ggml_tensor * norm(ggml_tensor * x, int b) {
        const int form = pick(4);
        if (form == 3) return x;
        ggml_tensor * n = ggml_rms_norm(ctx_, x, 1e-6f);
        name(n, "norm%d", b);
        if (form == 1) return n;
        ggml_tensor * s = ggml_new_tensor_1d(ctx_, GGML_TYPE_F32, D_);
        name(s, "norm%d.scale", b);
        leaf(s, 0.1f, 1.0f);
        ggml_tensor * h = form == 0 ? ggml_mul(ctx_, n, s) : ggml_mul_inplace(ctx_, n, s);
        name(h, form == 0 ? "norm%d*scale" : "norm%d*=scale", b);
        return h;
    }

    ggml_tensor * block(int b, ggml_tensor * x) {
        // attention-input side: a group of matmuls on the norm's result
        ggml_tensor * h = norm(x, b);
        const bool h_is_leaf = root(h)->op == GGML_OP_NONE;  // the graph's input: never written
        ggml_tensor * hin = coin(0.3) ? ggml_reshape_2d(ctx_, h, D_, T_) : h;
        static const int64_t widths[] = {32, 64, 96, 160, 256}, big_widths[] = {4096, 1024, 1024, 2560, 64};
        const int nproj = 1 + pick(3);
        const bool residual = coin(0.5);
        ggml_tensor * first = nullptr;
        for (int i = 0; i < nproj; i++) {
            const int64_t n = i == 0 && residual ? D_ : big_ ? big_widths[pick(5)] : widths[pick(5)];
            ggml_tensor * p = ggml_mul_mat(ctx_, new_weight(D_, n, type_for(D_), b), hin);
            name(p, i == 0 ? "proj%d.0" : i == 1 ? "proj%d.1" : "proj%d.2", b);
            if (i > 0 && coin(0.3)) {
                // a bias row added to every row of the projection (q/k/v biases)
                ggml_tensor * bias = ggml_new_tensor_1d(ctx_, GGML_TYPE_F32, n);
                name(bias, i == 1 ? "bias%d.1" : "bias%d.2", b);
                leaf(bias, 0.5f, 0.0f);
                p = ggml_add(ctx_, p, bias);
                name(p, i == 1 ? "proj%d.1+bias" : "proj%d.2+bias", b);
            }
            if (i == 0) first = p;
            if (i > 0 || !residual || coin(0.2)) output(p);
            last_proj_ = p;
        }
        if (coin(0.35)) rope_heads(last_proj_, b);
        if (residual) {
            x = coin(0.5) ? ggml_add(ctx_, first, x) : ggml_add(ctx_, x, first);
            name(x, "attn_out%d", b);
        }
        if (!h_is_leaf && coin(0.25)) {
            // the norm's result scaled in place after its matmuls, then multiplied again
            ggml_tensor * hs = ggml_scale_inplace(ctx_, h, 0.5f);
            name(hs, "norm%d*=0.5", b);
            ggml_tensor * e = ggml_mul_mat(ctx_, new_weight(D_, 64, type_for(D_), b), hs);
            name(e, "after_inplace%d", b);
            output(e);
        }
        if (!big_ && T_ > 4 && coin(0.25)) {
            // a matmul over a range of the norm's rows
            const int64_t r0 = 1 + pick((int) (T_ / 2)), r1 = r0 + 1 + pick((int) (T_ - r0 - 1));
            ggml_tensor * v = ggml_view_2d(ctx_, h, D_, r1 - r0, h->nb[1], (size_t) r0 * h->nb[1]);
            ggml_tensor * e = ggml_mul_mat(ctx_, new_weight(D_, 96, type_for(D_), b), v);
            name(e, "row_range%d", b);
            output(e);
        }

        // the FFN: gate/up, a GLU, the down projection, the residual
        ggml_tensor * h2 = norm(x, b + 10);
        const ggml_type gt = type_for(D_), dt = any_type();
        const int64_t F = big_ ? 9728 : super_blocks(dt) ? 256 * (1 + pick(3)) : 32 * (1 + pick(24));
        static const ggml_glu_op kinds[] = {GGML_GLU_OP_SWIGLU, GGML_GLU_OP_GEGLU, GGML_GLU_OP_REGLU,
                                            GGML_GLU_OP_GEGLU_ERF, GGML_GLU_OP_GEGLU_QUICK};
        const ggml_glu_op kind = kinds[pick(5)];
        ggml_tensor * act;
        if (coin(0.5)) {
            ggml_tensor * g = ggml_mul_mat(ctx_, new_weight(D_, F, gt, b), h2);
            ggml_tensor * u = ggml_mul_mat(ctx_, new_weight(D_, F, gt, b), h2);
            name(g, "gate%d", b);
            name(u, "up%d", b);
            if (coin(0.15)) output(g);
            act = ggml_glu_split(ctx_, g, u, kind);
        } else {
            ggml_tensor * gu = ggml_mul_mat(ctx_, new_weight(D_, 2 * F, gt, b), h2);
            name(gu, "gate_up%d", b);
            if (coin(0.15)) output(gu);
            act = ggml_glu(ctx_, gu, kind, coin(0.5));
        }
        name(act, "glu%d", b);
        if (coin(0.15)) output(act);
        ggml_tensor * dn = ggml_mul_mat(ctx_, new_weight(F, D_, dt, b), act);
        name(dn, "down%d", b);
        const int res = pick(4);
        ggml_tensor * out = res == 0   ? ggml_add(ctx_, dn, x)
                            : res == 1 ? ggml_add(ctx_, x, dn)
                            : res == 2 && root(x)->op != GGML_OP_NONE ? ggml_add_inplace(ctx_, x, dn)
                                                                                : dn;
        if (out != dn) name(out, "ffn_out%d", b);
        if (coin(0.3)) {
            out = coin(0.5) ? ggml_scale(ctx_, out, 0.75f) : ggml_scale_inplace(ctx_, out, 0.75f);
            name(out, "scaled%d", b);
        }
        char s[96];
        snprintf(s, sizeof(s), " | block %d: %d proj%s, F=%lld %s/%s, res %d", b, nproj, residual ? " +res" : "",
                 (long long) F, ggml_type_name_of(gt), ggml_type_name_of(dt), res);
        describe += s;
        return out;
    }

    static const char * ggml_type_name_of(ggml_type t) {
        switch (t) {
            case GGML_TYPE_Q4_K: return "q4_K";
            case GGML_TYPE_Q6_K: return "q6_K";
            case GGML_TYPE_Q8_0: return "q8_0";
            case GGML_TYPE_Q4_0: return "q4_0";
            case GGML_TYPE_Q5_1: return "q5_1";
            case GGML_TYPE_F16: return "f16";
            case GGML_TYPE_BF16: return "bf16";
            case GGML_TYPE_IQ4_XS: return "iq4_xs";
            case GGML_TYPE_Q3_K: return "q3_K";
            case GGML_TYPE_Q5_0: return "q5_0";
            default: return "?";
        }
    }

    // t's values in the CPU chain: its root's memory, whole or a range of rows
    fvec value(const ggml_tensor * t) const {
        const fvec & m = mem_.at(root(t));
        if (!t->view_src) return m;
        const size_t first = t->view_offs / sizeof(float);
        return fvec(m.begin() + (ptrdiff_t) first, m.begin() + (ptrdiff_t) (first + (size_t) ggml_nelements(t)));
    }

    void cpu_chain(const ggml_cgraph * gf) {
        for (auto & [t, v] : leaves_) mem_[t] = sampled(v, t->ne[1] == T_ && ggml_nrows(t) == T_ ? t->ne[0] : 0);
        std::unordered_map<const ggml_tensor *, std::vector<int32_t>> pos_of;
        for (auto & [t, v] : positions_) pos_of[t] = sampled(v, 1);
        for (int i = 0; i < gf->n_nodes; i++) {
            const ggml_tensor * n = gf->nodes[i];
            if (n->op == GGML_OP_NONE || n->op == GGML_OP_RESHAPE || n->op == GGML_OP_VIEW) continue;
            const int64_t w = n->ne[0], rows = rows_of(n);
            fvec y((size_t) (w * rows));
            switch (n->op) {
                case GGML_OP_MUL_MAT: {
                    const weight & wt = *weight_of_.at(n->src[0]);
                    const int64_t K = n->src[0]->ne[0];
                    const fvec x = bfp16(value(n->src[1]), rows, K);
                    std::vector<double> acc((size_t) (rows * w));
                    orc_mul_mat_f64(wt.deq.data(), w, K, x.data(), rows, acc.data(), nullptr, 8);
                    std::copy(acc.begin(), acc.end(), y.begin());
                    break;
                }
                case GGML_OP_RMS_NORM: {
                    float eps;
                    memcpy(&eps, &n->op_params[0], sizeof(eps));
                    orc_rms_norm(value(n->src[0]).data(), rows, w, eps, y.data());
                    break;
                }
                case GGML_OP_MUL: orc_mul_row(value(n->src[0]).data(), rows, w, value(n->src[1]).data(), y.data()); break;
                case GGML_OP_ADD:
                    if (ggml_nelements(n->src[1]) == w)  // a bias row
                        orc_add_row(value(n->src[0]).data(), rows, w, value(n->src[1]).data(), y.data());
                    else
                        orc_add(value(n->src[0]).data(), value(n->src[1]).data(), w * rows, y.data());
                    break;
                case GGML_OP_SCALE: {
                    float s, b;
                    memcpy(&s, &n->op_params[0], sizeof(s));
                    memcpy(&b, &n->op_params[1], sizeof(b));
                    orc_scale(value(n->src[0]).data(), w * rows, s, b, y.data());
                    break;
                }
                case GGML_OP_GLU: {
                    static const int kind_of[] = {ORC_GLU_REGLU, ORC_GLU_GEGLU, ORC_GLU_SWIGLU, -1, ORC_GLU_GEGLU_ERF,
                                                  ORC_GLU_GEGLU_QUICK};
                    const int kind = kind_of[n->op_params[0]];
                    const fvec a = value(n->src[0]);
                    if (n->src[1]) {
                        const fvec u = value(n->src[1]);
                        orc_glu(kind, a.data(), w, u.data(), w, rows, w, y.data());
                    } else {
                        const bool swapped = n->op_params[1] != 0;
                        orc_glu(kind, a.data() + (swapped ? w : 0), 2 * w, a.data() + (swapped ? 0 : w), 2 * w, rows, w,
                                y.data());
                    }
                    break;
                }
                case GGML_OP_ROPE: {
                    float fp[11];
                    memcpy(fp, n->op_params, sizeof(fp));
                    const fvec ff = n->src[2] ? value(n->src[2]) : fvec();
                    orc_rope(value(n->src[0]).data(), rows / n->ne[1], n->ne[1], n->ne[0], pos_of.at(n->src[1]).data(),
                             n->src[2] ? ff.data() : nullptr, n->op_params[1], n->op_params[2], n->op_params[4], fp[5],
                             fp[6], fp[7], fp[8], fp[9], fp[10], y.data());
                    break;
                }
                default: test_check(false, "cpu chain: unexpected op %d", (int) n->op); return;
            }
            mem_[root(n)] = std::move(y);  // an in-place result lands in its input's memory
        }
    }
};

}  // namespace

// The checker's own check, with no GPU: on ordinary cases (tensors in host
// memory), the CPU chain restricted to a few token rows gives exactly the
// full chain's values on those rows, as the model-sized cases assume.
static int self_check(int cases, uint64_t seed0) {
    int checked = 0;
    ggml_backend_buffer_type_t host = ggml_backend_dev_buffer_type(ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU));
    for (int c = 0; c < cases; c++) {
        random_piece p(seed0 + (uint64_t) c);
        p.build();
        if (!p.self_check(host, checked)) return 1;
    }
    printf("self-check: %d outputs, sampled rows equal to the full chain's\n", checked);
    printf("%s\n", checked > 0 && !test_failures() ? "ALL PASS" : "FAILED");
    return checked > 0 && !test_failures() ? 0 : 1;
}

// test_pieces_random [CASES [SEED [THREADS]]]: with THREADS > 1, each thread
// runs CASES cases of its own (seeds SEED + 1000 t + c) on a backend of its
// own, all at once, as llama.cpp contexts on several threads do: they share
// the library, the gate's reader log and the budget, and every write of a
// tensor looks through every context's weight cache.
int main(int argc, char ** argv) {
    if (argc > 1 && strcmp(argv[1], "--self-check") == 0) {
        ggml_backend_load_all();
        return self_check(60, 1000);
    }
    const int cases = argc > 1 ? atoi(argv[1]) : 24;
    const uint64_t seed0 = argc > 2 ? strtoull(argv[2], nullptr, 10) : 1000;
    const int threads = argc > 3 ? std::max(1, atoi(argv[3])) : 1;
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "XDNA device not registered - is GGML_BACKEND_PATH set?\n");
        return 2;
    }
    std::vector<ggml_backend_t> backends;
    for (int t = 0; t < threads; t++) {
        backends.push_back(ggml_backend_dev_init(dev, nullptr));
        if (!backends.back()) {
            fprintf(stderr, "cannot start the backend\n");
            return 2;
        }
    }
    auto work = [&](int t) {
        for (int c = 0; c < cases; c++) {
            const uint64_t seed = seed0 + 1000 * (uint64_t) t + (uint64_t) c;
            random_piece p(seed, c % 6 == 5);
            p.build();
            printf("thread %d case %d (seed %llu): %s\n", t, c, (unsigned long long) seed, p.describe.c_str());
            fflush(stdout);
            p.run(backends[t]);
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; t++) pool.emplace_back(work, t);
    work(0);
    for (std::thread & th : pool) th.join();
    for (ggml_backend_t be : backends) ggml_backend_free(be);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

// What the ggml scheduler may hand this backend, decided without reading any
// tensor data: the run mode, the gate (supports_op), the record of who reads
// what, the HBM budget of the weight cache, and the notes said once per
// model. The decisions follow the reference's contract (src/ggml-zest.cpp:
// 56-130 settings and run mode, 429-564 budget, 566-637 notes, 1066-1226
// gate; src/xdna-exec.cpp:85-131 what the executor runs; acceptance criteria
// XDNA-BATCH-GATE, XDNA-WORK-FLOOR, XDNA-MEMORY-BUDGET and XDNA-HOST-OPS in
// specs/xdna-backend/spec.md) for a GPU whose own memory holds the model.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <set>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "backend.h"
#include "zest_hip.h"

namespace zest {

void log(log_level level, const char * fmt, ...) {
    static const char * const tag[] = {"", "warning: ", "error: "};
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    fprintf(stderr, "xdna: %s%s", tag[level], buf);
}

const char * op_name(int op) {
    switch (op) {
        case GGML_OP_NONE: return "NONE";
        case GGML_OP_ADD: return "ADD";
        case GGML_OP_MUL: return "MUL";
        case GGML_OP_RMS_NORM: return "RMS_NORM";
        case GGML_OP_MUL_MAT: return "MUL_MAT";
        case GGML_OP_MUL_MAT_ID: return "MUL_MAT_ID";
        case GGML_OP_SCALE: return "SCALE";
        case GGML_OP_RESHAPE: return "RESHAPE";
        case GGML_OP_VIEW: return "VIEW";
        case GGML_OP_PERMUTE: return "PERMUTE";
        case GGML_OP_TRANSPOSE: return "TRANSPOSE";
        case GGML_OP_GET_ROWS: return "GET_ROWS";
        case GGML_OP_ROPE: return "ROPE";
        case GGML_OP_GLU: return "GLU";
        default: return "OTHER";
    }
}

// ---- settings ------------------------------------------------------------------

namespace {

// Every environment setting the policy reads, read together the first time
// one is needed (the reference's names and defaults; docs/technical-guide.md
// of the reference lists them).
struct settings {
    int device = 0;
    bool plan_only = false, host_only = false;
    int64_t min_batch = 1024, min_mflop = 256;
    bool blocks = true, trace = false, write_all = false;
    int trace_level = 0;
    // GGML_XDNA_BLOCK_OPS: the small ops block claiming may take, by ggml op
    // name (for tracking a wrong result down op by op); empty = all
    std::set<std::string> block_ops;

    settings() {
        device = (int) env_int("GGML_XDNA_DEVICE", device);
        plan_only = env_int("GGML_XDNA_PLAN_ONLY", 0) != 0;
        host_only = env_int("GGML_XDNA_HOST_ONLY", 0) != 0;
        min_batch = env_int("GGML_XDNA_MIN_BATCH", min_batch);
        min_mflop = env_int("GGML_XDNA_MIN_MFLOP", min_mflop);
        blocks = env_int("GGML_XDNA_BLOCKS", 1) != 0;
        trace_level = (int) env_int("GGML_XDNA_TRACE", 0);
        trace = trace_level != 0;
        write_all = env_int("GGML_XDNA_WRITE_ALL", 0) != 0;
        if (const char * s = env("GGML_XDNA_BLOCK_OPS")) {
            std::string list(s);
            size_t at = 0;
            while (at <= list.size()) {
                const size_t comma = std::min(list.find(',', at), list.size());
                if (comma > at) block_ops.insert(list.substr(at, comma - at));
                at = comma + 1;
            }
        }
    }
};

const settings & cfg() {
    static const settings s;
    return s;
}

}  // namespace

int device_index() { return cfg().device; }
bool plan_only() { return cfg().plan_only; }
int64_t min_batch() { return cfg().min_batch; }
int64_t min_mflop() { return cfg().min_mflop; }
bool trace() { return cfg().trace; }
bool blocks() { return cfg().blocks && mode() == run_mode::gpu; }

// ---- run mode --------------------------------------------------------------------

// Decided once, at registration: the GPU opens, is a gfx950, and gets the
// registration known-answer multiply right; or no device is offered. There is
// no host-only mode (no CPU path); planning-only mode offers the device
// without opening a GPU.
run_mode mode() {
    static const run_mode m = [] {
        if (cfg().host_only) {
            log(LOG_WARN, "GGML_XDNA_HOST_ONLY is not supported: this backend has no CPU path; not offering "
                          GGML_XDNA_DEVICE_NAME "\n");
            return run_mode::off;
        }
        if (cfg().plan_only) {
            log(LOG_INFO, "planning-only mode (GGML_XDNA_PLAN_ONLY): graphs will not run\n");
            return run_mode::gpu;
        }
        const int dev = cfg().device;
        if (zest_init(dev) != ZEST_OK || zest_self_test() != ZEST_OK) {
            log(LOG_WARN, "not offering " GGML_XDNA_DEVICE_NAME ": %s\n", zest_last_error());
            return run_mode::off;
        }
        log(LOG_INFO, "GPU %d (gfx950), registration test multiply right\n", dev);
        return run_mode::gpu;
    }();
    return m;
}

static std::atomic<bool> g_broken{false};
bool broken() { return g_broken.load(); }
void mark_broken(const std::string & why) {
    if (!g_broken.exchange(true))
        log(LOG_ERROR, "the GPU path failed (%s); from now on this backend claims nothing\n", why.c_str());
}

// ---- what the executor runs ---------------------------------------------------------

namespace {

bool dense_f32(const ggml_tensor * t) { return t && t->type == GGML_TYPE_F32 && is_contiguous(t); }

// `out` and `in` dense fp32 of one shape: a row-by-row op the kernels run in place or not
bool rowwise(const ggml_tensor * out, const ggml_tensor * in) {
    return dense_f32(out) && dense_f32(in) && same_shape(out, in);
}

// one dense fp32 row as wide as the rows of `of` (a norm's scale, a bias)
bool one_row_of(const ggml_tensor * r, const ggml_tensor * of) {
    return dense_f32(r) && r->ne[0] == of->ne[0] && nrows(r) == 1;
}

bool glu_op_runs(int g) {
    switch (g) {
        case GGML_GLU_OP_REGLU:
        case GGML_GLU_OP_GEGLU:
        case GGML_GLU_OP_SWIGLU:
        case GGML_GLU_OP_GEGLU_ERF:
        case GGML_GLU_OP_GEGLU_QUICK: return true;
        default: return false;  // SWIGLU_OAI and later kinds
    }
}

// Per small op: whether its shapes and types are ones the kernels take, and
// which of its inputs, if any, is a parameter that must be a kept leaf.
struct small_op {
    int op;
    bool (*runs)(const ggml_tensor *);
    const ggml_tensor * (*parameter)(const ggml_tensor *);
};

const small_op k_small_ops[] = {
    {GGML_OP_RESHAPE, [](const ggml_tensor * n) { return n->src[0] && is_contiguous(n->src[0]); }, nullptr},
    {GGML_OP_RMS_NORM, [](const ggml_tensor * n) { return dense_f32(n) && dense_f32(n->src[0]); }, nullptr},
    {GGML_OP_MUL,  // times a scale row broadcast over every row
     [](const ggml_tensor * n) { return rowwise(n, n->src[0]) && n->src[1] && one_row_of(n->src[1], n->src[0]); },
     [](const ggml_tensor * n) { return (const ggml_tensor *) n->src[1]; }},
    {GGML_OP_ADD,  // two of one shape, or a bias row added to every row
     [](const ggml_tensor * n) {
         const ggml_tensor * a = n->src[0], * b = n->src[1];
         return b && rowwise(n, a) && (rowwise(a, b) || one_row_of(b, a));
     },
     [](const ggml_tensor * n) {
         const ggml_tensor * a = n->src[0], * b = n->src[1];
         return a && b && !same_shape(a, b) && one_row_of(b, a) ? b : nullptr;
     }},
    {GGML_OP_SCALE, [](const ggml_tensor * n) { return rowwise(n, n->src[0]); }, nullptr},
    {GGML_OP_GLU,  // gate and up as two tensors, or as the halves of one
     [](const ggml_tensor * n) {
         const ggml_tensor * a = n->src[0], * b = n->src[1];
         if (!glu_op_runs(param_i32(n, 0)) || !dense_f32(a) || !dense_f32(n)) return false;
         if (!b) return a->ne[0] == 2 * n->ne[0] && nrows(a) == nrows(n);
         return param_i32(n, 1) == 0 && rowwise(n, a) && rowwise(a, b);
     },
     nullptr},
    {GGML_OP_ROPE,
     [](const ggml_tensor * n) {
         const ggml_tensor * x = n->src[0], * pos = n->src[1], * freq = n->src[2];
         if (!rowwise(n, x) || !pos || pos->type != GGML_TYPE_I32) return false;
         const int n_dims = param_i32(n, 1), kind = param_i32(n, 2);
         if (kind != GGML_ROPE_TYPE_NORMAL && kind != GGML_ROPE_TYPE_NEOX) return false;
         if (param_i32(n, 15) != 0) return false;  // position offsets
         // the kernel's angle table, 1.5 n_dims floats, must fit 64 KiB of LDS
         if (n_dims <= 0 || n_dims % 2 != 0 || n_dims > x->ne[0] || n_dims > 8192) return false;
         if (freq && (!dense_f32(freq) || freq->ne[0] < n_dims / 2)) return false;
         return x->ne[3] == 1 && pos->ne[0] == x->ne[2];
     },
     [](const ggml_tensor * n) { return (const ggml_tensor *) n->src[2]; }},
};

const small_op * small_op_of(int op) {
    for (const small_op & s : k_small_ops)
        if (s.op == op) return &s;
    return nullptr;
}

}  // namespace

bool exec_supports(const ggml_tensor * op) {
    if (op->op == GGML_OP_MUL_MAT) return true;  // the gate checks its weight side
    const small_op * s = small_op_of(op->op);
    return s && s->runs(op);
}

const ggml_tensor * exec_param(const ggml_tensor * op) {
    const small_op * s = small_op_of(op->op);
    return s && s->parameter ? s->parameter(op) : nullptr;
}

// ---- who reads what ------------------------------------------------------------------

namespace {

// The scheduler asks supports_op about every op it places, so the questions
// show every reader of every tensor; a result is written back for readers
// outside a piece only when one exists. Readers recorded for tensors ggml
// later reuses can linger: that only ever adds a write back, never drops one.
class reader_log {
    mutable std::shared_mutex mu_;
    std::unordered_map<const ggml_tensor *, std::vector<const ggml_tensor *>> by_tensor_;
    std::atomic<uint64_t> epoch_{0};

    // true if `op` was new among t's readers
    bool add(const ggml_tensor * t, const ggml_tensor * op) {
        std::vector<const ggml_tensor *> & r = by_tensor_[t];
        if (std::find(r.begin(), r.end(), op) != r.end()) return false;
        r.push_back(op);
        return true;
    }

public:
    // op reads each of its inputs, and every tensor an input is a view of
    void record(const ggml_tensor * op) {
        std::unique_lock<std::shared_mutex> lk(mu_);
        bool grew = false;
        for (const ggml_tensor * s : op->src)
            for (const ggml_tensor * t = s; t; t = t->view_src) grew |= add(t, op);
        if (grew) epoch_.fetch_add(1, std::memory_order_relaxed);
    }

    // whether a reader not in `piece` exists, or t was never seen read
    bool read_beyond(const ggml_tensor * t, const std::unordered_set<const ggml_tensor *> & piece) const {
        std::shared_lock<std::shared_mutex> lk(mu_);
        const auto it = by_tensor_.find(t);
        if (it == by_tensor_.end()) return true;
        return std::any_of(it->second.begin(), it->second.end(),
                           [&](const ggml_tensor * r) { return piece.count(r) == 0; });
    }

    uint64_t epoch() const { return epoch_.load(std::memory_order_relaxed); }
};

reader_log & readers() {
    static reader_log r;
    return r;
}

}  // namespace

void note_readers(const ggml_tensor * op) { readers().record(op); }
uint64_t readers_epoch() { return readers().epoch(); }

bool read_outside(const ggml_tensor * t, const std::unordered_set<const ggml_tensor *> & in_piece) {
    if (cfg().write_all || (t->flags & GGML_TENSOR_FLAG_OUTPUT)) return true;
    return readers().read_beyond(t, in_piece);
}

// ---- the weight-cache budget ------------------------------------------------------------

// A K x N weight's cache entry: 9 bytes per 8 values in the tile layout
// (rows padded to 256, columns to 64).
double copy_bytes(int64_t K, int64_t N) { return (double) zest_bfp16_bytes(N, K); }

namespace {

constexpr double kGiB = 1024.0 * 1024 * 1024;

// The layer of a weight named as llama.cpp names them ("blk.12.attn_q.weight"),
// -1 for the others (the output matrix).
int layer_number(const char * name) {
    if (strncmp(name, "blk.", 4) != 0) return -1;
    const char * p = name + 4;
    int layer = 0;
    if (*p < '0' || *p > '9') return -1;
    for (; *p >= '0' && *p <= '9'; p++) layer = layer * 10 + (*p - '0');
    return *p == '.' ? layer : -1;
}

// One process-wide budget (supports_op is asked with no context): the
// decision made for every weight asked about while a context lives, in the
// order asked. Weights are taken while the entries taken so far and the next
// fit the limit. The first that does not fit closes the budget: nothing new
// is taken afterwards, and, unless a graph has already run (its entries may
// exist by then), the weights already taken from that weight's layer are
// given back, so no layer is split between this backend and the next. Every
// decision then stands until the last context goes, which clears them all.
class weight_budget {
    struct key {
        const void * buffer, * data;
        int type;
        int64_t ne0, ne1;
        bool operator==(const key & o) const {
            return buffer == o.buffer && data == o.data && type == o.type && ne0 == o.ne0 && ne1 == o.ne1;
        }
    };
    struct key_hash {
        size_t operator()(const key & k) const {
            size_t h = std::hash<const void *>()(k.data);
            h = h * 1000003u ^ std::hash<const void *>()(k.buffer);
            return h * 1000003u ^ (size_t) (k.ne1 * 31 + k.ne0 + k.type);
        }
    };
    struct decision {
        int layer;
        double bytes;
        bool taken;
    };

    std::mutex mu_;
    int live_ = 0;  // contexts alive
    std::unordered_map<key, size_t, key_hash> index_;  // weight -> its place in log_
    std::vector<decision> log_;                          // in the order asked
    double taken_bytes_ = 0;
    bool closed_ = false;   // a weight did not fit
    bool ran_ = false;      // a graph has run
    // the limit, fixed when the first weight is asked about
    bool limit_known_ = false, limit_from_env_ = false;
    double limit_ = 0;

    void fix_limit() {
        limit_known_ = true;
        if (const char * s = env("GGML_XDNA_MAX_COPY_GB")) {
            limit_from_env_ = true;
            limit_ = atof(s) * kGiB;
            return;
        }
        if (cfg().plan_only) {
            limit_ = 1e30;  // no device to measure
            return;
        }
        // the device memory free now (the model is loaded by then), less what
        // llama.cpp's work buffers need: the larger of 4 GiB and a tenth of
        // the device. No fixed cap, unlike the NPU's 20 GB: the cache lives
        // in the GPU's own HBM.
        size_t free = 0, total = 0;
        if (hipMemGetInfo(&free, &total) != hipSuccess) free = total = 0;
        limit_ = (double) free - std::max(4 * kGiB, (double) total / 10);
    }

    // A weight did not fit: close the budget and give its layer back.
    void close(int layer) {
        closed_ = true;
        if (layer >= 0 && !ran_)
            for (decision & d : log_)
                if (d.taken && d.layer == layer) {
                    d.taken = false;
                    taken_bytes_ -= d.bytes;
                }
        std::set<int> layers;
        for (const decision & d : log_)
            if (d.taken && d.layer >= 0) layers.insert(d.layer);
        const std::string where =
            layers.empty() ? "no layer fits" : std::to_string(layers.size()) + " layers on the GPU path";
        log(LOG_WARN, "weight cache limited to %.2f GB (%s): %s\n", std::max(0.0, limit_) / kGiB,
            limit_from_env_ ? "GGML_XDNA_MAX_COPY_GB" : "device memory free less what is kept back", where.c_str());
    }

public:
    bool admit(const ggml_tensor * w) {
        // no entry is ever built for these, so they cost nothing: a weight
        // without data (llama.cpp's memory-fitting trial), a tensor outside a
        // weights buffer, or a question asked with no context alive
        if (!w->buffer || !w->data || !in_weight_buffer(w)) return true;
        std::lock_guard<std::mutex> lk(mu_);
        if (live_ == 0) return true;
        const key k{w->buffer, w->data, (int) w->type, w->ne[0], w->ne[1]};
        if (const auto it = index_.find(k); it != index_.end()) return log_[it->second].taken;
        if (!limit_known_) fix_limit();
        decision d{layer_number(w->name), copy_bytes(w->ne[0], w->ne[1]), false};
        if (!closed_ && taken_bytes_ + d.bytes <= limit_) {
            d.taken = true;
            taken_bytes_ += d.bytes;
        } else if (!closed_) {
            close(d.layer);
        }
        index_.emplace(k, log_.size());
        log_.push_back(d);
        return d.taken;
    }

    void context_opened() {
        std::lock_guard<std::mutex> lk(mu_);
        live_++;
    }

    // true when it was the last: the budget starts over
    bool context_closed() {
        std::lock_guard<std::mutex> lk(mu_);
        if (--live_ > 0) return false;
        index_.clear();
        log_.clear();
        taken_bytes_ = 0;
        closed_ = ran_ = limit_known_ = limit_from_env_ = false;
        limit_ = 0;
        return true;
    }

    // The first graph to run: one line on what the cache takes, when the
    // budget never closed (a closed budget said so when it closed).
    void first_graph() {
        std::lock_guard<std::mutex> lk(mu_);
        if (ran_) return;
        ran_ = true;
        if (!limit_known_ || closed_) return;
        size_t n = 0;
        for (const decision & d : log_) n += d.taken;
        log(LOG_INFO, "weight cache: %.2f GB for %zu weights (limit %.1f GB)\n", taken_bytes_ / kGiB, n,
            std::max(0.0, limit_) / kGiB);
    }
};

weight_budget & budget() {
    static weight_budget b;
    return b;
}

// What was noticed about the model while the scheduler planned it, said once
// when a graph first runs (llama.cpp's memory-fitting trial plans with
// warnings hidden but never computes).
std::atomic<bool> g_expert_step{false}, g_notes_said{false};

}  // namespace

bool budget_takes(const ggml_tensor * w) { return budget().admit(w); }
void budget_context_added() { budget().context_opened(); }
void budget_context_freed() {
    if (budget().context_closed()) {
        g_expert_step = false;
        g_notes_said = false;
    }
}
void budget_report() { budget().first_graph(); }

void note_model(const ggml_tensor * op) {
    if (op->op == GGML_OP_MUL_MAT_ID) g_expert_step = true;
}

void say_notes() {
    if (g_notes_said.exchange(true) || !g_expert_step.load()) return;
    log(LOG_WARN, "mixture-of-experts model: the expert step (MUL_MAT_ID) is not taken, only the dense matmuls\n");
}

// ---- the gate --------------------------------------------------------------------------

// The weight side of a matmul we can take: a plain 2-D leaf (not a view, not
// computed: keys and values read from the KV cache are views) of a type the
// converter handles.
bool is_weight(const ggml_tensor * w) {
    return w->op == GGML_OP_NONE && w->view_src == nullptr && w->ne[2] == 1 && w->ne[3] == 1 && is_contiguous(w) &&
           convertible(w->type);
}

bool gemm_shape_fits(int64_t M, int64_t K, int64_t N) {
    constexpr uint64_t lim = 1ull << 31;
    return zest_bfp16_bytes(N, K) < lim && zest_act_bytes(M, K) < lim && (uint64_t) N * 4 * 256 < lim;
}

namespace {

// Why a MUL_MAT is left to the scheduler, or nullptr when it is taken. The
// budget is asked last: only a matmul that passes everything else counts
// against it.
const char * mul_mat_refusal(const ggml_tensor * op) {
    const ggml_tensor * w = op->src[0], * x = op->src[1];
    const int64_t tokens = op->ne[1];
    if (tokens < cfg().min_batch) return "batch below GGML_XDNA_MIN_BATCH";
    if (!is_weight(w)) return "left side not a plain weight of a converted type";
    if (op->type != GGML_TYPE_F32 || x->type != GGML_TYPE_F32) return "not fp32 rows in and out";
    if (x->ne[2] != 1 || x->ne[3] != 1 || !is_contiguous(x)) return "right side not contiguous 2-D rows";
    if (x->view_src && x->view_offs % 16 != 0) return "right side's rows not 16-byte aligned";
    if (x->ne[0] != w->ne[0]) return "K differs";
    if (w->ne[0] % 8 != 0) return "K not a whole number of 8-value blocks";
    // what one launch can address (2 GiB buffer ranges): the weight's cache
    // entry and the expanded activations whole, the output in bands of 256
    // rows or more (the library splits a taller output into such bands)
    if (!gemm_shape_fits(tokens, w->ne[0], w->ne[1])) return "an operand reaches 2 GiB";
    const int64_t mflop = 2 * w->ne[0] * w->ne[1] * tokens / 1000000;
    if (mflop < cfg().min_mflop) return "work below GGML_XDNA_MIN_MFLOP";
    if (!budget_takes(w)) return "weight cache budget";
    return nullptr;
}

// Whether a tensor may live in host memory once allocated: a graph input, an
// embedding lookup (llama.cpp keeps the token embeddings on the CPU), or one
// already in a host buffer.
bool maybe_in_host_memory(const ggml_tensor * t) {
    for (; t; t = t->view_src)
        if ((t->flags & GGML_TENSOR_FLAG_INPUT) || t->op == GGML_OP_GET_ROWS || buffer_is_host(t->buffer)) return true;
    return false;
}

bool taken(const ggml_tensor * op, int depth);

// A small op next to our matmuls: run by the executor, over a big batch, its
// parameter a kept leaf, and safe from ggml's in-place reuse of a same-shape
// input (which, were that input in host memory, would put our result there
// too: LFM2's first residual add, add(embeddings, x)).
bool small_op_eligible(const ggml_tensor * op) {
    if (op->op != GGML_OP_RESHAPE && tokens_of(op) < cfg().min_batch) return false;
    if (!exec_supports(op)) return false;
    if (!cfg().block_ops.empty() && !cfg().block_ops.count(op_name(op->op))) return false;
    if (const ggml_tensor * p = exec_param(op); p && (p->op != GGML_OP_NONE || p->view_src)) return false;
    for (const ggml_tensor * s : op->src)
        if (s && same_shape(op, s) && maybe_in_host_memory(s)) return false;
    return true;
}

// A small op is taken only when one of its inputs is the result of an op we
// take: pieces grow out from our matmuls (norm -> q/k/v; o -> add -> norm ->
// gate/up -> GLU -> down -> add) and never pull in unrelated work, which
// would only cut the next backend's graph into pieces. The search looks at
// most eight ops back.
bool taken(const ggml_tensor * op, int depth) {
    if (mode() != run_mode::gpu || broken()) return false;
    if (op->op == GGML_OP_MUL_MAT) return claim_mul_mat(op);
    if (!blocks() || depth > 8 || !small_op_eligible(op)) return false;
    return std::any_of(std::begin(op->src), std::end(op->src), [depth](const ggml_tensor * s) {
        return s && s->op != GGML_OP_NONE && taken(s, depth + 1);
    });
}

}  // namespace

bool claim_mul_mat(const ggml_tensor * op) {
    const char * why = mul_mat_refusal(op);
    if (why && cfg().trace_level >= 2)
        log(LOG_INFO, "%s (%lld x %lld at batch %lld) left to the scheduler: %s\n", op->name,
            (long long) op->src[0]->ne[0], (long long) op->src[0]->ne[1], (long long) op->ne[1], why);
    return why == nullptr;
}

bool supports_op(const ggml_tensor * op) {
    if (blocks() || trace()) note_readers(op);
    note_model(op);
    return taken(op, 0);
}

} // namespace zest

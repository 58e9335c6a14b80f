// What the ggml scheduler may hand this backend: the run mode, the gate
// (supports_op), reader tracking, the HBM budget for weight-cache entries and
// the one-time model notes. Same policy and settings as the reference
// (src/ggml-zest.cpp:56-130, 429-637, 1066-1226; src/xdna-exec.cpp:85-131),
// for a GPU whose memory holds the model.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>

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

// ---- run mode ------------------------------------------------------------

int device_index() {
    static const int d = (int) env_int("GGML_XDNA_DEVICE", 0);
    return d;
}

// GGML_XDNA_PLAN_ONLY=1 offers the device for planning only (supports_op,
// the budget) without a GPU, so the gate can be tested on a machine without
// one; every graph_compute then fails.
bool plan_only() {
    static const bool v = env_int("GGML_XDNA_PLAN_ONLY", 0) != 0;
    return v;
}

run_mode mode() {
    static const run_mode m = [] {
        if (env_int("GGML_XDNA_HOST_ONLY", 0) != 0) {
            log(LOG_WARN, "GGML_XDNA_HOST_ONLY is not supported: this backend has no CPU path; not offering "
                          GGML_XDNA_DEVICE_NAME "\n");
            return run_mode::off;
        }
        if (plan_only()) {
            log(LOG_INFO, "planning-only mode (GGML_XDNA_PLAN_ONLY): graphs will not run\n");
            return run_mode::gpu;
        }
        if (zest_init(device_index()) != ZEST_OK) {
            log(LOG_WARN, "not offering " GGML_XDNA_DEVICE_NAME ": %s\n", zest_last_error());
            return run_mode::off;
        }
        if (zest_self_test() != ZEST_OK) {
            log(LOG_WARN, "not offering " GGML_XDNA_DEVICE_NAME ": %s\n", zest_last_error());
            return run_mode::off;
        }
        log(LOG_INFO, "GPU %d (gfx950), registration test multiply right\n", device_index());
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

int64_t min_batch() {
    static const int64_t v = env_int("GGML_XDNA_MIN_BATCH", 1024);
    return v;
}
int64_t min_mflop() {
    static const int64_t v = env_int("GGML_XDNA_MIN_MFLOP", 256);
    return v;
}
bool blocks() {
    static const bool v = env_int("GGML_XDNA_BLOCKS", 1) != 0;
    return v && mode() == run_mode::gpu;
}
bool trace() {
    static const bool v = env_int("GGML_XDNA_TRACE", 0) != 0;
    return v;
}

// ---- what the executor implements (src/xdna-exec.cpp:85-131) --------------

static bool f32_contig(const ggml_tensor * t) { return t && t->type == GGML_TYPE_F32 && is_contiguous(t); }

// a single row as wide as a's rows (a norm's scale, a bias)
static bool is_row_of(const ggml_tensor * r, const ggml_tensor * a) {
    return f32_contig(r) && r->ne[0] == a->ne[0] && r->ne[1] == 1 && r->ne[2] == 1 && r->ne[3] == 1;
}

static bool glu_kind(int g) {
    return g == GGML_GLU_OP_SWIGLU || g == GGML_GLU_OP_GEGLU || g == GGML_GLU_OP_GEGLU_ERF ||
           g == GGML_GLU_OP_GEGLU_QUICK || g == GGML_GLU_OP_REGLU;
}

const ggml_tensor * exec_param(const ggml_tensor * op) {
    switch (op->op) {
        case GGML_OP_MUL: return op->src[1];
        case GGML_OP_ADD:
            return op->src[1] && op->src[0] && is_row_of(op->src[1], op->src[0]) && !same_shape(op->src[0], op->src[1])
                       ? op->src[1]
                       : nullptr;
        case GGML_OP_ROPE: return op->src[2];
        default: return nullptr;
    }
}

bool exec_supports(const ggml_tensor * op) {
    const ggml_tensor * a = op->src[0], * b = op->src[1];
    switch (op->op) {
        case GGML_OP_MUL_MAT: return true;  // the gate checks the weight side
        case GGML_OP_RESHAPE: return a && is_contiguous(a);
        case GGML_OP_RMS_NORM: return f32_contig(a) && f32_contig(op);
        case GGML_OP_MUL: return f32_contig(a) && f32_contig(op) && b && is_row_of(b, a) && same_shape(a, op);
        case GGML_OP_ADD:
            return f32_contig(a) && f32_contig(b) && f32_contig(op) && same_shape(a, op) &&
                   (same_shape(a, b) || is_row_of(b, a));
        case GGML_OP_SCALE: return f32_contig(a) && f32_contig(op) && same_shape(a, op);
        case GGML_OP_GLU:
            if (!glu_kind(param_i32(op, 0)) || !f32_contig(a) || !f32_contig(op)) return false;
            if (b) return param_i32(op, 1) == 0 && f32_contig(b) && same_shape(a, b) && same_shape(a, op);
            return a->ne[0] == 2 * op->ne[0] && nrows(a) == nrows(op);
        case GGML_OP_ROPE: {
            if (!f32_contig(a) || !f32_contig(op) || !b || b->type != GGML_TYPE_I32) return false;
            const int n_dims = param_i32(op, 1), mode = param_i32(op, 2), n_offs = param_i32(op, 15);
            const ggml_tensor * ff = op->src[2];
            if (ff && (!f32_contig(ff) || ff->ne[0] < n_dims / 2)) return false;
            // n_dims <= 8192: the kernel's angle table (1.5 n_dims floats) fits 64 KiB of shared memory
            return (mode == GGML_ROPE_TYPE_NEOX || mode == GGML_ROPE_TYPE_NORMAL) && n_dims > 0 && n_dims % 2 == 0 &&
                   n_dims <= a->ne[0] && n_dims <= 8192 && n_offs == 0 && a->ne[3] == 1 && b->ne[0] == a->ne[2];
        }
        default: return false;
    }
}

// ---- reader tracking ---------------------------------------------------------

static std::mutex g_read_mu;
static std::unordered_map<const ggml_tensor *, std::unordered_set<const ggml_tensor *>> g_readers;
static std::atomic<uint64_t> g_read_epoch{0};  // counts the readers recorded

void note_readers(const ggml_tensor * op) {
    std::lock_guard<std::mutex> lk(g_read_mu);
    bool added = false;
    for (int j = 0; j < GGML_MAX_SRC; j++)
        if (const ggml_tensor * s = op->src[j]) {
            added |= g_readers[s].insert(op).second;
            for (const ggml_tensor * v = s->view_src; v; v = v->view_src) added |= g_readers[v].insert(op).second;
        }
    if (added) g_read_epoch.fetch_add(1, std::memory_order_relaxed);
}

uint64_t readers_epoch() { return g_read_epoch.load(std::memory_order_relaxed); }

bool read_outside(const ggml_tensor * t, const std::unordered_set<const ggml_tensor *> & in_piece) {
    static const bool all = env_int("GGML_XDNA_WRITE_ALL", 0) != 0;
    if (all || (t->flags & GGML_TENSOR_FLAG_OUTPUT)) return true;
    std::lock_guard<std::mutex> lk(g_read_mu);
    auto it = g_readers.find(t);
    if (it == g_readers.end()) return true;
    for (const ggml_tensor * r : it->second)
        if (!in_piece.count(r)) return true;
    return false;
}

// ---- the HBM budget -------------------------------------------------------------

static constexpr double GiB = 1024.0 * 1024 * 1024;

struct wkey {
    const void * buffer, * data;
    int type;
    int64_t ne0, ne1;
    bool operator==(const wkey & o) const {
        return buffer == o.buffer && data == o.data && type == o.type && ne0 == o.ne0 && ne1 == o.ne1;
    }
};
struct wkey_hash {
    size_t operator()(const wkey & k) const {
        return std::hash<const void *>()(k.buffer) ^ (std::hash<const void *>()(k.data) * 31) ^ (size_t) k.ne1;
    }
};

// A K x N weight's cache entry: 9 bytes per 8 values in the tile layout
// (rows padded to 256, columns to 64).
double copy_bytes(int64_t K, int64_t N) { return (double) zest_bfp16_bytes(N, K); }

static int layer_of(const ggml_tensor * w) {
    int layer = -1;
    return sscanf(w->name, "blk.%d.", &layer) == 1 ? layer : -1;
}

// Weights are taken in the order the scheduler asks about them until the next
// would pass the limit; that layer and every later weight then stay off the
// GPU path, and a decision never changes while a context lives. The limit is
// the device memory free when the first weight is asked about, less the larger
// of 4 GB and a tenth of the device (llama.cpp's work buffers), or
// GGML_XDNA_MAX_COPY_GB. Unlike the reference's 20 GB NPU cap there is no
// default cap: the cache lives in the GPU's own HBM.
struct budget {
    std::mutex mu;
    int contexts = 0;
    bool started = false, cut = false, running = false, overridden = false;
    double limit = 0, free = 0, kept_back = 0, taken = 0;
    struct entry {
        int layer;
        double bytes;
    };
    std::unordered_map<wkey, entry, wkey_hash> in, out;

    void reset() {
        started = cut = running = overridden = false;
        limit = free = kept_back = taken = 0;
        in.clear();
        out.clear();
    }
};
static budget g_budget;

void budget_context_added() {
    std::lock_guard<std::mutex> lk(g_budget.mu);
    g_budget.contexts++;
}

static void notes_reset();

void budget_context_freed() {
    std::lock_guard<std::mutex> lk(g_budget.mu);
    if (--g_budget.contexts == 0) {
        g_budget.reset();
        notes_reset();
    }
}

bool budget_takes(const ggml_tensor * w) {
    if (!w->buffer || !w->data || !in_weight_buffer(w)) return true;
    budget & b = g_budget;
    std::lock_guard<std::mutex> lk(b.mu);
    if (b.contexts == 0) return true;
    const wkey key = {w->buffer, w->data, (int) w->type, w->ne[0], w->ne[1]};
    if (b.in.count(key)) return true;
    if (b.out.count(key)) return false;
    if (!b.started) {
        b.started = true;
        size_t fr = 0, tot = 0;
        if (!plan_only() && hipMemGetInfo(&fr, &tot) == hipSuccess) {
            b.free = (double) fr;
            b.kept_back = std::max(4 * GiB, (double) tot / 10);
        }
        const char * s = env("GGML_XDNA_MAX_COPY_GB");
        b.overridden = s != nullptr;
        b.limit = s ? atof(s) * GiB : (plan_only() ? 1e30 : b.free - b.kept_back);
    }
    const budget::entry e = {layer_of(w), copy_bytes(w->ne[0], w->ne[1])};
    if (!b.cut && b.taken + e.bytes <= b.limit) {
        b.in[key] = e;
        b.taken += e.bytes;
        return true;
    }
    if (!b.cut) {
        b.cut = true;
        // the layer's weights taken so far go too, so no layer is split
        if (e.layer >= 0 && !b.running)
            for (auto it = b.in.begin(); it != b.in.end();) {
                if (it->second.layer != e.layer) {
                    ++it;
                    continue;
                }
                b.taken -= it->second.bytes;
                b.out.insert(*it);
                it = b.in.erase(it);
            }
        std::unordered_set<int> layers;
        for (const auto & kv : b.in)
            if (kv.second.layer >= 0) layers.insert(kv.second.layer);
        log(LOG_WARN, "weight cache limited to %.2f GB (%s): %s\n", std::max(0.0, b.limit) / GiB,
            b.overridden ? "GGML_XDNA_MAX_COPY_GB" : "device memory free less what is kept back",
            layers.empty() ? "no layer fits" : (std::to_string(layers.size()) + " layers on the GPU path").c_str());
    }
    b.out[key] = e;
    return false;
}

void budget_report() {
    budget & b = g_budget;
    std::lock_guard<std::mutex> lk(b.mu);
    if (b.running) return;
    b.running = true;
    if (!b.started || b.cut) return;
    log(LOG_INFO, "weight cache: %.2f GB for %zu weights (limit %.1f GB)\n", b.taken / GiB, b.in.size(),
        std::max(0.0, b.limit) / GiB);
}

// ---- model notes -------------------------------------------------------------

static std::atomic<bool> g_moe{false};
static std::atomic<int64_t> g_width{0};
static std::atomic<bool> g_said{false};
static void notes_reset() {
    g_moe = false;
    g_width = 0;
    g_said = false;
}

static bool name_in_layer(const char * name, const char * tail) {
    if (strncmp(name, "blk.", 4) != 0) return false;
    const char * p = name + 4;
    while (*p >= '0' && *p <= '9') p++;
    return *p == '.' && strcmp(p + 1, tail) == 0;
}

void note_model(const ggml_tensor * op) {
    if (op->op == GGML_OP_MUL_MAT_ID) g_moe = true;
    if (g_width.load() != 0) return;
    for (int j = 0; j < GGML_MAX_SRC; j++) {
        const ggml_tensor * s = op->src[j];
        if (!s) continue;
        if (strcmp(s->name, "token_embd.weight") == 0 || name_in_layer(s->name, "attn_q.weight") ||
            name_in_layer(s->name, "attn_qkv.weight")) {
            g_width = s->ne[0];
            return;
        }
    }
}

void say_notes() {
    if (g_said.exchange(true)) return;
    if (g_moe.load())
        log(LOG_WARN, "mixture-of-experts model: the expert step (MUL_MAT_ID) is not taken, only the dense matmuls\n");
}

// ---- the gate ------------------------------------------------------------------

// The weight side of a matmul we can take: a plain 2-D leaf (not a view, not
// computed) of a type the converter handles (src/ggml-zest.cpp:1066-1072).
bool is_weight(const ggml_tensor * w) {
    if (w->op != GGML_OP_NONE || w->view_src != nullptr) return false;
    if (w->ne[2] != 1 || w->ne[3] != 1 || !is_contiguous(w)) return false;
    return convertible(w->type);
}

// src/ggml-zest.cpp:1167-1180, with this path's shape rule (K a multiple of 8,
// the bfp16 block) in place of the NPU's instruction-stream sizes.
bool claim_mul_mat(const ggml_tensor * op) {
    const ggml_tensor * src0 = op->src[0], * src1 = op->src[1];
    if (op->ne[1] < min_batch()) return false;
    if (!is_weight(src0)) return false;
    if (op->type != GGML_TYPE_F32 || src1->type != GGML_TYPE_F32) return false;
    if (!is_contiguous(src1) || src1->ne[2] != 1 || src1->ne[3] != 1) return false;
    if (src0->ne[0] != src1->ne[0] || src0->ne[0] % 8 != 0) return false;
    const int64_t mflop = 2 * src0->ne[0] * src0->ne[1] * op->ne[1] / 1000000;
    return mflop >= min_mflop() && budget_takes(src0);
}

// Whether a tensor may live in host memory once allocated: a graph input, an
// embedding lookup, or one already in a host buffer.
static bool maybe_host(const ggml_tensor * t) {
    for (; t; t = t->view_src) {
        if ((t->flags & GGML_TENSOR_FLAG_INPUT) || t->op == GGML_OP_GET_ROWS) return true;
        if (buffer_is_host(t->buffer)) return true;
    }
    return false;
}

// src/ggml-zest.cpp:1191-1226: matmuls by claim_mul_mat; a small op only when
// the executor implements it, it covers a big batch, and one of its inputs
// comes from an op we would claim (pieces grow out from our matmuls).
static bool policy(const ggml_tensor * op, int depth) {
    if (mode() != run_mode::gpu || broken()) return false;
    if (op->op == GGML_OP_MUL_MAT) return claim_mul_mat(op);
    if (!blocks() || depth > 8) return false;
    if (op->op != GGML_OP_RESHAPE && tokens_of(op) < min_batch()) return false;
    if (!exec_supports(op)) return false;
    {
        static const std::string allow = [] {
            const char * s = env("GGML_XDNA_BLOCK_OPS");
            return s ? "," + std::string(s) + "," : std::string();
        }();
        if (!allow.empty() && allow.find("," + std::string(op_name(op->op)) + ",") == std::string::npos) return false;
    }
    if (const ggml_tensor * w = exec_param(op))
        if (w->op != GGML_OP_NONE || w->view_src) return false;
    for (int j = 0; j < GGML_MAX_SRC; j++)
        if (const ggml_tensor * s = op->src[j])
            if (maybe_host(s) && same_shape(op, s)) return false;
    for (int j = 0; j < GGML_MAX_SRC; j++) {
        const ggml_tensor * s = op->src[j];
        if (s && s->op != GGML_OP_NONE && policy(s, depth + 1)) return true;
    }
    return false;
}

bool supports_op(const ggml_tensor * op) {
    if (blocks() || trace()) note_readers(op);
    note_model(op);
    return policy(op, 0);
}

} // namespace zest

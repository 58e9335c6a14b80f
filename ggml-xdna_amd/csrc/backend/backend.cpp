// The ggml backend add-on: registration, the device, its HIP buffer type, and
// the backend whose graph_compute runs the scheduler's pieces on one GPU.
//
// The reference (src/ggml-zest.cpp) works next to a Vulkan GPU on a laptop:
// it reads every input out of Vulkan memory, runs the matmuls on the NPU and
// the small ops on the host, and writes results back. On an MI355X the model
// lives in the GPU's own HBM, so this device has its own HIP buffer type and a
// piece is a sequence of kernel launches on one HIP stream: inputs, weight
// cache, packed activations and results never leave HBM. Same registry and
// device names, same gate and settings (policy.cpp), same failure latch; no
// CPU path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "backend.h"
#include "zest_hip.h"

namespace zest {
namespace {

#define XDNA_DESCRIPTION "AMD Instinct MI355X (gfx950): bfp16 prefill MUL_MAT"

// ---- the HIP buffer type -------------------------------------------------------

struct buffer_ctx {
    void * base = nullptr;
    size_t size = 0;
};

void evict_buffer(const ggml_backend_buffer * b);
void forget_weight(const void * data);

void buf_free(ggml_backend_buffer_t b) {
    evict_buffer(b);  // its weights' cache entries go with it
    auto * c = (buffer_ctx *) b->context;
    if (c->base) (void) hipFree(c->base);
    delete c;  // the buffer object itself is deleted by ggml_backend_buffer_free
}
void * buf_base(ggml_backend_buffer_t b) { return ((buffer_ctx *) b->context)->base; }
ggml_status buf_init_tensor(ggml_backend_buffer_t, ggml_tensor *) { return GGML_STATUS_SUCCESS; }
// A tensor written from outside a graph may be a weight whose cache entries
// were converted from its old bytes: they are dropped first.
void buf_memset(ggml_backend_buffer_t, ggml_tensor * t, uint8_t value, size_t offset, size_t size) {
    forget_weight(t->data);
    (void) hipMemset((char *) t->data + offset, value, size);
}
void buf_set(ggml_backend_buffer_t, ggml_tensor * t, const void * data, size_t offset, size_t size) {
    forget_weight(t->data);
    (void) hipMemcpy((char *) t->data + offset, data, size, hipMemcpyHostToDevice);
}
void buf_get(ggml_backend_buffer_t, const ggml_tensor * t, void * data, size_t offset, size_t size) {
    (void) hipMemcpy(data, (const char *) t->data + offset, size, hipMemcpyDeviceToHost);
}
ggml_backend_buffer_type * our_buft();
bool buf_cpy(ggml_backend_buffer_t, const ggml_tensor * src, ggml_tensor * dst) {
    if (!src->buffer || src->buffer->buft != our_buft()) return false;
    forget_weight(dst->data);
    return hipMemcpy(dst->data, src->data, nbytes(src), hipMemcpyDeviceToDevice) == hipSuccess;
}
void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    evict_buffer(b);
    auto * c = (buffer_ctx *) b->context;
    (void) hipMemset(c->base, value, c->size);
}

const ggml_backend_buffer_i buffer_iface = {
    /* .free_buffer   = */ buf_free,
    /* .get_base      = */ buf_base,
    /* .init_tensor   = */ buf_init_tensor,
    /* .memset_tensor = */ buf_memset,
    /* .set_tensor    = */ buf_set,
    /* .get_tensor    = */ buf_get,
    /* .cpy_tensor    = */ buf_cpy,
    /* .clear         = */ buf_clear,
    /* .reset         = */ nullptr,
};

const char * buft_name(ggml_backend_buffer_type_t) { return GGML_XDNA_DEVICE_NAME; }
ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    auto * c = new buffer_ctx;
    c->size = size;
    if (hipMalloc(&c->base, size ? size : 1) != hipSuccess) {
        log(LOG_ERROR, "cannot allocate %zu bytes of device memory\n", size);
        delete c;
        return nullptr;
    }
    return new ggml_backend_buffer{buffer_iface, buft, c, size, GGML_BACKEND_BUFFER_USAGE_ANY};
}
size_t buft_alignment(ggml_backend_buffer_type_t) { return 256; }
size_t buft_max_size(ggml_backend_buffer_type_t) { return SIZE_MAX; }
bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

ggml_backend_device * our_device();

ggml_backend_buffer_type * our_buft() {
    static ggml_backend_buffer_type buft = {
        {buft_name, buft_alloc, buft_alignment, buft_max_size, nullptr, buft_is_host}, nullptr, nullptr};
    buft.device = our_device();
    return &buft;
}

// ---- the backend context ---------------------------------------------------

// A weight-cache entry's key: the weight's buffer, address, type and shape;
// for a fused gate/up entry also its partner, the up weight's address and
// buffer (or, for one weight of both halves, which half is the gate).
struct wkey {
    const void * buffer, * data;
    int type;
    int64_t ne0, ne1;
    const void * partner = nullptr, * partner_buffer = nullptr;
    bool operator==(const wkey & o) const {
        return buffer == o.buffer && data == o.data && type == o.type && ne0 == o.ne0 && ne1 == o.ne1 &&
               partner == o.partner;
    }
    bool uses(const void * d) const { return data == d || partner == d; }
};
struct wkey_hash {
    size_t operator()(const wkey & k) const {
        return std::hash<const void *>()(k.buffer) ^ (std::hash<const void *>()(k.data) * 31) ^ (size_t) k.ne1 ^
               (std::hash<const void *>()(k.partner) * 131);
    }
};
wkey key_of(const ggml_tensor * w) { return {w->buffer, w->data, (int) w->type, w->ne[0], w->ne[1]}; }

// A GLU over matmuls that one fused gate/up GEMM replaces (the reference's
// find_fusions, src/xdna-exec.cpp:399-431): gate and up matmuls on the same
// input, or one matmul whose weight holds both halves (up == nullptr; then
// `swapped` says the up rows come first), each read by nothing but the GLU.
struct fusion {
    const ggml_tensor * gate_mm, * up_mm;
    ggml_tensor * glu;
    bool swapped;
    int64_t F, K;
};

// The cache key of a fused pair: the gate weight's, type + 1000, 2F rows (as
// xdna_npu::fused_key, src/xdna-npu.h:65), and the up weight it is paired
// with, so that a gate met with another partner gets an entry of its own.
const char k_up_rows_first = 0;
wkey fused_key(const fusion & f) {
    const ggml_tensor * w = f.gate_mm->src[0], * u = f.up_mm ? f.up_mm->src[0] : nullptr;
    wkey k{w->buffer, w->data, 1000 + (int) w->type, f.K, 2 * f.F};
    k.partner = u ? u->data : f.swapped ? (const void *) &k_up_rows_first : nullptr;
    k.partner_buffer = u ? (const void *) u->buffer : nullptr;
    return k;
}

// GGML_XDNA_FAIL_AFTER=n: every GEMM submission after the n-th fails;
// GGML_XDNA_NAN_AFTER=n: every GEMM result after the n-th comes back as NaN
// (src/xdna-npu.cpp:89-112). Both forced from the host: kernels run normally.
int64_t fail_after() {
    static const int64_t v = env_int("GGML_XDNA_FAIL_AFTER", -1);
    return v;
}
int64_t nan_after() {
    static const int64_t v = env_int("GGML_XDNA_NAN_AFTER", -1);
    return v;
}
std::atomic<int64_t> g_submissions{0};

struct piece_plan;

struct context {
    hipStream_t stream = nullptr;  // compute
    hipStream_t loader = nullptr;  // weight conversion at load
    uint32_t * nonfinite = nullptr;       // device word the kernels OR 1 into
    uint32_t * nonfinite_host = nullptr;  // pinned host copy, read after each piece's synchronize

    struct weight_entry {
        void * packed = nullptr;
        hipEvent_t ready = nullptr;  // recorded on `loader` when built at load
    };
    // The cache, and the lock other threads take to drop entries from it (a
    // buffer freed or a weight rewritten while this context computes).
    std::unordered_map<wkey, weight_entry, wkey_hash> weights;
    std::mutex weights_mu;
    int64_t built_at_load = 0, built_in_graph = 0;

    // per-graph device workspace: grow-only blocks, handed out from the start
    // again by each graph
    struct block {
        char * p;
        size_t size, used;
    };
    std::vector<block> blocks;

    // trace
    double compute_ms = 0;
    int64_t matmuls = 0, pieces = 0;

    // the plans of the graphs computed lately, by graph (reused while the
    // graph is unchanged; at most PLAN_CACHE of them)
    static constexpr size_t PLAN_CACHE = 256;
    std::unordered_map<const ggml_cgraph *, std::shared_ptr<const piece_plan>> plans;
    std::shared_ptr<const piece_plan> plan_for(const ggml_cgraph * g);

    context();
    ~context();
    void evict(const ggml_backend_buffer * b);
    void forget(const void * data);
    void drop_where(const std::function<bool(const wkey &)> & stale);

    bool init(std::string & err) {
        if (hipSetDevice(device_index()) != hipSuccess || hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) ||
            hipStreamCreateWithFlags(&loader, hipStreamNonBlocking) || hipMalloc(&nonfinite, 256) ||
            hipHostMalloc(&nonfinite_host, sizeof(uint32_t), hipHostMallocDefault)) {
            err = "cannot create streams on the device";
            return false;
        }
        return true;
    }


    void ws_reset() {
        for (block & b : blocks) b.used = 0;
    }
    void * ws_alloc(size_t n) {
        n = (n + 255) / 256 * 256;
        for (block & b : blocks)
            if (b.size - b.used >= n) {
                void * p = b.p + b.used;
                b.used += n;
                return p;
            }
        const size_t sz = std::max(n, (size_t) 64 << 20);
        block b{nullptr, sz, n};
        if (hipMalloc((void **) &b.p, sz) != hipSuccess) return nullptr;
        blocks.push_back(b);
        return b.p;
    }

    // The weight's cache entry (its packed bytes into *packed), converted
    // from its raw GGUF bytes where they are (device memory in our buffers;
    // host memory goes up first) on `on_stream`; an entry built at load is
    // waited for on the compute stream.
    bool ensure_weight(const ggml_tensor * w, hipStream_t on_stream, bool at_load, std::string & err,
                       const void ** packed = nullptr) {
        std::lock_guard<std::mutex> lk(weights_mu);
        const wkey key = key_of(w);
        auto it = weights.find(key);
        if (it != weights.end()) {
            if (!at_load && it->second.ready) {
                if (hipStreamWaitEvent(stream, it->second.ready, 0) != hipSuccess) {
                    err = "waiting for a weight conversion failed";
                    return false;
                }
            }
            if (packed) *packed = it->second.packed;
            return true;
        }
        const int64_t K = w->ne[0], N = w->ne[1];
        weight_entry e;
        if (hipMalloc(&e.packed, zest_bfp16_bytes(N, K)) != hipSuccess) {
            err = "cannot allocate a weight-cache entry";
            return false;
        }
        const void * raw = w->data;
        void * tmp = nullptr;
        if (buffer_is_host(w->buffer)) {
            const size_t nb = nbytes(w);
            if (hipMalloc(&tmp, nb) != hipSuccess ||
                hipMemcpyAsync(tmp, w->data, nb, hipMemcpyHostToDevice, on_stream) != hipSuccess) {
                err = "cannot upload a host weight";
                (void) hipFree(e.packed);
                return false;
            }
            raw = tmp;
        }
        if (zest_convert_weight(w->type, raw, N, K, e.packed, on_stream) != ZEST_OK) {
            err = std::string(w->name) + ": " + zest_last_error();
            (void) hipFree(e.packed);
            return false;
        }
        if (tmp) {
            (void) hipStreamSynchronize(on_stream);
            (void) hipFree(tmp);
        }
        if (at_load) {
            (void) hipEventCreateWithFlags(&e.ready, hipEventDisableTiming);
            (void) hipEventRecord(e.ready, on_stream);
            built_at_load++;
        } else {
            built_in_graph++;
        }
        weights.emplace(key, e);
        if (packed) *packed = e.packed;
        return true;
    }

    // The same for a fused gate/up pair: both weights' rows, interleaved into
    // one entry (zest_convert_weight_gu).
    bool ensure_fused(const fusion & f, hipStream_t on_stream, bool at_load, std::string & err,
                      const void ** packed = nullptr) {
        std::lock_guard<std::mutex> lk(weights_mu);
        const wkey key = fused_key(f);
        auto it = weights.find(key);
        if (it != weights.end()) {
            if (!at_load && it->second.ready && hipStreamWaitEvent(stream, it->second.ready, 0) != hipSuccess) {
                err = "waiting for a weight conversion failed";
                return false;
            }
            if (packed) *packed = it->second.packed;
            return true;
        }
        const ggml_tensor * gw = f.gate_mm->src[0], * uw = f.up_mm ? f.up_mm->src[0] : nullptr;
        weight_entry e;
        if (hipMalloc(&e.packed, zest_bfp16_bytes(2 * f.F, f.K)) != hipSuccess) {
            err = "cannot allocate a weight-cache entry";
            return false;
        }
        // each weight's raw rows in device memory (host weights go up first)
        std::vector<void *> tmps;
        auto dev = [&](const ggml_tensor * w) -> const uint8_t * {
            if (!buffer_is_host(w->buffer)) return (const uint8_t *) w->data;
            void * t = nullptr;
            if (hipMalloc(&t, nbytes(w)) != hipSuccess ||
                hipMemcpyAsync(t, w->data, nbytes(w), hipMemcpyHostToDevice, on_stream) != hipSuccess)
                return nullptr;
            tmps.push_back(t);
            return (const uint8_t *) t;
        };
        const uint8_t * g = dev(gw), * u = uw ? dev(uw) : nullptr;
        int st = ZEST_E_HIP;
        if (g && (!uw || u)) {
            if (!uw) {
                // one weight: the gate's F rows, then the up's (or the reverse)
                const uint8_t * second = g + f.F * gw->nb[1];
                u = f.swapped ? g : second;
                g = f.swapped ? second : g;
            }
            st = zest_convert_weight_gu(gw->type, g, u, f.F, f.K, e.packed, on_stream);
        }
        if (!tmps.empty()) (void) hipStreamSynchronize(on_stream);
        for (void * t : tmps) (void) hipFree(t);
        if (st != ZEST_OK) {
            err = std::string(gw->name) + " (fused gate/up): " + (st == ZEST_E_HIP ? "upload failed" : zest_last_error());
            (void) hipFree(e.packed);
            return false;
        }
        if (at_load) {
            (void) hipEventCreateWithFlags(&e.ready, hipEventDisableTiming);
            (void) hipEventRecord(e.ready, on_stream);
            built_at_load++;
        } else {
            built_in_graph++;
        }
        weights.emplace(key, e);
        if (packed) *packed = e.packed;
        return true;
    }
};

// Live contexts, so that freeing one of our buffers drops the cache entries of
// the weights it held (a later buffer may reuse the address).
std::mutex g_ctx_mu;
std::unordered_set<context *> g_contexts;

context::context() {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    g_contexts.insert(this);
}

context::~context() {
    {
        std::lock_guard<std::mutex> lk(g_ctx_mu);
        g_contexts.erase(this);
    }
    if (stream) (void) hipStreamSynchronize(stream);
    if (loader) (void) hipStreamSynchronize(loader);
    for (auto & kv : weights) {
        if (kv.second.packed) (void) hipFree(kv.second.packed);
        if (kv.second.ready) (void) hipEventDestroy(kv.second.ready);
    }
    for (block & b : blocks) (void) hipFree(b.p);
    if (nonfinite) (void) hipFree(nonfinite);
    if (nonfinite_host) (void) hipHostFree(nonfinite_host);
    // the library's split-K workspaces for these streams go with them
    if (stream) (void) zest_release_stream(stream);
    if (loader) (void) zest_release_stream(loader);
    if (stream) (void) hipStreamDestroy(stream);
    if (loader) (void) hipStreamDestroy(loader);
}

// Drops the cache entries `stale` names, after the work that may read them
// (weights_mu held).
void context::drop_where(const std::function<bool(const wkey &)> & stale) {
    bool synced = false;
    for (auto it = weights.begin(); it != weights.end();) {
        if (!stale(it->first)) {
            ++it;
            continue;
        }
        if (!synced) {
            if (stream) (void) hipStreamSynchronize(stream);
            if (loader) (void) hipStreamSynchronize(loader);
            synced = true;
        }
        if (it->second.packed) (void) hipFree(it->second.packed);
        if (it->second.ready) (void) hipEventDestroy(it->second.ready);
        it = weights.erase(it);
    }
}

// every entry of a weight in buffer b, or paired with one there
void context::evict(const ggml_backend_buffer * b) {
    std::lock_guard<std::mutex> lk(weights_mu);
    drop_where([b](const wkey & k) { return k.buffer == b || k.partner_buffer == b; });
}

// every entry converted from the tensor at `data`
void context::forget(const void * data) {
    std::lock_guard<std::mutex> lk(weights_mu);
    if (weights.empty()) return;
    drop_where([data](const wkey & k) { return k.uses(data); });
}

void evict_buffer(const ggml_backend_buffer * b) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    for (context * c : g_contexts) c->evict(b);
}

void forget_weight(const void * data) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    for (context * c : g_contexts) c->forget(data);
}

// ---- graph execution ---------------------------------------------------------

int glu_kind_of(int g) {
    switch (g) {
        case GGML_GLU_OP_REGLU: return ZEST_GLU_REGLU;
        case GGML_GLU_OP_GEGLU: return ZEST_GLU_GEGLU;
        case GGML_GLU_OP_SWIGLU: return ZEST_GLU_SWIGLU;
        case GGML_GLU_OP_GEGLU_ERF: return ZEST_GLU_GEGLU_ERF;
        case GGML_GLU_OP_GEGLU_QUICK: return ZEST_GLU_GEGLU_QUICK;
        default: return -1;
    }
}

// ggml_rope_yarn_corr_dims (ggml-base; called by the reference at
// src/xdna-exec.cpp:221), from the published YaRN formula: the dimension
// where a frequency turns n_rot times over n_ctx_orig positions.
void rope_corr_dims(int n_dims, int n_ctx_orig, float base, float beta_fast, float beta_slow, float dims[2]) {
    auto dim = [&](float n_rot) {
        return (float) n_dims * logf((float) n_ctx_orig / (n_rot * 2.0f * (float) M_PI)) / (2.0f * logf(base));
    };
    dims[0] = std::max(0.0f, floorf(dim(beta_fast)));
    dims[1] = std::min((float) (n_dims - 1), ceilf(dim(beta_slow)));
}

// The tensor whose packed copy a matmul input x can use: its owner when x
// reads the owner's rows exactly (itself, or a reshape of the same rows),
// else x itself (no packed copy is ever made for a partial view).
const ggml_tensor * packed_key(const ggml_tensor * x) {
    const ggml_tensor * o = owner(x);
    if (x == o) return x;
    return x->data == o->data && x->ne[0] == o->ne[0] && nrows(x) == nrows(o) && is_contiguous(x) ? o : x;
}

// A matmul this backend runs as a GEMM: a weight (K % 8 == 0) times F32 rows.
bool gemm_matmul(const ggml_tensor * n) {
    return n->op == GGML_OP_MUL_MAT && is_weight(n->src[0]) && n->src[1]->type == GGML_TYPE_F32 &&
           is_contiguous(n->src[1]) && n->src[0]->ne[0] % 8 == 0;
}

// Readers of each tensor among a piece's nodes, owner(src) -> (node, source
// slot), built once per piece so that each reader question is one lookup
// rather than a pass over every node (a prompt graph of a whole model has
// hundreds of nodes, and the questions are asked per node).
using reader_list = std::vector<std::pair<const ggml_tensor *, int>>;
using reader_map = std::unordered_map<const ggml_tensor *, reader_list>;

reader_map index_readers(const std::vector<ggml_tensor *> & nodes) {
    reader_map r;
    for (const ggml_tensor * n : nodes)
        for (int j = 0; j < GGML_MAX_SRC; j++)
            if (n->src[j]) r[owner(n->src[j])].emplace_back(n, j);
    return r;
}

// whether a node of the piece other than `except` reads t
bool read_by_other(const reader_map & r, const ggml_tensor * t, const ggml_tensor * except) {
    const auto it = r.find(t);
    if (it == r.end()) return false;
    for (const auto & e : it->second)
        if (e.first != except) return true;
    return false;
}

// A node that writes into the memory of another tensor: an in-place op, whose
// result is a view of its input (ggml's *_inplace ops). Packed copies of that
// tensor's rows made before it no longer hold its values.
bool writes_in_place(const ggml_tensor * n) { return !is_noop(n) && n->view_src != nullptr; }

// The fusions of a piece (src/xdna-exec.cpp:399-431): a GLU whose gate and up
// are matmuls of the piece on the same input, with weights of one type and
// shape, read by nothing but the GLU, inside the piece or out; or a GLU over
// the halves of one such matmul's output. F % 32 == 0 (the fused GEMM's
// interleave). The reference fuses SwiGLU only; every GLU kind is fused here,
// the epilogue computing the same GLU the GLU kernel does. Gate and up must
// see the same values: no node between them writes into their input in place.
std::vector<fusion> find_fusions(const std::vector<ggml_tensor *> & nodes,
                                 const std::unordered_set<const ggml_tensor *> & in_piece, const reader_map & rd) {
    std::vector<fusion> out;
    std::unordered_map<const ggml_tensor *, size_t> at;
    for (size_t i = 0; i < nodes.size(); i++) at[nodes[i]] = i;
    auto rewritten_between = [&](const ggml_tensor * m1, const ggml_tensor * m2) {
        const ggml_tensor * o = owner(m1->src[1]);
        size_t i = at.at(m1), j = at.at(m2);
        if (i > j) std::swap(i, j);
        for (size_t k = i + 1; k < j; k++)
            if (writes_in_place(nodes[k]) && owner(nodes[k]) == o) return true;
        return false;
    };
    for (ggml_tensor * n : nodes) {
        if (n->op != GGML_OP_GLU || glu_kind_of(param_i32(n, 0)) < 0 || !is_contiguous(n)) continue;
        const ggml_tensor * gm = n->src[0], * um = n->src[1];
        if (!gemm_matmul(gm) || !in_piece.count(gm) || read_outside(gm, in_piece) || !is_contiguous(gm)) continue;
        const ggml_tensor * gw = gm->src[0];
        fusion f{gm, nullptr, n, false, 0, gw->ne[0]};
        if (um) {
            if (param_i32(n, 1) != 0 || !gemm_matmul(um) || !in_piece.count(um) || read_outside(um, in_piece) ||
                !is_contiguous(um) || packed_key(gm->src[1]) != packed_key(um->src[1]) || rewritten_between(gm, um))
                continue;
            const ggml_tensor * uw = um->src[0];
            if (uw->type != gw->type || uw->ne[0] != gw->ne[0] || uw->ne[1] != gw->ne[1]) continue;
            f.up_mm = um;
            f.F = gw->ne[1];
        } else {
            if (gw->ne[1] % 2) continue;
            f.F = gw->ne[1] / 2;
            f.swapped = param_i32(n, 1) != 0;
        }
        if (f.F % 32 || n->ne[0] != f.F || nrows(n) != gm->src[1]->ne[1]) continue;
        // one launch addresses the 2F-row weight and the packed h whole
        const int64_t M = gm->src[1]->ne[1];
        if (!gemm_shape_fits(M, f.K, 2 * f.F) || zest_act_bytes(M, f.F) >= (1ull << 31)) continue;
        // another reader of the gate's or up's result
        if (!read_by_other(rd, gm, n) && !(um && read_by_other(rd, um, n))) out.push_back(f);
    }
    return out;
}

// Residual adds: an ADD of a matmul's result and a same-shape F32 tensor whose
// rows are 16-byte aligned, the matmul read by nothing else, inside the piece
// or out, runs as one GEMM with the add in its store (zest_gemm_residual).
// Returns ADD -> its matmul.
std::unordered_map<const ggml_tensor *, const ggml_tensor *> find_residuals(
    const std::vector<ggml_tensor *> & nodes, const std::unordered_set<const ggml_tensor *> & in_piece,
    const std::unordered_set<const ggml_tensor *> & fused, const reader_map & rd) {
    std::unordered_map<const ggml_tensor *, const ggml_tensor *> out;
    for (ggml_tensor * a : nodes) {
        if (a->op != GGML_OP_ADD || !is_contiguous(a) || a->type != GGML_TYPE_F32) continue;
        for (int side = 0; side < 2; side++) {
            const ggml_tensor * n = a->src[side], * r = a->src[1 - side];
            if (!n || !r || !gemm_matmul(n) || fused.count(n) || !in_piece.count(n) || read_outside(n, in_piece) ||
                !same_shape(a, n) || !same_shape(a, r) || r->type != GGML_TYPE_F32 || r->nb[0] != 4 ||
                r->nb[1] % 16 != 0 || (r->view_src && r->view_offs % 16 != 0) || nrows(a) != a->ne[1] ||
                (uint64_t) std::max(r->nb[1], a->nb[1]) * 256 >= (1ull << 31))
                continue;
            if (read_by_other(rd, n, a)) continue;  // another reader of the matmul's result
            out[a] = n;
            break;
        }
    }
    return out;
}

// What graph_compute works out about a piece before launching anything: its
// nodes, their readers, the gate/up fusions and the residual adds. It depends
// only on the graph's structure (ops, sources, shapes, strides, data
// addresses, flags, op parameters) and on the readers recorded by
// supports_op, so a graph computed again unchanged (llama.cpp reuses its
// prompt graph from one batch to the next) reuses it.
struct piece_plan {
    std::vector<ggml_tensor *> nodes;
    std::unordered_set<const ggml_tensor *> in_piece;
    reader_map readers;                                     // owner -> its readers in the piece
    std::unordered_set<const ggml_tensor *> matmul_inputs;  // packed_key of every MUL_MAT's input
    std::vector<fusion> fusions;
    std::unordered_map<const ggml_tensor *, const fusion *> fused_mm;      // gate/up matmul -> its fusion
    std::unordered_map<const ggml_tensor *, const fusion *> fused_glu;     // GLU -> its fusion
    std::unordered_map<const ggml_tensor *, const ggml_tensor *> res_add;  // ADD -> its matmul
    std::unordered_set<const ggml_tensor *> res_mm;                        // matmuls run by their ADD
    uint64_t key = 0, epoch = 0;  // graph_key and readers_epoch it was made at

    explicit piece_plan(const ggml_cgraph * g) {
        for (int i = 0; i < g->n_nodes; i++) {
            nodes.push_back(g->nodes[i]);
            in_piece.insert(g->nodes[i]);
            if (g->nodes[i]->op == GGML_OP_MUL_MAT) matmul_inputs.insert(packed_key(g->nodes[i]->src[1]));
        }
        readers = index_readers(nodes);
        fusions = find_fusions(nodes, in_piece, readers);
        std::unordered_set<const ggml_tensor *> fused;
        for (const fusion & f : fusions) {
            fused_mm[f.gate_mm] = &f;
            if (f.up_mm) fused_mm[f.up_mm] = &f;
            fused_glu[f.glu] = &f;
            fused.insert(f.gate_mm);
            if (f.up_mm) fused.insert(f.up_mm);
        }
        res_add = find_residuals(nodes, in_piece, fused, readers);
        for (const auto & kv : res_add) res_mm.insert(kv.second);
    }
};

// A 64-bit digest of everything a piece_plan reads from a graph.
uint64_t graph_key(const ggml_cgraph * g) {
    uint64_t h = 0x9E3779B97F4A7C15ull ^ (uint64_t) g->n_nodes;
    auto mix = [&h](uint64_t v) {
        h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
        h *= 0xBF58476D1CE4E5B9ull;
    };
    auto tensor = [&mix](const ggml_tensor * t) {
        mix((uint64_t) (uintptr_t) t);
        mix(((uint64_t) t->op << 32) | ((uint64_t) t->type << 8) | (uint64_t) (uint32_t) t->flags);
        for (int d = 0; d < GGML_MAX_DIMS; d++) {
            mix((uint64_t) t->ne[d]);
            mix((uint64_t) t->nb[d]);
        }
        mix((uint64_t) (uintptr_t) t->data);
        mix((uint64_t) (uintptr_t) t->view_src);
        mix((uint64_t) (uintptr_t) t->buffer);
        mix(t->buffer ? (uint64_t) t->buffer->usage : 0);
    };
    for (int i = 0; i < g->n_nodes; i++) {
        const ggml_tensor * n = g->nodes[i];
        tensor(n);
        for (int j = 0; j < GGML_MAX_OP_PARAMS / 4; j += 2)
            mix(((uint64_t) (uint32_t) n->op_params[j] << 32) | (uint32_t) n->op_params[j + 1]);
        for (int j = 0; j < GGML_MAX_SRC; j++)
            if (n->src[j]) tensor(n->src[j]);
            else mix(j);
    }
    return h;
}

std::shared_ptr<const piece_plan> context::plan_for(const ggml_cgraph * g) {
    const uint64_t key = graph_key(g), epoch = readers_epoch();
    auto it = plans.find(g);
    if (it != plans.end() && it->second->key == key && it->second->epoch == epoch &&
        it->second->nodes.size() == (size_t) g->n_nodes &&
        std::equal(it->second->nodes.begin(), it->second->nodes.end(), g->nodes))
        return it->second;
    auto pl = std::make_shared<piece_plan>(g);
    pl->key = key;
    pl->epoch = epoch;
    if (plans.size() >= PLAN_CACHE) plans.clear();
    plans[g] = pl;
    return pl;
}

struct piece {
    context & ctx;
    const ggml_cgraph * g;
    std::shared_ptr<const piece_plan> plan;
    const std::vector<ggml_tensor *> & nodes;
    const std::unordered_set<const ggml_tensor *> & in_piece;
    std::unordered_map<const ggml_tensor *, void *> staged;   // host inputs copied up
    std::unordered_map<const ggml_tensor *, void *> packed;   // owner -> packed bfp16 activations
    // matmuls run later with their GLU or ADD -> their input packed where they stand
    std::unordered_map<const ggml_tensor *, const void *> deferred_in;
    struct pending_out {
        ggml_tensor * t;
        void * dev;
    };
    std::vector<pending_out> host_outs;  // results of nodes whose memory is on the host
    std::string err;

    const std::unordered_map<const ggml_tensor *, const fusion *> & fused_mm;
    const std::unordered_map<const ggml_tensor *, const fusion *> & fused_glu;
    const std::unordered_map<const ggml_tensor *, const ggml_tensor *> & res_add;
    const std::unordered_set<const ggml_tensor *> & res_mm;
    const reader_map & readers;
    const std::unordered_set<const ggml_tensor *> & matmul_inputs;
    int launches = 0, fused_launches = 0, grouped_launches = 0;  // GEMM launches of the piece
    int residual_launches = 0;

    piece(context & c, const ggml_cgraph * graph, std::shared_ptr<const piece_plan> pl)
        : ctx(c), g(graph), plan(std::move(pl)), nodes(plan->nodes), in_piece(plan->in_piece),
          fused_mm(plan->fused_mm), fused_glu(plan->fused_glu), res_add(plan->res_add), res_mm(plan->res_mm),
          readers(plan->readers), matmul_inputs(plan->matmul_inputs) {}

    bool fail(const std::string & e) {
        err = e;
        return false;
    }

    // A device pointer to t's data (host tensors are copied up once per piece).
    const void * in(const ggml_tensor * t) {
        if (!buffer_is_host(t->buffer)) return t->data;
        auto it = staged.find(t);
        if (it != staged.end()) return it->second;
        const size_t nb = nbytes(t);
        void * p = ctx.ws_alloc(nb);
        if (!p || hipMemcpyAsync(p, t->data, nb, hipMemcpyHostToDevice, ctx.stream) != hipSuccess) return nullptr;
        staged[t] = p;
        return p;
    }
    // Where a node writes: its own memory, or device scratch copied down after.
    void * out(ggml_tensor * t) {
        if (!buffer_is_host(t->buffer)) return t->data;
        void * p = ctx.ws_alloc(nbytes(t));
        if (p) {
            host_outs.push_back({t, p});
            staged[t] = p;
        }
        return p;
    }

    // whether some MUL_MAT of this piece reads t's rows as its input
    bool feeds_matmul(const ggml_tensor * t) const { return matmul_inputs.count(t) != 0; }
    // the only reader of t, inside the piece and out, is `only`
    bool only_reader(const ggml_tensor * t, const ggml_tensor * only) const {
        return !read_by_other(readers, t, only) && !read_outside(t, in_piece);
    }
    // Every reader of t is a matmul of this piece taking t's rows as its
    // input (views in between are free): its packed copy then serves them
    // all and its fp32 values need not be written (src/ggml-zest.cpp:1100-1109).
    bool only_matmuls_read(const ggml_tensor * t) const {
        bool any = false;
        const auto it = readers.find(t);
        if (it != readers.end())
            for (const auto & e : it->second) {
                const ggml_tensor * n = e.first;
                if (is_noop(n)) continue;
                if (n->op != GGML_OP_MUL_MAT || e.second != 1 || packed_key(n->src[1]) != t) return false;
                any = true;
            }
        return any && !read_outside(t, in_piece);
    }
    // packed bfp16 space for a matmul input produced in this piece
    void * packed_for(const ggml_tensor * t, int64_t rows, int64_t K) {
        if (K % 8 != 0 || !feeds_matmul(t)) return nullptr;
        void * p = ctx.ws_alloc(zest_act_bytes(rows, K));
        if (p) packed[t] = p;
        return p;
    }

    bool check(int st, const char * what) {
        if (st == ZEST_OK) return true;
        return fail(std::string(what) + ": " + zest_last_error());
    }

    // Node n is about to write into another tensor's memory (in place): the
    // packed copies of that tensor's rows, whole or a row range, are dropped,
    // so later matmuls pack its new values.
    void invalidate(const ggml_tensor * n) {
        if (!writes_in_place(n)) return;
        const ggml_tensor * o = owner(n);
        for (auto it = packed.begin(); it != packed.end();)
            it = owner(it->first) == o ? packed.erase(it) : std::next(it);
    }

    // The expanded bfp16 operand of matmul input x: the packed copy made with
    // x (a fused norm or GLU), or packed here, once per piece.
    const void * packed_input(const ggml_tensor * x) {
        auto it = packed.find(packed_key(x));
        if (it != packed.end()) return it->second;
        const int64_t M = x->ne[1], K = x->ne[0];
        const void * xd = in(x);
        void * ap = ctx.ws_alloc(zest_act_bytes(M, K));
        if (!xd || !ap) {
            fail("out of device memory for a matmul input");
            return nullptr;
        }
        if (!check(zest_pack_act_x((const float *) xd, M, K, (int64_t) (x->nb[1] / 4), ap, ctx.stream), "pack"))
            return nullptr;
        packed[packed_key(x)] = ap;
        return ap;
    }

    // The input of a matmul run with its GLU or ADD, as packed where the
    // matmul stands (its input may be rewritten in place before then).
    const void * deferred_input(const ggml_tensor * mm) {
        const auto it = deferred_in.find(mm);
        return it != deferred_in.end() ? it->second : packed_input(mm->src[1]);
    }

    // One GEMM submission: GGML_XDNA_FAIL_AFTER fails it; GGML_XDNA_NAN_AFTER
    // then turns its results into NaN (src/xdna-npu.cpp:89-112).
    bool injected_failure(int64_t & s) {
        s = ++g_submissions;
        if (fail_after() >= 0 && s > fail_after()) return fail("an injected failure (GGML_XDNA_FAIL_AFTER)");
        return true;
    }
    bool inject_nan(int64_t s, float * y, int64_t M, int64_t N, int64_t ldc) {
        if (nan_after() < 0 || s <= nan_after()) return true;
        if (y) {
            (void) hipMemsetAsync(y, 0xff, (size_t) ((M - 1) * ldc + N) * 4, ctx.stream);
            return check(zest_check_finite(y, M, N, ldc, ctx.nonfinite, ctx.stream), "finite check");
        }
        return hipMemsetAsync(ctx.nonfinite, 0x01, sizeof(uint32_t), ctx.stream) == hipSuccess ||
               fail("flagging an injected NaN failed");
    }

    // Matmuls on one input, consecutive in the piece: one launch (the
    // reference's group of calls on one input, src/xdna-exec.cpp:509-547).
    bool mul_mats(const std::vector<ggml_tensor *> & ms) {
        const ggml_tensor * x = ms[0]->src[1];
        const int64_t K = x->ne[0], M = x->ne[1];
        for (ggml_tensor * n : ms)
            if (!gemm_matmul(n)) return fail("a matmul this backend does not take");
        const void * ap = packed_input(x);
        if (!ap) return false;
        const void * w[ZEST_GEMM_MAX_GROUP];
        int64_t N[ZEST_GEMM_MAX_GROUP], ldc[ZEST_GEMM_MAX_GROUP];
        float * y[ZEST_GEMM_MAX_GROUP];
        for (size_t i = 0; i < ms.size(); i++) {
            const ggml_tensor * wt = ms[i]->src[0];
            if (!ctx.ensure_weight(wt, ctx.stream, false, err, &w[i])) return false;
            N[i] = wt->ne[1];
            ldc[i] = (int64_t) (ms[i]->nb[1] / 4);
            y[i] = (float *) out(ms[i]);
            if (!y[i]) return fail("out of device memory for a matmul result");
        }
        int64_t s = 0;
        if (!injected_failure(s)) return false;
        if (!check(zest_gemm_group(ap, M, K, (int) ms.size(), w, N, y, ldc, ctx.nonfinite, ctx.stream), "gemm"))
            return false;
        for (size_t i = 0; i < ms.size(); i++)
            if (!inject_nan(s, y[i], M, N[i], ldc[i])) return false;
        ctx.matmuls += (int64_t) ms.size();
        launches++;
        if (ms.size() > 1) grouped_launches++;
        return true;
    }

    // A matmul and the ADD of its result, run where the ADD stands: one GEMM
    // storing acc + the other operand into the ADD's output.
    bool residual_gemm(ggml_tensor * a, const ggml_tensor * n) {
        const ggml_tensor * r = a->src[0] == n ? a->src[1] : a->src[0];
        const ggml_tensor * wt = n->src[0], * x = n->src[1];
        const int64_t K = wt->ne[0], N = wt->ne[1], M = x->ne[1];
        const void * ap = deferred_input(n);
        if (!ap) return false;
        const void * wp = nullptr;
        if (!ctx.ensure_weight(wt, ctx.stream, false, err, &wp)) return false;
        const float * rd = (const float *) in(r);
        float * y = (float *) out(a);
        if (!rd || !y) return fail("out of device memory for a residual add");
        if ((reinterpret_cast<uintptr_t>(rd) & 15) != 0) return fail("a residual whose rows are not 16-byte aligned");
        int64_t s = 0;
        if (!injected_failure(s)) return false;
        const int64_t ldc = (int64_t) (a->nb[1] / 4);
        if (!check(zest_gemm_residual(ap, M, wp, N, K, rd, (int64_t) (r->nb[1] / 4), y, ldc, ctx.nonfinite,
                                      ctx.stream),
                   "gemm+add"))
            return false;
        if (!inject_nan(s, y, M, N, ldc)) return false;
        ctx.matmuls++;
        launches++;
        residual_launches++;
        return true;
    }

    // A fused gate/up GEMM, run where its GLU stands: the GLU's fp32 rows
    // where something other than a matmul reads them, and its packed copy
    // where a matmul of the piece does.
    bool fused_glu_gemm(const fusion & f) {
        const ggml_tensor * x = f.gate_mm->src[1];
        const int64_t M = x->ne[1];
        const void * ap = deferred_input(f.gate_mm);
        if (!ap) return false;
        const void * wp = nullptr;
        if (!ctx.ensure_fused(f, ctx.stream, false, err, &wp)) return false;
        ggml_tensor * n = f.glu;
        void * pk = packed_for(n, M, f.F);
        float * y = pk && only_matmuls_read(n) ? nullptr : (float *) out(n);
        if (!y && !pk) return fail("out of device memory for a fused GLU result");
        int64_t s = 0;
        if (!injected_failure(s)) return false;
        if (!check(zest_gemm_glu(glu_kind_of(param_i32(n, 0)), ap, M, wp, f.F, f.K, pk, y, y ? (int64_t) (n->nb[1] / 4) : 0,
                                 ctx.nonfinite, ctx.stream),
                   "fused gate/up gemm"))
            return false;
        if (!inject_nan(s, y, M, f.F, y ? (int64_t) (n->nb[1] / 4) : 0)) return false;
        ctx.matmuls += f.up_mm ? 2 : 1;
        launches++;
        fused_launches++;
        return true;
    }

    bool rms_norm(ggml_tensor * n, size_t & i) {
        const ggml_tensor * x = n->src[0];
        const float eps = param_f32(n, 0);
        const int64_t d = x->ne[0], rows = nrows(x);
        const void * xd = in(x);
        if (!xd) return fail("out of device memory");
        // RMS_NORM then MUL by a scale row, the norm read by nothing else: one kernel
        ggml_tensor * next = i + 1 < nodes.size() ? nodes[i + 1] : nullptr;
        if (next && next->op == GGML_OP_MUL && next->src[0] == n && exec_supports(next) && only_reader(n, next)) {
            invalidate(next);
            const void * wd = in(next->src[1]);
            void * pk = packed_for(next, rows, d);
            float * y = pk && only_matmuls_read(next) ? nullptr : (float *) out(next);
            if (!wd || (!y && !pk)) return fail("out of device memory");
            i++;
            return check(zest_rms_norm((const float *) xd, rows, d, eps, (const float *) wd, y, pk, ctx.stream),
                         "rms_norm+mul");
        }
        void * pk = packed_for(n, rows, d);
        float * y = pk && only_matmuls_read(n) ? nullptr : (float *) out(n);
        if (!y && !pk) return fail("out of device memory");
        return check(zest_rms_norm((const float *) xd, rows, d, eps, nullptr, y, pk, ctx.stream), "rms_norm");
    }

    bool glu(ggml_tensor * n) {
        const ggml_tensor * a = n->src[0], * b = n->src[1];
        const int kind = glu_kind_of(param_i32(n, 0));
        const int64_t f = n->ne[0], rows = nrows(n);
        const float * ad = (const float *) in(a);
        const float * gd, * ud;
        int64_t sg, su;
        if (b) {
            gd = ad;
            ud = (const float *) in(b);
            sg = (int64_t) (a->nb[1] / 4);
            su = (int64_t) (b->nb[1] / 4);
        } else {
            const bool swapped = param_i32(n, 1) != 0;
            gd = ad ? ad + (swapped ? f : 0) : nullptr;
            ud = ad ? ad + (swapped ? 0 : f) : nullptr;
            sg = su = (int64_t) (a->nb[1] / 4);
        }
        void * pk = packed_for(n, rows, f);
        float * y = pk && only_matmuls_read(n) ? nullptr : (float *) out(n);
        if (!gd || !ud || (!y && !pk) || kind < 0) return fail("bad GLU");
        return check(zest_glu(kind, gd, sg, ud, su, rows, f, y, pk, ctx.stream), "glu");
    }

    bool rope(ggml_tensor * n) {
        const ggml_tensor * x = n->src[0], * pos = n->src[1], * ff = n->src[2];
        const int n_dims = param_i32(n, 1), mode = param_i32(n, 2), n_ctx_orig = param_i32(n, 4);
        const float base = param_f32(n, 5), fs = param_f32(n, 6), ext = param_f32(n, 7), attn = param_f32(n, 8);
        float corr[2];
        rope_corr_dims(n_dims, n_ctx_orig, base, param_f32(n, 9), param_f32(n, 10), corr);
        const void * xd = in(x), * pd = in(pos), * fd = ff ? in(ff) : nullptr;
        float * y = (float *) out(n);
        if (!xd || !pd || (ff && !fd) || !y) return fail("out of device memory");
        return check(zest_rope((const float *) xd, x->ne[2], x->ne[1], x->ne[0], (const int32_t *) pd,
                               (const float *) fd, n_dims, mode, base, fs, ext, attn, corr[0], corr[1], y, ctx.stream),
                     "rope");
    }

    bool run() {
        for (size_t i = 0; i < nodes.size(); i++) {
            ggml_tensor * n = nodes[i];
            if (is_noop(n)) continue;
            invalidate(n);
            bool ok = true;
            switch (n->op) {
                case GGML_OP_MUL_MAT: {
                    if (fused_mm.count(n) || res_mm.count(n)) {
                        // runs with its GLU or ADD; its input is packed now, as it stands here
                        const void * ap = packed_input(n->src[1]);
                        ok = ap != nullptr;
                        deferred_in[n] = ap;
                        break;
                    }
                    // the run of matmuls on the same input that follows
                    std::vector<ggml_tensor *> ms{n};
                    size_t last = i;
                    for (size_t j = i + 1; j < nodes.size() && ms.size() < ZEST_GEMM_MAX_GROUP; j++) {
                        ggml_tensor * m = nodes[j];
                        if (is_noop(m)) continue;
                        if (m->op != GGML_OP_MUL_MAT || fused_mm.count(m) || res_mm.count(m) ||
                            packed_key(m->src[1]) != packed_key(n->src[1]))
                            break;
                        ms.push_back(m);
                        last = j;
                    }
                    ok = mul_mats(ms);
                    i = last;
                    break;
                }
                case GGML_OP_RMS_NORM: ok = rms_norm(n, i); break;
                case GGML_OP_GLU: {
                    auto f = fused_glu.find(n);
                    ok = f != fused_glu.end() ? fused_glu_gemm(*f->second) : glu(n);
                    break;
                }
                case GGML_OP_ROPE: ok = rope(n); break;
                case GGML_OP_MUL: {
                    const void * xd = in(n->src[0]), * wd = in(n->src[1]);
                    float * y = (float *) out(n);
                    ok = xd && wd && y &&
                         check(zest_mul_row((const float *) xd, (const float *) wd, nrows(n), n->ne[0], y, ctx.stream),
                               "mul");
                    break;
                }
                case GGML_OP_ADD: {
                    if (auto rm = res_add.find(n); rm != res_add.end()) {
                        ok = residual_gemm(n, rm->second);
                        break;
                    }
                    const ggml_tensor * a = n->src[0], * b = n->src[1];
                    const void * ad = in(a), * bd = in(b);
                    float * y = (float *) out(n);
                    const int row = !same_shape(a, b);
                    ok = ad && bd && y &&
                         check(zest_add((const float *) ad, (const float *) bd, nrows(n), n->ne[0], row, y, ctx.stream),
                               "add");
                    break;
                }
                case GGML_OP_SCALE: {
                    const void * xd = in(n->src[0]);
                    float * y = (float *) out(n);
                    ok = xd && y &&
                         check(zest_scale((const float *) xd, nelements(n), param_f32(n, 0), param_f32(n, 1), y,
                                          ctx.stream),
                               "scale");
                    break;
                }
                default: return fail(std::string("unsupported op ") + op_name(n->op) + " (" + n->name + ")");
            }
            if (!ok) {
                // the small ops' paths stop at a missing pointer without a reason of their own
                if (err.empty())
                    err = std::string(op_name(n->op)) + " (" + n->name +
                          "): an input or the result has no memory (device scratch exhausted, a host copy failed, "
                          "or a tensor left unallocated)";
                return false;
            }
        }
        for (const pending_out & o : host_outs)
            if (hipMemcpyAsync(o.t->data, o.dev, nbytes(o.t), hipMemcpyDeviceToHost, ctx.stream) != hipSuccess)
                return fail("copying a result to host memory failed");
        // the non-finite flag comes back with the piece's one synchronize
        if (hipMemcpyAsync(ctx.nonfinite_host, ctx.nonfinite, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx.stream) !=
            hipSuccess)
            return fail("reading the non-finite flag failed");
        return true;
    }
};

// ---- the backend ---------------------------------------------------------------

const char * backend_name(ggml_backend_t) { return GGML_XDNA_DEVICE_NAME; }

void backend_free(ggml_backend_t backend) {
    delete (context *) backend->context;
    delete backend;
    budget_context_freed();
}

ggml_status graph_compute(ggml_backend_t backend, ggml_cgraph * cgraph) {
    context & ctx = *(context *) backend->context;
    budget_report();
    say_notes();
    if (mode() != run_mode::gpu || !ctx.stream) {
        log(LOG_ERROR, "graph_compute without a GPU\n");
        return GGML_STATUS_FAILED;
    }
    if (broken()) {
        log(LOG_ERROR, "graph_compute after the GPU path failed\n");
        return GGML_STATUS_FAILED;
    }
    using clock = std::chrono::steady_clock;
    const auto ms = [](clock::time_point a, clock::time_point b) {
        return std::chrono::duration<double, std::milli>(b - a).count();
    };
    const auto t0 = clock::now();
    ctx.ws_reset();
    (void) hipMemsetAsync(ctx.nonfinite, 0, sizeof(uint32_t), ctx.stream);
    piece p(ctx, cgraph, ctx.plan_for(cgraph));  // the piece's fusions, residual adds and readers
    const auto t1 = clock::now();
    bool ok = p.run();     // its launches
    const auto t2 = clock::now();
    const hipError_t se = hipStreamSynchronize(ctx.stream);
    const auto t3 = clock::now();
    if (ok && se != hipSuccess) ok = p.fail(std::string("the GPU reported ") + hipGetErrorString(se));
    if (ok && *ctx.nonfinite_host) ok = p.fail("the results held NaN or infinity");
    ctx.compute_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    ctx.pieces++;
    static const int64_t trace_level = env_int("GGML_XDNA_TRACE", 0);
    if (trace_level >= 2)
        fprintf(stderr,
                "xdna piece: %d nodes, %d GEMM launches (%d fused gate/up, %d grouped, %d with a residual add); "
                "host ms: plan %.3f, launch %.3f, wait %.3f\n",
                (int) p.nodes.size(), p.launches, p.fused_launches, p.grouped_launches, p.residual_launches,
                ms(t0, t1), ms(t1, t2), ms(t2, t3));
    if (trace() && ctx.matmuls >= 196) {
        fprintf(stderr, "xdna times, %lld matmuls in %lld pieces: all %.1f ms; weight copies %lld at load, %lld in pieces\n",
                (long long) ctx.matmuls, (long long) ctx.pieces, ctx.compute_ms, (long long) ctx.built_at_load,
                (long long) ctx.built_in_graph);
        ctx.compute_ms = 0;
        ctx.matmuls = ctx.pieces = 0;
    }
    if (!ok) {
        mark_broken(p.err);
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

// The first time a piece's weights appear (llama.cpp plans graphs at load),
// their cache entries start converting on a stream of their own, so the first
// prompt does not wait for them (src/ggml-zest.cpp:928-965).
// GGML_XDNA_COPY_AT_LOAD=0 leaves them to the first graph_compute.
void graph_optimize(ggml_backend_t backend, ggml_cgraph * cgraph, ggml_backend_graph_optimize_params *) {
    static const bool at_load = env_int("GGML_XDNA_COPY_AT_LOAD", 1) != 0;
    if (!at_load || mode() != run_mode::gpu || broken()) return;
    context & ctx = *(context *) backend->context;
    if (!ctx.loader) return;
    // the fusions graph_compute will make: their interleaved entries instead
    std::vector<ggml_tensor *> nodes(cgraph->nodes, cgraph->nodes + cgraph->n_nodes);
    const std::unordered_set<const ggml_tensor *> in_piece(nodes.begin(), nodes.end());
    std::unordered_set<const ggml_tensor *> fused;
    std::string err;
    for (const fusion & f : find_fusions(nodes, in_piece, index_readers(nodes))) {
        const ggml_tensor * gw = f.gate_mm->src[0], * uw = f.up_mm ? f.up_mm->src[0] : nullptr;
        if (!gw->data || !in_weight_buffer(gw) || (uw && (!uw->data || !in_weight_buffer(uw)))) continue;
        if (!ctx.ensure_fused(f, ctx.loader, true, err)) {
            mark_broken("building a weight-cache entry at load: " + err);
            return;
        }
        fused.insert(f.gate_mm);
        if (f.up_mm) fused.insert(f.up_mm);
    }
    for (const ggml_tensor * n : nodes) {
        if (n->op != GGML_OP_MUL_MAT || fused.count(n)) continue;
        const ggml_tensor * w = n->src[0];
        if (!w->data || !in_weight_buffer(w) || !is_weight(w) || w->ne[0] % 8) continue;
        if (!ctx.ensure_weight(w, ctx.loader, true, err)) {
            mark_broken("building a weight-cache entry at load: " + err);
            return;
        }
    }
}

ggml_guid_t backend_guid() {
    static ggml_guid guid = {0x5a, 0x35, 0x35, 0x58, 0x9d, 0x3a, 0x4e, 0x12, 0xb6, 0x0f, 0x8c, 0x71, 0x2d, 0xe4, 0x90, 0x33};
    return &guid;
}

const ggml_backend_i backend_iface = {
    /* .get_name            = */ backend_name,
    /* .free                = */ backend_free,
    /* .set_tensor_async    = */ nullptr,
    /* .get_tensor_async    = */ nullptr,
    /* .set_tensor_2d_async = */ nullptr,
    /* .get_tensor_2d_async = */ nullptr,
    /* .cpy_tensor_async    = */ nullptr,
    /* .synchronize         = */ nullptr,
    /* .graph_plan_create   = */ nullptr,
    /* .graph_plan_free     = */ nullptr,
    /* .graph_plan_update   = */ nullptr,
    /* .graph_plan_compute  = */ nullptr,
    /* .graph_compute       = */ graph_compute,
    /* .event_record        = */ nullptr,
    /* .event_wait          = */ nullptr,
    /* .graph_optimize      = */ graph_optimize,
};

// ---- the device ------------------------------------------------------------------

const char * dev_name(ggml_backend_dev_t) { return GGML_XDNA_DEVICE_NAME; }
const char * dev_description(ggml_backend_dev_t) { return XDNA_DESCRIPTION; }

// The GPU's own memory: the model's weights live there with their cache.
void dev_memory(ggml_backend_dev_t, size_t * free, size_t * total) {
    *free = *total = 0;
    if (mode() == run_mode::gpu && !plan_only() && hipMemGetInfo(free, total) != hipSuccess) *free = *total = 0;
}
ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_props(ggml_backend_dev_t dev, ggml_backend_dev_props * props) {
    props->name = dev_name(dev);
    props->description = dev_description(dev);
    props->type = dev_type(dev);
    props->device_id = nullptr;
    dev_memory(dev, &props->memory_free, &props->memory_total);
    // graph_compute returns with its results done: no async, no events
    props->caps = {false, false, false, false, false};
}

ggml_backend_t dev_init(ggml_backend_dev_t dev, const char *) {
    if (mode() != run_mode::gpu) return nullptr;
    auto * ctx = new context;
    std::string err;
    if (!plan_only() && !ctx->init(err)) {
        log(LOG_ERROR, "%s\n", err.c_str());
        delete ctx;
        return nullptr;
    }
    budget_context_added();
    return new ggml_backend{backend_guid(), backend_iface, dev, ctx};
}

ggml_backend_buffer_type_t dev_buffer_type(ggml_backend_dev_t) { return our_buft(); }

bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor * op) { return supports_op(op); }

// Our device memory, and host buffers (graph inputs such as positions are read
// from there directly, copied up inside graph_compute).
bool dev_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t buft) {
    return buft == our_buft() || (buft->iface.is_host && buft->iface.is_host(buft));
}

const ggml_backend_device_i device_iface = {
    /* .get_name             = */ dev_name,
    /* .get_description      = */ dev_description,
    /* .get_memory           = */ dev_memory,
    /* .get_type             = */ dev_type,
    /* .get_props            = */ dev_props,
    /* .init_backend         = */ dev_init,
    /* .get_buffer_type      = */ dev_buffer_type,
    /* .get_host_buffer_type = */ nullptr,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    // deliberately no offload_op: that path copies the weights per op
    /* .offload_op           = */ nullptr,
    /* .event_new            = */ nullptr,
    /* .event_free           = */ nullptr,
    /* .event_synchronize    = */ nullptr,
};

// ---- the registry -----------------------------------------------------------------

const char * reg_name(ggml_backend_reg_t) { return GGML_XDNA_NAME; }
size_t reg_device_count(ggml_backend_reg_t) { return mode() == run_mode::off ? 0 : 1; }
ggml_backend_dev_t reg_device_get(ggml_backend_reg_t, size_t index) { return index == 0 ? our_device() : nullptr; }

const ggml_backend_reg_i reg_iface = {
    /* .get_name         = */ reg_name,
    /* .get_device_count = */ reg_device_count,
    /* .get_device       = */ reg_device_get,
    /* .get_proc_address = */ nullptr,
};

ggml_backend_device * our_device() {
    static ggml_backend_device dev = {device_iface, nullptr, nullptr};
    dev.reg = ggml_backend_xdna_reg();
    return &dev;
}

} // namespace
} // namespace zest

extern "C" {

ggml_backend_reg_t ggml_backend_xdna_reg(void) {
    static ggml_backend_reg reg = {GGML_BACKEND_API_VERSION, zest::reg_iface, nullptr};
    return &reg;
}

ggml_backend_reg_t ggml_backend_init(void) { return ggml_backend_xdna_reg(); }

int ggml_backend_score(void) { return 1; }

} // extern "C"

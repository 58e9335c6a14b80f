// Implementation of the ggml stand-in declared in mini_ggml.h (test
// infrastructure). Field conventions follow ggml's public headers: nb[] in
// bytes from the type's block size, views rooted at their owning tensor with
// an accumulated view_offs, op_params as ggml's op constructors fill them.
#include "mini_ggml.h"

#include <dlfcn.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <string>
#include <unordered_set>

#include "zest_oracle.h"

// ---- types and tensors ----------------------------------------------------------

namespace {

struct blk {
    int64_t n;
    size_t bytes;
};
blk blk_of(ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return {1, 4};
        case GGML_TYPE_F16: return {1, 2};
        case GGML_TYPE_BF16: return {1, 2};
        case GGML_TYPE_Q4_0: return {32, 18};
        case GGML_TYPE_Q4_1: return {32, 20};
        case GGML_TYPE_Q5_0: return {32, 22};
        case GGML_TYPE_Q5_1: return {32, 24};
        case GGML_TYPE_Q8_0: return {32, 34};
        case GGML_TYPE_Q2_K: return {256, 84};
        case GGML_TYPE_Q3_K: return {256, 110};
        case GGML_TYPE_Q4_K: return {256, 144};
        case GGML_TYPE_Q5_K: return {256, 176};
        case GGML_TYPE_Q6_K: return {256, 210};
        case GGML_TYPE_Q8_K: return {256, 292};
        case GGML_TYPE_IQ4_NL: return {32, 18};
        case GGML_TYPE_IQ4_XS: return {256, 136};
        case GGML_TYPE_IQ2_XXS: return {256, 66};
        case GGML_TYPE_IQ2_XS: return {256, 74};
        case GGML_TYPE_IQ2_S: return {256, 82};
        case GGML_TYPE_IQ3_XXS: return {256, 98};
        case GGML_TYPE_IQ3_S: return {256, 110};
        case GGML_TYPE_IQ1_S: return {256, 50};
        case GGML_TYPE_IQ1_M: return {256, 56};
        case GGML_TYPE_I32: return {1, 4};
        default: fprintf(stderr, "mini_ggml: type %d not known\n", (int) t); abort();
    }
}

} // namespace

// a graph and the arrays its nodes/leafs point into (the graph is the first
// member, so a ggml_cgraph * converts back)
struct graph_store {
    ggml_cgraph g;
    std::vector<ggml_tensor *> nodes, leafs;
};

struct ggml_context {
    std::deque<ggml_tensor> tensors;
    std::deque<graph_store> graphs;
};

size_t ggml_tensor_overhead() { return sizeof(ggml_tensor) + 32; }
size_t ggml_graph_overhead() { return 4096; }
ggml_context * ggml_init(ggml_init_params) { return new ggml_context; }
void ggml_free(ggml_context * ctx) { delete ctx; }

static void set_strides(ggml_tensor * t) {
    const blk b = blk_of(t->type);
    t->nb[0] = b.bytes;
    t->nb[1] = b.bytes * (size_t) (t->ne[0] / b.n);
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
}

static ggml_tensor * new_tensor(ggml_context * ctx, ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    ctx->tensors.emplace_back();
    ggml_tensor * t = &ctx->tensors.back();
    memset(t, 0, sizeof(*t));
    t->type = type;
    t->ne[0] = ne0;
    t->ne[1] = ne1;
    t->ne[2] = ne2;
    t->ne[3] = ne3;
    set_strides(t);
    t->op = GGML_OP_NONE;
    return t;
}

ggml_tensor * ggml_new_tensor_1d(ggml_context * c, ggml_type t, int64_t a) { return new_tensor(c, t, a, 1, 1, 1); }
ggml_tensor * ggml_new_tensor_2d(ggml_context * c, ggml_type t, int64_t a, int64_t b) { return new_tensor(c, t, a, b, 1, 1); }
ggml_tensor * ggml_new_tensor_3d(ggml_context * c, ggml_type t, int64_t a, int64_t b, int64_t d) {
    return new_tensor(c, t, a, b, d, 1);
}
void ggml_set_name(ggml_tensor * t, const char * name) { snprintf(t->name, sizeof(t->name), "%s", name); }
void ggml_set_input(ggml_tensor * t) { t->flags |= GGML_TENSOR_FLAG_INPUT; }
void ggml_set_output(ggml_tensor * t) { t->flags |= GGML_TENSOR_FLAG_OUTPUT; }

int64_t ggml_nelements(const ggml_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t ggml_nrows(const ggml_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }
size_t ggml_row_size(ggml_type type, int64_t ne) {
    const blk b = blk_of(type);
    return b.bytes * (size_t) (ne / b.n);
}
size_t ggml_nbytes(const ggml_tensor * t) {
    const blk b = blk_of(t->type);
    size_t n = b.n == 1 ? b.bytes : (size_t) (t->ne[0] / b.n) * t->nb[0];
    for (int i = b.n == 1 ? 0 : 1; i < GGML_MAX_DIMS; i++) n += (size_t) (t->ne[i] - 1) * t->nb[i];
    return n;
}

// ---- ops ------------------------------------------------------------------------

static ggml_tensor * op_result(ggml_context * ctx, ggml_op op, ggml_type type, const int64_t ne[4]) {
    ggml_tensor * t = new_tensor(ctx, type, ne[0], ne[1], ne[2], ne[3]);
    t->op = op;
    return t;
}

static ggml_tensor * view_of(ggml_context * ctx, ggml_tensor * a, ggml_op op, size_t offset) {
    ggml_tensor * t = new_tensor(ctx, a->type, 1, 1, 1, 1);
    t->op = op;
    t->src[0] = a;
    t->view_src = a->view_src ? a->view_src : a;
    t->view_offs = offset + (a->view_src ? a->view_offs : 0);
    snprintf(t->name, sizeof(t->name), "%.50s (view)", a->name);
    return t;
}

ggml_tensor * ggml_view_2d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) {
    ggml_tensor * t = view_of(ctx, a, GGML_OP_VIEW, offset);
    t->ne[0] = ne0;
    t->ne[1] = ne1;
    t->nb[0] = a->nb[0];
    t->nb[1] = nb1;
    t->nb[2] = t->nb[3] = nb1 * (size_t) ne1;
    memcpy(t->op_params, &offset, sizeof(offset));
    return t;
}

ggml_tensor * ggml_reshape_2d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1) {
    ggml_tensor * t = view_of(ctx, a, GGML_OP_RESHAPE, 0);
    t->ne[0] = ne0;
    t->ne[1] = ne1;
    set_strides(t);
    return t;
}

ggml_tensor * ggml_reshape_3d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2) {
    ggml_tensor * t = view_of(ctx, a, GGML_OP_RESHAPE, 0);
    t->ne[0] = ne0;
    t->ne[1] = ne1;
    t->ne[2] = ne2;
    set_strides(t);
    return t;
}

ggml_tensor * ggml_mul_mat(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    const int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    ggml_tensor * t = op_result(ctx, GGML_OP_MUL_MAT, GGML_TYPE_F32, ne);
    t->src[0] = a;
    t->src[1] = b;
    return t;
}

ggml_tensor * ggml_mul_mat_id(ggml_context * ctx, ggml_tensor * as, ggml_tensor * b, ggml_tensor * ids) {
    const int64_t ne[4] = {as->ne[1], ids->ne[0], b->ne[2], 1};
    ggml_tensor * t = op_result(ctx, GGML_OP_MUL_MAT_ID, GGML_TYPE_F32, ne);
    t->src[0] = as;
    t->src[1] = b;
    t->src[2] = ids;
    return t;
}

static ggml_tensor * binary(ggml_context * ctx, ggml_op op, ggml_tensor * a, ggml_tensor * b) {
    ggml_tensor * t = op_result(ctx, op, a->type, a->ne);
    t->src[0] = a;
    t->src[1] = b;
    return t;
}
ggml_tensor * ggml_add(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) { return binary(ctx, GGML_OP_ADD, a, b); }
ggml_tensor * ggml_mul(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) { return binary(ctx, GGML_OP_MUL, a, b); }

static void set_f32(ggml_tensor * t, int i, float v) { memcpy(&t->op_params[i], &v, sizeof(v)); }

ggml_tensor * ggml_scale_bias(ggml_context * ctx, ggml_tensor * a, float s, float b) {
    ggml_tensor * t = op_result(ctx, GGML_OP_SCALE, a->type, a->ne);
    t->src[0] = a;
    set_f32(t, 0, s);
    set_f32(t, 1, b);
    return t;
}
ggml_tensor * ggml_scale(ggml_context * ctx, ggml_tensor * a, float s) { return ggml_scale_bias(ctx, a, s, 0.0f); }

// a whole-tensor view of `a` computed by `op` (its result lands in a's memory)
static ggml_tensor * in_place(ggml_context * ctx, ggml_op op, ggml_tensor * a, ggml_tensor * b) {
    ggml_tensor * t = view_of(ctx, a, op, 0);
    memcpy(t->ne, a->ne, sizeof(t->ne));
    memcpy(t->nb, a->nb, sizeof(t->nb));
    t->src[1] = b;
    return t;
}
ggml_tensor * ggml_add_inplace(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    return in_place(ctx, GGML_OP_ADD, a, b);
}
ggml_tensor * ggml_mul_inplace(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    return in_place(ctx, GGML_OP_MUL, a, b);
}
ggml_tensor * ggml_scale_inplace(ggml_context * ctx, ggml_tensor * a, float s) {
    ggml_tensor * t = in_place(ctx, GGML_OP_SCALE, a, nullptr);
    set_f32(t, 0, s);
    set_f32(t, 1, 0.0f);
    return t;
}

ggml_tensor * ggml_rms_norm(ggml_context * ctx, ggml_tensor * a, float eps) {
    ggml_tensor * t = op_result(ctx, GGML_OP_RMS_NORM, a->type, a->ne);
    t->src[0] = a;
    set_f32(t, 0, eps);
    return t;
}

ggml_tensor * ggml_get_rows(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    const int64_t ne[4] = {a->ne[0], b->ne[0], 1, 1};
    ggml_tensor * t = op_result(ctx, GGML_OP_GET_ROWS, GGML_TYPE_F32, ne);
    t->src[0] = a;
    t->src[1] = b;
    return t;
}

ggml_tensor * ggml_glu(ggml_context * ctx, ggml_tensor * a, ggml_glu_op op, bool swapped) {
    const int64_t ne[4] = {a->ne[0] / 2, a->ne[1], a->ne[2], a->ne[3]};
    ggml_tensor * t = op_result(ctx, GGML_OP_GLU, a->type, ne);
    t->src[0] = a;
    t->op_params[0] = (int32_t) op;
    t->op_params[1] = swapped ? 1 : 0;
    return t;
}

ggml_tensor * ggml_glu_split(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, ggml_glu_op op) {
    ggml_tensor * t = op_result(ctx, GGML_OP_GLU, a->type, a->ne);
    t->src[0] = a;
    t->src[1] = b;
    t->op_params[0] = (int32_t) op;
    t->op_params[1] = 0;
    return t;
}

ggml_tensor * ggml_rope_ext(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, ggml_tensor * c, int n_dims, int mode,
                            int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                            float beta_fast, float beta_slow) {
    ggml_tensor * t = op_result(ctx, GGML_OP_ROPE, a->type, a->ne);
    t->src[0] = a;
    t->src[1] = b;
    t->src[2] = c;
    t->op_params[1] = n_dims;
    t->op_params[2] = mode;
    t->op_params[4] = n_ctx_orig;
    set_f32(t, 5, freq_base);
    set_f32(t, 6, freq_scale);
    set_f32(t, 7, ext_factor);
    set_f32(t, 8, attn_factor);
    set_f32(t, 9, beta_fast);
    set_f32(t, 10, beta_slow);
    return t;
}

// ---- graphs ------------------------------------------------------------------------

ggml_cgraph * ggml_new_graph(ggml_context * ctx) {
    ctx->graphs.emplace_back();
    graph_store & st = ctx->graphs.back();
    memset(&st.g, 0, sizeof(st.g));
    return &st.g;
}

static void visit(ggml_tensor * t, std::unordered_set<ggml_tensor *> & seen, graph_store & st) {
    if (!t || seen.count(t)) return;
    seen.insert(t);
    for (int j = 0; j < GGML_MAX_SRC; j++) visit(t->src[j], seen, st);
    (t->op == GGML_OP_NONE ? st.leafs : st.nodes).push_back(t);
}

void ggml_build_forward_expand(ggml_cgraph * g, ggml_tensor * t) {
    graph_store & st = *reinterpret_cast<graph_store *>(g);
    std::unordered_set<ggml_tensor *> seen(st.nodes.begin(), st.nodes.end());
    seen.insert(st.leafs.begin(), st.leafs.end());
    visit(t, seen, st);
    g->nodes = st.nodes.data();
    g->leafs = st.leafs.data();
    g->n_nodes = (int) st.nodes.size();
    g->n_leafs = (int) st.leafs.size();
    g->size = (int) (st.nodes.size() + st.leafs.size());
}

// ---- quantisers ----------------------------------------------------------------------

size_t ggml_quantize_chunk(ggml_type type, const float * src, void * dst, int64_t start, int64_t nrows,
                           int64_t n_per_row, const float *) {
    const size_t rb = ggml_row_size(type, n_per_row);
    uint8_t * out = (uint8_t *) dst + (size_t) (start / n_per_row) * rb;
    for (int64_t r = 0; r < nrows; r++) {
        const float * x = src + start + r * n_per_row;
        uint8_t * o = out + (size_t) r * rb;
        if (orc_quantize_row((int) type, x, o, n_per_row) != 0) {
            fprintf(stderr, "mini_ggml: no quantiser for type %d\n", (int) type);
            abort();
        }
    }
    return rb * (size_t) nrows;
}

void ggml_dequantize_row(ggml_type type, const void * src, float * dst, int64_t k) {
    orc_dequant_row((int) type, src, dst, k);
}

// ---- the host ("CPU") device: memory only ----------------------------------------------

namespace {

const char * host_buft_name(ggml_backend_buffer_type_t) { return "CPU"; }
void host_free(ggml_backend_buffer_t b) { free(b->context); }
void * host_base(ggml_backend_buffer_t b) { return b->context; }
void host_memset(ggml_backend_buffer_t, ggml_tensor * t, uint8_t v, size_t off, size_t n) {
    memset((char *) t->data + off, v, n);
}
void host_set(ggml_backend_buffer_t, ggml_tensor * t, const void * d, size_t off, size_t n) {
    memcpy((char *) t->data + off, d, n);
}
void host_get(ggml_backend_buffer_t, const ggml_tensor * t, void * d, size_t off, size_t n) {
    memcpy(d, (const char *) t->data + off, n);
}
void host_clear(ggml_backend_buffer_t b, uint8_t v) { memset(b->context, v, b->size); }
const ggml_backend_buffer_i host_buffer_iface = {host_free, host_base,  nullptr,    host_memset, host_set,
                                                 host_get,  nullptr,    host_clear, nullptr};
ggml_backend_buffer_t host_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    void * p = aligned_alloc(256, (size + 255) / 256 * 256 + 256);
    return new ggml_backend_buffer{host_buffer_iface, buft, p, size, GGML_BACKEND_BUFFER_USAGE_ANY};
}
size_t host_align(ggml_backend_buffer_type_t) { return 64; }
size_t host_max(ggml_backend_buffer_type_t) { return SIZE_MAX; }
bool host_is_host(ggml_backend_buffer_type_t) { return true; }
ggml_backend_buffer_type host_buft = {{host_buft_name, host_alloc, host_align, host_max, nullptr, host_is_host},
                                      nullptr, nullptr};

const char * host_dev_name(ggml_backend_dev_t) { return "CPU"; }
enum ggml_backend_dev_type host_dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_CPU; }
ggml_backend_buffer_type_t host_dev_buft(ggml_backend_dev_t) { return &host_buft; }
void host_dev_memory(ggml_backend_dev_t, size_t * f, size_t * t) { *f = *t = 0; }
ggml_backend_device host_dev = {{host_dev_name, host_dev_name, host_dev_memory, host_dev_type, nullptr, nullptr,
                                 host_dev_buft, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr},
                                nullptr, nullptr};

std::vector<ggml_backend_dev_t> g_devices;

} // namespace

// ---- ggml-backend -----------------------------------------------------------------------

void ggml_backend_load_all() {
    static bool done = false;
    if (done) return;
    done = true;
    const char * path = getenv("GGML_BACKEND_PATH");
    if (path && *path) {
        void * h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
        if (!h) {
            fprintf(stderr, "mini_ggml: cannot load %s: %s\n", path, dlerror());
        } else {
            auto score = (int (*)()) dlsym(h, "ggml_backend_score");
            auto init = (ggml_backend_reg_t (*)()) dlsym(h, "ggml_backend_init");
            if (!init) {
                fprintf(stderr, "mini_ggml: %s has no ggml_backend_init\n", path);
            } else if (score && score() == 0) {
                fprintf(stderr, "mini_ggml: %s scores 0, not loaded\n", path);
            } else {
                ggml_backend_reg_t reg = init();
                if (!reg || reg->api_version != GGML_BACKEND_API_VERSION) {
                    fprintf(stderr, "mini_ggml: %s: wrong API version\n", path);
                } else {
                    for (size_t i = 0; i < reg->iface.get_device_count(reg); i++)
                        g_devices.push_back(reg->iface.get_device(reg, i));
                }
            }
        }
    }
    g_devices.push_back(&host_dev);
}

size_t ggml_backend_dev_count() { return g_devices.size(); }
ggml_backend_dev_t ggml_backend_dev_get(size_t i) { return i < g_devices.size() ? g_devices[i] : nullptr; }
ggml_backend_dev_t ggml_backend_dev_by_name(const char * name) {
    for (ggml_backend_dev_t d : g_devices)
        if (strcmp(d->iface.get_name(d), name) == 0) return d;
    return nullptr;
}
ggml_backend_dev_t ggml_backend_dev_by_type(enum ggml_backend_dev_type type) {
    for (ggml_backend_dev_t d : g_devices)
        if (d->iface.get_type(d) == type) return d;
    return nullptr;
}
const char * ggml_backend_dev_name(ggml_backend_dev_t d) { return d->iface.get_name(d); }
enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t d) { return d->iface.get_type(d); }
ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t d) { return d->iface.get_buffer_type(d); }
bool ggml_backend_dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t b) {
    return d->iface.supports_buft && d->iface.supports_buft(d, b);
}
bool ggml_backend_dev_supports_op(ggml_backend_dev_t d, const ggml_tensor * op) {
    return d->iface.supports_op && d->iface.supports_op(d, op);
}
bool ggml_backend_dev_offload_op(ggml_backend_dev_t d, const ggml_tensor * op) {
    return d->iface.offload_op && d->iface.offload_op(d, op);
}
void ggml_backend_dev_memory(ggml_backend_dev_t d, size_t * f, size_t * t) { d->iface.get_memory(d, f, t); }
void ggml_backend_dev_get_props(ggml_backend_dev_t d, ggml_backend_dev_props * p) {
    memset(p, 0, sizeof(*p));
    d->iface.get_props(d, p);
}
ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t d, const char * params) {
    return d->iface.init_backend ? d->iface.init_backend(d, params) : nullptr;
}
void ggml_backend_free(ggml_backend_t b) {
    if (b) b->iface.free(b);
}
ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t b) {
    return ggml_backend_dev_buffer_type(b->device);
}
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t b) { return b->iface.is_host && b->iface.is_host(b); }

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(ggml_context * ctx, ggml_backend_buffer_type_t buft) {
    const size_t align = buft->iface.get_alignment(buft);
    size_t total = 0;
    for (ggml_tensor & t : ctx->tensors)
        if (!t.view_src && !t.data) total += (ggml_nbytes(&t) + align - 1) / align * align;
    if (total == 0) return nullptr;
    ggml_backend_buffer_t buf = buft->iface.alloc_buffer(buft, total);
    if (!buf) return nullptr;
    char * base = (char *) buf->iface.get_base(buf);
    size_t off = 0;
    for (ggml_tensor & t : ctx->tensors)
        if (!t.view_src && !t.data) {
            t.data = base + off;
            t.buffer = buf;
            if (buf->iface.init_tensor) buf->iface.init_tensor(buf, &t);
            off += (ggml_nbytes(&t) + align - 1) / align * align;
        }
    // views, of this buffer's tensors or of any tensor already allocated (as
    // ggml_backend_view_init does)
    for (ggml_tensor & t : ctx->tensors)
        if (t.view_src && t.view_src->buffer && !t.data) {
            t.data = (char *) t.view_src->data + t.view_offs;
            t.buffer = t.view_src->buffer;
        }
    return buf;
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(ggml_context * ctx, ggml_backend_t backend) {
    return ggml_backend_alloc_ctx_tensors_from_buft(ctx, ggml_backend_get_default_buffer_type(backend));
}
void ggml_backend_buffer_set_usage(ggml_backend_buffer_t b, ggml_backend_buffer_usage u) { b->usage = u; }
// as ggml does: the buffer type's free_buffer, then the object itself
void ggml_backend_buffer_free(ggml_backend_buffer_t b) {
    if (!b) return;
    if (b->iface.free_buffer) b->iface.free_buffer(b);
    delete b;
}
void ggml_backend_tensor_set(ggml_tensor * t, const void * d, size_t off, size_t n) {
    t->buffer->iface.set_tensor(t->buffer, t, d, off, n);
}
void ggml_backend_tensor_get(const ggml_tensor * t, void * d, size_t off, size_t n) {
    t->buffer->iface.get_tensor(t->buffer, t, d, off, n);
}

ggml_status ggml_backend_graph_compute(ggml_backend_t b, ggml_cgraph * gf) {
    const ggml_status s = b->iface.graph_compute(b, gf);
    if (b->iface.synchronize) b->iface.synchronize(b);
    return s;
}

void ggml_backend_plan_graph(ggml_backend_t b, ggml_cgraph * gf) {
    for (int i = 0; i < gf->n_nodes; i++) ggml_backend_dev_supports_op(b->device, gf->nodes[i]);
    if (b->iface.graph_optimize) b->iface.graph_optimize(b, gf, nullptr);
}

// ---- helpers ----------------------------------------------------------------------------------

float test_rng::normal(float mean, float sd) {
    if (have) {
        have = false;
        return mean + sd * (float) spare;
    }
    double u1 = uniform(), u2 = uniform();
    if (u1 < 1e-300) u1 = 1e-300;
    const double r = std::sqrt(-2.0 * std::log(u1)), th = 2.0 * M_PI * u2;
    spare = r * std::sin(th);
    have = true;
    return mean + sd * (float) (r * std::cos(th));
}

static std::atomic<int> g_failures{0};  // programs may check from several threads
int test_check(bool ok, const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    printf("%s %s\n", ok ? "PASS" : "FAIL", buf);
    fflush(stdout);
    if (!ok) g_failures++;
    return ok;
}
int test_failures() { return g_failures; }

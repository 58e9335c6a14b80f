// Helpers over ggml tensors for the backend, computed from the tensor fields
// and the public GGUF block sizes, so the add-on needs nothing from
// ggml-base at run time; plus the environment settings and logging.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "ggml-zest.h"

namespace zest {

// --- settings: environment variables, an empty value counts as unset
// (src/xdna-env.h:9-17)
inline const char * env(const char * name) {
    const char * s = getenv(name);
    return s && *s ? s : nullptr;
}
inline int64_t env_int(const char * name, int64_t def) {
    const char * s = env(name);
    return s ? atoll(s) : def;
}

enum log_level { LOG_INFO, LOG_WARN, LOG_ERROR };
void log(log_level level, const char * fmt, ...) __attribute__((format(printf, 2, 3)));

// --- types: (block size, bytes per block) of the GGUF formats
struct type_traits {
    int64_t blck;
    size_t size;
};
inline type_traits traits_of(int type) {
    switch (type) {
        case GGML_TYPE_F32: return {1, 4};
        case GGML_TYPE_F16: return {1, 2};
        case GGML_TYPE_BF16: return {1, 2};
        case GGML_TYPE_Q4_0: return {32, 18};
        case GGML_TYPE_Q4_1: return {32, 20};
        case GGML_TYPE_Q5_0: return {32, 22};
        case GGML_TYPE_Q5_1: return {32, 24};
        case GGML_TYPE_Q8_0: return {32, 34};
        case GGML_TYPE_Q8_1: return {32, 36};
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
        case GGML_TYPE_I8: return {1, 1};
        case GGML_TYPE_I16: return {1, 2};
        case GGML_TYPE_I32: return {1, 4};
        case GGML_TYPE_I64: return {1, 8};
        case GGML_TYPE_F64: return {1, 8};
        default: return {0, 0};
    }
}

// weight types the converter turns into bfp16 (zest_convert_weight): the
// reference takes any type with a to_float (src/ggml-zest.cpp:1066-1072);
// these are GGUF's float and block types and the two 4-bit non-uniform grid
// types (not the codebook IQ types, whose grids are ggml-base tables, Q8_1 or
// Q8_K)
inline bool convertible(int type) {
    switch (type) {
        case GGML_TYPE_F32:
        case GGML_TYPE_F16:
        case GGML_TYPE_BF16:
        case GGML_TYPE_Q4_0:
        case GGML_TYPE_Q4_1:
        case GGML_TYPE_Q5_0:
        case GGML_TYPE_Q5_1:
        case GGML_TYPE_Q8_0:
        case GGML_TYPE_Q2_K:
        case GGML_TYPE_Q3_K:
        case GGML_TYPE_Q4_K:
        case GGML_TYPE_Q5_K:
        case GGML_TYPE_Q6_K:
        case GGML_TYPE_IQ4_NL:
        case GGML_TYPE_IQ4_XS: return true;
        default: return false;
    }
}

inline int64_t nelements(const ggml_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
inline int64_t nrows(const ggml_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

inline size_t row_size(int type, int64_t ne0) {
    const type_traits tr = traits_of(type);
    return tr.blck ? tr.size * (size_t) (ne0 / tr.blck) : 0;
}

// bytes spanned by a tensor, as ggml counts them (last element's end)
inline size_t nbytes(const ggml_tensor * t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] <= 0) return 0;
    const type_traits tr = traits_of(t->type);
    if (!tr.blck) return 0;
    size_t n = tr.blck == 1 ? tr.size : (size_t) (t->ne[0] * (int64_t) t->nb[0] / tr.blck);
    for (int i = tr.blck == 1 ? 0 : 1; i < GGML_MAX_DIMS; i++) n += (size_t) (t->ne[i] - 1) * t->nb[i];
    return n;
}

// rows packed back to back, no gaps (dimensions of extent 1 are skipped)
inline bool is_contiguous(const ggml_tensor * t) {
    const type_traits tr = traits_of(t->type);
    if (!tr.blck) return false;
    size_t next = tr.size;
    if (t->ne[0] != tr.blck && t->nb[0] != next) return false;
    next *= (size_t) (t->ne[0] / tr.blck);
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] == 1) continue;
        if (t->nb[i] != next) return false;
        next *= (size_t) t->ne[i];
    }
    return true;
}

inline bool same_shape(const ggml_tensor * a, const ggml_tensor * b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}

inline bool is_noop(const ggml_tensor * n) {
    return n->op == GGML_OP_NONE || n->op == GGML_OP_RESHAPE || n->op == GGML_OP_VIEW || n->op == GGML_OP_PERMUTE ||
           n->op == GGML_OP_TRANSPOSE;
}

inline const ggml_tensor * owner(const ggml_tensor * t) {
    while (t->view_src) t = t->view_src;
    return t;
}

inline int32_t param_i32(const ggml_tensor * t, int i) { return t->op_params[i]; }
inline float param_f32(const ggml_tensor * t, int i) {
    float v;
    memcpy(&v, &t->op_params[i], sizeof(v));
    return v;
}

inline bool buffer_is_host(const ggml_backend_buffer * b) {
    return b && b->buft && b->buft->iface.is_host && b->buft->iface.is_host(b->buft);
}
inline bool in_weight_buffer(const ggml_tensor * t) {
    return t->buffer && t->buffer->usage == GGML_BACKEND_BUFFER_USAGE_WEIGHTS;
}

// Rows are prompt tokens, along a tensor's last dimension in use
// (src/xdna-exec.cpp:29-33).
inline int64_t tokens_of(const ggml_tensor * t) {
    return t->ne[3] > 1 ? t->ne[3] : t->ne[2] > 1 ? t->ne[2] : t->ne[1];
}

const char * op_name(int op);

} // namespace zest

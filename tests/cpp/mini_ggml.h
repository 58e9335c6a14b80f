// A small stand-in for the parts of ggml's public API that the reference's
// backend tests call (tests/test-dispatch-gate.cpp, test-memory-budget.cpp,
// test-mul-mat.cpp, test-host-ops.cpp, test-safe-start.cpp of
// Cyronius/ggml-xdna): tensor and graph construction with ggml's field
// conventions (ne/nb, op_params, views, flags), and the ggml-backend calls that
// load an add-on from GGML_BACKEND_PATH and drive its iface tables. llama.cpp
// itself is not available here; these tests reach libggml-zest.so only through
// its exported ggml_backend_init, exactly as ggml_backend_load does.
//
// Test infrastructure: the weight dequantiser and the CPU references come from
// the oracle library (oracle/zest_oracle.h).
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

#include "ggml_abi.h"

struct ggml_context;
struct ggml_init_params {
    size_t mem_size;
    void * mem_buffer;
    bool no_alloc;
};

size_t ggml_tensor_overhead();
size_t ggml_graph_overhead();
ggml_context * ggml_init(ggml_init_params params);
void ggml_free(ggml_context * ctx);

ggml_tensor * ggml_new_tensor_1d(ggml_context * ctx, ggml_type type, int64_t ne0);
ggml_tensor * ggml_new_tensor_2d(ggml_context * ctx, ggml_type type, int64_t ne0, int64_t ne1);
ggml_tensor * ggml_new_tensor_3d(ggml_context * ctx, ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2);
void ggml_set_name(ggml_tensor * t, const char * name);
void ggml_set_input(ggml_tensor * t);
void ggml_set_output(ggml_tensor * t);

int64_t ggml_nelements(const ggml_tensor * t);
int64_t ggml_nrows(const ggml_tensor * t);
size_t ggml_nbytes(const ggml_tensor * t);
size_t ggml_row_size(ggml_type type, int64_t ne);

// ops, with ggml's op_params conventions
ggml_tensor * ggml_view_2d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset);
ggml_tensor * ggml_reshape_2d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1);
ggml_tensor * ggml_reshape_3d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2);
ggml_tensor * ggml_mul_mat(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b);
ggml_tensor * ggml_mul_mat_id(ggml_context * ctx, ggml_tensor * as, ggml_tensor * b, ggml_tensor * ids);
ggml_tensor * ggml_add(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b);
ggml_tensor * ggml_mul(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b);
ggml_tensor * ggml_scale(ggml_context * ctx, ggml_tensor * a, float s);
ggml_tensor * ggml_scale_bias(ggml_context * ctx, ggml_tensor * a, float s, float b);
// in place, as ggml's *_inplace ops: the result is a view of `a` and the op writes a's memory
ggml_tensor * ggml_add_inplace(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b);
ggml_tensor * ggml_mul_inplace(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b);
ggml_tensor * ggml_scale_inplace(ggml_context * ctx, ggml_tensor * a, float s);
ggml_tensor * ggml_rms_norm(ggml_context * ctx, ggml_tensor * a, float eps);
ggml_tensor * ggml_get_rows(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b);
ggml_tensor * ggml_glu(ggml_context * ctx, ggml_tensor * a, ggml_glu_op op, bool swapped);
ggml_tensor * ggml_glu_split(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, ggml_glu_op op);
inline ggml_tensor * ggml_swiglu(ggml_context * c, ggml_tensor * a) { return ggml_glu(c, a, GGML_GLU_OP_SWIGLU, false); }
inline ggml_tensor * ggml_swiglu_swapped(ggml_context * c, ggml_tensor * a) { return ggml_glu(c, a, GGML_GLU_OP_SWIGLU, true); }
inline ggml_tensor * ggml_geglu(ggml_context * c, ggml_tensor * a) { return ggml_glu(c, a, GGML_GLU_OP_GEGLU, false); }
inline ggml_tensor * ggml_geglu_erf(ggml_context * c, ggml_tensor * a) { return ggml_glu(c, a, GGML_GLU_OP_GEGLU_ERF, false); }
inline ggml_tensor * ggml_swiglu_split(ggml_context * c, ggml_tensor * a, ggml_tensor * b) { return ggml_glu_split(c, a, b, GGML_GLU_OP_SWIGLU); }
inline ggml_tensor * ggml_geglu_split(ggml_context * c, ggml_tensor * a, ggml_tensor * b) { return ggml_glu_split(c, a, b, GGML_GLU_OP_GEGLU); }
inline ggml_tensor * ggml_geglu_erf_split(ggml_context * c, ggml_tensor * a, ggml_tensor * b) { return ggml_glu_split(c, a, b, GGML_GLU_OP_GEGLU_ERF); }
inline ggml_tensor * ggml_geglu_quick_split(ggml_context * c, ggml_tensor * a, ggml_tensor * b) { return ggml_glu_split(c, a, b, GGML_GLU_OP_GEGLU_QUICK); }
inline ggml_tensor * ggml_reglu_split(ggml_context * c, ggml_tensor * a, ggml_tensor * b) { return ggml_glu_split(c, a, b, GGML_GLU_OP_REGLU); }
ggml_tensor * ggml_rope_ext(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, ggml_tensor * c, int n_dims, int mode,
                            int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                            float beta_fast, float beta_slow);

ggml_cgraph * ggml_new_graph(ggml_context * ctx);
void ggml_build_forward_expand(ggml_cgraph * gf, ggml_tensor * t);

// GGUF quantisers for synthetic weights (valid blocks, not ggml's search):
// F32, Q8_0 (d = absmax/127), Q4_K (per-sub-block min/scale, 6-bit codes)
size_t ggml_quantize_chunk(ggml_type type, const float * src, void * dst, int64_t start, int64_t nrows,
                           int64_t n_per_row, const float * imatrix);
// one row back to floats (the oracle's dequantiser)
void ggml_dequantize_row(ggml_type type, const void * src, float * dst, int64_t k);

// ---- ggml-backend ---------------------------------------------------------

void ggml_backend_load_all();  // the add-on named by GGML_BACKEND_PATH, plus a host ("CPU") device
size_t ggml_backend_dev_count();
ggml_backend_dev_t ggml_backend_dev_get(size_t i);
ggml_backend_dev_t ggml_backend_dev_by_name(const char * name);
ggml_backend_dev_t ggml_backend_dev_by_type(enum ggml_backend_dev_type type);
const char * ggml_backend_dev_name(ggml_backend_dev_t dev);
enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t dev);
ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t dev);
bool ggml_backend_dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft);
bool ggml_backend_dev_supports_op(ggml_backend_dev_t dev, const ggml_tensor * op);
bool ggml_backend_dev_offload_op(ggml_backend_dev_t dev, const ggml_tensor * op);
void ggml_backend_dev_memory(ggml_backend_dev_t dev, size_t * free, size_t * total);
void ggml_backend_dev_get_props(ggml_backend_dev_t dev, ggml_backend_dev_props * props);
ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t dev, const char * params);
void ggml_backend_free(ggml_backend_t backend);
ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend);
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft);

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(ggml_context * ctx, ggml_backend_buffer_type_t buft);
ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(ggml_context * ctx, ggml_backend_t backend);
void ggml_backend_buffer_set_usage(ggml_backend_buffer_t buf, ggml_backend_buffer_usage usage);
void ggml_backend_buffer_free(ggml_backend_buffer_t buf);
void ggml_backend_tensor_set(ggml_tensor * t, const void * data, size_t offset, size_t size);
void ggml_backend_tensor_get(const ggml_tensor * t, void * data, size_t offset, size_t size);

ggml_status ggml_backend_graph_compute(ggml_backend_t backend, ggml_cgraph * gf);
// What ggml_backend_sched does before running a split on a backend: asks
// supports_op about every node (the add-on's reader tracking sees the graph)
// and lets the backend optimise the graph (load-time weight conversion).
void ggml_backend_plan_graph(ggml_backend_t backend, ggml_cgraph * gf);

// ---- test helpers ------------------------------------------------------------

// mt19937_64 with a Box-Muller normal of our own (std::normal_distribution is
// implementation-defined)
struct test_rng {
    std::mt19937_64 eng;
    bool have = false;
    double spare = 0;
    explicit test_rng(uint64_t seed) : eng(seed) {}
    double uniform() { return (double) (eng() >> 11) * 0x1.0p-53; }  // [0, 1)
    float normal(float mean, float sd);
};

int test_check(bool ok, const char * fmt, ...) __attribute__((format(printf, 2, 3)));
int test_failures();

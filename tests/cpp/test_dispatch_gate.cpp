// What the backend takes lives in supports_op, the device type and the buffer
// type: the three things ggml's scheduler reads to decide. Checked directly,
// as the reference's tests/test-dispatch-gate.cpp does, with
// GGML_XDNA_MIN_BATCH and GGML_XDNA_MIN_MFLOP at their defaults. Runs on the
// GPU, or without one under GGML_XDNA_PLAN_ONLY=1 (planning only).
#include <cstdio>
#include <cstdlib>

#include "mini_ggml.h"

static ggml_tensor * make_mul_mat(ggml_context * ctx, ggml_type wtype, int64_t k, int64_t n, int64_t batch) {
    ggml_tensor * a = ggml_new_tensor_2d(ctx, wtype, k, n);
    ggml_tensor * b = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, batch);
    return ggml_mul_mat(ctx, a, b);
}

int main() {
    ggml_backend_load_all();
    ggml_backend_dev_t dev = ggml_backend_dev_by_name("XDNA0");
    if (!dev) {
        fprintf(stderr, "XDNA0 device not registered - is GGML_BACKEND_PATH set, and is there a GPU?\n");
        return 2;
    }
    const char * po = getenv("GGML_XDNA_PLAN_ONLY");
    const bool plan_only = po && *po && po[0] != '0';

    test_check(ggml_backend_dev_type(dev) == GGML_BACKEND_DEVICE_TYPE_GPU,
               "device registers as a GPU (the model's memory is on it)");
    ggml_backend_buffer_type_t own = ggml_backend_dev_buffer_type(dev);
    test_check(own && !ggml_backend_buft_is_host(own), "its buffer type is its own device memory");
    test_check(ggml_backend_dev_supports_buft(dev, own), "it reads its own buffers");
    ggml_backend_dev_t cpu = ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU);
    test_check(cpu && ggml_backend_dev_supports_buft(dev, ggml_backend_dev_buffer_type(cpu)),
               "it reads host buffers (graph inputs such as positions)");
    size_t free = 1, total = 0;
    ggml_backend_dev_memory(dev, &free, &total);
    if (plan_only)
        test_check(free == 0 && total == 0, "planning only: no memory reported");
    else
        test_check(total > 0 && free > 0 && free <= total, "reports the GPU's HBM (free %.1f of %.1f GB)", free / 1e9,
                   total / 1e9);
    ggml_backend_dev_props props;
    ggml_backend_dev_get_props(dev, &props);
    test_check(!props.caps.async && !props.caps.events, "no async or events: graph_compute returns with results done");

    ggml_init_params ip = {ggml_tensor_overhead() * 256, nullptr, true};
    ggml_context * ctx = ggml_init(ip);
    const int64_t k = 2048, n = 2048;

    test_check(!ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_K, k, n, 1)),
               "batch 1 (reply generation) is not claimed");
    test_check(!ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_K, k, n, 512)),
               "batch 512 (llama.cpp's default chunk) is not claimed");
    test_check(!ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_K, k, n, 1023)),
               "batch 1023 is not claimed (below the default threshold of 1024)");
    test_check(ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_K, k, n, 1024)),
               "batch 1024, q4_K 2048x2048 is claimed");
    test_check(ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_0, k, n, 2048)),
               "batch 2048, q4_0 is claimed");
    test_check(ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_F32, k, n, 2048)),
               "batch 2048, f32 is claimed");
    // every GGUF float and block type has a converter; Q8_K (a dot-product
    // intermediate, no weight of a model file) has none and is not claimed
    for (ggml_type t : {GGML_TYPE_F16, GGML_TYPE_BF16, GGML_TYPE_Q4_1, GGML_TYPE_Q5_0, GGML_TYPE_Q5_1, GGML_TYPE_Q8_0,
                        GGML_TYPE_Q2_K, GGML_TYPE_Q3_K, GGML_TYPE_Q5_K, GGML_TYPE_Q6_K}) {
        char what[64];
        snprintf(what, sizeof what, "batch 2048, type %d is claimed", (int) t);
        test_check(ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, t, k, n, 2048)), "%s", what);
    }
    test_check(!ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q8_K, k, n, 2048)),
               "a type with no converter (q8_K) is not claimed");
    // 2*1024*64*1024 = 134 MFLOP, under the 256 MFLOP floor
    test_check(!ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_K, 1024, 64, 1024)),
               "a tiny matmul is not claimed even at a large batch");
    // 2*1024*128*1024 = 268 MFLOP: just over
    test_check(ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q8_0, 1024, 128, 1024)),
               "a matmul just over the floor is claimed");
    test_check(!ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_F32, 2052, n, 2048)),
               "K not a multiple of the 8-value block is not claimed");
    {
        ggml_tensor * a = ggml_new_tensor_2d(ctx, GGML_TYPE_Q8_0, k, n);
        ggml_tensor * b = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, k, 1024, 2);
        test_check(!ggml_backend_dev_supports_op(dev, ggml_mul_mat(ctx, a, b)), "a batched (3-D) input is not claimed");
    }

    // attention's matmuls read keys from the cache through views, not weights
    {
        ggml_tensor * cache = ggml_new_tensor_2d(ctx, GGML_TYPE_F16, k, 4 * n);
        ggml_tensor * view = ggml_view_2d(ctx, cache, k, n, cache->nb[1], 0);
        ggml_tensor * b = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, 1024);
        test_check(!ggml_backend_dev_supports_op(dev, ggml_mul_mat(ctx, view, b)),
                   "a matmul whose left side is a view (a cache read, not a weight) is not claimed");
        ggml_tensor * computed =
            ggml_add(ctx, ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, n), ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, n));
        test_check(!ggml_backend_dev_supports_op(dev, ggml_mul_mat(ctx, computed, b)),
                   "a matmul whose left side is computed (not a weight) is not claimed");
        test_check(!ggml_backend_dev_supports_op(dev, computed), "other ops (ADD) on their own are not claimed");
    }

    // small ops next to our matmuls (block claiming), except those reading a
    // same-shape tensor that may sit in host memory
    {
        ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, 2048);
        ggml_tensor * mm1 = ggml_mul_mat(ctx, ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, k, n), x);
        ggml_tensor * mm2 = ggml_mul_mat(ctx, ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, k, n), x);
        test_check(ggml_backend_dev_supports_op(dev, ggml_add(ctx, mm1, mm2)),
                   "an ADD of two claimed matmuls is claimed (block claiming)");
        ggml_tensor * emb = ggml_get_rows(ctx, ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, k, 32000),
                                          ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 2048));
        test_check(!ggml_backend_dev_supports_op(dev, ggml_add(ctx, emb, mm1)),
                   "an ADD of a claimed matmul and the token embeddings (GET_ROWS) is not claimed");
        test_check(!ggml_backend_dev_supports_op(dev, ggml_add(ctx, mm1, emb)), "... in either order");
        ggml_tensor * in = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, 2048);
        ggml_set_input(in);
        test_check(!ggml_backend_dev_supports_op(dev, ggml_add(ctx, in, mm1)),
                   "an ADD of a claimed matmul and a graph input is not claimed");
        ggml_tensor * bias = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n);
        test_check(ggml_backend_dev_supports_op(dev, ggml_add(ctx, mm1, bias)),
                   "an ADD of a bias row to a claimed matmul is claimed");
        ggml_tensor * made = ggml_scale(ctx, ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n), 2.0f);
        test_check(!ggml_backend_dev_supports_op(dev, ggml_add(ctx, mm1, made)),
                   "an ADD of a computed row (not a kept leaf) is not claimed");
        test_check(ggml_backend_dev_supports_op(dev, ggml_scale(ctx, mm1, 0.25f)), "a SCALE of a claimed matmul is claimed");
        test_check(ggml_backend_dev_supports_op(dev, ggml_geglu_split(ctx, mm1, mm2)),
                   "a GeGLU of two claimed matmuls is claimed");
        ggml_tensor * fused = ggml_mul_mat(ctx, ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, k, 2 * n), x);
        test_check(ggml_backend_dev_supports_op(dev, ggml_swiglu(ctx, fused)),
                   "a SwiGLU on one claimed matmul holding gate and up is claimed");
        ggml_tensor * norm = ggml_rms_norm(ctx, mm1, 1e-6f);
        test_check(ggml_backend_dev_supports_op(dev, norm), "an RMS_NORM of a claimed matmul is claimed");
        test_check(ggml_backend_dev_supports_op(dev, ggml_mul(ctx, norm, ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n))),
                   "... and its MUL by a scale row");
        ggml_tensor * small_x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, 512);
        ggml_tensor * mm_small = ggml_mul_mat(ctx, ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_K, k, n), small_x);
        test_check(!ggml_backend_dev_supports_op(dev, ggml_scale(ctx, mm_small, 0.5f)),
                   "a small op next to an unclaimed (small-batch) matmul is not claimed");
        // ROPE on the q projection, viewed as heads
        ggml_tensor * q = ggml_reshape_2d(ctx, mm1, 128, 16 * 2048);
        ggml_tensor * q3 = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, 128, 16, 2048);
        q3->op = GGML_OP_RESHAPE;
        q3->src[0] = q;
        q3->view_src = mm1;
        ggml_tensor * pos = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 2048);
        test_check(ggml_backend_dev_supports_op(dev, ggml_rope_ext(ctx, q3, pos, nullptr, 128, GGML_ROPE_TYPE_NEOX, 0,
                                                                   1e6f, 1.0f, 0.0f, 1.0f, 32.0f, 1.0f)),
                   "a NeoX ROPE of a claimed projection is claimed");
        test_check(!ggml_backend_dev_supports_op(dev, ggml_rope_ext(ctx, q3, pos, nullptr, 128, 8, 0, 1e6f, 1.0f,
                                                                    0.0f, 1.0f, 32.0f, 1.0f)),
                   "a ROPE of another mode (multi-section) is not claimed");
    }

    // A mixture-of-experts model's expert step is a MUL_MAT_ID: not taken, but
    // the model's ordinary matmuls still are (the backend warns instead).
    {
        ggml_tensor * experts = ggml_new_tensor_3d(ctx, GGML_TYPE_Q4_0, k, n, 8);
        ggml_tensor * rows = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, k, 1, 2048);
        ggml_tensor * ids = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, 1, 2048);
        test_check(!ggml_backend_dev_supports_op(dev, ggml_mul_mat_id(ctx, experts, rows, ids)),
                   "the expert step (MUL_MAT_ID) is not claimed");
        test_check(ggml_backend_dev_supports_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_0, k, n, 2048)),
                   "... and an ordinary matmul is still claimed afterwards");
    }

    test_check(!ggml_backend_dev_offload_op(dev, make_mul_mat(ctx, GGML_TYPE_Q4_K, k, n, 2048)),
               "offload_op never claims an op (no per-op weight copies)");

    ggml_free(ctx);
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

// The dispatch gate: which ops the backend takes from ggml's scheduler, read
// through the three things the scheduler asks (the device's type and buffer
// types, and supports_op for each node).
//
// Contract (reference: src/ggml-zest.cpp:56-81 thresholds and batch,
// :1066-1072 what a weight is, :1160-1226 claim and policy; acceptance
// criteria in specs/xdna-backend/spec.md, XDNA-BATCH-GATE, XDNA-WORK-FLOOR,
// XDNA-SIZE-POLICY):
//   batch    a MUL_MAT is taken only when its batch (dst ne[1]) is at least
//            GGML_XDNA_MIN_BATCH (1024);
//   floor    and its work 2*K*N*batch / 1e6 (integer MFLOP) is at least
//            GGML_XDNA_MIN_MFLOP (256);
//   weight   and its left side is a plain 2-D leaf (not a view, not computed)
//            of a type the converter handles, the right side fp32 and 2-D,
//            and K a whole number of 8-value blocks (this build's shape rule);
//   block    a small op (RMS_NORM, MUL by a row, ADD, SCALE, GLU, ROPE) is
//            taken when one input comes from a taken op, it covers the batch,
//            its row inputs are kept leaves, and no same-shape input may sit
//            in host memory (graph inputs, GET_ROWS results);
//   size     one launch addresses the weight's cache entry and the expanded
//            activations whole and the output in bands of 256 rows or more,
//            each under 2 GiB: an operand no band fits is left, a tall
//            output is taken (the library cuts it into bands); the right
//            side's rows are 16-byte aligned;
//   never    MUL_MAT_ID and every other op; offload_op claims nothing.
// Each rule is checked on both sides of its boundary, with the expected
// answer computed here from the rule where it is arithmetic. BASELINE's
// small-model configuration (hidden 1024, Q8_0, chunks of 256 to 4096
// tokens) is checked launch by launch. Runs with the thresholds at their
// defaults, on the GPU or under GGML_XDNA_PLAN_ONLY=1.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include "mini_ggml.h"

namespace {

ggml_context * g_ctx;
ggml_backend_dev_t g_dev;
int g_cases;

ggml_tensor * weight(ggml_type t, int64_t k, int64_t n) { return ggml_new_tensor_2d(g_ctx, t, k, n); }
ggml_tensor * rows(int64_t k, int64_t m) { return ggml_new_tensor_2d(g_ctx, GGML_TYPE_F32, k, m); }
ggml_tensor * matmul(ggml_type t, int64_t k, int64_t n, int64_t m) { return ggml_mul_mat(g_ctx, weight(t, k, n), rows(k, m)); }

// Asks supports_op about `op` and checks the answer is `want`.
void expect(ggml_tensor * op, bool want, const char * rule, const char * fmt, ...) __attribute__((format(printf, 4, 5)));
void expect(ggml_tensor * op, bool want, const char * rule, const char * fmt, ...) {
    char what[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(what, sizeof what, fmt, ap);
    va_end(ap);
    const bool got = ggml_backend_dev_supports_op(g_dev, op);
    test_check(got == want, "[%s] %s: %s", rule, what, want ? "taken" : "left to the scheduler");
    g_cases++;
}

// the integer MFLOP the floor compares
int64_t mflop(int64_t k, int64_t n, int64_t m) { return 2 * k * n * m / 1000000; }

void batch_rule() {
    // below, at and above the threshold, for a 2048 x 2048 q4_K weight
    for (int64_t m : {1, 256, 512, 1000, 1023, 1024, 1025, 1536, 2048, 4096, 8192})
        expect(matmul(GGML_TYPE_Q4_K, 2048, 2048, m), m >= 1024, "batch", "q4_K 2048x2048 at batch %lld",
               (long long) m);
}

void floor_rule() {
    // at batch 1024 and K 1024, the floor of 256 MFLOP falls between N = 122 and 123
    for (int64_t n : {32, 64, 120, 122, 123, 128, 4096}) {
        const int64_t w = mflop(1024, n, 1024);
        expect(matmul(GGML_TYPE_Q8_0, 1024, n, 1024), w >= 256, "floor", "q8_0 1024x%lld at batch 1024 (%lld MFLOP)",
               (long long) n, (long long) w);
    }
    // a wide batch does not lift a matmul over the floor by itself: 64 rows of K 256 at 4096 tokens
    expect(matmul(GGML_TYPE_Q8_0, 256, 64, 4096), mflop(256, 64, 4096) >= 256, "floor",
           "q8_0 256x64 at batch 4096 (%lld MFLOP)", (long long) mflop(256, 64, 4096));
}

void weight_rule() {
    const ggml_type convertible[] = {GGML_TYPE_F32,  GGML_TYPE_F16,  GGML_TYPE_BF16, GGML_TYPE_Q4_0, GGML_TYPE_Q4_1,
                                     GGML_TYPE_Q5_0, GGML_TYPE_Q5_1, GGML_TYPE_Q8_0, GGML_TYPE_Q2_K, GGML_TYPE_Q3_K,
                                     GGML_TYPE_Q4_K, GGML_TYPE_Q5_K, GGML_TYPE_Q6_K, GGML_TYPE_IQ4_NL,
                                     GGML_TYPE_IQ4_XS};
    for (ggml_type t : convertible) expect(matmul(t, 2048, 2048, 2048), true, "weight", "ggml type %d", (int) t);
    expect(matmul(GGML_TYPE_Q8_K, 2048, 2048, 2048), false, "weight", "q8_K (a dot-product intermediate, no converter)");
    // the codebook IQ types (their grids are ggml-base tables): left to the next backend
    const ggml_type codebook[] = {GGML_TYPE_IQ2_XXS, GGML_TYPE_IQ2_XS, GGML_TYPE_IQ3_XXS, GGML_TYPE_IQ1_S,
                                  GGML_TYPE_IQ3_S,   GGML_TYPE_IQ2_S,  GGML_TYPE_IQ1_M};
    for (ggml_type t : codebook) expect(matmul(t, 2048, 2048, 2048), false, "weight", "codebook type %d", (int) t);
    expect(matmul(GGML_TYPE_F32, 2052, 2048, 2048), false, "weight", "K = 2052, not a whole number of blocks");
    expect(matmul(GGML_TYPE_F32, 2056, 2048, 2048), true, "weight", "K = 2056, a whole number of blocks");
    // keys read from the cache are views; the score matrix is computed
    ggml_tensor * cache = ggml_new_tensor_2d(g_ctx, GGML_TYPE_F16, 2048, 8192);
    expect(ggml_mul_mat(g_ctx, ggml_view_2d(g_ctx, cache, 2048, 2048, cache->nb[1], 0), rows(2048, 2048)), false,
           "weight", "left side a view of a larger tensor");
    ggml_tensor * made = ggml_add(g_ctx, weight(GGML_TYPE_F32, 2048, 2048), weight(GGML_TYPE_F32, 2048, 2048));
    expect(ggml_mul_mat(g_ctx, made, rows(2048, 2048)), false, "weight", "left side computed by another op");
    expect(made, false, "never", "an ADD of two leaves");
    expect(ggml_mul_mat(g_ctx, weight(GGML_TYPE_Q8_0, 2048, 2048), ggml_new_tensor_3d(g_ctx, GGML_TYPE_F32, 2048, 1024, 2)),
           false, "weight", "a 3-D right side");
}

// What one launch addresses: the packed weight and the expanded activations
// whole, the output in bands of 256 rows or more, each under 2 GiB (32-bit
// buffer ranges). A taller output is cut into bands by the library, so it is
// taken; an operand that no band can fit is left to the scheduler.
void size_rule() {
    constexpr double lim = 2147483648.0;
    auto rnd = [](int64_t v, int64_t a) { return (double) ((v + a - 1) / a * a); };
    // an all-logits output projection: vocab 151,936 at a 4096-token ubatch,
    // 2.49 GB of fp32 output, runs as bands of 3328 rows
    const double out_bytes = 151936.0 * 4096 * 4;
    test_check(out_bytes > lim, "[size] the logits output spans %.2f GB", out_bytes / 1e9);
    expect(matmul(GGML_TYPE_Q6_K, 2560, 151936, 4096), true, "size",
           "output projection 2560x151936 at batch 4096 (%.2f GB of output, cut into bands)", out_bytes / 1e9);
    expect(matmul(GGML_TYPE_Q8_0, 5120, 262144, 8192), true, "size", "a 262,144-word vocabulary at batch 8192");
    // a weight whose cache entry reaches 2 GiB: 131072 x 16384 at 9/8 bytes a value
    const double w_bytes = rnd(131072, 256) * rnd(16384, 64) * 9 / 8;
    expect(matmul(GGML_TYPE_Q4_K, 16384, 131072, 2048), w_bytes < lim, "size", "a weight of %.2f GB as bfp16",
           w_bytes / 1e9);
    expect(matmul(GGML_TYPE_Q4_K, 16384, 65536, 2048), true, "size", "half that weight (%.2f GB)", w_bytes / 2e9);
    // activations whose expanded operand (2 bytes a value) reaches 2 GiB
    const double a_bytes = rnd(65536, 256) * rnd(16384, 64) * 2;
    expect(matmul(GGML_TYPE_Q8_0, 16384, 1024, 65536), a_bytes < lim, "size",
           "65536 rows of 16384 (%.2f GB expanded)", a_bytes / 1e9);
    expect(matmul(GGML_TYPE_Q8_0, 16384, 1024, 32768), true, "size", "32768 rows of 16384");
    // 256 output rows of N floats must fit one band
    expect(matmul(GGML_TYPE_Q8_0, 256, 2097152, 1024), 256.0 * 2097152 * 4 < lim, "size",
           "N = 2,097,152: 256 output rows take 2 GiB");
    expect(matmul(GGML_TYPE_Q8_0, 256, 2097136, 1024), true, "size", "N = 2,097,136: 256 rows just fit");
    // the right side's rows must be 16-byte aligned (the pack's 16-byte loads)
    ggml_tensor * big = rows(2048, 2048 + 4);
    expect(ggml_mul_mat(g_ctx, weight(GGML_TYPE_Q8_0, 2048, 2048), ggml_view_2d(g_ctx, big, 2048, 2048, big->nb[1], 4)),
           false, "size", "right side a view 4 bytes into its tensor");
    expect(ggml_mul_mat(g_ctx, weight(GGML_TYPE_Q8_0, 2048, 2048), ggml_view_2d(g_ctx, big, 2048, 2048, big->nb[1], 64)),
           true, "size", "right side a view 64 bytes into its tensor");
}

void block_rule() {
    ggml_tensor * x = rows(2048, 2048);
    ggml_tensor * up = ggml_mul_mat(g_ctx, weight(GGML_TYPE_Q4_0, 2048, 2048), x);
    ggml_tensor * gate = ggml_mul_mat(g_ctx, weight(GGML_TYPE_Q4_0, 2048, 2048), x);
    ggml_tensor * short_mm = matmul(GGML_TYPE_Q4_K, 2048, 2048, 512);
    ggml_tensor * embd = ggml_get_rows(g_ctx, weight(GGML_TYPE_Q4_0, 2048, 32000), ggml_new_tensor_1d(g_ctx, GGML_TYPE_I32, 2048));
    ggml_tensor * input = rows(2048, 2048);
    ggml_set_input(input);
    ggml_tensor * bias = ggml_new_tensor_1d(g_ctx, GGML_TYPE_F32, 2048);
    ggml_tensor * made_row = ggml_scale(g_ctx, ggml_new_tensor_1d(g_ctx, GGML_TYPE_F32, 2048), 3.0f);

    expect(ggml_add(g_ctx, up, gate), true, "block", "ADD of two taken matmuls");
    expect(ggml_add(g_ctx, up, bias), true, "block", "ADD of a kept bias row to a taken matmul");
    expect(ggml_add(g_ctx, up, made_row), false, "block", "ADD of a computed row");
    expect(ggml_add(g_ctx, embd, up), false, "block", "ADD of the token embeddings (GET_ROWS) and a taken matmul");
    expect(ggml_add(g_ctx, up, embd), false, "block", "the same ADD with its inputs swapped");
    expect(ggml_add(g_ctx, input, up), false, "block", "ADD of a graph input and a taken matmul");
    expect(ggml_scale(g_ctx, up, 0.5f), true, "block", "SCALE of a taken matmul");
    expect(ggml_scale(g_ctx, short_mm, 0.5f), false, "block", "SCALE of a matmul the batch rule left");
    expect(ggml_geglu_split(g_ctx, gate, up), true, "block", "GeGLU over two taken matmuls");
    expect(ggml_swiglu_split(g_ctx, gate, up), true, "block", "SwiGLU over two taken matmuls");
    expect(ggml_swiglu(g_ctx, ggml_mul_mat(g_ctx, weight(GGML_TYPE_Q4_0, 2048, 4096), x)), true, "block",
           "SwiGLU over one taken matmul holding gate and up");
    ggml_tensor * norm = ggml_rms_norm(g_ctx, up, 1e-6f);
    expect(norm, true, "block", "RMS_NORM of a taken matmul");
    expect(ggml_mul(g_ctx, norm, ggml_new_tensor_1d(g_ctx, GGML_TYPE_F32, 2048)), true, "block",
           "MUL of that norm by a kept scale row");
    // ROPE over the heads of a projection: NeoX is run, a multi-section mode is not
    ggml_tensor * heads = ggml_new_tensor_3d(g_ctx, GGML_TYPE_F32, 128, 16, 2048);
    heads->op = GGML_OP_RESHAPE;
    heads->src[0] = ggml_reshape_2d(g_ctx, up, 128, 16 * 2048);
    heads->view_src = up;
    ggml_tensor * pos = ggml_new_tensor_1d(g_ctx, GGML_TYPE_I32, 2048);
    expect(ggml_rope_ext(g_ctx, heads, pos, nullptr, 128, GGML_ROPE_TYPE_NEOX, 0, 1e6f, 1.0f, 0.0f, 1.0f, 32.0f, 1.0f),
           true, "block", "NeoX ROPE of a taken projection's heads");
    expect(ggml_rope_ext(g_ctx, heads, pos, nullptr, 128, 8, 0, 1e6f, 1.0f, 0.0f, 1.0f, 32.0f, 1.0f), false, "block",
           "ROPE in a multi-section mode");
}

void never_rule() {
    ggml_tensor * experts = ggml_new_tensor_3d(g_ctx, GGML_TYPE_Q4_0, 2048, 2048, 8);
    ggml_tensor * ids = ggml_new_tensor_2d(g_ctx, GGML_TYPE_I32, 1, 2048);
    expect(ggml_mul_mat_id(g_ctx, experts, ggml_new_tensor_3d(g_ctx, GGML_TYPE_F32, 2048, 1, 2048), ids), false, "never",
           "an expert step (MUL_MAT_ID)");
    expect(matmul(GGML_TYPE_Q4_0, 2048, 2048, 2048), true, "never", "a plain matmul asked after it");
    test_check(!ggml_backend_dev_offload_op(g_dev, matmul(GGML_TYPE_Q4_K, 2048, 2048, 4096)),
               "[never] offload_op claims nothing (the cache is built per weight, not per op)");
}

// a hidden-1024 Q8_0 layer at each chunk size
void small_model_config() {
    struct mm { const char * name; int64_t k, n; };
    const mm layer[] = {{"q", 1024, 1024}, {"k", 1024, 1024}, {"v", 1024, 1024}, {"o", 1024, 1024},
                        {"gate", 1024, 4096}, {"up", 1024, 4096}, {"down", 4096, 1024}};
    for (int64_t m : {256, 512, 1024, 1536, 4096})
        for (const mm & w : layer) {
            const bool want = m >= 1024 && mflop(w.k, w.n, m) >= 256;
            expect(matmul(GGML_TYPE_Q8_0, w.k, w.n, m), want, "config 4", "%s (%lldx%lld) at a %lld-token chunk", w.name,
                   (long long) w.k, (long long) w.n, (long long) m);
        }
}

}  // namespace

int main() {
    ggml_backend_load_all();
    g_dev = ggml_backend_dev_by_name("XDNA0");
    if (!g_dev) {
        fprintf(stderr, "no XDNA0 device: set GGML_BACKEND_PATH to libggml-zest.so (and run on a GPU, or planning only)\n");
        return 2;
    }
    const char * po = getenv("GGML_XDNA_PLAN_ONLY");
    const bool planning = po && *po && po[0] != '0';

    // what the scheduler reads before any op
    test_check(ggml_backend_dev_type(g_dev) == GGML_BACKEND_DEVICE_TYPE_GPU, "[device] a GPU device");
    ggml_backend_buffer_type_t own = ggml_backend_dev_buffer_type(g_dev);
    test_check(own && !ggml_backend_buft_is_host(own) && ggml_backend_dev_supports_buft(g_dev, own),
               "[device] its buffer type is device memory it reads");
    ggml_backend_dev_t host = ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU);
    test_check(host && ggml_backend_dev_supports_buft(g_dev, ggml_backend_dev_buffer_type(host)),
               "[device] host buffers are readable too, so pieces never wait on copied inputs");
    size_t free = 7, total = 7;
    ggml_backend_dev_memory(g_dev, &free, &total);
    test_check(planning ? free == 0 && total == 0 : total > 0 && free > 0 && free <= total,
               "[device] memory: %zu free of %zu (none when planning only)", free, total);
    ggml_backend_dev_props props;
    ggml_backend_dev_get_props(g_dev, &props);
    test_check(!props.caps.async && !props.caps.events, "[device] synchronous: graph_compute returns with results done");

    ggml_init_params ip = {ggml_tensor_overhead() * 1024, nullptr, true};
    g_ctx = ggml_init(ip);
    batch_rule();
    floor_rule();
    weight_rule();
    size_rule();
    block_rule();
    never_rule();
    small_model_config();
    ggml_free(g_ctx);
    printf("%d supports_op cases\n%s\n", g_cases, test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}

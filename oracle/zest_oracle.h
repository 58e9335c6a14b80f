/*
 * zest_oracle — CPU restatement of the reference's bfp16 prefill MUL_MAT path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library, the ggml
 * backend) links, loads or calls this code. Only tests/, the smoke check in
 * __graft_entry__.py and bench.py's cpu_baseline leg use it, and only as the
 * checker or as the timed CPU baseline.
 *
 * Each function names the reference file:line it restates (paths relative to
 * the Cyronius/ggml-xdna tree). Pinning status of each part:
 *   bfp16 encode/decode ....... pinned: golden vectors from the reference's own
 *                                packer (oracle/_ref), the reference test's KATs,
 *                                and a brute-force sweep of all exponent bytes
 *   NPU tile order (A/B) ....... pinned: byte-equal to the reference packer's
 *                                pack_a/pack_b output on the golden shapes
 *   GGUF dequant (F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K,
 *   Q5_K, Q6_K) ................ pinned by closed form (every product is exact
 *                                in fp32), hand-built blocks with known values,
 *                                relations between the types (Q5_K with no
 *                                fifth bits is Q4_K, Q4_1 with m = -8d is Q4_0,
 *                                ...) and quantise/dequantise error bounds;
 *                                ggml's own to_float is absent (third-party,
 *                                not vendored)
 *   GGUF dequant (IQ4_NL, IQ4_XS) closed form over the published 16-level grid,
 *                                hand-built blocks, IQ4_XS with every scale
 *                                32 + 1 is IQ4_NL; the grid itself is parity
 *                                unpinned (ggml absent)
 *   ref_mul_mat ................ pinned: integer KAT (exact under any order),
 *                                fp64 recomputation bound
 *   host ops ................... RMS_NORM/MUL/ADD/SCALE/GLU pinned by closed forms
 *                                and fp64 recomputation; ROPE's YaRN part
 *                                (ggml_rope_yarn_corr_dims is absent) pinned by
 *                                YaRN's definitions: the correction dims are the
 *                                pairs turning beta_fast / beta_slow times over
 *                                n_ctx_orig, pairs below and above them take the
 *                                extrapolated and interpolated angles, the
 *                                magnitude is 1 + 0.1 ln(1/s)
 */
#ifndef ZEST_ORACLE_H
#define ZEST_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bfp16 block format (src/npu/bfp16_pack.h:28-35) ---------------------- */
void orc_bfp16_encode_block(const float *x, uint8_t *out9);
void orc_bfp16_decode_block(const uint8_t *in9, float *x);
/* row-major blocks: x[rows][K] -> out[rows][K/8][9] */
void orc_bfp16_encode_rows(const float *x, int64_t rows, int64_t K, uint8_t *out);
void orc_bfp16_decode_rows(const uint8_t *in, int64_t rows, int64_t K, float *x);

/* ---- the NPU tile order (src/npu/bfp16_pack.cpp:143-197, 286-302) --------- */
size_t orc_a_offset(int64_t r, int64_t cb, int64_t K, int m, int k);
size_t orc_b_offset(int64_t r, int64_t cb, int64_t N, int64_t K, int n, int k, int cols);
void orc_pack_a(const float *x, int64_t M, int64_t K, int m, int k, uint8_t *out);
void orc_pack_b(const float *w, int64_t N, int64_t K, int n, int k, int cols, uint8_t *out);

/* ---- GGUF dequant (ggml to_float, called at src/xdna-ref.cpp:44) ----------- */
enum {
    ORC_TYPE_F32 = 0, ORC_TYPE_F16 = 1, ORC_TYPE_Q4_0 = 2, ORC_TYPE_Q4_1 = 3, ORC_TYPE_Q5_0 = 6, ORC_TYPE_Q5_1 = 7,
    ORC_TYPE_Q8_0 = 8, ORC_TYPE_Q2_K = 10, ORC_TYPE_Q3_K = 11, ORC_TYPE_Q4_K = 12, ORC_TYPE_Q5_K = 13,
    ORC_TYPE_Q6_K = 14, ORC_TYPE_IQ4_NL = 20, ORC_TYPE_IQ4_XS = 23, ORC_TYPE_BF16 = 30
};
size_t orc_row_bytes(int type, int64_t K);
void orc_dequant_row(int type, const void *raw, float *y, int64_t K);
float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f); /* round to nearest even */

/* Synthetic GGUF rows for the tests (what ggml_quantize_chunk is to the
 * reference's tests, tests/test-mul-mat.cpp:174): valid blocks of every type
 * above from float rows. A simple min/max search, not ggml's own quantiser:
 * the bytes are the shared input of every path under test. Returns 0, or -1
 * for a type or K it does not cover. */
int orc_quantize_row(int type, const float *x, void *out, int64_t K);

/* ---- CPU reference matmul (src/xdna-ref.cpp:10-97) ------------------------
 * y[M][N] = x[M][K] . W[N][K]^T; W as raw GGUF rows of `type`. One weight row
 * dequantised at a time, fp32 sequential dot per token, rows split over
 * n_threads as ceil(N / n_threads). */
void orc_ref_mul_mat(int type, const void *w_raw, int64_t N, int64_t K, const float *x, int64_t M, float *y,
                     int n_threads);
/* The same loop over already-float weights (the bfp16-decoded operands). */
void orc_ref_mul_mat_f32(const float *w, int64_t N, int64_t K, const float *x, int64_t M, float *y, int n_threads);
/* fp64 accumulation of the same products, and sum_k |a_k b_k| per output
 * (the rounding-error bound's scale). Either output may be NULL. */
void orc_mul_mat_f64(const float *w, int64_t N, int64_t K, const float *x, int64_t M, double *y, double *absdot,
                     int n_threads);

/* ---- host ops (src/xdna-exec.cpp:253-346) --------------------------------- */
void orc_rms_norm(const float *x, int64_t rows, int64_t d, float eps, float *y);
void orc_mul_row(const float *x, int64_t rows, int64_t d, const float *w, float *y);
void orc_add(const float *a, const float *b, int64_t n, float *y);
void orc_add_row(const float *x, int64_t rows, int64_t d, const float *w, float *y);
void orc_scale(const float *x, int64_t n, float s, float b, float *y);
enum { ORC_GLU_REGLU = 0, ORC_GLU_GEGLU = 1, ORC_GLU_SWIGLU = 2, ORC_GLU_GEGLU_ERF = 3, ORC_GLU_GEGLU_QUICK = 4 };
/* g/u rows of f floats with row strides sg/su; y rows of f floats */
void orc_glu(int kind, const float *g, int64_t sg, const float *u, int64_t su, int64_t rows, int64_t f, float *y);
/* ROPE over x[T][heads][d], positions pos[T]; mode 0 normal, 2 neox */
void orc_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow,
                             float dims[2]);
void orc_rope(const float *x, int64_t T, int64_t heads, int64_t d, const int32_t *pos, const float *freq_factors,
              int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
              float attn_factor, float beta_fast, float beta_slow, float *y);

/* ---- the GPU-side known-answer generators --------------------------------
 * npu_self_test's integer inputs (src/xdna-npu.cpp:142-156): LCG seed 1,
 * a[M][K] in -2..2 then w[N][K] in -3..3, as floats. */
void orc_self_test_inputs(int64_t M, int64_t K, int64_t N, float *a, float *w);

#ifdef __cplusplus
}
#endif
#endif

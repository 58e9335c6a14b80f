/*
 * zest_hip.h — the thin C ABI between the C++ host side (the ggml backend in
 * ggml-xdna_amd/csrc/backend) and the hand-written CDNA4 kernels of the bfp16
 * prefill MUL_MAT path. Plain pointers, sizes and int status codes; no C++ or
 * torch types. Device pointers are HIP device memory; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream). Every call only
 * enqueues work on `stream` and returns; results are ready when the stream is.
 *
 * Errors: a negative status, with zest_last_error() (thread-local) saying why.
 *
 * Each entry point names the reference interface it replaces (paths in the
 * Cyronius/ggml-xdna tree).
 */
#ifndef ZEST_HIP_H
#define ZEST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZEST_API __attribute__((visibility("default")))

enum zest_status {
    ZEST_OK = 0,
    ZEST_E_ARG = -1,         /* a bad size, pointer or type */
    ZEST_E_HIP = -2,         /* the HIP runtime failed */
    ZEST_E_UNSUPPORTED = -3, /* no kernel for this case */
    ZEST_E_SELF_TEST = -4,   /* the known-answer multiply came out wrong */
};

/* Weight types, numbered as ggml's enum ggml_type. */
enum zest_type {
    ZEST_TYPE_F32 = 0,
    ZEST_TYPE_F16 = 1,
    ZEST_TYPE_Q4_0 = 2,
    ZEST_TYPE_Q4_1 = 3,
    ZEST_TYPE_Q5_0 = 6,
    ZEST_TYPE_Q5_1 = 7,
    ZEST_TYPE_Q8_0 = 8,
    ZEST_TYPE_Q2_K = 10,
    ZEST_TYPE_Q3_K = 11,
    ZEST_TYPE_Q4_K = 12,
    ZEST_TYPE_Q5_K = 13,
    ZEST_TYPE_Q6_K = 14,
    ZEST_TYPE_IQ4_NL = 20,
    ZEST_TYPE_IQ4_XS = 23,
    ZEST_TYPE_BF16 = 30
};

/* GLU kinds. Not ggml's numbering (ggml_glu_op has SWIGLU_OAI at 3, which
 * this library does not run): a ggml caller maps by kind. */
enum zest_glu_kind {
    ZEST_GLU_REGLU = 0,
    ZEST_GLU_GEGLU = 1,
    ZEST_GLU_SWIGLU = 2,
    ZEST_GLU_GEGLU_ERF = 3,
    ZEST_GLU_GEGLU_QUICK = 4,
};

/* Makes `device` current for the calling thread and checks it is a gfx950
 * (MI355X-class) GPU. Replaces the device-open half of xdna_npu_usable
 * (src/xdna-npu.cpp:255-291). */
ZEST_API int zest_init(int device);

/* The registration known-answer test: npu_self_test's integer multiply
 * (src/xdna-npu.cpp:142-184) run through the pack and GEMM kernels on the
 * current device; every output must equal the exact integer. 0 when it
 * passes. Synchronous. */
ZEST_API int zest_self_test(void);

/* What the last failing call on this thread said. */
ZEST_API const char *zest_last_error(void);

/* ---- the tile layout (ggml-xdna_amd/csrc/zest_layout.h) ----------------- */
ZEST_API int64_t zest_rows_pad(int64_t rows);          /* rows rounded up to 256 */
ZEST_API int64_t zest_k_pad(int64_t K);                /* K rounded up to 64 */
ZEST_API size_t zest_bfp16_bytes(int64_t rows, int64_t K); /* bytes of a packed operand */
ZEST_API size_t zest_act_bytes(int64_t rows, int64_t K);   /* bytes of an expanded activation operand */
ZEST_API size_t zest_raw_row_bytes(int type, int64_t K);  /* bytes of one GGUF row */

/* fp32 activations x[M][K] (row stride ldx floats) -> packed bfp16, bit-exact
 * with the reference encoder; rows M..rows_pad(M)-1 and columns K..k_pad(K)-1
 * become zero blocks. K % 8 == 0. Replaces bfp16_pack_a_into
 * (src/npu/bfp16_pack.h:58) / xdna_npu::encode_row (src/xdna-npu.h:96). */
ZEST_API int zest_pack_act(const float *x, int64_t M, int64_t K, int64_t ldx, void *dst, void *stream);

/* The same pack, written as the GEMM's activation operand: every bfp16 block
 * stored decoded, each value as the bf16 it is exactly (zest_act_bytes(M, K)
 * bytes, in 32-row x 16-column sub-tiles laid out as the GEMM's MFMA reads
 * them: zest_layout.h). Equals zest_expand_act of
 * zest_pack_act's bytes. Replaces the same reference functions: the NPU
 * expands its bfp16 operands inside the kernel, here the activations are
 * expanded once when packed. */
ZEST_API int zest_pack_act_x(const float *x, int64_t M, int64_t K, int64_t ldx, void *dst, void *stream);

/* Packed bfp16 activations (zest_pack_act's output, M rows, K columns) -> the
 * expanded operand, losslessly (bfp16_decode_block, src/npu/bfp16_pack.cpp:
 * 129-144, as bf16). */
ZEST_API int zest_expand_act(const void *src, int64_t M, int64_t K, void *dst, void *stream);

/* A GGUF weight raw[N][K] of `type` (any zest_type, rows as ggml stores
 * them) -> packed bfp16 weight cache entry (zest_bfp16_bytes(N, K) bytes).
 * Dequantisation as ggml's to_float, then the same encoder. K must be a
 * multiple of the type's block (32 for Q4_0..Q8_0 and IQ4_NL, 256 for the
 * K-quants and IQ4_XS). Row alignment: 16 bytes for F32, F16, BF16, Q4_K and
 * Q5_K, 8 for IQ4_XS, 4 for Q4_1, Q5_1 and Q2_K, 2 for the rest. Replaces xdna_npu::add_weight's unpack +
 * bfp16_pack_b (src/xdna-npu.cpp:339-378), which converts any type with a
 * to_float (src/ggml-zest.cpp:1066-1072). */
ZEST_API int zest_convert_weight(int type, const void *raw, int64_t N, int64_t K, void *dst, void *stream);

/* c[M][N] (row stride ldc floats) = A . W^T, a the expanded activation
 * operand (M rows, as zest_pack_act_x, the fused norm and GLU packs and
 * zest_gemm_glu write it: its padding rows and columns zero, so they add
 * nothing) and w a packed bfp16 weight (N rows), K
 * columns each: the weight's bfp16 tiles expanded to bf16 in LDS, bf16 MFMA,
 * fp32 accumulation, fp32 store. If `nonfinite` (a device word) is non-NULL,
 * it is OR-ed with 1 when any stored value is NaN or infinite. Replaces
 * xdna_npu::mul_mat (src/xdna-npu.cpp:392-444) and the NPU kernel's
 * mm_f32_first/mid + output mode 0 (kernels/bfp16_gemm/aie_kernels/aie2p/
 * mm_bfp_acc.cc:44-116, 258-278). */
ZEST_API int zest_gemm(const void *a, int64_t M, const void *w, int64_t N, int64_t K, float *c, int64_t ldc,
                       uint32_t *nonfinite, void *stream);
/* Limits of zest_gemm, zest_gemm_residual and zest_gemm_group: a and every
 * w 16-byte aligned (as the packers and converters write them), outputs and
 * `nonfinite` 4-byte aligned; the expanded
 * activations and each packed weight under 2 GiB, and 256 rows of the output
 * (and of the residual) under 2 GiB. A taller output runs as launches over
 * bands of rows, each band's output span under 2 GiB (whole 256-row tiles;
 * the plan, and so the K split, is made per band). */

/* c[M][N] = A . W^T + res[M][N] (row stride ldr floats, 16-byte aligned
 * rows; res may be c itself, for an in-place residual add): zest_gemm with
 * the ADD that follows a matmul fused into its store, bit-exact with zest_gemm
 * then zest_add. Replaces the matmul + ADD of the reference's row pass
 * (src/xdna-exec.cpp:278-289 after xdna_npu::mul_mat). */
ZEST_API int zest_gemm_residual(const void *a, int64_t M, const void *w, int64_t N, int64_t K, const float *res,
                                int64_t ldr, float *c, int64_t ldc, uint32_t *nonfinite, void *stream);

/* Up to ZEST_GEMM_MAX_GROUP weights that share one activation operand, in one
 * launch: c[i][M][N[i]] (row stride ldc[i]) = A . w[i]^T, as zest_gemm
 * computes each (the same products; the launch's split of K among
 * workgroups, and so the fp32 summation order, can differ). Replaces
 * the reference's group of calls on one input (q, k and v): xdna_npu::begin /
 * submit (src/xdna-npu.h:88-107) over the group built in xdna-exec.cpp
 * (:509-547). A launch whose whole tiles would leave CUs idle splits each
 * tile's K among workgroups (split-K) and sums the splits in a fixed order,
 * through a workspace the library allocates per device and stream on first
 * use (and grows, synchronizing the stream; zest_release_stream frees it):
 * calls that share a stream run in order and never share it concurrently. A launch of at most one small
 * tile a CU may instead split each tile's K between two groups of waves in
 * one workgroup (K-groups), whose sums meet in LDS, also in a fixed order.
 * The same holds for zest_gemm and zest_gemm_glu, which run through the
 * same launch. */
#define ZEST_GEMM_MAX_GROUP 4
ZEST_API int zest_gemm_group(const void *a, int64_t M, int64_t K, int n, const void *const *w, const int64_t *N,
                             float *const *c, const int64_t *ldc, uint32_t *nonfinite, void *stream);

/* Frees the split-K workspace the library holds for `stream` (on every
 * device), after the launches queued on it finish. Call it before destroying
 * a stream that GEMMs ran on: the library cannot see a stream go, and a
 * process that makes and destroys streams would otherwise keep one workspace
 * per stream it ever used. A later GEMM on the stream allocates a new one;
 * a stream that holds none is left as it is. It has no counterpart in the
 * reference, whose NPU buffers live with its context. */
ZEST_API int zest_release_stream(void *stream);

/* zest_gemm_group for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc). It
 * has no counterpart in the reference. It runs the launch zest_gemm_group
 * plans for the same arguments (the same tiles, K splits and summation order,
 * so the same results), but a split-K plan takes its workspace from a static
 * device array the library holds on each GPU (ZEST_NOALLOC_PARTIAL_BYTES of
 * partial sums and ZEST_NOALLOC_COUNTERS counters, kept until the process
 * ends) instead of allocating one. A call whose plan needs more than that
 * fails with ZEST_E_ARG and runs nothing; plans without split-K need none.
 * It allocates nothing: no hipMalloc, no hipFree, no library allocation. The
 * device address of the array is looked up once per device, by zest_init or
 * else by the first call on that device (which should then not be under
 * capture). Every call on one GPU shares that GPU's array, whose counters
 * each call clears (with a kernel on `stream`) before use: calls that overlap
 * on one GPU, on any streams, race. */
#define ZEST_NOALLOC_PARTIAL_BYTES (64u << 20)
#define ZEST_NOALLOC_COUNTERS 16384
ZEST_API int zest_gemm_group_noalloc(const void *a, int64_t M, int64_t K, int n, const void *const *w,
                                     const int64_t *N, float *const *c, const int64_t *ldc, uint32_t *nonfinite,
                                     void *stream);

/* A GLU's gate[F][K] and up[F][K] weights (GGUF rows of `type`, the same for
 * both; for a weight holding the gate and then the up, up = gate + F rows)
 * -> one packed weight of 2F rows for zest_gemm_glu (zest_bfp16_bytes(2F, K)
 * bytes), its rows interleaved by 32-row groups: 32 gate rows, the 32 up
 * rows that pair with them, and so on. Each row's bytes are zest_convert_
 * weight's. F % 32 == 0. Replaces xdna_npu::add_fused (src/xdna-npu.cpp:
 * 380-390) and bfp16_interleave_gate_up (src/npu/bfp16_pack.cpp:231-237),
 * which interleave by the NPU tile's 8 rows where this uses the MFMA's 32. */
ZEST_API int zest_convert_weight_gu(int type, const void *gate, const void *up, int64_t F, int64_t K, void *dst,
                                    void *stream);

/* The fused gate/up GEMM: with w_gu from zest_convert_weight_gu, computes
 * g = A . gate^T and u = A . up^T as zest_gemm does, and in the same kernel
 * h[M][F] = glu(g, u) of `kind` (zest_glu's arithmetic), written as the next
 * matmul's operand (xout, as zest_pack_act_x writes it, zest_act_bytes(M, F)
 * bytes) and/or as fp32 rows (h, row stride ldh floats); either may be NULL,
 * not both. This launch splits K among workgroups and K-groups exactly as
 * zest_gemm(a, w_gu) of 2F columns does, so its gate and up sums are that
 * call's, bit for bit, and h is bit-exact with zest_glu over the gate and up columns of
 * zest_gemm(a, w_gu) whenever that call runs as one launch (its fp32 output,
 * M x 2F floats, under 2 GiB); xout is then zest_pack_act_x of that h.
 * `nonfinite` as for zest_gemm, over g, u and h.
 * F % 32 == 0; a, w_gu and xout 16-byte aligned, h 4.
 * Replaces the reference's fused SwiGLU matmul: find_fusions
 * (src/xdna-exec.cpp:399-431) and the NPU kernel's output mode 2
 * (kernels/bfp16_gemm/aie_kernels/aie2p/mm_bfp_acc.cc:258-278), which stores
 * SiLU(gate)*up as bf16. */
ZEST_API int zest_gemm_glu(int kind, const void *a, int64_t M, const void *w_gu, int64_t F, int64_t K, void *xout,
                           float *h, int64_t ldh, uint32_t *nonfinite, void *stream);

/* ---- the fused host ops (piece::run_rows, src/xdna-exec.cpp:253-346) ---- */

/* y = RMS_NORM(x) (eps), optionally times a scale row w[d] (the MUL that
 * follows a norm, :258-277). y (fp32 rows, may be NULL) and/or packed (the
 * next matmul's input as zest_pack_act_x writes it, zest_act_bytes(rows, d)
 * bytes, 16-byte aligned, may be NULL). */
ZEST_API int zest_rms_norm(const float *x, int64_t rows, int64_t d, float eps, const float *w, float *y, void *packed,
                           void *stream);

/* y[r][j] = act(g[r][j]) * u[r][j] for the GLU kinds (:296-320); g and u rows
 * have strides sg/su floats (one tensor's halves, or two tensors). y and/or
 * packed as for zest_rms_norm. */
ZEST_API int zest_glu(int kind, const float *g, int64_t sg, const float *u, int64_t su, int64_t rows, int64_t f,
                      float *y, void *packed, void *stream);

/* y = a + b, b either the same shape or one row of d broadcast (:278-289). */
ZEST_API int zest_add(const float *a, const float *b, int64_t rows, int64_t d, int b_is_row, float *y, void *stream);

/* y = x * w, w one row of d broadcast over rows (:271-277). */
ZEST_API int zest_mul_row(const float *x, const float *w, int64_t rows, int64_t d, float *y, void *stream);

/* y = x * s + b over n floats (:290-295). */
ZEST_API int zest_scale(const float *x, int64_t n, float s, float b, float *y, void *stream);

/* ROPE over x[T][heads][d] with positions pos[T] (device int32), normal
 * (mode 0) or NeoX (mode 2), rotating the first n_dims of each head, with
 * YaRN and optional per-frequency factors ff[n_dims/2] (:203-239, :321-342).
 * corr_dims are ggml_rope_yarn_corr_dims' two values, computed by the host. */
ZEST_API int zest_rope(const float *x, int64_t T, int64_t heads, int64_t d, const int32_t *pos, const float *ff,
                       int n_dims, int mode, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                       float corr0, float corr1, float *y, void *stream);

/* Sets *flag (device memory, nonzero stays) when any of rows x cols floats at
 * y (row stride ld) is NaN or infinite: the check the reference makes on each
 * NPU result before using it (src/xdna-npu.cpp:57-85), for results that
 * no zest_gemm produced. */
ZEST_API int zest_check_finite(const float *y, int64_t rows, int64_t cols, int64_t ld, uint32_t *flag, void *stream);

#ifdef __cplusplus
}
#endif
#endif

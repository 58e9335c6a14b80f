/*
 * zest_oracle.c — CPU restatement of the reference path. TEST INFRASTRUCTURE:
 * used only by tests/, the smoke check and bench.py's cpu_baseline leg.
 * See zest_oracle.h for what pins each part.
 */
#include "zest_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * bfp16 block: one exponent byte = the largest biased exponent field of the
 * eight floats; mantissa q = round-to-nearest-even(x * 2^(133 - e)) clamped to
 * [-128, 127].  src/npu/bfp16_pack.cpp:85-127 (the scalar path; the AVX2 path
 * computes the same bytes for finite inputs), tests/test-bfp16-pack.cpp:21-38.
 * ------------------------------------------------------------------------- */
void orc_bfp16_encode_block(const float *x, uint8_t *out) {
    uint32_t maxe = 0;
    for (int i = 0; i < 8; i++) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        const uint32_t e = (u >> 23) & 0xffu;
        if (e > maxe) maxe = e;
    }
    out[0] = (uint8_t) maxe;
    const int sh = 133 - (int) maxe;
    for (int i = 0; i < 8; i++) {
        float q = nearbyintf(ldexpf(x[i], sh));
        if (q > 127.0f) q = 127.0f;
        if (q < -128.0f) q = -128.0f;
        out[1 + i] = (uint8_t) (int8_t) q;
    }
}

/* m * 2^(e - 133): src/npu/bfp16_pack.cpp:129-144 */
void orc_bfp16_decode_block(const uint8_t *in, float *x) {
    const int sh = (int) in[0] - 133;
    for (int i = 0; i < 8; i++) x[i] = ldexpf((float) (int8_t) in[1 + i], sh);
}

void orc_bfp16_encode_rows(const float *x, int64_t rows, int64_t K, uint8_t *out) {
    const int64_t nb = rows * (K / 8);
    for (int64_t b = 0; b < nb; b++) orc_bfp16_encode_block(x + b * 8, out + b * 9);
}

void orc_bfp16_decode_rows(const uint8_t *in, int64_t rows, int64_t K, float *x) {
    const int64_t nb = rows * (K / 8);
    for (int64_t b = 0; b < nb; b++) orc_bfp16_decode_block(in + b * 9, x + b * 8);
}

/* ---------------------------------------------------------------------------
 * NPU tile order.  Inside an (rows x k) tile the blocks go 16-row pair by
 * pair, block column by block column, the pair's first eight rows then its
 * second (src/npu/bfp16_pack.cpp:143-151, 286-291).  A: row block of m rows,
 * then K/k tiles (:153-168, 293-296).  B: array column c, the column's n-row
 * groups (c + cols*t), then K/k tiles (:176-191, 298-302).
 * ------------------------------------------------------------------------- */
static int64_t in_tile(int64_t rr, int64_t cb, int k) {
    const int64_t tkb = k / 8;
    return ((rr / 16) * tkb + cb % tkb) * 16 + rr % 16;
}

size_t orc_a_offset(int64_t r, int64_t cb, int64_t K, int m, int k) {
    const int64_t nk = K / k, tile = (r / m) * nk + cb / (k / 8);
    return (size_t) (tile * m * (k / 8) + in_tile(r % m, cb, k)) * 9;
}

size_t orc_b_offset(int64_t r, int64_t cb, int64_t N, int64_t K, int n, int k, int cols) {
    const int64_t per_col = N / n / cols, nk = K / k, g = r / n;
    const int64_t tile = ((g % cols) * per_col + g / cols) * nk + cb / (k / 8);
    return (size_t) (tile * n * (k / 8) + in_tile(r % n, cb, k)) * 9;
}

void orc_pack_a(const float *x, int64_t M, int64_t K, int m, int k, uint8_t *out) {
    for (int64_t r = 0; r < M; r++)
        for (int64_t cb = 0; cb < K / 8; cb++) orc_bfp16_encode_block(x + r * K + cb * 8, out + orc_a_offset(r, cb, K, m, k));
}

void orc_pack_b(const float *w, int64_t N, int64_t K, int n, int k, int cols, uint8_t *out) {
    for (int64_t r = 0; r < N; r++)
        for (int64_t cb = 0; cb < K / 8; cb++)
            orc_bfp16_encode_block(w + r * K + cb * 8, out + orc_b_offset(r, cb, N, K, n, k, cols));
}

/* ---------------------------------------------------------------------------
 * GGUF dequant, the public block formats (ggml-base of llama.cpp b10944,
 * called by the reference at src/xdna-ref.cpp:44 and src/xdna-npu.cpp:345).
 * ------------------------------------------------------------------------- */
float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t s = (uint32_t) (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal half: m * 2^-24, exact in float */
            float f = ldexpf((float) m, -24);
            memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

size_t orc_row_bytes(int type, int64_t K) {
    switch (type) {
        case ORC_TYPE_F32: return (size_t) K * 4;
        case ORC_TYPE_Q8_0: return (size_t) (K / 32) * 34;
        case ORC_TYPE_Q4_K: return (size_t) (K / 256) * 144;
        default: return 0;
    }
}

/* Q8_0: 32 values per block, fp16 d then 32 int8; y = d * q (exact in fp32). */
static void dequant_q8_0(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, src += 34) {
        uint16_t dh;
        memcpy(&dh, src, 2);
        const float d = orc_fp16_to_fp32(dh);
        for (int j = 0; j < 32; j++) y[b * 32 + j] = (float) (int8_t) src[2 + j] * d;
    }
}

/* Q4_K's 6-bit (scale, min) pair j of 8, from the 12 packed bytes. */
static void q4k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Q4_K: 256 values per super-block: fp16 d, fp16 dmin, 12 bytes of 6-bit
 * scales/mins, 128 bytes of nibbles. Group j of 64 values: low nibbles of
 * qs[32j..32j+32) with pair 2j, then the high nibbles with pair 2j+1;
 * y = (d*sc)*q - (dmin*m). d*sc, (d*sc)*q and dmin*m are exact in fp32, so the
 * one rounding is the subtraction's and a fused multiply-add gives the same. */
static void dequant_q4_k(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, src += 144) {
        uint16_t dh, mh;
        memcpy(&dh, src, 2);
        memcpy(&mh, src + 2, 2);
        const float d = orc_fp16_to_fp32(dh), dmin = orc_fp16_to_fp32(mh);
        const uint8_t *scales = src + 4, *qs = src + 16;
        float *out = y + b * 256;
        for (int j = 0; j < 4; j++) {
            uint8_t sc, m;
            q4k_scale_min(2 * j, scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            q4k_scale_min(2 * j + 1, scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; l++) out[64 * j + l] = d1 * (float) (qs[32 * j + l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) out[64 * j + 32 + l] = d2 * (float) (qs[32 * j + l] >> 4) - m2;
        }
    }
}

void orc_dequant_row(int type, const void *raw, float *y, int64_t K) {
    switch (type) {
        case ORC_TYPE_F32: memcpy(y, raw, (size_t) K * 4); break;
        case ORC_TYPE_Q8_0: dequant_q8_0((const uint8_t *) raw, y, K); break;
        case ORC_TYPE_Q4_K: dequant_q4_k((const uint8_t *) raw, y, K); break;
        default: memset(y, 0, (size_t) K * 4); break;
    }
}

/* ---------------------------------------------------------------------------
 * xdna_ref_mul_mat (src/xdna-ref.cpp:10-97): weight rows split over threads
 * in chunks of ceil(N / n_threads); each dequantises one row at a time and
 * runs an fp32 sequential dot against every token.
 * ------------------------------------------------------------------------- */
typedef struct {
    int type;
    const void *w_raw;
    const float *w_f32;
    int64_t N, K, M, r0, r1;
    const float *x;
    float *y;
    double *y64, *absdot;
} mm_job;

static void *mm_rows(void *arg) {
    const mm_job *j = (const mm_job *) arg;
    float *row = j->w_f32 ? NULL : (float *) malloc((size_t) j->K * sizeof(float));
    const size_t rb = j->w_f32 ? 0 : orc_row_bytes(j->type, j->K);
    for (int64_t n = j->r0; n < j->r1 && n < j->N; n++) {
        const float *w;
        if (j->w_f32) {
            w = j->w_f32 + n * j->K;
        } else {
            orc_dequant_row(j->type, (const uint8_t *) j->w_raw + (size_t) n * rb, row, j->K);
            w = row;
        }
        for (int64_t t = 0; t < j->M; t++) {
            const float *s1 = j->x + t * j->K;
            if (j->y) {
                float acc = 0.0f;
                for (int64_t k = 0; k < j->K; k++) acc += w[k] * s1[k];
                j->y[t * j->N + n] = acc;
            }
            if (j->y64 || j->absdot) {
                double acc = 0.0, ab = 0.0;
                for (int64_t k = 0; k < j->K; k++) {
                    const double p = (double) w[k] * (double) s1[k];
                    acc += p;
                    ab += fabs(p);
                }
                if (j->y64) j->y64[t * j->N + n] = acc;
                if (j->absdot) j->absdot[t * j->N + n] = ab;
            }
        }
    }
    free(row);
    return NULL;
}

static void run_split(mm_job base, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if ((int64_t) n_threads > base.N) n_threads = (int) base.N;
    const int64_t chunk = (base.N + n_threads - 1) / n_threads;
    mm_job *jobs = (mm_job *) calloc((size_t) n_threads, sizeof(mm_job));
    pthread_t *th = (pthread_t *) calloc((size_t) n_threads, sizeof(pthread_t));
    int started = 0;
    for (int t = 1; t < n_threads; t++) {
        const int64_t b = t * chunk;
        if (b >= base.N) break;
        jobs[t] = base;
        jobs[t].r0 = b;
        jobs[t].r1 = b + chunk;
        pthread_create(&th[t], NULL, mm_rows, &jobs[t]);
        started = t;
    }
    jobs[0] = base;
    jobs[0].r0 = 0;
    jobs[0].r1 = chunk;
    mm_rows(&jobs[0]);
    for (int t = 1; t <= started; t++) pthread_join(th[t], NULL);
    free(jobs);
    free(th);
}

void orc_ref_mul_mat(int type, const void *w_raw, int64_t N, int64_t K, const float *x, int64_t M, float *y,
                     int n_threads) {
    mm_job j = {type, w_raw, NULL, N, K, M, 0, 0, x, y, NULL, NULL};
    run_split(j, n_threads);
}

void orc_ref_mul_mat_f32(const float *w, int64_t N, int64_t K, const float *x, int64_t M, float *y, int n_threads) {
    mm_job j = {ORC_TYPE_F32, NULL, w, N, K, M, 0, 0, x, y, NULL, NULL};
    run_split(j, n_threads);
}

void orc_mul_mat_f64(const float *w, int64_t N, int64_t K, const float *x, int64_t M, double *y, double *absdot,
                     int n_threads) {
    mm_job j = {ORC_TYPE_F32, NULL, w, N, K, M, 0, 0, x, NULL, y, absdot};
    run_split(j, n_threads);
}

/* ---------------------------------------------------------------------------
 * Host ops: piece::run_rows (src/xdna-exec.cpp:253-346), with the activation
 * helpers of :55-59 and rope_yarn of :66-78.
 * ------------------------------------------------------------------------- */
void orc_rms_norm(const float *x, int64_t rows, int64_t d, float eps, float *y) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * d;
        float ss = 0.0f;
        for (int64_t j = 0; j < d; j++) ss += xr[j] * xr[j];
        const float sc = 1.0f / sqrtf(ss / (float) d + eps);
        for (int64_t j = 0; j < d; j++) y[r * d + j] = xr[j] * sc;
    }
}

void orc_mul_row(const float *x, int64_t rows, int64_t d, const float *w, float *y) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t j = 0; j < d; j++) y[r * d + j] = x[r * d + j] * w[j];
}

void orc_add(const float *a, const float *b, int64_t n, float *y) {
    for (int64_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

void orc_add_row(const float *x, int64_t rows, int64_t d, const float *w, float *y) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t j = 0; j < d; j++) y[r * d + j] = x[r * d + j] + w[j];
}

void orc_scale(const float *x, int64_t n, float s, float b, float *y) {
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * s + b;
}

static float silu(float x) { return x / (1.0f + expf(-x)); }
static float gelu(float x) { return 0.5f * x * (1.0f + tanhf(0.7978845608f * x * (1.0f + 0.044715f * x * x))); }
static float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067812f)); }
static float gelu_quick(float x) { return x / (1.0f + expf(-1.702f * x)); }

void orc_glu(int kind, const float *g, int64_t sg, const float *u, int64_t su, int64_t rows, int64_t f, float *y) {
    for (int64_t r = 0; r < rows; r++) {
        const float *gr = g + r * sg, *ur = u + r * su;
        float *o = y + r * f;
        for (int64_t j = 0; j < f; j++) {
            switch (kind) {
                case ORC_GLU_SWIGLU: o[j] = silu(gr[j]) * ur[j]; break;
                case ORC_GLU_GEGLU: o[j] = gelu(gr[j]) * ur[j]; break;
                case ORC_GLU_GEGLU_ERF: o[j] = gelu_erf(gr[j]) * ur[j]; break;
                case ORC_GLU_GEGLU_QUICK: o[j] = gelu_quick(gr[j]) * ur[j]; break;
                default: o[j] = gr[j] > 0.0f ? gr[j] * ur[j] : 0.0f; break;
            }
        }
    }
}

/* ggml_rope_yarn_corr_dims (ggml-base, absent here; called at
 * src/xdna-exec.cpp:221), restated from ggml's published YaRN formula:
 * the dimension where a rotation completes n_rot turns over n_ctx_orig. */
static float corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return (float) n_dims * logf((float) n_ctx_orig / (n_rot * 2.0f * (float) M_PI)) / (2.0f * logf(base));
}

void orc_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow,
                             float dims[2]) {
    const float start = floorf(corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base));
    const float end = ceilf(corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base));
    dims[0] = start > 0.0f ? start : 0.0f;
    dims[1] = end < (float) (n_dims - 1) ? end : (float) (n_dims - 1);
}

static void rope_yarn(float theta_extrap, float freq_scale, const float corr[2], int64_t pair, float ext_factor,
                      float mscale, float *c, float *s) {
    float theta = freq_scale * theta_extrap;
    if (ext_factor != 0.0f) {
        float den = corr[1] - corr[0];
        if (den < 0.001f) den = 0.001f;
        const float y = ((float) pair - corr[0]) / den;
        float cl = y < 0.0f ? 0.0f : (y > 1.0f ? 1.0f : y);
        const float ramp_mix = (1.0f - cl) * ext_factor;
        theta = theta * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
    }
    *c = cosf(theta) * mscale;
    *s = sinf(theta) * mscale;
}

/* rope_table (src/xdna-exec.cpp:203-239) then the ROPE case of run_rows
 * (:321-342): pairs (i, i+1) for normal, (i/2, i/2 + n_dims/2) for neox;
 * dimensions past n_dims are copied. */
void orc_rope(const float *x, int64_t T, int64_t heads, int64_t d, const int32_t *pos, const float *ff, int n_dims,
              int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
              float beta_fast, float beta_slow, float *y) {
    float corr[2];
    orc_rope_yarn_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, corr);
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    float *cs = (float *) malloc((size_t) n_dims * sizeof(float));
    const int neox = mode == 2;
    const int64_t off_n = neox ? n_dims / 2 : 1;
    for (int64_t t = 0; t < T; t++) {
        float theta = (float) pos[t];
        for (int p = 0; p < n_dims / 2; p++) {
            rope_yarn(ff ? theta / ff[p] : theta, freq_scale, corr, p, ext_factor, attn_factor, &cs[2 * p],
                      &cs[2 * p + 1]);
            theta *= theta_scale;
        }
        for (int64_t h = 0; h < heads; h++) {
            const float *src = x + (t * heads + h) * d;
            float *dst = y + (t * heads + h) * d;
            for (int64_t i = 0; i < n_dims; i += 2) {
                const int64_t ic = neox ? i / 2 : i;
                const float c = cs[i], sn = cs[i + 1];
                const float x0 = src[ic], x1 = src[ic + off_n];
                dst[ic] = x0 * c - x1 * sn;
                dst[ic + off_n] = x0 * sn + x1 * c;
            }
            for (int64_t i = n_dims; i < d; i++) dst[i] = src[i];
        }
    }
    free(cs);
}

/* npu_self_test's operands (src/xdna-npu.cpp:142-156). */
void orc_self_test_inputs(int64_t M, int64_t K, int64_t N, float *a, float *w) {
    uint32_t seed = 1;
    for (int64_t i = 0; i < M * K; i++) {
        seed = seed * 1664525u + 1013904223u;
        a[i] = (float) (int8_t) ((int) (seed >> 24) % 5 - 5 / 2);
    }
    for (int64_t i = 0; i < N * K; i++) {
        seed = seed * 1664525u + 1013904223u;
        w[i] = (float) (int8_t) ((int) (seed >> 24) % 7 - 7 / 2);
    }
}

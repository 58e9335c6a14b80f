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

/* bytes per block and values per block of each GGUF type (ggml-common.h's
 * block structs: the field order below is the struct's) */
size_t orc_row_bytes(int type, int64_t K) {
    switch (type) {
        case ORC_TYPE_F32: return (size_t) K * 4;
        case ORC_TYPE_F16:
        case ORC_TYPE_BF16: return (size_t) K * 2;
        case ORC_TYPE_Q4_0: return (size_t) (K / 32) * 18;  /* d, qs[16] */
        case ORC_TYPE_Q4_1: return (size_t) (K / 32) * 20;  /* d, m, qs[16] */
        case ORC_TYPE_Q5_0: return (size_t) (K / 32) * 22;  /* d, qh[4], qs[16] */
        case ORC_TYPE_Q5_1: return (size_t) (K / 32) * 24;  /* d, m, qh[4], qs[16] */
        case ORC_TYPE_Q8_0: return (size_t) (K / 32) * 34;  /* d, qs[32] */
        case ORC_TYPE_Q2_K: return (size_t) (K / 256) * 84;  /* scales[16], qs[64], d, dmin */
        case ORC_TYPE_Q3_K: return (size_t) (K / 256) * 110; /* hmask[32], qs[64], scales[12], d */
        case ORC_TYPE_Q4_K: return (size_t) (K / 256) * 144; /* d, dmin, scales[12], qs[128] */
        case ORC_TYPE_Q5_K: return (size_t) (K / 256) * 176; /* d, dmin, scales[12], qh[32], qs[128] */
        case ORC_TYPE_Q6_K: return (size_t) (K / 256) * 210; /* ql[128], qh[64], scales[16], d */
        case ORC_TYPE_IQ4_NL: return (size_t) (K / 32) * 18;   /* d, qs[16] */
        case ORC_TYPE_IQ4_XS: return (size_t) (K / 256) * 136; /* d, scales_h, scales_l[4], qs[128] */
        default: return 0;
    }
}

static float f16_at(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return orc_fp16_to_fp32(h);
}

/* F16 / BF16: one value per 2 bytes, widened exactly */
static void dequant_f16(const uint8_t *src, float *y, int64_t K) {
    for (int64_t i = 0; i < K; i++) y[i] = f16_at(src + 2 * i);
}

static void dequant_bf16(const uint8_t *src, float *y, int64_t K) {
    for (int64_t i = 0; i < K; i++) {
        uint16_t h;
        memcpy(&h, src + 2 * i, 2);
        const uint32_t bits = (uint32_t) h << 16;
        memcpy(&y[i], &bits, 4);
    }
}

/* The 32-value types. Byte j of qs holds value j (low nibble) and value
 * j + 16 (high nibble). Q5: bit j of the little-endian 32-bit qh is the fifth
 * bit of value j. Q4_0 q - 8 and Q5_0 q - 16 are signed and y = d*q, exact;
 * Q4_1 / Q5_1 are unsigned and y = d*q + m: d*q is exact, so the one rounding
 * is the addition's (an fma gives the same float). */
static void dequant_q4_0(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, src += 18, y += 32) {
        const float d = f16_at(src);
        for (int j = 0; j < 16; j++) {
            y[j] = (float) ((src[2 + j] & 0xF) - 8) * d;
            y[j + 16] = (float) ((src[2 + j] >> 4) - 8) * d;
        }
    }
}

static void dequant_q4_1(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, src += 20, y += 32) {
        const float d = f16_at(src), m = f16_at(src + 2);
        for (int j = 0; j < 16; j++) {
            y[j] = (float) (src[4 + j] & 0xF) * d + m;
            y[j + 16] = (float) (src[4 + j] >> 4) * d + m;
        }
    }
}

static void dequant_q5_0(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, src += 22, y += 32) {
        const float d = f16_at(src);
        uint32_t qh;
        memcpy(&qh, src + 2, 4);
        for (int j = 0; j < 16; j++) {
            const int lo = (src[6 + j] & 0xF) | (int) (((qh >> j) & 1u) << 4);
            const int hi = (src[6 + j] >> 4) | (int) (((qh >> (j + 16)) & 1u) << 4);
            y[j] = (float) (lo - 16) * d;
            y[j + 16] = (float) (hi - 16) * d;
        }
    }
}

static void dequant_q5_1(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, src += 24, y += 32) {
        const float d = f16_at(src), m = f16_at(src + 2);
        uint32_t qh;
        memcpy(&qh, src + 4, 4);
        for (int j = 0; j < 16; j++) {
            const int lo = (src[8 + j] & 0xF) | (int) (((qh >> j) & 1u) << 4);
            const int hi = (src[8 + j] >> 4) | (int) (((qh >> (j + 16)) & 1u) << 4);
            y[j] = (float) lo * d + m;
            y[j + 16] = (float) hi * d + m;
        }
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

/* Q2_K: 256 values in two halves of 128; half h uses qs[32h..32h+32). Its
 * value group g (0..7) of 16 takes 2-bit field g/2 of qs[32h + 16(g%2) + l]
 * and scale byte s = scales[8h + g]: y = (d*(s & 15))*q - dmin*(s >> 4).
 * The products are exact, so the one rounding is the subtraction's. */
static void dequant_q2_k(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, src += 84) {
        const uint8_t *scales = src, *qs = src + 16;
        const float d = f16_at(src + 80), dmin = f16_at(src + 82);
        for (int h = 0; h < 2; h++)
            for (int g = 0; g < 8; g++) {
                const uint8_t s = scales[8 * h + g];
                const float dl = d * (float) (s & 0xF), ml = dmin * (float) (s >> 4);
                const uint8_t *q = qs + 32 * h + 16 * (g & 1);
                for (int l = 0; l < 16; l++) *y++ = dl * (float) ((q[l] >> (2 * (g >> 1))) & 3) - ml;
            }
    }
}

/* Q3_K's 6-bit scale i of 16: low 4 bits from nibble i/8 of byte i%8, high
 * 2 bits from bits 2(i/4).. of byte 8 + i%4; biased by 32. */
static int q3k_scale(const uint8_t *sc, int i) {
    const int lo = i < 8 ? (sc[i] & 0xF) : (sc[i - 8] >> 4);
    const int hi = (sc[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

/* Q3_K: as Q2_K's 2-bit fields, with a third bit from hmask: value group g
 * (0..7) of half h takes bit 4h + g/2 of hmask[16(g%2) + l]; q = field - 4
 * where that bit is clear. y = (d*scale)*q with scale 16*h + g, exact. */
static void dequant_q3_k(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, src += 110) {
        const uint8_t *hmask = src, *qs = src + 32, *sc = src + 96;
        const float d = f16_at(src + 108);
        for (int h = 0; h < 2; h++)
            for (int g = 0; g < 8; g++) {
                const float dl = d * (float) q3k_scale(sc, 8 * h + g);
                const int j = g >> 1, off = 16 * (g & 1);
                const uint8_t *q = qs + 32 * h + off, *hm = hmask + off;
                for (int l = 0; l < 16; l++) {
                    const int v = ((q[l] >> (2 * j)) & 3) - ((hm[l] >> (4 * h + j)) & 1 ? 0 : 4);
                    *y++ = dl * (float) v;
                }
            }
    }
}

/* Q5_K: Q4_K's scales and nibbles plus a fifth bit: in group j of 64, value
 * l takes bit 2j of qh[l], value 32 + l bit 2j + 1. y = (d*sc)*q - dmin*m,
 * one rounding (the subtraction's). */
static void dequant_q5_k(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, src += 176) {
        const float d = f16_at(src), dmin = f16_at(src + 2);
        const uint8_t *scales = src + 4, *qh = src + 16, *qs = src + 48;
        for (int j = 0; j < 4; j++) {
            uint8_t sc, m;
            q4k_scale_min(2 * j, scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            q4k_scale_min(2 * j + 1, scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; l++) {
                const int q = (qs[32 * j + l] & 0xF) | (((qh[l] >> (2 * j)) & 1) << 4);
                *y++ = d1 * (float) q - m1;
            }
            for (int l = 0; l < 32; l++) {
                const int q = (qs[32 * j + l] >> 4) | (((qh[l] >> (2 * j + 1)) & 1) << 4);
                *y++ = d2 * (float) q - m2;
            }
        }
    }
}

/* Q6_K: two halves of 128; half h uses ql[64h..64h+64), qh[32h..32h+32) and
 * the int8 scales[8h..8h+8). For l < 32, value 32c + l (c = 0..3) is
 *   nibble (c >= 2 ? high : low) of ql[64h + l + 32(c%2)]
 *   | bits 2c..2c+1 of qh[32h + l] << 4,  minus 32,
 * times d*scales[8h + 2c + l/16]. d*scale (<= 18 bits) and its product with
 * q (<= 23 bits) are exact in fp32. */
static void dequant_q6_k(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, src += 210) {
        const uint8_t *ql = src, *qh = src + 128;
        const int8_t *sc = (const int8_t *) (src + 192);
        const float d = f16_at(src + 208);
        for (int h = 0; h < 2; h++)
            for (int c = 0; c < 4; c++)
                for (int l = 0; l < 32; l++) {
                    const uint8_t lq = ql[64 * h + l + 32 * (c & 1)];
                    const int q = ((c >= 2 ? lq >> 4 : lq & 0xF) | (((qh[32 * h + l] >> (2 * c)) & 3) << 4)) - 32;
                    *y++ = (d * (float) sc[8 * h + 2 * c + l / 16]) * (float) q;
                }
    }
}

/* IQ4_NL and IQ4_XS code into GGUF's sixteen non-uniform levels
 * (ggml-common.h kvalues_iq4nl). */
static const int8_t iq4_grid[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* IQ4_NL (ggml-quants.c dequantize_row_iq4_nl): blocks of 32, byte j of qs
 * holds value j (low nibble) and j + 16 (high); y = d * grid[code]. */
static void dequant_iq4_nl(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 32; b++, src += 18, y += 32) {
        const float d = f16_at(src);
        for (int j = 0; j < 16; j++) {
            y[j] = d * (float) iq4_grid[src[2 + j] & 0xF];
            y[j + 16] = d * (float) iq4_grid[src[2 + j] >> 4];
        }
    }
}

/* IQ4_XS (dequantize_row_iq4_xs): super-blocks of 256 = 8 sub-blocks of 32.
 * Sub-block s: ls = nibble s%2 of scales_l[s/2] | bits 2s..2s+1 of scales_h
 * << 4, dl = d * (ls - 32), y = dl * grid[code], its 16 qs bytes as IQ4_NL's. */
static void dequant_iq4_xs(const uint8_t *src, float *y, int64_t K) {
    for (int64_t b = 0; b < K / 256; b++, src += 136) {
        const float d = f16_at(src);
        const uint16_t sh = (uint16_t) (src[2] | (src[3] << 8));
        const uint8_t *sl = src + 4, *qs = src + 8;
        for (int s = 0; s < 8; s++, qs += 16, y += 32) {
            const int ls = ((sl[s / 2] >> (4 * (s % 2))) & 0xF) | (((sh >> (2 * s)) & 3) << 4);
            const float dl = d * (float) (ls - 32);
            for (int j = 0; j < 16; j++) {
                y[j] = dl * (float) iq4_grid[qs[j] & 0xF];
                y[j + 16] = dl * (float) iq4_grid[qs[j] >> 4];
            }
        }
    }
}

void orc_dequant_row(int type, const void *raw, float *y, int64_t K) {
    const uint8_t *r = (const uint8_t *) raw;
    switch (type) {
        case ORC_TYPE_F32: memcpy(y, raw, (size_t) K * 4); break;
        case ORC_TYPE_F16: dequant_f16(r, y, K); break;
        case ORC_TYPE_BF16: dequant_bf16(r, y, K); break;
        case ORC_TYPE_Q4_0: dequant_q4_0(r, y, K); break;
        case ORC_TYPE_Q4_1: dequant_q4_1(r, y, K); break;
        case ORC_TYPE_Q5_0: dequant_q5_0(r, y, K); break;
        case ORC_TYPE_Q5_1: dequant_q5_1(r, y, K); break;
        case ORC_TYPE_Q8_0: dequant_q8_0(r, y, K); break;
        case ORC_TYPE_Q2_K: dequant_q2_k(r, y, K); break;
        case ORC_TYPE_Q3_K: dequant_q3_k(r, y, K); break;
        case ORC_TYPE_Q4_K: dequant_q4_k(r, y, K); break;
        case ORC_TYPE_Q5_K: dequant_q5_k(r, y, K); break;
        case ORC_TYPE_Q6_K: dequant_q6_k(r, y, K); break;
        case ORC_TYPE_IQ4_NL: dequant_iq4_nl(r, y, K); break;
        case ORC_TYPE_IQ4_XS: dequant_iq4_xs(r, y, K); break;
        default: memset(y, 0, (size_t) K * 4); break;
    }
}

/* ---------------------------------------------------------------------------
 * Synthetic GGUF rows (test inputs, see zest_oracle.h). Each scheme fits a
 * block's range with the type's fields and rounds to the nearest code; the
 * fields are computed from the fp16 values actually stored.
 * ------------------------------------------------------------------------- */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); /* 65520 and up round to infinity */
    if (ax < 0x38800000u) {                                    /* below 2^-14: a subnormal half */
        float v;
        memcpy(&v, &ax, 4);
        return (uint16_t) (sign | (uint32_t) nearbyintf(v * 16777216.0f));
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t) (sign | h);
}

static void put_f16(uint8_t *p, float v, float *stored) {
    const uint16_t h = orc_fp32_to_fp16(v);
    memcpy(p, &h, 2);
    if (stored) *stored = orc_fp16_to_fp32(h);
}

static int clampi(float v, int lo, int hi) {
    const float r = nearbyintf(v);
    return r < (float) lo ? lo : r > (float) hi ? hi : (int) r;
}

static float inv_or_zero(float d) { return d != 0.0f ? 1.0f / d : 0.0f; }

/* the value of largest magnitude, with its sign */
static float signed_absmax(const float *x, int n) {
    float v = 0.0f;
    for (int i = 0; i < n; i++)
        if (fabsf(x[i]) > fabsf(v)) v = x[i];
    return v;
}

static void min_max(const float *x, int n, float *lo, float *hi) {
    *lo = *hi = x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < *lo) *lo = x[i];
        if (x[i] > *hi) *hi = x[i];
    }
}

/* symmetric 32-value blocks: d = v / -half (v the signed absmax), code = q + half */
static void quant_sym32(const float *x, uint8_t *o, int bits, int hdr) {
    const int half = 1 << (bits - 1);
    float d;
    put_f16(o, signed_absmax(x, 32) / (float) -half, &d);
    const float id = inv_or_zero(d);
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        const int lo = clampi(x[j] * id, -half, half - 1) + half, hi = clampi(x[j + 16] * id, -half, half - 1) + half;
        o[hdr + j] = (uint8_t) ((lo & 0xF) | ((hi & 0xF) << 4));
        qh |= (uint32_t) (lo >> 4) << j | (uint32_t) (hi >> 4) << (j + 16);
    }
    if (bits == 5) memcpy(o + 2, &qh, 4);
}

/* affine 32-value blocks: m = min, d = (max - min) / (2^bits - 1) */
static void quant_affine32(const float *x, uint8_t *o, int bits, int hdr) {
    const int top = (1 << bits) - 1;
    float lo, hi, d, m;
    min_max(x, 32, &lo, &hi);
    put_f16(o, (hi - lo) / (float) top, &d);
    put_f16(o + 2, lo, &m);
    const float id = inv_or_zero(d);
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        const int a = clampi((x[j] - m) * id, 0, top), b = clampi((x[j + 16] - m) * id, 0, top);
        o[hdr + j] = (uint8_t) ((a & 0xF) | ((b & 0xF) << 4));
        qh |= (uint32_t) (a >> 4) << j | (uint32_t) (b >> 4) << (j + 16);
    }
    if (bits == 5) memcpy(o + 4, &qh, 4);
}

static void quant_q8_0(const float *x, uint8_t *o) {
    float amax = 0.0f, d;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    put_f16(o, amax / 127.0f, &d);
    const float id = inv_or_zero(d);
    for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t) (int8_t) clampi(x[i] * id, -128, 127);
}

/* Unsigned sub-block codes with a (scale, min) pair per sub-block of n values:
 * m = max(0, -min x), s = (max x + m) / top; the pairs are quantised to
 * `sbits` against super-block scales d = max s / (2^sbits - 1), dmin likewise,
 * then q = round((x + dmin*mq) / (d*sc)) in 0..top. */
static void quant_scale_min(const float *x, int nsub, int n, int top, int sbits, uint8_t *sc, uint8_t *mq, uint8_t *q,
                            uint8_t *d_out, uint8_t *dmin_out) {
    float s[16], m[16], smax = 0.0f, mmax = 0.0f, d, dmin;
    const int stop = (1 << sbits) - 1;
    for (int j = 0; j < nsub; j++) {
        float lo, hi;
        min_max(x + n * j, n, &lo, &hi);
        m[j] = fmaxf(0.0f, -lo);
        s[j] = fmaxf(0.0f, (hi + m[j]) / (float) top);
        smax = fmaxf(smax, s[j]);
        mmax = fmaxf(mmax, m[j]);
    }
    put_f16(d_out, smax / (float) stop, &d);
    put_f16(dmin_out, mmax / (float) stop, &dmin);
    for (int j = 0; j < nsub; j++) {
        sc[j] = (uint8_t) (d > 0.0f ? clampi(s[j] / d, 0, stop) : 0);
        mq[j] = (uint8_t) (dmin > 0.0f ? clampi(m[j] / dmin, 0, stop) : 0);
        const float step = d * sc[j], off = dmin * mq[j], is = inv_or_zero(step);
        for (int i = 0; i < n; i++) q[n * j + i] = (uint8_t) (step > 0.0f ? clampi((x[n * j + i] + off) * is, 0, top) : 0);
    }
}

/* Q4_K / Q5_K's 12 bytes of 6-bit pairs: the inverse of q4k_scale_min */
static void pack_k4_scales(const uint8_t *sc, const uint8_t *mq, uint8_t *S) {
    for (int j = 0; j < 4; j++) {
        S[j] = (uint8_t) (sc[j] | ((sc[j + 4] >> 4) << 6));
        S[j + 4] = (uint8_t) (mq[j] | ((mq[j + 4] >> 4) << 6));
        S[j + 8] = (uint8_t) ((sc[j + 4] & 0xF) | ((mq[j + 4] & 0xF) << 4));
    }
}

static void quant_q4_k(const float *x, uint8_t *o) {
    uint8_t sc[8], mq[8], q[256];
    quant_scale_min(x, 8, 32, 15, 6, sc, mq, q, o, o + 2);
    pack_k4_scales(sc, mq, o + 4);
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++) o[16 + 32 * j + l] = (uint8_t) (q[64 * j + l] | (q[64 * j + 32 + l] << 4));
}

static void quant_q5_k(const float *x, uint8_t *o) {
    uint8_t sc[8], mq[8], q[256];
    quant_scale_min(x, 8, 32, 31, 6, sc, mq, q, o, o + 2);
    pack_k4_scales(sc, mq, o + 4);
    memset(o + 16, 0, 32);
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++) {
            const uint8_t a = q[64 * j + l], b = q[64 * j + 32 + l];
            o[48 + 32 * j + l] = (uint8_t) ((a & 0xF) | ((b & 0xF) << 4));
            o[16 + l] |= (uint8_t) (((a >> 4) << (2 * j)) | ((b >> 4) << (2 * j + 1)));
        }
}

static void quant_q2_k(const float *x, uint8_t *o) {
    uint8_t sc[16], mq[16], q[256];
    quant_scale_min(x, 16, 16, 3, 4, sc, mq, q, o + 80, o + 82);
    memset(o + 16, 0, 64);
    for (int h = 0; h < 2; h++)
        for (int g = 0; g < 8; g++) {
            o[8 * h + g] = (uint8_t) (sc[8 * h + g] | (mq[8 * h + g] << 4));
            for (int l = 0; l < 16; l++)
                o[16 + 32 * h + 16 * (g & 1) + l] |= (uint8_t) (q[128 * h + 16 * g + l] << (2 * (g >> 1)));
        }
}

/* Signed sub-blocks of 16 with an integer scale each: s = v / -2^(qbits-1)
 * (v the signed absmax), d = max|s| / smax, sc = round(s/d) in [-smax-1, smax],
 * q = round(x / (d*sc)) in [-2^(qbits-1), 2^(qbits-1) - 1]. */
static void quant_signed16(const float *x, int qbits, int smax, int *sc, int *q, uint8_t *d_out) {
    const int half = 1 << (qbits - 1);
    float s[16], amax = 0.0f, d;
    for (int g = 0; g < 16; g++) {
        s[g] = signed_absmax(x + 16 * g, 16) / (float) -half;
        amax = fmaxf(amax, fabsf(s[g]));
    }
    put_f16(d_out, amax / (float) smax, &d);
    const float id = inv_or_zero(d);
    for (int g = 0; g < 16; g++) {
        sc[g] = clampi(s[g] * id, -smax - 1, smax);
        const float il = inv_or_zero(d * (float) sc[g]);
        for (int l = 0; l < 16; l++) q[16 * g + l] = clampi(x[16 * g + l] * il, -half, half - 1);
    }
}

static void quant_q3_k(const float *x, uint8_t *o) {
    int sc[16], q[256];
    quant_signed16(x, 3, 31, sc, q, o + 108);
    memset(o, 0, 108);
    for (int i = 0; i < 16; i++) {
        const int u = sc[i] + 32;
        o[96 + (i & 7)] |= (uint8_t) ((u & 0xF) << (i < 8 ? 0 : 4));
        o[96 + 8 + (i & 3)] |= (uint8_t) ((u >> 4) << (2 * (i >> 2)));
    }
    for (int h = 0; h < 2; h++)
        for (int g = 0; g < 8; g++)
            for (int l = 0; l < 16; l++) {
                const int v = q[128 * h + 16 * g + l], j = g >> 1, off = 16 * (g & 1) + l;
                o[32 + 32 * h + off] |= (uint8_t) ((v & 3) << (2 * j)); /* v + 4 and v agree in the low 2 bits */
                if (v >= 0) o[off] |= (uint8_t) (1u << (4 * h + j));
            }
}

static void quant_q6_k(const float *x, uint8_t *o) {
    int sc[16], q[256];
    quant_signed16(x, 6, 127, sc, q, o + 208);
    memset(o, 0, 192);
    for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t) (int8_t) sc[i];
    for (int h = 0; h < 2; h++)
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                const int u = q[128 * h + 32 * c + l] + 32;
                o[64 * h + l + 32 * (c & 1)] |= (uint8_t) ((u & 0xF) << (c >= 2 ? 4 : 0));
                o[128 + 32 * h + l] |= (uint8_t) ((u >> 4) << (2 * c));
            }
}

/* the grid level nearest x */
static int iq4_nearest(float x) {
    int best = 0;
    for (int i = 1; i < 16; i++)
        if (fabsf(x - (float) iq4_grid[i]) < fabsf(x - (float) iq4_grid[best])) best = i;
    return best;
}

/* IQ4_NL: d = v / -127 (v the signed absmax, so it lands on level -127) */
static void quant_iq4_nl(const float *x, uint8_t *o) {
    float d;
    put_f16(o, signed_absmax(x, 32) / -127.0f, &d);
    const float id = inv_or_zero(d);
    for (int j = 0; j < 16; j++)
        o[2 + j] = (uint8_t) (iq4_nearest(x[j] * id) | (iq4_nearest(x[j + 16] * id) << 4));
}

/* IQ4_XS: each sub-block's own d_s = v_s / -127 against d = max|d_s| / 32,
 * ls - 32 = round(d_s / d) in [-32, 31] */
static void quant_iq4_xs(const float *x, uint8_t *o) {
    float ds[8], amax = 0.0f, d;
    for (int s = 0; s < 8; s++) {
        ds[s] = signed_absmax(x + 32 * s, 32) / -127.0f;
        amax = fmaxf(amax, fabsf(ds[s]));
    }
    put_f16(o, amax / 32.0f, &d);
    const float id = inv_or_zero(d);
    uint16_t sh = 0;
    memset(o + 4, 0, 4);
    for (int s = 0; s < 8; s++) {
        const int ls = clampi(ds[s] * id, -32, 31) + 32;
        o[4 + s / 2] |= (uint8_t) ((ls & 0xF) << (4 * (s % 2)));
        sh |= (uint16_t) ((ls >> 4) << (2 * s));
        const float il = inv_or_zero(d * (float) (ls - 32));
        for (int j = 0; j < 16; j++)
            o[8 + 16 * s + j] =
                (uint8_t) (iq4_nearest(x[32 * s + j] * il) | (iq4_nearest(x[32 * s + j + 16] * il) << 4));
    }
    memcpy(o + 2, &sh, 2);
}

int orc_quantize_row(int type, const float *x, void *out, int64_t K) {
    uint8_t *o = (uint8_t *) out;
    const size_t rb = orc_row_bytes(type, K);
    if (rb == 0 || K <= 0) return -1;
    switch (type) {
        case ORC_TYPE_F32: memcpy(o, x, rb); return 0;
        case ORC_TYPE_F16:
            for (int64_t i = 0; i < K; i++) put_f16(o + 2 * i, x[i], NULL);
            return 0;
        case ORC_TYPE_BF16:
            for (int64_t i = 0; i < K; i++) {
                uint32_t u;
                memcpy(&u, &x[i], 4);
                const uint16_t h = (uint16_t) ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
                memcpy(o + 2 * i, &h, 2);
            }
            return 0;
        default: break;
    }
    const int blk = type == ORC_TYPE_Q2_K || type == ORC_TYPE_Q3_K || type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q5_K ||
                            type == ORC_TYPE_Q6_K || type == ORC_TYPE_IQ4_XS
                        ? 256
                        : 32;
    if (K % blk) return -1;
    const size_t bb = rb / (size_t) (K / blk);
    for (int64_t b = 0; b < K / blk; b++, x += blk, o += bb) switch (type) {
            case ORC_TYPE_Q4_0: quant_sym32(x, o, 4, 2); break;
            case ORC_TYPE_Q5_0: quant_sym32(x, o, 5, 6); break;
            case ORC_TYPE_Q4_1: quant_affine32(x, o, 4, 4); break;
            case ORC_TYPE_Q5_1: quant_affine32(x, o, 5, 8); break;
            case ORC_TYPE_Q8_0: quant_q8_0(x, o); break;
            case ORC_TYPE_Q2_K: quant_q2_k(x, o); break;
            case ORC_TYPE_Q3_K: quant_q3_k(x, o); break;
            case ORC_TYPE_Q4_K: quant_q4_k(x, o); break;
            case ORC_TYPE_Q5_K: quant_q5_k(x, o); break;
            case ORC_TYPE_Q6_K: quant_q6_k(x, o); break;
            case ORC_TYPE_IQ4_NL: quant_iq4_nl(x, o); break;
            case ORC_TYPE_IQ4_XS: quant_iq4_xs(x, o); break;
            default: return -1;
        }
    return 0;
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

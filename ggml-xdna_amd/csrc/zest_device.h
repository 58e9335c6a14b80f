// Device helpers shared by the kernels: the bfp16 block encoder and the
// lossless bfp16 -> bf16 expansion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "zest_hip.h"
#include "zest_layout.h"

namespace zest {

// One block of eight floats -> exponent byte (returned) and eight mantissa
// bytes (m0 = bytes 0..3, m1 = bytes 4..7). The reference's arithmetic
// (src/npu/bfp16_pack.cpp:85-127): e = the largest biased exponent field;
// q = RNE(x * 2^(133 - e)) saturated to [-128, 127].
//
// For e in 6..254 (every finite block but the tiniest) 2^(133-e) is a normal
// float s, and one fma computes x*s exactly and adds 1.5 * 2^23, whose
// binade has ulp 1: the sum is 1.5 * 2^23 + q with q = RNE(x*s) (|x*s| < 128,
// so it stays in the binade), and q's two's-complement byte is the sum's low
// byte (1.5 * 2^23 has a zero low byte). med3 on the sum saturates q to
// [-128, 127]; v_perm gathers the low bytes. Three VALU ops per value.
// Other blocks (zeros and subnormals, infinities, NaN) take the direct form:
// ldexp (exact: |x * 2^(133-e)| < 128, and anything it would round in
// underflow is below one half), rint to nearest even, med3.
__device__ inline uint32_t lo_bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u), cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Mantissas of a block whose exponent byte e is known.
__device__ inline void encode8_mant(const float v[8], uint32_t e, uint32_t & m0, uint32_t & m1) {
    if (__builtin_expect(e - 6u < 249u, 1)) {
        constexpr float MAGIC = 12582912.0f;  // 1.5 * 2^23
        const float s = __uint_as_float((260u - e) << 23);  // 2^(133 - e)
        uint32_t t[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            t[i] = __float_as_uint(__builtin_amdgcn_fmed3f(fmaf(v[i], s, MAGIC), MAGIC - 128.0f, MAGIC + 127.0f));
        m0 = lo_bytes4(t[0], t[1], t[2], t[3]);
        m1 = lo_bytes4(t[4], t[5], t[6], t[7]);
        return;
    }
    const int sh = 133 - (int) e;
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(__builtin_ldexpf(v[i], sh)), -128.0f, 127.0f);
        b[i] = (uint32_t) (int32_t) q & 0xffu;
    }
    m0 = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    m1 = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
}

__device__ inline uint32_t encode8(const float v[8], uint32_t & m0, uint32_t & m1) {
    uint32_t e = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) e = max(e, (__float_as_uint(v[i]) >> 23) & 0xffu);
    encode8_mant(v, e, m0, m1);
    return e;
}

// encode8 for a block that holds no NaN: the largest exponent field is the
// exponent of the largest magnitude (v_max3_f32 with free abs modifiers, four
// ops for the eight values; a NaN would be skipped by the max, which is why
// the general encoder reads the fields one by one).
__device__ inline uint32_t encode8_no_nan(const float v[8], uint32_t & m0, uint32_t & m1) {
    const float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fabsf(v[2]));
    const float b = fmaxf(fmaxf(a, fabsf(v[3])), fabsf(v[4]));
    const float c = fmaxf(fmaxf(b, fabsf(v[5])), fabsf(v[6]));
    const uint32_t e = __float_as_uint(fmaxf(c, fabsf(v[7]))) >> 23;
    encode8_mant(v, e, m0, m1);
    return e;
}

// 2^(e - 133) as a float: normal for e >= 7, subnormal below.
__device__ inline float block_scale(uint32_t e) {
    return e >= 7u ? __uint_as_float((e - 6u) << 23) : __uint_as_float(1u << (e + 16u));
}

// Eight mantissas (two dwords) with one exponent -> eight bf16 (four dwords),
// each exactly the decoded value q * 2^(e-133) (bfp16_decode_block,
// src/npu/bfp16_pack.cpp:129-144). A signed 8-bit mantissa times a power of
// two has at most 8 significant bits, so it is exact in bf16; the bf16 is the
// top half of the exact float (whose low half is zero).
//
// For exponent bytes 7..253 (every block of realistic data) 2^(e-133) and
// 128 * 2^(e-133) are normal floats: each byte is read unsigned after
// flipping its sign bit (u = q + 128) and fma(u, s, -128 s) = q * s exactly,
// two VALU ops per value. The other bytes (zero and tiny blocks, 0..6; the
// top of the float range, 254..255) take the plain q * s, where fp32
// rounding of the product gives what the reference's decode gives.
__device__ inline void expand8(uint32_t w0, uint32_t w1, uint32_t e, uint32_t out[4]) {
    const float s = block_scale(e);
    float f[8];
    if (__builtin_expect(e - 7u < 247u, 1)) {
        const float off = -128.0f * s;
        const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
        f[0] = fmaf((float) (u0 & 0xffu), s, off);
        f[1] = fmaf((float) ((u0 >> 8) & 0xffu), s, off);
        f[2] = fmaf((float) ((u0 >> 16) & 0xffu), s, off);
        f[3] = fmaf((float) (u0 >> 24), s, off);
        f[4] = fmaf((float) (u1 & 0xffu), s, off);
        f[5] = fmaf((float) ((u1 >> 8) & 0xffu), s, off);
        f[6] = fmaf((float) ((u1 >> 16) & 0xffu), s, off);
        f[7] = fmaf((float) (u1 >> 24), s, off);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            f[i] = (float) (int8_t) (w0 >> (8 * i)) * s;
            f[4 + i] = (float) (int8_t) (w1 >> (8 * i)) * s;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __builtin_amdgcn_perm(__float_as_uint(f[2 * i + 1]), __float_as_uint(f[2 * i]), 0x07060302u);
}

typedef unsigned short zest_u16x2 __attribute__((ext_vector_type(2)));

// Sixteen mantissas (one 16-byte unit: two blocks) with their two exponent
// bytes -> sixteen bf16, the same values as expand8 with fewer VALU ops when
// both exponent bytes are in 7..133 (blocks whose largest magnitude is below
// 128 and above 2^-120: the activations and weights of real models):
//   float(q) by a byte-select convert with sign extension (exact), its top
//   half is bf16(q) (exact: |q| <= 128 has at most 8 significant bits), and
//   q * 2^(e-133) is that bf16 with (133 - e) subtracted from its exponent
//   field: a 16-bit saturating subtract on both halves of a dword. The
//   exponent field of a nonzero bf16(q) is at least 127 and 133 - e is at
//   most 126, so the sign bit never borrows, and q = 0 saturates to 0.
// Two ops per value. Other exponent bytes go through expand8.
//
// expand16_fast is that fast path alone, branch-free so it can be scheduled
// between MFMAs; it returns true when the unit needs expand8 instead (its
// output is then not the decoded values and must be replaced).
__device__ inline bool expand16_fast(const uint4 & m, uint32_t e2, uint32_t out[8]) {
    // (133 - e) << 7 for each block
    const int32_t d0 = 133 * 128 - (int32_t) ((e2 & 0xffu) << 7);
    const int32_t d1 = 133 * 128 - (int32_t) ((e2 >> 8) << 7);
    const zest_u16x2 dv0 = {(unsigned short) d0, (unsigned short) d0};
    const zest_u16x2 dv1 = {(unsigned short) d1, (unsigned short) d1};
    const uint32_t w[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t wd = w[i >> 1];
        const int sh = (i & 1) * 16;
        const float lo = (float) (int8_t) (wd >> sh), hi = (float) (int8_t) (wd >> (sh + 8));
        const uint32_t b = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
        const zest_u16x2 r = __builtin_elementwise_sub_sat(__builtin_bit_cast(zest_u16x2, b), i < 4 ? dv0 : dv1);
        out[i] = __builtin_bit_cast(uint32_t, r);
    }
    // exponent bytes 7..133 <=> 0 <= (133 - e) * 128 <= 126 * 128
    return max((uint32_t) d0, (uint32_t) d1) > 126u * 128u;
}

__device__ inline void expand16(const uint4 & m, uint32_t e2, uint32_t out[8]) {
    const uint32_t e0 = e2 & 0xffu, e1 = e2 >> 8;
    if (__builtin_expect((e0 - 7u <= 126u) & (e1 - 7u <= 126u), 1)) {
        const uint32_t d0 = (133u - e0) * 0x00800080u, d1 = (133u - e1) * 0x00800080u;
        const uint32_t w[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t wd = w[i >> 1];
            const int sh = (i & 1) * 16;
            const float lo = (float) (int8_t) (wd >> sh), hi = (float) (int8_t) (wd >> (sh + 8));
            const uint32_t b = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
            const zest_u16x2 r = __builtin_elementwise_sub_sat(__builtin_bit_cast(zest_u16x2, b),
                                                               __builtin_bit_cast(zest_u16x2, i < 4 ? d0 : d1));
            out[i] = __builtin_bit_cast(uint32_t, r);
        }
    } else {
        expand8(m.x, m.y, e0, out);
        expand8(m.z, m.w, e1, out + 4);
    }
}

// e^-x as the hardware exp2 of -x log2(e) (v_exp_f32, about 1 ulp), and
// 1 / (1 + e^-x) through the hardware reciprocal (v_rcp_f32, 1 ulp): the
// logistic function in 4 VALU ops, against about 30 for libm's expf and a
// correctly rounded divide. Its relative error (a few ulp, ~3e-7) is far
// inside the 1e-5 nrmse the host ops are held to against the CPU's
// x / (1 + expf(-x)). x -> -inf gives 1 / inf = 0, x -> +inf gives 1.
__device__ inline float sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// The GLU of one gate value g and up value u (src/xdna-exec.cpp:296-320):
// act(g) * u, ReGLU as g > 0 ? g * u : 0. Shared by the GLU kernel and the
// fused gate/up GEMM's epilogue, so both give the same floats.
__device__ inline float glu(int kind, float g, float u) {
    switch (kind) {
        case ZEST_GLU_SWIGLU: return g * sigmoid(g) * u;
        case ZEST_GLU_GEGLU: return 0.5f * g * (1.0f + tanhf(0.7978845608f * g * (1.0f + 0.044715f * g * g))) * u;
        case ZEST_GLU_GEGLU_ERF: return 0.5f * g * (1.0f + erff(g * 0.7071067812f)) * u;
        case ZEST_GLU_GEGLU_QUICK: return g * sigmoid(1.702f * g) * u;
        default: return g > 0.0f ? g * u : 0.0f;
    }
}

// Encodes 16 values (two blocks) and writes them decoded into row r, columns
// [col, col+16) of an expanded operand (col % 16 == 0): the 32 contiguous
// bytes of the row in its sub-tile, as two 16-byte stores of the bf16 values
// the packed bytes stand for.
__device__ inline void store_expanded16(uint8_t * xop, int64_t R_pad, int64_t r, int64_t col, const float v[16]) {
    uint4 m;
    const uint32_t e0 = encode8(v, m.x, m.y);
    const uint32_t e1 = encode8(v + 8, m.z, m.w);
    uint32_t b[8];
    expand16(m, e0 | (e1 << 8), b);
    uint4 * p = reinterpret_cast<uint4 *>(xop + zest_xoffset(r, col, R_pad));
    p[0] = make_uint4(b[0], b[1], b[2], b[3]);
    p[1] = make_uint4(b[4], b[5], b[6], b[7]);
}

} // namespace zest

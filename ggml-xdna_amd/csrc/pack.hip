// The HBM-bound converters of the path:
//   zest_pack_act        fp32 activations -> packed bfp16 (per chunk)
//   zest_pack_act_x      fp32 activations -> the GEMM's expanded operand: the
//                        same bfp16 blocks, stored decoded as bf16
//   zest_expand_act      packed bfp16 -> expanded operand
//   zest_convert_weight  GGUF weights (F32, F16, BF16, Q4_0..Q8_0, Q2_K..Q6_K, IQ4_NL, IQ4_XS)
//                        -> packed bfp16 (once, into the resident weight cache)
// All write the layouts of zest_layout.h with 16-byte stores.
#include "zest_common.h"
#include "zest_device.h"

namespace {

using zest::encode8;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Row r of a weight in the packed operand: itself, or (gu = 0 / 1) its place
// in a gate/up pair interleaved by 32-row groups: rows 64g..64g+31 hold gate
// rows 32g..32g+31 and rows 64g+32..64g+63 the matching up rows (the
// reference's bfp16_interleave_gate_up, src/npu/bfp16_pack.cpp:231-237, at
// the GEMM's 32-row MFMA granularity), so one output tile of the fused GEMM
// holds a gate value and its up value in the same lane.
__device__ inline int64_t dst_row(int64_t r, int gu) { return gu < 0 ? r : (r >> 5) * 64 + gu * 32 + (r & 31); }

// One workgroup packs a 16-row band of 256 columns (four tiles). Load i reads
// columns 64i..64i+63 of the band (a column past K reads as zero): thread t
// takes row t/16 and the 4 floats
// at column 64i + 4(t%16), so the 16 threads of a row read 256 contiguous
// bytes. A bfp16 block is 8 columns, two threads: the pair's exponent is the
// larger of their two maxima (one lane exchange); each thread then encodes
// its 4 values exactly as encode8 does, into one mantissa dword at tile i,
// row t/16, byte 4(t%16), so a wave's store covers 4 whole tile rows (256
// contiguous bytes). The 8 exponent bytes of a tile row come from threads
// t%16 = 0 and 8, which gather 4 each and store a dword. Rows past M and
// columns past K become zero blocks.
// XOUT: write the expanded operand instead (the 4 decoded values as bf16,
// 8 bytes, in row t/16's 32 bytes of the sub-tile: a wave's store covers four
// 128-byte runs, one per 16-column quarter).
// STREAM: read x with nontemporal loads, for inputs too large to be held in
// the 256 MB MALL; a smaller input (an activation its producer has just
// written) is read with ordinary loads, which find it there (2048 x 4096 to
// the expanded operand: 9.1 -> 6.8 us with ordinary loads when x is
// resident; 8192 x 5120 from HBM: 41 us with nontemporal loads, 44 us with
// ordinary ones).
template <bool XOUT, bool STREAM>
__global__ __launch_bounds__(256) void pack_act_kernel(const float * __restrict__ x, int64_t M, int64_t K, int64_t ldx,
                                                       uint8_t * __restrict__ dst, int64_t R_pad, int64_t K_pad, int gu) {
    const int t = threadIdx.x, j = t & 15, rr = t >> 4;
    const int64_t r = (int64_t) blockIdx.y * ZEST_TILE_ROWS + rr;
    const int64_t rt = dst_row((int64_t) blockIdx.y * ZEST_TILE_ROWS, gu) / ZEST_TILE_ROWS;  // 16-row groups stay whole
    const bool row_ok = r < M, vec = (ldx & 3) == 0;
    // all four loads first, then the encodes: 64 bytes in flight per thread
    float va[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t col = (int64_t) blockIdx.x * 256 + i * 64 + j * 4;
        if (row_ok && col + 4 <= K && vec) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            const f32x4 * p = reinterpret_cast<const f32x4 *>(x + r * ldx + col);
            const f32x4 q = STREAM ? __builtin_nontemporal_load(p) : *p;
            va[i][0] = q.x;
            va[i][1] = q.y;
            va[i][2] = q.z;
            va[i][3] = q.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) va[i][q] = (row_ok && col + q < K) ? x[r * ldx + col + q] : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t c0 = (int64_t) blockIdx.x * 256 + i * 64;  // the tile's first column
        if (c0 >= K_pad) break;
        const float * v = va[i];
        uint32_t e = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) e = max(e, (__float_as_uint(v[q]) >> 23) & 0xffu);
        e = max(e, (uint32_t) __shfl_xor((int) e, 1));
        const int sh = 133 - (int) e;
        int32_t qi[4];
#pragma unroll
        for (int q = 0; q < 4; q++)
            qi[q] = (int32_t) __builtin_amdgcn_fmed3f(__builtin_rintf(__builtin_ldexpf(v[q], sh)), -128.0f, 127.0f);
        const int64_t kc = c0 / ZEST_TILE_K;
        if (XOUT) {
            // q * 2^(e-133) is exact in fp32 and in bf16 (at most 8 significant bits)
            const float sc = zest::block_scale(e);
            uint32_t b[4];
#pragma unroll
            for (int q = 0; q < 4; q++) b[q] = __float_as_uint((float) qi[q] * sc) >> 16;
            // nontemporal: the operand is written once per chunk and read by the GEMMs after
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 bb = {b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
            __builtin_nontemporal_store(
                bb, reinterpret_cast<u32x2 *>(dst + zest_xoffset(rt * ZEST_TILE_ROWS + rr, c0 + j * 4, R_pad)));
        } else {
            uint8_t * tile = dst + zest_tile_offset(rt, kc, R_pad);
            *reinterpret_cast<uint32_t *>(tile + rr * ZEST_TILE_K + j * 4) =
                ((uint32_t) qi[0] & 0xffu) | (((uint32_t) qi[1] & 0xffu) << 8) | (((uint32_t) qi[2] & 0xffu) << 16) |
                (((uint32_t) qi[3] & 0xffu) << 24);
            // blocks j/2, j/2+1, j/2+2, j/2+3 of the row, from threads j, j+2, j+4, j+6
            const uint32_t e1 = (uint32_t) __shfl_down((int) e, 2), e2 = (uint32_t) __shfl_down((int) e, 4),
                           e3 = (uint32_t) __shfl_down((int) e, 6);
            if ((j & 7) == 0)
                *reinterpret_cast<uint32_t *>(tile + ZEST_TILE_MANT + rr * 8 + (j >> 3) * 4) =
                    e | (e1 << 8) | (e2 << 16) | (e3 << 24);
        }
    }
}

// One thread per 16-value unit of a packed operand: its mantissas and two
// exponent bytes -> 16 bf16 of the expanded operand (32 contiguous bytes).
__global__ __launch_bounds__(256) void expand_act_kernel(const uint8_t * __restrict__ src, uint8_t * __restrict__ dst,
                                                         int64_t units, int64_t R_pad) {
    const int64_t u = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const int64_t tile = u / 64, c = u % 64;  // unit c of a tile: row c/4, 16-column quarter c%4
    const int64_t tiles_per_chunk = R_pad / ZEST_TILE_ROWS;
    const int64_t r = (tile % tiles_per_chunk) * ZEST_TILE_ROWS + c / 4;
    const int64_t col = (tile / tiles_per_chunk) * ZEST_TILE_K + (c % 4) * 16;
    const uint8_t * t = src + tile * ZEST_TILE_BYTES;
    const uint4 m = *reinterpret_cast<const uint4 *>(t + c * 16);
    const uint32_t e = *reinterpret_cast<const uint16_t *>(t + ZEST_TILE_MANT + c * 2);
    uint32_t b[8];
    zest::expand16(m, e, b);
    uint4 * p = reinterpret_cast<uint4 *>(dst + zest_xoffset(r, col, R_pad));
    p[0] = make_uint4(b[0], b[1], b[2], b[3]);
    p[1] = make_uint4(b[4], b[5], b[6], b[7]);
}

__device__ inline float half_to_float(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }

// ---- every GGUF type: one thread per half tile row ----------------------------
// One thread dequantises 32 consecutive values of a row (col % 32 == 0) as
// ggml's to_float does and encodes them (four bfp16 blocks). Every product
// below is exact in fp32 (an fp16 scale times integers of at most 8 bits,
// or a 6-bit scale product times at most 6 bits), so each form written as
// fma(u, d, c) with an offset code u = q + bias gives the reference's value:
// where the reference computes d*q exactly (Q4_0, Q5_0, Q8_0, Q3_K, Q6_K),
// the fma's exact result is representable and no rounding happens; where it
// adds an offset after an exact product (Q4_1, Q5_1, Q2_K, Q4_K, Q5_K), the
// one rounding is the same addition's.
//
// Codes are assembled four at a time, one per byte of a 32-bit word, so
// each value costs one byte-to-float convert (v_cvt_f32_ubyte0..3) and one
// fma. `finite` says the block's scale fields are finite, so its values hold
// no NaN and the encoder may take the exponent from the largest magnitude.

__device__ inline uint32_t ld16(const uint8_t * p) { return *reinterpret_cast<const uint16_t *>(p); }  // 2-aligned
__device__ inline uint32_t ld32(const uint8_t * p) { return *reinterpret_cast<const uint32_t *>(p); }  // 4-aligned
__device__ inline uint32_t ld32h(const uint8_t * p) { return ld16(p) | (ld16(p + 2) << 16); }          // 2-aligned
__device__ inline uint32_t byte_of(const uint32_t * w, int i) { return (w[i >> 2] >> ((i & 3) * 8)) & 0xffu; }

// v[0..3] = fma(byte k of u, d, c). The empty asm hides how u was masked,
// so each byte converts with one v_cvt_f32_ubyte<k> (the compiler would
// otherwise fold the mask into a bit-field extract plus a convert).
__device__ inline void fma_bytes(uint32_t u, float d, float c, float * v) {
    asm("" : "+v"(u));
    v[0] = fmaf((float) (u & 0xffu), d, c);
    v[1] = fmaf((float) ((u >> 8) & 0xffu), d, c);
    v[2] = fmaf((float) ((u >> 16) & 0xffu), d, c);
    v[3] = fmaf((float) (u >> 24), d, c);
}

// bits 0..3 of x -> bit 0 of bytes 0..3 (the four terms x << 7k do not overlap)
__device__ inline uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }

__device__ inline bool finite(float x) { return __builtin_isfinite(x); }

// IQ4_NL / IQ4_XS: four codes (0..15, one a byte) -> their levels + 128 as
// unsigned bytes. The sixteen levels are GGUF's non-uniform 4-bit grid
// (ggml-common.h kvalues_iq4nl): -127 -104 -83 -65 -49 -35 -22 -10 1 13 25
// 38 53 69 89 113. Two byte permutes look up the low and the high eight, and
// bit 3 of each code picks between them.
__device__ inline uint32_t iq4_levels(uint32_t n) {
    constexpr uint32_t T0 = 1u | 24u << 8 | 45u << 16 | 63u << 24, T1 = 79u | 93u << 8 | 106u << 16 | 118u << 24;
    constexpr uint32_t T2 = 129u | 141u << 8 | 153u << 16 | 166u << 24, T3 = 181u | 197u << 8 | 217u << 16 | 241u << 24;
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// 32-value blocks: byte j of qs holds value j (low nibble) and j + 16 (high);
// bit j of the little-endian 32-bit qh is value j's fifth bit.
template <int TYPE>
__device__ inline bool dq_32(const uint8_t * p, float * v) {
    constexpr bool Q5 = TYPE == ZEST_TYPE_Q5_0 || TYPE == ZEST_TYPE_Q5_1;
    constexpr bool AFFINE = TYPE == ZEST_TYPE_Q4_1 || TYPE == ZEST_TYPE_Q5_1;  // y = d*q + m
    float d, c;
    uint32_t qh = 0, qs[4];
    if (TYPE == ZEST_TYPE_Q4_0) {  // d, qs[16]: 18 bytes
        d = half_to_float((uint16_t) ld16(p));
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32h(p + 2 + 4 * i);
    } else if (TYPE == ZEST_TYPE_Q4_1) {  // d, m, qs[16]: 20 bytes
        const uint32_t h = ld32(p);
        d = half_to_float((uint16_t) (h & 0xffff));
        c = half_to_float((uint16_t) (h >> 16));
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32(p + 4 + 4 * i);
    } else if (TYPE == ZEST_TYPE_Q5_0) {  // d, qh[4], qs[16]: 22 bytes
        d = half_to_float((uint16_t) ld16(p));
        qh = ld32h(p + 2);
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32h(p + 6 + 4 * i);
    } else {  // Q5_1: d, m, qh[4], qs[16]: 24 bytes
        const uint32_t h = ld32(p);
        d = half_to_float((uint16_t) (h & 0xffff));
        c = half_to_float((uint16_t) (h >> 16));
        qh = ld32(p + 4);
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32(p + 8 + 4 * i);
    }
    if (!AFFINE) c = (Q5 ? -16.0f : -8.0f) * d;  // signed codes: y = d*(u - bias)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t lo = qs[i] & 0x0F0F0F0Fu, hi = (qs[i] >> 4) & 0x0F0F0F0Fu;
        if (Q5) {
            lo |= spread4(qh >> (4 * i)) << 4;
            hi |= spread4(qh >> (16 + 4 * i)) << 4;
        }
        fma_bytes(lo, d, c, v + 4 * i);
        fma_bytes(hi, d, c, v + 16 + 4 * i);
    }
    return AFFINE ? finite(d) && finite(c) : finite(d);
}

// Values [col, col + 32) of one row (col % 32 == 0, col < K): half a tile
// row. Returns whether they are NaN-free by construction.
template <int TYPE>
__device__ inline bool dq_half(const uint8_t * row, int64_t col, int64_t K, float v[32]) {
    if (TYPE == ZEST_TYPE_F16 || TYPE == ZEST_TYPE_BF16) {
        // K % 8 == 0 but maybe not % 32: 8-value chunks past K read as zero
        const uint4 * p = reinterpret_cast<const uint4 *>(row + col * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 q = col + 8 * i < K ? p[i] : make_uint4(0, 0, 0, 0);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (TYPE == ZEST_TYPE_F16) {
                    v[8 * i + 2 * k] = half_to_float((uint16_t) (w[k] & 0xffff));
                    v[8 * i + 2 * k + 1] = half_to_float((uint16_t) (w[k] >> 16));
                } else {
                    v[8 * i + 2 * k] = __uint_as_float(w[k] << 16);
                    v[8 * i + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
                }
            }
        }
        return false;  // the values are the file's own: NaN is possible
    } else if (TYPE == ZEST_TYPE_Q4_0 || TYPE == ZEST_TYPE_Q4_1 || TYPE == ZEST_TYPE_Q5_0 ||
               TYPE == ZEST_TYPE_Q5_1) {
        constexpr int B = TYPE == ZEST_TYPE_Q4_0 ? 18 : TYPE == ZEST_TYPE_Q4_1 ? 20 : TYPE == ZEST_TYPE_Q5_0 ? 22 : 24;
        return dq_32<TYPE>(row + (col / 32) * B, v);
    } else if (TYPE == ZEST_TYPE_IQ4_NL || TYPE == ZEST_TYPE_IQ4_XS) {
        // IQ4_NL: d, qs[16] (18 bytes), y = d*level[q]. IQ4_XS: d,
        // scales_h, scales_l[4], qs[128] (136 bytes); sub-block s (32
        // values) has the 6-bit scale ls = nibble s%2 of scales_l[s/2] |
        // bits 2s..2s+1 of scales_h << 4, dl = d*(ls - 32), y = dl*level[q].
        // Byte j of a block's (sub-block's) 16 qs holds value j (low nibble)
        // and j + 16 (high). d*(ls - 32) has at most 17 significant bits and
        // its product with a level at most 24, so both are exact, and
        // fma(level + 128, dl, -128*dl) is the reference's product.
        float d;
        bool ok;
        uint32_t qs[4];
        if (TYPE == ZEST_TYPE_IQ4_NL) {
            const uint8_t * p = row + (col / 32) * 18;
            d = half_to_float((uint16_t) ld16(p));
            ok = finite(d);
#pragma unroll
            for (int i = 0; i < 4; i++) qs[i] = ld32h(p + 2 + 4 * i);
        } else {
            const int s = (int) ((col % 256) / 32);
            const uint8_t * p = row + (col / 256) * 136;  // rows 8-byte aligned
            const uint2 hdr = *reinterpret_cast<const uint2 *>(p);
            const uint2 qa = *reinterpret_cast<const uint2 *>(p + 8 + 16 * s);
            const uint2 qb = *reinterpret_cast<const uint2 *>(p + 16 + 16 * s);
            const float d0 = half_to_float((uint16_t) (hdr.x & 0xffff));
            const uint32_t ls = ((hdr.y >> (4 * s)) & 0xFu) | (((hdr.x >> (16 + 2 * s)) & 3u) << 4);
            d = d0 * (float) ((int) ls - 32);
            ok = finite(d0);
            qs[0] = qa.x;
            qs[1] = qa.y;
            qs[2] = qb.x;
            qs[3] = qb.y;
        }
        const float c = -128.0f * d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            fma_bytes(iq4_levels(qs[i] & 0x0F0F0F0Fu), d, c, v + 4 * i);
            fma_bytes(iq4_levels((qs[i] >> 4) & 0x0F0F0F0Fu), d, c, v + 16 + 4 * i);
        }
        return ok;
    } else if (TYPE == ZEST_TYPE_Q8_0) {
        // d, qs[32]: 34 bytes; y = d*q = d*(u - 128) with u = q ^ 0x80
        const uint8_t * p = row + (col / 32) * 34;
        const float d = half_to_float((uint16_t) ld16(p)), c = -128.0f * d;
#pragma unroll
        for (int i = 0; i < 8; i++) fma_bytes(ld32h(p + 2 + 4 * i) ^ 0x80808080u, d, c, v + 4 * i);
        return finite(d);
    } else if (TYPE == ZEST_TYPE_Q2_K || TYPE == ZEST_TYPE_Q3_K) {
        // Q2_K: scales[16], qs[64], d, dmin (84 bytes); Q3_K: hmask[32],
        // qs[64], scales[12], d (110 bytes). Eighth e8 = half h, shift 2j
        // (j = e8 % 4): groups g = 2j (qs[32h + l], l < 16) and 2j + 1
        // (qs[32h + 16 + l]), scale 8h + g.
        //   Q2_K: scale byte s: y = (d*(s & 15))*q - dmin*(s >> 4)
        //   Q3_K: q = field - 4 where bit 4h + j of hmask[16(g%2) + l] is
        //         clear; 6-bit signed scale: y = (d*scale)*q = dl*(u - 4)
        //         with u = field | hbit << 2
        const int64_t sb = col / 256;
        const int e8 = (int) ((col % 256) / 32), h = e8 >> 2, j = e8 & 3;
        const bool q3 = TYPE == ZEST_TYPE_Q3_K;
        const uint8_t * p = row + sb * (q3 ? 110 : 84);
        const uint8_t * qs = p + (q3 ? 32 : 16) + 32 * h;
        float dl[2], c[2];
        bool ok;
        if (!q3) {
            const uint32_t dd = ld32(p + 80), sw = ld16(p + 8 * h + 2 * j);
            const float d = half_to_float((uint16_t) (dd & 0xffff)), dmin = half_to_float((uint16_t) (dd >> 16));
#pragma unroll
            for (int gi = 0; gi < 2; gi++) {
                const uint32_t sc = (sw >> (8 * gi)) & 0xffu;
                dl[gi] = d * (float) (sc & 0xF);
                c[gi] = -(dmin * (float) (sc >> 4));
            }
            ok = finite(d) && finite(dmin);
        } else {
            const float d = half_to_float((uint16_t) ld16(p + 108));
            uint32_t sc[3];
#pragma unroll
            for (int i = 0; i < 3; i++) sc[i] = ld32h(p + 96 + 4 * i);
#pragma unroll
            for (int gi = 0; gi < 2; gi++) {
                const int si = 8 * h + 2 * j + gi;
                const int lo = si < 8 ? (int) (byte_of(sc, si) & 0xF) : (int) (byte_of(sc, si - 8) >> 4);
                const int hi = (int) ((byte_of(sc, 8 + (si & 3)) >> (2 * (si >> 2))) & 3u);
                dl[gi] = d * (float) ((lo | (hi << 4)) - 32);
                c[gi] = -4.0f * dl[gi];
            }
            ok = finite(d);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t u = (ld32h(qs + 4 * i) >> (2 * j)) & 0x03030303u;
            if (q3) u |= ((ld32h(p + 4 * i) >> (4 * h + j)) & 0x01010101u) << 2;
            fma_bytes(u, dl[i >> 2], c[i >> 2], v + 4 * i);
        }
        return ok;
    } else if (TYPE == ZEST_TYPE_Q4_K || TYPE == ZEST_TYPE_Q5_K) {
        // Q4_K: d, dmin, scales[12], qs[128] (144 bytes); Q5_K adds qh[32]
        // before qs (176 bytes). Sub-block s (eighth): nibble s % 2 of
        // qs[32(s/2) + l], fifth bit s of qh[l], 6-bit pair s:
        // y = (d*sc)*q - dmin*m.
        constexpr int BB = TYPE == ZEST_TYPE_Q4_K ? 144 : 176, QS = TYPE == ZEST_TYPE_Q4_K ? 16 : 48;
        const int64_t sb = col / 256;
        const int s = (int) ((col % 256) / 32);
        const uint8_t * p = row + sb * BB;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(p);
        const uint4 qa = *reinterpret_cast<const uint4 *>(p + QS + 32 * (s >> 1));
        const uint4 qb = *reinterpret_cast<const uint4 *>(p + QS + 16 + 32 * (s >> 1));
        const float d = half_to_float((uint16_t) (hdr.x & 0xffff)), dmin = half_to_float((uint16_t) (hdr.x >> 16));
        const uint32_t scw[3] = {hdr.y, hdr.z, hdr.w};
        uint32_t scv, mv;
        if (s < 4) {
            scv = byte_of(scw, s) & 63;
            mv = byte_of(scw, s + 4) & 63;
        } else {
            scv = (byte_of(scw, s + 4) & 0xF) | ((byte_of(scw, s - 4) >> 6) << 4);
            mv = (byte_of(scw, s + 4) >> 4) | ((byte_of(scw, s) >> 6) << 4);
        }
        const float d1 = d * (float) scv, c = -(dmin * (float) mv);
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t qh[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (TYPE == ZEST_TYPE_Q5_K) {
            const uint4 h0 = *reinterpret_cast<const uint4 *>(p + 16), h1 = *reinterpret_cast<const uint4 *>(p + 32);
            const uint32_t hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) qh[i] = hv[i];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t u = (w[i] >> (4 * (s & 1))) & 0x0F0F0F0Fu;
            if (TYPE == ZEST_TYPE_Q5_K) u |= ((qh[i] >> s) & 0x01010101u) << 4;
            fma_bytes(u, d1, c, v + 4 * i);
        }
        return finite(d) && finite(dmin);
    } else {  // Q6_K
        // ql[128], qh[64], int8 scales[16], d: 210 bytes. Eighth e8 = half
        // h, quarter c = e8 % 4: value l's low 4 bits are nibble c/2 of
        // ql[64h + 32(c%2) + l], its high 2 bits bits 2c of qh[32h + l];
        // y = (d*scales[8h + 2c + l/16])*(u - 32).
        const int64_t sb = col / 256;
        const int e8 = (int) ((col % 256) / 32), h = e8 >> 2, c = e8 & 3;
        const uint8_t * p = row + sb * 210;
        const float d = half_to_float((uint16_t) ld16(p + 208));
        const uint32_t sw = ld16(p + 192 + 8 * h + 2 * c);
        const float ds[2] = {d * (float) (int8_t) (sw & 0xffu), d * (float) (int8_t) (sw >> 8)};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t lo = (ld32h(p + 64 * h + 32 * (c & 1) + 4 * i) >> (4 * (c >> 1))) & 0x0F0F0F0Fu;
            const uint32_t hi = (ld32h(p + 128 + 32 * h + 4 * i) >> (2 * c)) & 0x03030303u;
            fma_bytes(lo | (hi << 4), ds[i >> 2], -32.0f * ds[i >> 2], v + 4 * i);
        }
        return finite(d);
    }
}

// Encodes 32 consecutive values of one row (half a tile row: 4 blocks):
// 32 mantissa bytes and the 4 exponent bytes.
__device__ inline void encode_half_row(const float v[32], bool no_nan, uint4 & m0, uint4 & m1, uint32_t & ex) {
    uint32_t e[4];
    if (no_nan) {
        e[0] = zest::encode8_no_nan(v, m0.x, m0.y);
        e[1] = zest::encode8_no_nan(v + 8, m0.z, m0.w);
        e[2] = zest::encode8_no_nan(v + 16, m1.x, m1.y);
        e[3] = zest::encode8_no_nan(v + 24, m1.z, m1.w);
    } else {
        e[0] = encode8(v, m0.x, m0.y);
        e[1] = encode8(v + 8, m0.z, m0.w);
        e[2] = encode8(v + 16, m1.x, m1.y);
        e[3] = encode8(v + 24, m1.z, m1.w);
    }
    ex = e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24);
}

#ifndef ZEST_CONVERT_ROWS
#define ZEST_CONVERT_ROWS 16
#endif

// Workgroup: ROWS rows x 128/ROWS tile columns (256 threads, a half tile row
// each). Lane t dequantises and encodes row t / (256/ROWS), half tile row
// t % (256/ROWS) of the band (the lanes of a row read one contiguous run of
// its GGUF bytes) into LDS, laid out as the destination's own bytes. With
// ROWS >= 16 a tile column's ROWS/16 tiles are consecutive in the packed
// operand, so the workgroup stores each tile column as one contiguous run,
// 16 bytes a lane, consecutive lanes on consecutive bytes (with ROWS = 8, a
// run of 512 mantissa bytes and one of 64 exponent bytes per tile).
//
// Workgroup order (a 1-D grid of nbx column blocks x a multiple of 8 row
// bands): workgroups go to the eight XCDs in turn, and every column block of
// a row band is sent to the same XCD, one after another. A band's GGUF row
// runs are not line-aligned at the column-block boundaries (Q8_0: 544 bytes
// a block), so neighbouring blocks share a line; on one XCD the second reads
// it from L2 instead of fetching it again (Q8_0 17408 x 5120: 112 -> 95 MB
// fetched, the GGUF bytes exactly).
template <int TYPE, int ROWS>
__global__ __launch_bounds__(256) void convert_kernel(const uint8_t * __restrict__ raw, size_t row_bytes, int64_t N,
                                                      int64_t K, uint8_t * __restrict__ dst, int64_t R_pad,
                                                      int64_t K_pad, int gu, int nbx) {
    static_assert(ROWS == 8 || ROWS == 16 || ROWS == 32, "rows per workgroup");
    constexpr int TILES = 128 / ROWS, HALVES = 2 * TILES;
    // LDS bytes of one tile column: ROWS rows of 64 mantissas and 8 exponents
    constexpr int RUN = ROWS * (ZEST_TILE_K + 8);
    __shared__ uint4 stage[TILES * RUN / 16];
    uint8_t * sb = reinterpret_cast<uint8_t *>(stage);
    const int64_t id = blockIdx.x, k8 = id / 8;
    const int64_t by = id % 8 + 8 * (k8 / nbx), bx = k8 % nbx;  // row band, column block
    const int t = threadIdx.x, rl = t / HALVES, hl = t % HALVES;
    const int64_t r = by * ROWS + rl;
    const int64_t col = (bx * HALVES + hl) * 32;
    uint4 m0 = make_uint4(0, 0, 0, 0), m1 = m0;
    uint32_t ex = 0;
    if (r < N && col < K) {  // else padding: zero blocks (exponent 0, mantissas 0)
        float v[32];
        const bool no_nan = dq_half<TYPE>(raw + r * (int64_t) row_bytes, col, K, v);
        encode_half_row(v, no_nan, m0, m1, ex);
    }
    const int j = hl >> 1, hf = hl & 1;
    // ROWS = 8: mantissas (8 rows of 64) then exponents (8 rows of 8);
    // else whole tiles in the packed layout, ROWS/16 of them
    const int mo = ROWS == 8 ? j * RUN + rl * ZEST_TILE_K
                             : j * RUN + (rl >> 4) * ZEST_TILE_BYTES + (rl & 15) * ZEST_TILE_K;
    const int eo = ROWS == 8 ? j * RUN + 8 * ZEST_TILE_K + rl * 8
                             : j * RUN + (rl >> 4) * ZEST_TILE_BYTES + ZEST_TILE_MANT + (rl & 15) * 8;
    uint4 * ms = reinterpret_cast<uint4 *>(sb + mo + hf * 32);
    ms[0] = m0;
    ms[1] = m1;
    *reinterpret_cast<uint32_t *>(sb + eo + hf * 4) = ex;
    __syncthreads();
    // the row band stays whole in the destination (dst_row keeps 32-row runs)
    const int64_t dr0 = dst_row(by * ROWS, gu), rt = dr0 / ZEST_TILE_ROWS, rr0 = dr0 % ZEST_TILE_ROWS;
    const int64_t kc0 = bx * TILES;
    const int ntiles = (int) min((int64_t) TILES, K_pad / ZEST_TILE_K - kc0);
    for (int c = t; c < ntiles * (RUN / 16); c += 256) {
        const int tj = c / (RUN / 16), q = c % (RUN / 16);
        uint8_t * tile = dst + zest_tile_offset(rt, kc0 + tj, R_pad);
        const int64_t off =
            ROWS == 8 ? (q < 32 ? rr0 * ZEST_TILE_K + q * 16 : ZEST_TILE_MANT + rr0 * 8 + (q - 32) * 16) : q * 16;
        // nontemporal: the operand is written once and read much later
        const uint4 v = stage[c];
        const u32x4 vv = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(vv, reinterpret_cast<u32x4 *>(tile + off));
    }
}

bool aligned(const void * p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Inputs larger than this (half the 256 MB MALL) are read with nontemporal loads.
constexpr int64_t STREAM_BYTES = 128ll << 20;

} // namespace

extern "C" {

int64_t zest_rows_pad(int64_t rows) { return zest_rows_padded(rows); }
int64_t zest_k_pad(int64_t K) { return zest_k_padded(K); }
size_t zest_bfp16_bytes(int64_t rows, int64_t K) {
    return (size_t) (zest_rows_padded(rows) * zest_k_padded(K) / 8 * 9);
}

size_t zest_raw_row_bytes(int type, int64_t K) {
    switch (type) {
        case ZEST_TYPE_F32: return (size_t) K * 4;
        case ZEST_TYPE_F16:
        case ZEST_TYPE_BF16: return (size_t) K * 2;
        case ZEST_TYPE_Q4_0: return K % 32 ? 0 : (size_t) (K / 32) * 18;
        case ZEST_TYPE_Q4_1: return K % 32 ? 0 : (size_t) (K / 32) * 20;
        case ZEST_TYPE_Q5_0: return K % 32 ? 0 : (size_t) (K / 32) * 22;
        case ZEST_TYPE_Q5_1: return K % 32 ? 0 : (size_t) (K / 32) * 24;
        case ZEST_TYPE_Q8_0: return K % 32 ? 0 : (size_t) (K / 32) * 34;
        case ZEST_TYPE_Q2_K: return K % 256 ? 0 : (size_t) (K / 256) * 84;
        case ZEST_TYPE_Q3_K: return K % 256 ? 0 : (size_t) (K / 256) * 110;
        case ZEST_TYPE_Q4_K: return K % 256 ? 0 : (size_t) (K / 256) * 144;
        case ZEST_TYPE_Q5_K: return K % 256 ? 0 : (size_t) (K / 256) * 176;
        case ZEST_TYPE_Q6_K: return K % 256 ? 0 : (size_t) (K / 256) * 210;
        case ZEST_TYPE_IQ4_NL: return K % 32 ? 0 : (size_t) (K / 32) * 18;
        case ZEST_TYPE_IQ4_XS: return K % 256 ? 0 : (size_t) (K / 256) * 136;
        default: return 0;
    }
}

// required alignment of a weight's rows, by the widest load its converter makes
static size_t row_align(int type) {
    switch (type) {
        case ZEST_TYPE_F32:
        case ZEST_TYPE_F16:
        case ZEST_TYPE_BF16:
        case ZEST_TYPE_Q4_K:
        case ZEST_TYPE_Q5_K: return 16;
        case ZEST_TYPE_IQ4_XS: return 8;
        case ZEST_TYPE_Q4_1:
        case ZEST_TYPE_Q5_1:
        case ZEST_TYPE_Q2_K: return 4;
        default: return 2;
    }
}

size_t zest_act_bytes(int64_t rows, int64_t K) { return (size_t) (zest_rows_padded(rows) * zest_k_padded(K) * 2); }

static int pack_act(bool xout, const float * x, int64_t M, int64_t K, int64_t ldx, void * dst, void * stream,
                    const char * name) {
    ZEST_REQUIRE(x && dst, "%s: null pointer", name);
    ZEST_REQUIRE(M > 0 && K > 0 && K % 8 == 0, "%s: M=%lld K=%lld (K must be a positive multiple of 8)", name,
                 (long long) M, (long long) K);
    ZEST_REQUIRE(ldx >= K, "%s: row stride %lld < K %lld", name, (long long) ldx, (long long) K);
    ZEST_REQUIRE(aligned(x, 16) && aligned(dst, 16), "%s: pointers must be 16-byte aligned", name);
    const int64_t R_pad = zest_rows_padded(M), K_pad = zest_k_padded(K);
    const dim3 grid((unsigned) ((K_pad + 255) / 256), (unsigned) (R_pad / ZEST_TILE_ROWS));
    // an input over half the MALL cannot be resident there: stream it
    const bool stream_x = (double) M * (double) ldx * 4.0 > (double) STREAM_BYTES;
    hipStream_t s = zest::as_stream(stream);
    uint8_t * d8 = (uint8_t *) dst;
    if (xout && stream_x)
        hipLaunchKernelGGL((pack_act_kernel<true, true>), grid, dim3(256), 0, s, x, M, K, ldx, d8, R_pad, K_pad, -1);
    else if (xout)
        hipLaunchKernelGGL((pack_act_kernel<true, false>), grid, dim3(256), 0, s, x, M, K, ldx, d8, R_pad, K_pad, -1);
    else if (stream_x)
        hipLaunchKernelGGL((pack_act_kernel<false, true>), grid, dim3(256), 0, s, x, M, K, ldx, d8, R_pad, K_pad, -1);
    else
        hipLaunchKernelGGL((pack_act_kernel<false, false>), grid, dim3(256), 0, s, x, M, K, ldx, d8, R_pad, K_pad, -1);
    return zest::check_launch(name);
}

int zest_pack_act(const float * x, int64_t M, int64_t K, int64_t ldx, void * dst, void * stream) {
    return pack_act(false, x, M, K, ldx, dst, stream, "zest_pack_act");
}

int zest_pack_act_x(const float * x, int64_t M, int64_t K, int64_t ldx, void * dst, void * stream) {
    return pack_act(true, x, M, K, ldx, dst, stream, "zest_pack_act_x");
}

int zest_expand_act(const void * src, int64_t M, int64_t K, void * dst, void * stream) {
    ZEST_REQUIRE(src && dst, "zest_expand_act: null pointer");
    ZEST_REQUIRE(M > 0 && K > 0 && K % 8 == 0, "zest_expand_act: M=%lld K=%lld", (long long) M, (long long) K);
    ZEST_REQUIRE(aligned(src, 16) && aligned(dst, 16), "zest_expand_act: pointers must be 16-byte aligned");
    const int64_t units = zest_rows_padded(M) * zest_k_padded(K) / 16;
    hipLaunchKernelGGL(expand_act_kernel, dim3((unsigned) ((units + 255) / 256)), dim3(256), 0,
                       zest::as_stream(stream), (const uint8_t *) src, (uint8_t *) dst, units, zest_rows_padded(M));
    return zest::check_launch("zest_expand_act");
}

// Converts one weight (N rows) into dst, a packed operand of R_pad rows:
// rows as they are (gu < 0), or into the gate (0) / up (1) slots of an
// interleaved pair (then R_pad is the pair's and N % 32 == 0).
static int convert(int type, const void * raw, int64_t N, int64_t K, void * dst, int64_t R_pad, int gu,
                   hipStream_t s, const char * name) {
    const int64_t K_pad = zest_k_padded(K), R_src = gu < 0 ? R_pad : R_pad / 2;
    switch (type) {
        case ZEST_TYPE_F32: {
            ZEST_REQUIRE(aligned(raw, 16), "%s: F32 rows must be 16-byte aligned", name);
            const dim3 grid((unsigned) ((K_pad + 255) / 256), (unsigned) (R_src / ZEST_TILE_ROWS));
            // a weight is read once, from wherever it was uploaded: streamed
            hipLaunchKernelGGL((pack_act_kernel<false, true>), grid, dim3(256), 0, s, (const float *) raw, N, K, K,
                               (uint8_t *) dst, R_pad, K_pad, gu);
            return zest::check_launch(name);
        }
        default: break;
    }
    const size_t rb = zest_raw_row_bytes(type, K);
    if (rb == 0) {
        if (zest_raw_row_bytes(type, 256) == 0)
            return zest::fail(ZEST_E_UNSUPPORTED, "%s: weight type %d has no converter", name, type);
        return zest::fail(ZEST_E_ARG, "%s: K=%lld is not a multiple of type %d's block", name, (long long) K,
                          type);
    }
    ZEST_REQUIRE(aligned(raw, row_align(type)), "%s: type %d rows must be %zu-byte aligned", name, type,
                 row_align(type));
    constexpr int RW = ZEST_CONVERT_ROWS;
    // nbx column blocks x nby row bands, the bands a multiple of 8 (R_src is a
    // multiple of 128), as one 1-D grid in the kernel's XCD order
    const int64_t nbx = (K_pad / ZEST_TILE_K + 128 / RW - 1) / (128 / RW), nby = R_src / RW;
    ZEST_REQUIRE(nby % 8 == 0 && nbx * nby < (1ll << 31), "%s: %lld x %lld workgroups", name, (long long) nbx,
                 (long long) nby);
    const dim3 grid((unsigned) (nbx * nby));
    const uint8_t * r8 = (const uint8_t *) raw;
    uint8_t * d8 = (uint8_t *) dst;
#define ZEST_CONVERT(T)                                                                                      \
    case T:                                                                                                  \
        hipLaunchKernelGGL((convert_kernel<T, RW>), grid, dim3(256), 0, s, r8, rb, N, K, d8, R_pad, K_pad, gu, \
                           (int) nbx);                                                                       \
        break
    switch (type) {
        ZEST_CONVERT(ZEST_TYPE_F16);
        ZEST_CONVERT(ZEST_TYPE_Q8_0);
        ZEST_CONVERT(ZEST_TYPE_BF16);
        ZEST_CONVERT(ZEST_TYPE_Q4_0);
        ZEST_CONVERT(ZEST_TYPE_Q4_1);
        ZEST_CONVERT(ZEST_TYPE_Q5_0);
        ZEST_CONVERT(ZEST_TYPE_Q5_1);
        ZEST_CONVERT(ZEST_TYPE_Q2_K);
        ZEST_CONVERT(ZEST_TYPE_Q3_K);
        ZEST_CONVERT(ZEST_TYPE_Q4_K);
        ZEST_CONVERT(ZEST_TYPE_Q5_K);
        ZEST_CONVERT(ZEST_TYPE_Q6_K);
        ZEST_CONVERT(ZEST_TYPE_IQ4_NL);
        ZEST_CONVERT(ZEST_TYPE_IQ4_XS);
        default: return zest::fail(ZEST_E_UNSUPPORTED, "%s: weight type %d has no converter", name, type);
    }
#undef ZEST_CONVERT
    return zest::check_launch(name);
}

int zest_convert_weight(int type, const void * raw, int64_t N, int64_t K, void * dst, void * stream) {
    ZEST_REQUIRE(raw && dst, "zest_convert_weight: null pointer");
    ZEST_REQUIRE(N > 0 && K > 0 && K % 8 == 0, "zest_convert_weight: N=%lld K=%lld", (long long) N, (long long) K);
    ZEST_REQUIRE(aligned(dst, 16), "zest_convert_weight: dst must be 16-byte aligned");
    return convert(type, raw, N, K, dst, zest_rows_padded(N), -1, zest::as_stream(stream), "zest_convert_weight");
}

int zest_convert_weight_gu(int type, const void * gate, const void * up, int64_t F, int64_t K, void * dst,
                           void * stream) {
    ZEST_REQUIRE(gate && up && dst, "zest_convert_weight_gu: null pointer");
    ZEST_REQUIRE(F > 0 && F % 32 == 0 && K > 0 && K % 8 == 0,
                 "zest_convert_weight_gu: F=%lld K=%lld (F must be a multiple of 32)", (long long) F, (long long) K);
    ZEST_REQUIRE(aligned(dst, 16), "zest_convert_weight_gu: dst must be 16-byte aligned");
    const int64_t R_pad = zest_rows_padded(2 * F);
    hipStream_t s = zest::as_stream(stream);
    const int st = convert(type, gate, F, K, dst, R_pad, 0, s, "zest_convert_weight_gu(gate)");
    return st != ZEST_OK ? st : convert(type, up, F, K, dst, R_pad, 1, s, "zest_convert_weight_gu(up)");
}

} // extern "C"

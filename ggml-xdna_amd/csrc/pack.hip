// The HBM-bound converters of the path:
//   zest_pack_act        fp32 activations -> packed bfp16 (per chunk)
//   zest_pack_act_x      fp32 activations -> the GEMM's expanded operand: the
//                        same bfp16 blocks, stored decoded as bf16
//   zest_expand_act      packed bfp16 -> expanded operand
//   zest_convert_weight  GGUF weights (F32, F16, BF16, Q4_0..Q8_0, Q2_K..Q6_K)
//                        -> packed bfp16 (once, into the resident weight cache)
// All write the layouts of zest_layout.h with 16-byte stores.
#include "zest_common.h"
#include "zest_device.h"

namespace {

using zest::encode8;

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
// 8 bytes, at row t/16 of the 2048-byte tile).
template <bool XOUT>
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
            const f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + r * ldx + col));
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
            *reinterpret_cast<uint2 *>(dst + zest_xtile_offset(rt, kc, R_pad) + rr * 128 + j * 8) =
                make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
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
// exponent bytes -> 16 bf16 of the expanded operand.
__global__ __launch_bounds__(256) void expand_act_kernel(const uint8_t * __restrict__ src, uint8_t * __restrict__ dst,
                                                         int64_t units) {
    const int64_t u = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const int64_t tile = u / 64, c = u % 64;  // unit c of a tile: row c/4, 16-column quarter c%4
    const uint8_t * t = src + tile * ZEST_TILE_BYTES;
    const uint4 m = *reinterpret_cast<const uint4 *>(t + c * 16);
    const uint32_t e = *reinterpret_cast<const uint16_t *>(t + ZEST_TILE_MANT + c * 2);
    uint32_t b[8];
    zest::expand16(m, e, b);
    uint4 * p = reinterpret_cast<uint4 *>(dst + tile * ZEST_XTILE_BYTES + c * 32);
    p[0] = make_uint4(b[0], b[1], b[2], b[3]);
    p[1] = make_uint4(b[4], b[5], b[6], b[7]);
}

__device__ inline float half_to_float(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }

// Q8_0: 34-byte blocks of fp16 d + 32 int8; y = d * q, exact in fp32. One
// thread takes one GGUF block = half a tile row: 32 mantissa bytes (two
// 16-byte stores) and four exponent bytes. Workgroup: 8 rows x 32 blocks.
__global__ __launch_bounds__(256) void convert_q8_0_kernel(const uint8_t * __restrict__ raw, int64_t N, int64_t K,
                                                           uint8_t * __restrict__ dst, int64_t R_pad, int64_t K_pad,
                                                           int64_t R_src, int gu) {
    const int t = threadIdx.x;
    const int64_t r = (int64_t) blockIdx.y * 8 + (t >> 5);
    const int64_t jb = (int64_t) blockIdx.x * 32 + (t & 31);  // 32-column block
    const int64_t col = jb * 32;
    if (col >= K_pad || r >= R_src) return;
    uint4 m0 = make_uint4(0, 0, 0, 0), m1 = make_uint4(0, 0, 0, 0);
    uint32_t ex = 0;
    if (r < N && col < K) {
        const uint8_t * b = raw + r * (K / 32 * 34) + jb * 34;
        const uint16_t * h = reinterpret_cast<const uint16_t *>(b);  // 2-byte aligned
        const float d = half_to_float(h[0]);
        float v[32];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint16_t pair = h[1 + i];
            v[2 * i] = (float) (int8_t) (pair & 0xff) * d;
            v[2 * i + 1] = (float) (int8_t) (pair >> 8) * d;
        }
        uint32_t e[4];
        e[0] = encode8(v, m0.x, m0.y);
        e[1] = encode8(v + 8, m0.z, m0.w);
        e[2] = encode8(v + 16, m1.x, m1.y);
        e[3] = encode8(v + 24, m1.z, m1.w);
        ex = e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24);
    }
    const int64_t dr = dst_row(r, gu);
    uint8_t * tile = dst + zest_tile_offset(dr / ZEST_TILE_ROWS, col / ZEST_TILE_K, R_pad);
    const int64_t rr = dr % ZEST_TILE_ROWS, half = (col % ZEST_TILE_K) / 32;
    uint4 * mp = reinterpret_cast<uint4 *>(tile + rr * ZEST_TILE_K + half * 32);
    mp[0] = m0;
    mp[1] = m1;
    *reinterpret_cast<uint32_t *>(tile + ZEST_TILE_MANT + rr * 8 + half * 4) = ex;
}

// Encodes 64 consecutive values of one row (a tile row: 8 blocks) and stores
// them at row dr of tile column kc: 64 mantissa bytes (four 16-byte stores)
// and the 8 exponent bytes (one 8-byte store).
__device__ inline void store_tile_row(uint8_t * dst, int64_t R_pad, int64_t dr, int64_t kc, const float v[64]) {
    uint4 m[4];
    uint32_t e[8];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        e[2 * u] = encode8(v + 16 * u, m[u].x, m[u].y);
        e[2 * u + 1] = encode8(v + 16 * u + 8, m[u].z, m[u].w);
    }
    uint8_t * tile = dst + zest_tile_offset(dr / ZEST_TILE_ROWS, kc, R_pad);
    const int64_t rr = dr % ZEST_TILE_ROWS;
    uint4 * mp = reinterpret_cast<uint4 *>(tile + rr * ZEST_TILE_K);
#pragma unroll
    for (int u = 0; u < 4; u++) mp[u] = m[u];
    *reinterpret_cast<uint2 *>(tile + ZEST_TILE_MANT + rr * 8) =
        make_uint2(e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24), e[4] | (e[5] << 8) | (e[6] << 16) | (e[7] << 24));
}

// Q4_K: 144-byte super-blocks of 256: fp16 d, fp16 dmin, 12 bytes of 6-bit
// (scale, min) pairs, 128 bytes of nibbles. Sub-block s (0..7) is 32 values:
// the low (s even) or high (s odd) nibbles of qs[32*(s/2) ..+32), with pair s:
// y = (d*sc)*q - dmin*m. The products are exact in fp32, so the one rounding
// is the subtraction's and fma gives the same float. One thread per quarter
// super-block: sub-blocks 2p and 2p+1, the two nibbles of the same 32 bytes,
// i.e. 64 consecutive values, one tile row. Three aligned 16-byte loads (the
// 16-byte header; the 32 nibble bytes). Workgroup: 16 rows x 4 super-blocks.
__global__ __launch_bounds__(256) void convert_q4_k_kernel(const uint8_t * __restrict__ raw, int64_t N, int64_t K,
                                                           uint8_t * __restrict__ dst, int64_t R_pad, int64_t K_pad,
                                                           int64_t R_src, int gu) {
    const int t = threadIdx.x, p = t & 3;
    const int64_t r = (int64_t) blockIdx.y * ZEST_TILE_ROWS + (t >> 4);
    const int64_t sb = (int64_t) blockIdx.x * 4 + ((t >> 2) & 3);
    const int64_t col = sb * 256 + p * 64;
    if (col >= K_pad || r >= R_src) return;
    float v[64];
    if (r < N && col < K) {
        const uint8_t * blk = raw + r * (K / 256 * 144) + sb * 144;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * p);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * p);
        const float d = half_to_float((uint16_t) (hdr.x & 0xffff)), dmin = half_to_float((uint16_t) (hdr.x >> 16));
        const uint32_t scw[3] = {hdr.y, hdr.z, hdr.w};
        auto sc = [&](int i) { return (scw[i >> 2] >> ((i & 3) * 8)) & 0xffu; };
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int s = 2 * p + h;
            uint32_t scv, mv;
            if (s < 4) {
                scv = sc(s) & 63;
                mv = sc(s + 4) & 63;
            } else {
                scv = (sc(s + 4) & 0xF) | ((sc(s - 4) >> 6) << 4);
                mv = (sc(s + 4) >> 4) | ((sc(s) >> 6) << 4);
            }
            const float d1 = d * (float) scv, m1f = dmin * (float) mv;
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const uint32_t nib = (w[i >> 2] >> ((i & 3) * 8 + h * 4)) & 0xF;
                v[32 * h + i] = fmaf(d1, (float) nib, -m1f);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = 0.0f;
    }
    store_tile_row(dst, R_pad, dst_row(r, gu), col / ZEST_TILE_K, v);
}

// ---- the other GGUF types ------------------------------------------------------
// One thread per 64 consecutive values of a row (one tile row of one tile
// column), dequantised as ggml's to_float does: every product below is exact
// in fp32 (fp16 scale x small integers), so where the format adds an offset
// the one rounding is the addition's and fmaf gives the same float.

__device__ inline uint32_t ld16(const uint8_t * p) { return *reinterpret_cast<const uint16_t *>(p); }  // 2-aligned
__device__ inline uint32_t ld32(const uint8_t * p) { return *reinterpret_cast<const uint32_t *>(p); }  // 4-aligned
__device__ inline uint32_t ld32h(const uint8_t * p) { return ld16(p) | (ld16(p + 2) << 16); }          // 2-aligned
__device__ inline uint32_t byte_of(const uint32_t * w, int i) { return (w[i >> 2] >> ((i & 3) * 8)) & 0xffu; }

// 32-value blocks: byte j of qs holds value j (low nibble) and j + 16 (high);
// bit j of the 32-bit qh is value j's fifth bit. SIGNED: q - 2^(bits-1)
// times d; else q*d + m.
template <int BITS, bool SIGNED>
__device__ inline void dq_block32(float d, float m, uint32_t qh, const uint32_t qs[4], float * v) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t b = byte_of(qs, j);
        int lo = (int) (b & 0xF), hi = (int) (b >> 4);
        if (BITS == 5) {
            lo |= (int) ((qh >> j) & 1u) << 4;
            hi |= (int) ((qh >> (j + 16)) & 1u) << 4;
        }
        if (SIGNED) {
            v[j] = (float) (lo - (1 << (BITS - 1))) * d;
            v[j + 16] = (float) (hi - (1 << (BITS - 1))) * d;
        } else {
            v[j] = fmaf((float) lo, d, m);
            v[j + 16] = fmaf((float) hi, d, m);
        }
    }
}

template <int TYPE>
__device__ inline void dq_32(const uint8_t * p, float * v) {
    uint32_t qs[4];
    if (TYPE == ZEST_TYPE_Q4_0) {  // d, qs[16]: 18 bytes
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32h(p + 2 + 4 * i);
        dq_block32<4, true>(half_to_float((uint16_t) ld16(p)), 0.0f, 0, qs, v);
    } else if (TYPE == ZEST_TYPE_Q4_1) {  // d, m, qs[16]: 20 bytes
        const uint32_t h = ld32(p);
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32(p + 4 + 4 * i);
        dq_block32<4, false>(half_to_float((uint16_t) (h & 0xffff)), half_to_float((uint16_t) (h >> 16)), 0, qs, v);
    } else if (TYPE == ZEST_TYPE_Q5_0) {  // d, qh[4], qs[16]: 22 bytes
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32h(p + 6 + 4 * i);
        dq_block32<5, true>(half_to_float((uint16_t) ld16(p)), 0.0f, ld32h(p + 2), qs, v);
    } else {  // Q5_1: d, m, qh[4], qs[16]: 24 bytes
        const uint32_t h = ld32(p);
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = ld32(p + 8 + 4 * i);
        dq_block32<5, false>(half_to_float((uint16_t) (h & 0xffff)), half_to_float((uint16_t) (h >> 16)), ld32(p + 4),
                             qs, v);
    }
}

// Values [col, col + 64) of one row (col % 64 == 0, col < K).
template <int TYPE>
__device__ inline void dq_64(const uint8_t * row, int64_t col, int64_t K, float v[64]) {
    if (TYPE == ZEST_TYPE_F16 || TYPE == ZEST_TYPE_BF16) {
        // K % 8 == 0 but maybe not % 64: 8-value chunks past K read as zero
        const uint4 * p = reinterpret_cast<const uint4 *>(row + col * 2);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint4 q = col + 8 * i < K ? p[i] : make_uint4(0, 0, 0, 0);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = w[k] & 0xffff, hi = w[k] >> 16;
                if (TYPE == ZEST_TYPE_F16) {
                    v[8 * i + 2 * k] = half_to_float((uint16_t) lo);
                    v[8 * i + 2 * k + 1] = half_to_float((uint16_t) hi);
                } else {
                    v[8 * i + 2 * k] = __uint_as_float(lo << 16);
                    v[8 * i + 2 * k + 1] = __uint_as_float(hi << 16);
                }
            }
        }
    } else if (TYPE == ZEST_TYPE_Q4_0 || TYPE == ZEST_TYPE_Q4_1 || TYPE == ZEST_TYPE_Q5_0 ||
               TYPE == ZEST_TYPE_Q5_1) {
        constexpr int B = TYPE == ZEST_TYPE_Q4_0 ? 18 : TYPE == ZEST_TYPE_Q4_1 ? 20 : TYPE == ZEST_TYPE_Q5_0 ? 22 : 24;
        const uint8_t * p = row + (col / 32) * B;
        dq_32<TYPE>(p, v);
        if (col + 32 < K) {
            dq_32<TYPE>(p + B, v + 32);
        } else {
#pragma unroll
            for (int i = 32; i < 64; i++) v[i] = 0.0f;
        }
    } else if (TYPE == ZEST_TYPE_Q2_K) {
        // scales[16], qs[64], d, dmin: 84 bytes. Quarter c4 = half h, groups
        // 4c..4c+3 of 16 (c = c4 % 2); group g takes 2-bit field g/2 of
        // qs[32h + 16(g%2) + l], scale byte 8h + g: y = (d*(s&15))*q - dmin*(s>>4)
        const int64_t sb = col / 256;
        const int c4 = (int) ((col % 256) / 64), h = c4 >> 1, c = c4 & 1;
        const uint8_t * p = row + sb * 84;
        const uint32_t dd = ld32(p + 80), sw = ld32(p + 8 * h + 4 * c);
        const float d = half_to_float((uint16_t) (dd & 0xffff)), dmin = half_to_float((uint16_t) (dd >> 16));
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = ld32(p + 16 + 32 * h + 4 * i);
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            const int g = 4 * c + gi, sh = 2 * (g >> 1);
            const uint32_t s = (sw >> (8 * gi)) & 0xffu;
            const float dl = d * (float) (s & 0xF), ml = dmin * (float) (s >> 4);
#pragma unroll
            for (int l = 0; l < 16; l++)
                v[16 * gi + l] = fmaf(dl, (float) ((byte_of(q, 16 * (gi & 1) + l) >> sh) & 3u), -ml);
        }
    } else if (TYPE == ZEST_TYPE_Q3_K) {
        // hmask[32], qs[64], scales[12], d: 110 bytes. As Q2_K's fields, with
        // q = field - 4 where bit 4h + g/2 of hmask[16(g%2) + l] is clear, and
        // 6-bit signed scales: y = (d*scale)*q, exact.
        const int64_t sb = col / 256;
        const int c4 = (int) ((col % 256) / 64), h = c4 >> 1, c = c4 & 1;
        const uint8_t * p = row + sb * 110;
        const float d = half_to_float((uint16_t) ld16(p + 108));
        uint32_t hm[8], q[8], sc[3];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hm[i] = ld32h(p + 4 * i);
            q[i] = ld32h(p + 32 + 32 * h + 4 * i);
        }
#pragma unroll
        for (int i = 0; i < 3; i++) sc[i] = ld32h(p + 96 + 4 * i);
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            const int g = 4 * c + gi, j = g >> 1, si = 8 * h + g;
            const int lo = si < 8 ? (int) (byte_of(sc, si) & 0xF) : (int) (byte_of(sc, si - 8) >> 4);
            const int hi = (int) ((byte_of(sc, 8 + (si & 3)) >> (2 * (si >> 2))) & 3u);
            const float dl = d * (float) ((lo | (hi << 4)) - 32);
#pragma unroll
            for (int l = 0; l < 16; l++) {
                const int o = 16 * (gi & 1) + l;
                const int f = (int) ((byte_of(q, o) >> (2 * j)) & 3u) - ((byte_of(hm, o) >> (4 * h + j)) & 1u ? 0 : 4);
                v[16 * gi + l] = dl * (float) f;
            }
        }
    } else if (TYPE == ZEST_TYPE_Q5_K) {
        // d, dmin, scales[12], qh[32], qs[128]: 176 bytes. Group j of 64:
        // Q4_K's nibbles of qs[32j..32j+32) and pairs 2j, 2j+1, fifth bits
        // 2j (low nibbles) and 2j + 1 (high) of qh[l].
        const int64_t sb = col / 256;
        const int jq = (int) ((col % 256) / 64);
        const uint8_t * p = row + sb * 176;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(p);
        const uint4 h0 = *reinterpret_cast<const uint4 *>(p + 16), h1 = *reinterpret_cast<const uint4 *>(p + 32);
        const uint4 qa = *reinterpret_cast<const uint4 *>(p + 48 + 32 * jq);
        const uint4 qb = *reinterpret_cast<const uint4 *>(p + 64 + 32 * jq);
        const float d = half_to_float((uint16_t) (hdr.x & 0xffff)), dmin = half_to_float((uint16_t) (hdr.x >> 16));
        const uint32_t scw[3] = {hdr.y, hdr.z, hdr.w};
        const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int s = 2 * jq + e;
            uint32_t scv, mv;
            if (s < 4) {
                scv = byte_of(scw, s) & 63;
                mv = byte_of(scw, s + 4) & 63;
            } else {
                scv = (byte_of(scw, s + 4) & 0xF) | ((byte_of(scw, s - 4) >> 6) << 4);
                mv = (byte_of(scw, s + 4) >> 4) | ((byte_of(scw, s) >> 6) << 4);
            }
            const float d1 = d * (float) scv, m1 = dmin * (float) mv;
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const uint32_t qv = ((byte_of(w, l) >> (4 * e)) & 0xF) | (((byte_of(qh, l) >> s) & 1u) << 4);
                v[32 * e + l] = fmaf(d1, (float) qv, -m1);
            }
        }
    } else {  // Q6_K
        // ql[128], qh[64], int8 scales[16], d: 210 bytes. Half h, quarters
        // c = 2c2 + e: value l's low 4 bits are nibble c2 of
        // ql[64h + 32e + l], its high 2 bits bits 2c of qh[32h + l]; minus
        // 32, times d*scales[8h + 2c + l/16] (products exact in fp32).
        const int64_t sb = col / 256;
        const int c4 = (int) ((col % 256) / 64), h = c4 >> 1, c2 = c4 & 1;
        const uint8_t * p = row + sb * 210;
        const float d = half_to_float((uint16_t) ld16(p + 208));
        const uint32_t sw = ld32h(p + 192 + 8 * h + 4 * c2);
        uint32_t ql[16], qh[8];
#pragma unroll
        for (int i = 0; i < 16; i++) ql[i] = ld32h(p + 64 * h + 4 * i);
#pragma unroll
        for (int i = 0; i < 8; i++) qh[i] = ld32h(p + 128 + 32 * h + 4 * i);
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int cq = 2 * c2 + e;
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const int lo = (int) ((byte_of(ql, 32 * e + l) >> (4 * c2)) & 0xF);
                const int hi = (int) ((byte_of(qh, l) >> (2 * cq)) & 3u);
                const int8_t s = (int8_t) ((sw >> (8 * (2 * e + l / 16))) & 0xffu);
                v[32 * e + l] = (d * (float) s) * (float) ((lo | (hi << 4)) - 32);
            }
        }
    }
}

// Workgroup: 16 rows x 16 tile columns (1024 values of each row); lane t
// takes row t/16 and tile column t%16, so the 16 lanes of a row read one
// contiguous run of its GGUF bytes.
template <int TYPE>
__global__ __launch_bounds__(256) void convert_kernel(const uint8_t * __restrict__ raw, size_t row_bytes, int64_t N,
                                                      int64_t K, uint8_t * __restrict__ dst, int64_t R_pad,
                                                      int64_t K_pad, int64_t R_src, int gu) {
    const int t = threadIdx.x;
    const int64_t r = (int64_t) blockIdx.y * ZEST_TILE_ROWS + (t >> 4);
    const int64_t kc = (int64_t) blockIdx.x * 16 + (t & 15), col = kc * ZEST_TILE_K;
    if (col >= K_pad || r >= R_src) return;
    float v[64];
    if (r < N && col < K) {
        dq_64<TYPE>(raw + r * (int64_t) row_bytes, col, K, v);
    } else {
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = 0.0f;
    }
    store_tile_row(dst, R_pad, dst_row(r, gu), kc, v);
}

bool aligned(const void * p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

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
    if (xout)
        hipLaunchKernelGGL(pack_act_kernel<true>, grid, dim3(256), 0, zest::as_stream(stream), x, M, K, ldx,
                           (uint8_t *) dst, R_pad, K_pad, -1);
    else
        hipLaunchKernelGGL(pack_act_kernel<false>, grid, dim3(256), 0, zest::as_stream(stream), x, M, K, ldx,
                           (uint8_t *) dst, R_pad, K_pad, -1);
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
                       zest::as_stream(stream), (const uint8_t *) src, (uint8_t *) dst, units);
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
            hipLaunchKernelGGL(pack_act_kernel<false>, grid, dim3(256), 0, s, (const float *) raw, N, K, K,
                               (uint8_t *) dst, R_pad, K_pad, gu);
            return zest::check_launch(name);
        }
        case ZEST_TYPE_Q8_0: {
            ZEST_REQUIRE(K % 32 == 0, "%s: Q8_0 needs K %% 32 == 0 (K=%lld)", name, (long long) K);
            ZEST_REQUIRE(aligned(raw, 2), "%s: Q8_0 rows must be 2-byte aligned", name);
            const dim3 grid((unsigned) ((K_pad / 32 + 31) / 32), (unsigned) (R_src / 8));
            hipLaunchKernelGGL(convert_q8_0_kernel, grid, dim3(256), 0, s, (const uint8_t *) raw, N, K, (uint8_t *) dst,
                               R_pad, K_pad, R_src, gu);
            return zest::check_launch(name);
        }
        case ZEST_TYPE_Q4_K: {
            ZEST_REQUIRE(K % 256 == 0, "%s: Q4_K needs K %% 256 == 0 (K=%lld)", name, (long long) K);
            ZEST_REQUIRE(aligned(raw, 16), "%s: Q4_K rows must be 16-byte aligned", name);
            const dim3 grid((unsigned) ((K_pad / 256 + 3) / 4), (unsigned) (R_src / ZEST_TILE_ROWS));
            hipLaunchKernelGGL(convert_q4_k_kernel, grid, dim3(256), 0, s, (const uint8_t *) raw, N, K, (uint8_t *) dst,
                               R_pad, K_pad, R_src, gu);
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
    const dim3 grid((unsigned) ((K_pad / ZEST_TILE_K + 15) / 16), (unsigned) (R_src / ZEST_TILE_ROWS));
    const uint8_t * r8 = (const uint8_t *) raw;
    uint8_t * d8 = (uint8_t *) dst;
#define ZEST_CONVERT(T)                                                                                         \
    case T: hipLaunchKernelGGL(convert_kernel<T>, grid, dim3(256), 0, s, r8, rb, N, K, d8, R_pad, K_pad, R_src, gu); \
        break
    switch (type) {
        ZEST_CONVERT(ZEST_TYPE_F16);
        ZEST_CONVERT(ZEST_TYPE_BF16);
        ZEST_CONVERT(ZEST_TYPE_Q4_0);
        ZEST_CONVERT(ZEST_TYPE_Q4_1);
        ZEST_CONVERT(ZEST_TYPE_Q5_0);
        ZEST_CONVERT(ZEST_TYPE_Q5_1);
        ZEST_CONVERT(ZEST_TYPE_Q2_K);
        ZEST_CONVERT(ZEST_TYPE_Q3_K);
        ZEST_CONVERT(ZEST_TYPE_Q5_K);
        ZEST_CONVERT(ZEST_TYPE_Q6_K);
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

// The small fp32 ops between the matmuls (piece::run_rows,
// src/xdna-exec.cpp:253-346), as HBM-bound row kernels. RMS_NORM (+ the scale
// row MUL after it) and the GLUs can also write the next matmul's input (the
// bfp16 pack, stored expanded) directly, so a normalised or gated row goes
// HBM -> registers -> matmul operand without a round trip through an fp32
// tensor.
#include <algorithm>

#include "zest_common.h"
#include "zest_device.h"

namespace {

using zest::encode8;

// Writes 16 values of row r, columns [col, col+16) (col % 16 == 0), of the
// next matmul's input: the bfp16 pack, stored expanded.
__device__ inline void pack16(uint8_t * packed, int64_t R_pad, int64_t r, int64_t col, const float v[16]) {
    zest::store_expanded16(packed, R_pad, r, col, v);
}

__device__ inline void load16(const float * p, float v[16], int64_t valid) {
    if (valid >= 16 && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 q = reinterpret_cast<const float4 *>(p)[i];
            v[4 * i] = q.x;
            v[4 * i + 1] = q.y;
            v[4 * i + 2] = q.z;
            v[4 * i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = i < valid ? p[i] : 0.0f;
    }
}

__device__ inline void store16(float * p, const float v[16], int64_t valid) {
    if (valid >= 16 && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            reinterpret_cast<float4 *>(p)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i < valid) p[i] = v[i];
    }
}

constexpr int NORM_ROWS = 4;  // rows per workgroup, one wave each

// Writes 4 values of row r at columns [c, c+4) (c % 4 == 0) of the next
// matmul's input, the bfp16 pack stored expanded: the 8-column block is this
// lane's 4 and its neighbour's (lane ^ 1), whose largest exponent field one
// lane exchange finds; the 4 values are encoded as encode8 does and stored as
// the bf16 they stand for (8 bytes). Both lanes of a pair must call it.
__device__ inline void pack4_expanded(uint8_t * packed, int64_t R_pad, int64_t r, int64_t c, const float v[4]) {
    uint32_t e = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) e = max(e, (__float_as_uint(v[q]) >> 23) & 0xffu);
    e = max(e, (uint32_t) __shfl_xor((int) e, 1));
    const int sh = 133 - (int) e;
    const float sc = zest::block_scale(e);
    uint32_t b[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int32_t qi =
            (int32_t) __builtin_amdgcn_fmed3f(__builtin_rintf(__builtin_ldexpf(v[q], sh)), -128.0f, 127.0f);
        b[q] = __float_as_uint((float) qi * sc) >> 16;  // exact: at most 8 significant bits
    }
    *reinterpret_cast<uint2 *>(packed + zest_xoffset(r, c, R_pad)) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
}

// Zeroes row r of an expanded operand (d_pad columns): a padding row past the
// last real row, which the GEMM reads as zero.
__device__ inline void zero_row_expanded(uint8_t * packed, int64_t R_pad, int64_t r, int64_t d_pad, int lane) {
    for (int64_t c = lane * 4; c < d_pad; c += 256)
        *reinterpret_cast<uint2 *>(packed + zest_xoffset(r, c, R_pad)) = make_uint2(0, 0);
}

// Rows wider than rms_norm_row_kernel takes: one wave per row, sum of
// squares (fp32), sc = 1/sqrt(ss/d + eps),
// y = x * sc (* w). Lane l takes the 4 floats at columns 4l + 256i, so a
// wave's load covers 1 KB of the row; the sum is a wave reduction, no LDS.
// The second pass re-reads the row (from L2) and writes y and/or the packed
// row, including the zero blocks of the K padding when d % 64 != 0; waves
// past the last row zero the packed operand's padding rows.
__global__ __launch_bounds__(NORM_ROWS * 64) void rms_norm_kernel(const float * __restrict__ x, int64_t rows,
                                                                  int64_t d, float eps, const float * __restrict__ w,
                                                                  float * __restrict__ y, uint8_t * __restrict__ packed,
                                                                  int64_t R_pad) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t) blockIdx.x * NORM_ROWS + (threadIdx.x >> 6);
    const int64_t d_pad = zest_k_padded(d);
    if (r >= rows) {
        if (packed && r < R_pad) zero_row_expanded(packed, R_pad, r, d_pad, lane);
        return;
    }
    const float * xr = x + r * d;
    const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    auto load4 = [&](const float * p, int64_t c, float v[4]) {
        if (vec && c + 4 <= d) {
            const float4 q = *reinterpret_cast<const float4 *>(p + c);
            v[0] = q.x;
            v[1] = q.y;
            v[2] = q.z;
            v[3] = q.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = c + i < d ? p[c + i] : 0.0f;
        }
    };
    float ss = 0.0f;
    for (int64_t c = lane * 4; c < d; c += 256) {
        float v[4];
        load4(xr, c, v);
#pragma unroll
        for (int i = 0; i < 4; i++) ss += v[i] * v[i];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float sc = 1.0f / sqrtf(ss / (float) d + eps);
    const bool wvec = w && vec && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    for (int64_t c = lane * 4; c < (packed ? d_pad : d); c += 256) {
        float o[4];
        load4(xr, c, o);
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] *= sc;
        if (w) {
            float wv[4];
            if (wvec && c + 4 <= d) {
                const float4 q = *reinterpret_cast<const float4 *>(w + c);
                wv[0] = q.x;
                wv[1] = q.y;
                wv[2] = q.z;
                wv[3] = q.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) wv[i] = c + i < d ? w[c + i] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] *= wv[i];
        }
        if (y && c < d) {
            float * yr = y + r * d;
            if (vec && c + 4 <= d) {
                *reinterpret_cast<float4 *>(yr + c) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (c + i < d) yr[c + i] = o[i];
            }
        }
        if (packed) pack4_expanded(packed, R_pad, r, c, o);
    }
}

// One workgroup (four waves) per row, for rows of at most 1024*NCH columns
// (padding included): thread t holds the 4 floats at columns 4t + 1024i,
// loaded at once; the sum of squares is a wave reduction and then a sum of
// the four waves' partials through LDS. Four times the waves of
// rms_norm_kernel for the same rows, so more loads are in flight.
//
// Row order: workgroups are dealt to the eight XCDs in turn (workgroup b to
// XCD b % 8), and a row writes only 32 bytes of each 128-byte line of the
// expanded operand (the other 96 are rows r^1..r^3 of its 4-row quartet).
// With a grid of 8k workgroups, workgroup b takes row (b % 8) * k + b / 8,
// so each XCD owns a contiguous run of k rows, every line is completed
// inside one XCD's L2, and no line leaves an L2 partly written
// (2048 x 2560 with the pack: 9.5 -> 7.3 us).
template <int NCH>
__global__ __launch_bounds__(256) void rms_norm_row_kernel(const float * __restrict__ x, int64_t rows, int64_t d,
                                                           float eps, const float * __restrict__ w,
                                                           float * __restrict__ y, uint8_t * __restrict__ packed,
                                                           int64_t R_pad) {
    __shared__ float part[4];
    const int t = threadIdx.x, lane = t & 63;
    const int64_t G = gridDim.x, b = blockIdx.x;
    const int64_t r = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    const int64_t d_pad = zest_k_padded(d);
    if (r >= rows) {  // a padding row of the packed operand (the whole workgroup takes this branch)
        for (int64_t c = t * 4; c < d_pad; c += 1024)
            *reinterpret_cast<uint2 *>(packed + zest_xoffset(r, c, R_pad)) = make_uint2(0, 0);
        return;
    }
    const float * xr = x + r * d;
    const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    float v[NCH][4];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int64_t c = t * 4 + 1024 * i;
        if (vec && c + 4 <= d) {
            const float4 q = *reinterpret_cast<const float4 *>(xr + c);
            v[i][0] = q.x;
            v[i][1] = q.y;
            v[i][2] = q.z;
            v[i][3] = q.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) v[i][q] = c + q < d ? xr[c + q] : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < NCH; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) ss += v[i][q] * v[i][q];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) part[t >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float sc = 1.0f / sqrtf(ss / (float) d + eps);
    const bool wvec = w && vec && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    const int64_t c_end = packed ? d_pad : d;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int64_t c = t * 4 + 1024 * i;
        if (c >= c_end) continue;  // pair-uniform: c_end is a multiple of 8
        float o[4];
#pragma unroll
        for (int q = 0; q < 4; q++) o[q] = v[i][q] * sc;
        if (w) {
            if (wvec && c + 4 <= d) {
                const float4 q = *reinterpret_cast<const float4 *>(w + c);
                o[0] *= q.x;
                o[1] *= q.y;
                o[2] *= q.z;
                o[3] *= q.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) o[q] *= c + q < d ? w[c + q] : 0.0f;
            }
        }
        if (y && c < d) {
            float * yr = y + r * d;
            if (vec && c + 4 <= d) {
                *reinterpret_cast<float4 *>(yr + c) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (c + q < d) yr[c + q] = o[q];
            }
        }
        if (packed) pack4_expanded(packed, R_pad, r, c, o);
    }
}

// One thread per 16 outputs of one row: y = act(g) * u (REGLU as g > 0 ? g*u : 0).
// With a packed output the grid also covers its padding rows, written as zeros.
template <int KIND>
__global__ __launch_bounds__(256) void glu_kernel(const float * __restrict__ g, int64_t sg, const float * __restrict__ u,
                                                  int64_t su, int64_t rows, int64_t f, float * __restrict__ y,
                                                  uint8_t * __restrict__ packed, int64_t R_pad, int64_t grid_rows) {
    const int64_t units = zest_k_padded(f) / 16;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= grid_rows * units) return;
    const int64_t r = idx / units, c = (idx % units) * 16;
    float o[16];
    if (r < rows && c < f) {
        float gv[16], uv[16];
        load16(g + r * sg + c, gv, f - c);
        load16(u + r * su + c, uv, f - c);
#pragma unroll
        for (int i = 0; i < 16; i++) o[i] = zest::glu(KIND, gv[i], uv[i]);
        if (y) store16(y + r * f + c, o, f - c);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) o[i] = 0.0f;
    }
    if (packed) {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (c + i >= f) o[i] = 0.0f;
        pack16(packed, R_pad, r, c, o);
    }
}

// Row-wise binary ops over rows x d (row-major, contiguous): y = a OP b,
// with b either the same shape or one row broadcast to every row (b_row).
// Thread t of column block x takes columns 4t + 1024x of rows y, y + Y, ...
// (a 2-D grid: no division per element), four at a time with 16-byte loads
// and stores when VEC (d % 4 == 0 and every pointer 16-byte aligned).
template <int OP, bool VEC>  // OP 0: add, 1: mul
__global__ __launch_bounds__(256) void binary_rows_kernel(const float * __restrict__ a, const float * __restrict__ b,
                                                          int64_t rows, int64_t d, int b_row, float * __restrict__ y) {
    const int64_t c = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= d) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float * ar = a + r * d;
        const float * br = b_row ? b : b + r * d;
        float * yr = y + r * d;
        if (VEC) {
            const float4 u = *reinterpret_cast<const float4 *>(ar + c), v = *reinterpret_cast<const float4 *>(br + c);
            *reinterpret_cast<float4 *>(yr + c) = OP == 0 ? make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w)
                                                          : make_float4(u.x * v.x, u.y * v.y, u.z * v.z, u.w * v.w);
        } else {
            for (int64_t i = c; i < c + 4 && i < d; i++) yr[i] = OP == 0 ? ar[i] + br[i] : ar[i] * br[i];
        }
    }
}

// y = x * s + b over n floats, four a thread (16-byte accesses when VEC).
template <bool VEC>
__global__ __launch_bounds__(256) void scale_kernel(const float * __restrict__ x, int64_t n, float s, float b,
                                                    float * __restrict__ y) {
    const int64_t i = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    if (VEC && i + 4 <= n) {
        const float4 u = *reinterpret_cast<const float4 *>(x + i);
        *reinterpret_cast<float4 *>(y + i) = make_float4(u.x * s + b, u.y * s + b, u.z * s + b, u.w * s + b);
    } else {
        for (int64_t k = i; k < i + 4 && k < n; k++) y[k] = x[k] * s + b;
    }
}

// NaN or infinity anywhere in rows x cols (row stride ld) sets *flag. The test
// is on the bits (exponent field all ones), so no fast-math can fold it away.
// 2-D grid as binary_rows_kernel, four columns a thread.
__global__ __launch_bounds__(256) void check_finite_kernel(const float * __restrict__ y, int64_t rows, int64_t cols,
                                                           int64_t ld, uint32_t * flag) {
    const int64_t c = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= cols) return;
    bool bad = false;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y)
        for (int64_t i = c; i < c + 4 && i < cols; i++)
            bad |= (__float_as_uint(y[r * ld + i]) & 0x7f800000u) == 0x7f800000u;
    if (bad) atomicOr(flag, 1u);
}

// ROPE: one workgroup per token. Thread 0 walks θ through the pairs as the
// reference's table loop does (src/xdna-exec.cpp:225-233): θ_0 = pos, and
// θ_{p+1} = θ_p * theta_scale, one float multiplication a pair; each thread
// then forms the cos and sin of its pairs (rope_yarn), and the token's heads
// are rotated from that table (the rotation of :326-339); dimensions past
// n_dims are copied. Shared memory: n_dims/2 angles, then n_dims/2 (cos, sin).
__global__ __launch_bounds__(256) void rope_kernel(const float * __restrict__ x, int64_t heads, int64_t d,
                                                   const int32_t * __restrict__ pos, const float * __restrict__ ff,
                                                   int n_dims, int neox, float theta_scale, float freq_scale,
                                                   float ext_factor, float attn_factor, float corr0, float corr1,
                                                   float * __restrict__ y) {
    extern __shared__ float rope_sh[];
    const int half = n_dims / 2;
    float * theta = rope_sh;
    float2 * cs = reinterpret_cast<float2 *>(rope_sh + ((half + 1) & ~1));
    const int64_t t = blockIdx.x;
    if (threadIdx.x == 0) {
        float th = (float) pos[t];
        for (int p = 0; p < half; p++) {
            theta[p] = th;
            th *= theta_scale;
        }
    }
    __syncthreads();
    for (int p = threadIdx.x; p < half; p += blockDim.x) {
        const float theta_extrap = ff ? theta[p] / ff[p] : theta[p];
        float th = freq_scale * theta_extrap, mscale = attn_factor;
        if (ext_factor != 0.0f) {
            // every operation rounded on its own, as the CPU's expression is:
            // a fused multiply-add moves the angle by an ulp, which at
            // positions in the tens of thousands shows in its sine and cosine
#pragma clang fp contract(off)
            const float yv = ((float) p - corr0) / fmaxf(0.001f, corr1 - corr0);
            const float ramp_mix = (1.0f - fminf(1.0f, fmaxf(0.0f, yv))) * ext_factor;
            th = th * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
        }
        cs[p] = make_float2(cosf(th) * mscale, sinf(th) * mscale);
    }
    __syncthreads();
    const int64_t off = neox ? half : 1;
    for (int64_t k = threadIdx.x; k < heads * half; k += blockDim.x) {
        const int64_t h = k / half, p = k - h * half;
        const float * src = x + (t * heads + h) * d;
        float * dst = y + (t * heads + h) * d;
        const int64_t ic = neox ? p : 2 * p;
        const float2 r = cs[p];
        const float x0 = src[ic], x1 = src[ic + off];
        dst[ic] = x0 * r.x - x1 * r.y;
        dst[ic + off] = x0 * r.y + x1 * r.x;
    }
    const int64_t rest = d - n_dims;
    if (rest > 0)
        for (int64_t k = threadIdx.x; k < heads * rest; k += blockDim.x) {
            const int64_t h = k / rest, i = n_dims + (k - h * rest);
            y[(t * heads + h) * d + i] = x[(t * heads + h) * d + i];
        }
}

unsigned blocks_for(int64_t n, int per) { return (unsigned) ((n + per - 1) / per); }

// rows x d as (column blocks of 1024, up to 65535 row slots)
dim3 row_grid(int64_t rows, int64_t d) {
    return dim3(blocks_for(d, 1024), (unsigned) std::min<int64_t>(rows, 65535));
}

bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int OP>
void binary_rows(const float * a, const float * b, int64_t rows, int64_t d, int b_row, float * y,
                        hipStream_t s) {
    if (d % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(y))
        hipLaunchKernelGGL((binary_rows_kernel<OP, true>), row_grid(rows, d), dim3(256), 0, s, a, b, rows, d, b_row, y);
    else
        hipLaunchKernelGGL((binary_rows_kernel<OP, false>), row_grid(rows, d), dim3(256), 0, s, a, b, rows, d, b_row, y);
}


} // namespace

extern "C" {

int zest_rms_norm(const float * x, int64_t rows, int64_t d, float eps, const float * w, float * y, void * packed,
                  void * stream) {
    ZEST_REQUIRE(x && (y || packed), "zest_rms_norm: null pointer");
    ZEST_REQUIRE(rows > 0 && d > 0, "zest_rms_norm: rows=%lld d=%lld", (long long) rows, (long long) d);
    ZEST_REQUIRE(!packed || d % 8 == 0, "zest_rms_norm: packing needs d %% 8 == 0");
    ZEST_REQUIRE(aligned16(packed), "zest_rms_norm: packed must be 16-byte aligned");
    // with a packed output, the grid also covers its padding rows (zeroed)
    const int64_t R_pad = zest_rows_padded(rows), grid_rows = packed ? R_pad : rows;
    const int64_t chunks = (zest_k_padded(d) + 255) / 256;  // the output pass covers the padded width
    hipStream_t s = zest::as_stream(stream);
    uint8_t * pk = (uint8_t *) packed;
    if (chunks <= 4)  // up to 1024 columns: one workgroup per row
        hipLaunchKernelGGL(rms_norm_row_kernel<1>, dim3((unsigned) grid_rows), dim3(256), 0, s, x, rows, d, eps, w, y,
                           pk, R_pad);
    else if (chunks <= 12)  // up to 3072
        hipLaunchKernelGGL(rms_norm_row_kernel<3>, dim3((unsigned) grid_rows), dim3(256), 0, s, x, rows, d, eps, w, y,
                           pk, R_pad);
    else if (chunks <= 24)  // up to 6144
        hipLaunchKernelGGL(rms_norm_row_kernel<6>, dim3((unsigned) grid_rows), dim3(256), 0, s, x, rows, d, eps, w, y,
                           pk, R_pad);
    else
        hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned) ((grid_rows + NORM_ROWS - 1) / NORM_ROWS)),
                           dim3(NORM_ROWS * 64), 0, s, x, rows, d, eps, w, y, pk, R_pad);
    return zest::check_launch("zest_rms_norm");
}

int zest_glu(int kind, const float * g, int64_t sg, const float * u, int64_t su, int64_t rows, int64_t f, float * y,
             void * packed, void * stream) {
    ZEST_REQUIRE(g && u && (y || packed), "zest_glu: null pointer");
    ZEST_REQUIRE(rows > 0 && f > 0 && sg >= f && su >= f, "zest_glu: bad shape");
    ZEST_REQUIRE(!packed || f % 8 == 0, "zest_glu: packing needs f %% 8 == 0");
    ZEST_REQUIRE(aligned16(packed), "zest_glu: packed must be 16-byte aligned");
    const int64_t R_pad = zest_rows_padded(rows), gr = packed ? R_pad : rows;
    const int64_t n = gr * (zest_k_padded(f) / 16);
    const dim3 grid(blocks_for(n, 256));
    hipStream_t s = zest::as_stream(stream);
    uint8_t * p = (uint8_t *) packed;
    switch (kind) {
        case ZEST_GLU_SWIGLU: hipLaunchKernelGGL(glu_kernel<ZEST_GLU_SWIGLU>, grid, dim3(256), 0, s, g, sg, u, su, rows, f, y, p, R_pad, gr); break;
        case ZEST_GLU_GEGLU: hipLaunchKernelGGL(glu_kernel<ZEST_GLU_GEGLU>, grid, dim3(256), 0, s, g, sg, u, su, rows, f, y, p, R_pad, gr); break;
        case ZEST_GLU_GEGLU_ERF: hipLaunchKernelGGL(glu_kernel<ZEST_GLU_GEGLU_ERF>, grid, dim3(256), 0, s, g, sg, u, su, rows, f, y, p, R_pad, gr); break;
        case ZEST_GLU_GEGLU_QUICK: hipLaunchKernelGGL(glu_kernel<ZEST_GLU_GEGLU_QUICK>, grid, dim3(256), 0, s, g, sg, u, su, rows, f, y, p, R_pad, gr); break;
        case ZEST_GLU_REGLU: hipLaunchKernelGGL(glu_kernel<ZEST_GLU_REGLU>, grid, dim3(256), 0, s, g, sg, u, su, rows, f, y, p, R_pad, gr); break;
        default: return zest::fail(ZEST_E_UNSUPPORTED, "zest_glu: GLU kind %d", kind);
    }
    return zest::check_launch("zest_glu");
}

int zest_add(const float * a, const float * b, int64_t rows, int64_t d, int b_is_row, float * y, void * stream) {
    ZEST_REQUIRE(a && b && y && rows > 0 && d > 0, "zest_add: bad arguments");
    binary_rows<0>(a, b, rows, d, b_is_row != 0, y, zest::as_stream(stream));
    return zest::check_launch("zest_add");
}

int zest_mul_row(const float * x, const float * w, int64_t rows, int64_t d, float * y, void * stream) {
    ZEST_REQUIRE(x && w && y && rows > 0 && d > 0, "zest_mul_row: bad arguments");
    binary_rows<1>(x, w, rows, d, 1, y, zest::as_stream(stream));
    return zest::check_launch("zest_mul_row");
}

int zest_scale(const float * x, int64_t n, float s, float b, float * y, void * stream) {
    ZEST_REQUIRE(x && y && n > 0, "zest_scale: bad arguments");
    const dim3 grid(blocks_for(n, 1024));
    if (aligned16(x) && aligned16(y))
        hipLaunchKernelGGL((scale_kernel<true>), grid, dim3(256), 0, zest::as_stream(stream), x, n, s, b, y);
    else
        hipLaunchKernelGGL((scale_kernel<false>), grid, dim3(256), 0, zest::as_stream(stream), x, n, s, b, y);
    return zest::check_launch("zest_scale");
}

int zest_rope(const float * x, int64_t T, int64_t heads, int64_t d, const int32_t * pos, const float * ff, int n_dims,
              int mode, float freq_base, float freq_scale, float ext_factor, float attn_factor, float corr0, float corr1,
              float * y, void * stream) {
    ZEST_REQUIRE(x && pos && y && T > 0 && heads > 0 && d > 0, "zest_rope: bad arguments");
    ZEST_REQUIRE(n_dims > 0 && n_dims % 2 == 0 && n_dims <= d, "zest_rope: n_dims=%d d=%lld", n_dims, (long long) d);
    ZEST_REQUIRE(mode == 0 || mode == 2, "zest_rope: mode %d (normal 0 or neox 2)", mode);
    ZEST_REQUIRE(T <= 0x7fffffff, "zest_rope: %lld tokens", (long long) T);
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    const int half = n_dims / 2;
    const size_t lds = (size_t) (((half + 1) & ~1) + 2 * half) * sizeof(float);
    ZEST_REQUIRE(lds <= 65536, "zest_rope: n_dims=%d needs %zu bytes of shared memory (at most 65536)", n_dims, lds);
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned) T), dim3(256), lds, zest::as_stream(stream), x, heads, d, pos, ff,
                       n_dims, mode == 2, theta_scale, freq_scale, ext_factor, attn_factor, corr0, corr1, y);
    return zest::check_launch("zest_rope");
}

int zest_check_finite(const float * y, int64_t rows, int64_t cols, int64_t ld, uint32_t * flag, void * stream) {
    ZEST_REQUIRE(y && flag && rows > 0 && cols > 0 && ld >= cols, "zest_check_finite: bad arguments");
    ZEST_REQUIRE((reinterpret_cast<uintptr_t>(flag) & 3) == 0, "zest_check_finite: flag must be 4-byte aligned");
    hipLaunchKernelGGL(check_finite_kernel, row_grid(rows, cols), dim3(256), 0, zest::as_stream(stream), y, rows, cols,
                       ld, flag);
    return zest::check_launch("zest_check_finite");
}

} // extern "C"

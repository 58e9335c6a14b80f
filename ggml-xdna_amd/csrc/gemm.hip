// The bfp16 GEMM: C[M][N] = A[M][K] . W[N][K]^T over packed bfp16 operands.
//
// Per workgroup a BM x BN output tile; per K-step of 64 (one tile-layout
// column chunk) it
//   1. reads the A and W slabs (BM/16 and BN/16 contiguous 1152-byte tiles)
//      with 16-byte loads: each thread one or more "units" = 16 mantissas of
//      one row plus their two exponent bytes;
//   2. expands every unit once, losslessly, to 16 bf16 (zest::expand8) and
//      stores them to LDS, rows of 64 bf16 with the 16-byte chunks XOR-swizzled
//      by row so the MFMA reads are bank-conflict free;
//   3. runs v_mfma_f32_32x32x16_bf16: each lane's eight K values of an operand
//      are exactly one bfp16 block.
// LDS is double-buffered and the next K-step's global loads are in flight
// while the current one's MFMAs run; one barrier per K-step. Accumulation is
// fp32 throughout, and the store is fp32 row-major, as the reference's output
// mode 0 (kernels/bfp16_gemm/aie_kernels/aie2p/mm_bfp_acc.cc:106-116, 258-278).
#include "zest_common.h"
#include "zest_device.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct unit_regs {
    uint4 m;
    uint32_t e;
};

template <int BM, int BN, int WGM, int WGN>
struct gemm_cfg {
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int TI = WM / 32, TJ = WN / 32;
    static constexpr int AU = BM * 4 / NT, BU = BN * 4 / NT;  // units per thread per K-step
    static constexpr int LDS_CHUNKS = (BM + BN) * 8;         // 16-byte chunks per buffer
    static_assert(BM * 4 % NT == 0 && BN * 4 % NT == 0, "units must divide evenly");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
};

// Unit u of a slab: tile u/64, within it row (u%64)/4 and column quarter u%4.
// Its mantissas are at tile*1152 + (u%64)*16, its exponents at
// tile*1152 + 1024 + (u%64)*2.
__device__ inline unit_regs load_unit(const uint8_t * slab, int u) {
    const uint8_t * t = slab + (u >> 6) * ZEST_TILE_BYTES;
    const int c = u & 63;
    unit_regs r;
    r.m = *reinterpret_cast<const uint4 *>(t + c * 16);
    r.e = *reinterpret_cast<const uint16_t *>(t + ZEST_TILE_MANT + c * 2);
    return r;
}

// Expands unit u (row (u/64)*16 + (u%64)/4 of the slab, chunks 2q and 2q+1 of
// that row) into LDS rows starting at `row0`.
__device__ inline void store_unit(uint4 * lds, int row0, int u, const unit_regs & r) {
    const int row = row0 + (u >> 6) * 16 + ((u & 63) >> 2);
    const int q = u & 3;
    uint32_t b0[4], b1[4];
    zest::expand8(r.m.x, r.m.y, r.e & 0xffu, b0);
    zest::expand8(r.m.z, r.m.w, r.e >> 8, b1);
    const int sw = row & 7;
    lds[row * 8 + ((2 * q) ^ sw)] = make_uint4(b0[0], b0[1], b0[2], b0[3]);
    lds[row * 8 + ((2 * q + 1) ^ sw)] = make_uint4(b1[0], b1[1], b1[2], b1[3]);
}

__device__ inline bf16x8 lds_frag(const uint4 * lds, int row, int chunk) {
    const uint4 v = lds[row * 8 + (chunk ^ (row & 7))];
    return __builtin_bit_cast(bf16x8, v);
}

template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_kernel(const uint8_t * __restrict__ A, int64_t M_pad,
                                                               const uint8_t * __restrict__ W, int64_t N_pad, int nk,
                                                               float * __restrict__ C, int64_t M, int64_t N,
                                                               int64_t ldc, uint32_t * nonfinite) {
    using cfg = gemm_cfg<BM, BN, WGM, WGN>;
    __shared__ uint4 lds[2][cfg::LDS_CHUNKS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int64_t m0 = (int64_t) blockIdx.y * BM, n0 = (int64_t) blockIdx.x * BN;

    const int64_t a_kstride = (M_pad / ZEST_TILE_ROWS) * ZEST_TILE_BYTES;
    const int64_t w_kstride = (N_pad / ZEST_TILE_ROWS) * ZEST_TILE_BYTES;
    const uint8_t * a_slab = A + (m0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES;
    const uint8_t * w_slab = W + (n0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES;

    unit_regs ar[cfg::AU], br[cfg::BU];
#pragma unroll
    for (int i = 0; i < cfg::AU; i++) ar[i] = load_unit(a_slab, tid + i * cfg::NT);
#pragma unroll
    for (int i = 0; i < cfg::BU; i++) br[i] = load_unit(w_slab, tid + i * cfg::NT);
#pragma unroll
    for (int i = 0; i < cfg::AU; i++) store_unit(lds[0], 0, tid + i * cfg::NT, ar[i]);
#pragma unroll
    for (int i = 0; i < cfg::BU; i++) store_unit(lds[0], BM, tid + i * cfg::NT, br[i]);
    __syncthreads();

    f32x16 acc[cfg::TI][cfg::TJ];
#pragma unroll
    for (int i = 0; i < cfg::TI; i++)
#pragma unroll
        for (int j = 0; j < cfg::TJ; j++) acc[i][j] = f32x16{};

    const int a_row = wm * cfg::WM + (lane & 31);
    const int w_row = BM + wn * cfg::WN + (lane & 31);
    const int khalf = lane >> 5;

    for (int kc = 0; kc < nk; kc++) {
        const int cur = kc & 1;
        const bool more = kc + 1 < nk;
        if (more) {
            a_slab += a_kstride;
            w_slab += w_kstride;
#pragma unroll
            for (int i = 0; i < cfg::AU; i++) ar[i] = load_unit(a_slab, tid + i * cfg::NT);
#pragma unroll
            for (int i = 0; i < cfg::BU; i++) br[i] = load_unit(w_slab, tid + i * cfg::NT);
        }
        const uint4 * L = lds[cur];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            bf16x8 af[cfg::TI], bfr[cfg::TJ];
#pragma unroll
            for (int i = 0; i < cfg::TI; i++) af[i] = lds_frag(L, a_row + i * 32, 2 * s + khalf);
#pragma unroll
            for (int j = 0; j < cfg::TJ; j++) bfr[j] = lds_frag(L, w_row + j * 32, 2 * s + khalf);
#pragma unroll
            for (int i = 0; i < cfg::TI; i++)
#pragma unroll
                for (int j = 0; j < cfg::TJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < cfg::AU; i++) store_unit(lds[cur ^ 1], 0, tid + i * cfg::NT, ar[i]);
#pragma unroll
            for (int i = 0; i < cfg::BU; i++) store_unit(lds[cur ^ 1], BM, tid + i * cfg::NT, br[i]);
        }
        __syncthreads();
    }

    // 32x32 accumulator layout: lane l, register v holds row
    // (v/4)*8 + (l/32)*4 + v%4 and column l%32 of the tile.
    bool bad = false;
#pragma unroll
    for (int i = 0; i < cfg::TI; i++)
#pragma unroll
        for (int j = 0; j < cfg::TJ; j++) {
            const int64_t col = n0 + wn * cfg::WN + j * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int64_t row = m0 + wm * cfg::WM + i * 32 + (v >> 2) * 8 + khalf * 4 + (v & 3);
                if (row < M && col < N) {
                    const float x = acc[i][j][v];
                    bad |= (__float_as_uint(x) & 0x7f800000u) == 0x7f800000u;
                    C[row * ldc + col] = x;
                }
            }
        }
    if (nonfinite && __any(bad) && lane == 0) atomicOr(nonfinite, 1u);
}

template <int BM, int BN, int WGM, int WGN>
int launch(const void * a, int64_t M, const void * w, int64_t N, int64_t K, float * c, int64_t ldc, uint32_t * nf,
           hipStream_t s) {
    const int64_t M_pad = zest_rows_padded(M), N_pad = zest_rows_padded(N), K_pad = zest_k_padded(K);
    const dim3 grid((unsigned) ((N + BN - 1) / BN), (unsigned) ((M + BM - 1) / BM));
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WGM, WGN>), grid, dim3(64 * WGM * WGN), 0, s, (const uint8_t *) a, M_pad,
                       (const uint8_t *) w, N_pad, (int) (K_pad / ZEST_TILE_K), c, M, N, ldc, nf);
    return zest::check_launch("zest_gemm");
}

} // namespace

extern "C" int zest_gemm(const void * a, int64_t M, const void * w, int64_t N, int64_t K, float * c, int64_t ldc,
                         uint32_t * nonfinite, void * stream) {
    ZEST_REQUIRE(a && w && c, "zest_gemm: null pointer");
    ZEST_REQUIRE(M > 0 && N > 0 && K > 0 && K % 8 == 0, "zest_gemm: M=%lld N=%lld K=%lld", (long long) M,
                 (long long) N, (long long) K);
    ZEST_REQUIRE(ldc >= N, "zest_gemm: ldc %lld < N %lld", (long long) ldc, (long long) N);
    return launch<128, 128, 2, 2>(a, M, w, N, K, c, ldc, nonfinite, zest::as_stream(stream));
}

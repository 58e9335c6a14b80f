// The bfp16 GEMM: C[M][N] = A[M][K] . W[N][K]^T over packed bfp16 operands.
//
// Per workgroup a BM x BN output tile; per K-step of 64 (one tile-layout
// column chunk) it
//   1. reads the A and W slabs (BM/16 and BN/16 contiguous 1152-byte tiles)
//      with 16-byte buffer loads: each thread one or more "units" = 16
//      mantissas of one row plus their two exponent bytes;
//   2. expands every unit once, losslessly, to 16 bf16 (zest::expand16) and
//      stores them to LDS, rows of 64 bf16 with the 16-byte chunks XOR-swizzled
//      by row so the stores and the MFMA reads are bank-conflict free;
//   3. runs v_mfma_f32_32x32x16_bf16: each lane's eight K values of an operand
//      are exactly one bfp16 block.
// Software pipeline: the global loads of K-step k+1 are issued as step k
// starts, and step k+1 is expanded into the other LDS buffer in between step
// k's later MFMAs; one barrier closes each step. Accumulation is fp32 throughout,
// and the store is fp32 row-major, as the reference's output mode 0
// (kernels/bfp16_gemm/aie_kernels/aie2p/mm_bfp_acc.cc:106-116, 258-278).
//
// LDS: [A buf 0][A buf 1][W buf 0][W buf 1], each BM (or BN) rows of 128
// bytes, so every fragment and store address is a per-lane base plus an
// immediate offset (buffer, MFMA tile, unit) and the address registers stay
// few.
#include "zest_common.h"
#include "zest_device.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct unit_regs {
    uint4 m;
    uint32_t e;
};

// BM x BN tile over WGM x WGN waves; DEPTH 1 or 2 staging register sets (how
// many K-steps ahead the global loads run); the next step's expansion starts
// after sub-step EXP_START of the current one.
template <int BM_, int BN_, int WGM_, int WGN_, int DEPTH_ = 2, int EXP_START_ = 0>
struct gemm_cfg {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, DEPTH = DEPTH_, EXP_START = EXP_START_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int TI = WM / 32, TJ = WN / 32;
    static constexpr int AU = BM * 4 / NT, BU = BN * 4 / NT;  // units per thread per K-step
    static constexpr int U = AU + BU;
    static constexpr int ROWB = 128;                          // LDS bytes per row (64 bf16)
    static constexpr int A_BUF = BM * ROWB, W_BUF = BN * ROWB;
    static constexpr int W_BASE = 2 * A_BUF;
    static constexpr size_t LDS_BYTES = 2 * (A_BUF + W_BUF);
    static constexpr int UNIT_ROWS = NT / 4;                  // rows between a thread's units
    static_assert(BM * 4 % NT == 0 && BN * 4 % NT == 0, "units must divide evenly");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
};

// Unit u of a slab: tile u/64, within it row (u%64)/4 and column quarter u%4.
// Its mantissas are at tile*1152 + (u%64)*16, its exponents at
// tile*1152 + 1024 + (u%64)*2. Loads go through buffer resources: the slab's
// byte offset is wave-uniform (a scalar offset), the lane's place in it a
// fixed vector offset, and a read past the operand returns zeros.
struct slab_reader {
    __amdgpu_buffer_rsrc_t rsrc;
    int vm, ve;  // lane offsets of unit `tid`'s mantissas and exponents
};

// Lane -> unit within each 64-unit (one tile) group: row l%16, column
// quarter l/16, so 16 consecutive lanes handle 16 consecutive rows (see the
// LDS swizzle). A wave's load still covers the tile's 1 KB of mantissas and
// 128 bytes of exponents exactly.
__device__ inline int unit_of_lane(int tid) { return (tid & 15) * 4 + ((tid >> 4) & 3); }

__device__ inline slab_reader make_reader(const uint8_t * base, int64_t bytes, int tid) {
    slab_reader r;
    r.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short) 0, (int) bytes, 0x00020000);
    const int c = unit_of_lane(tid);
    r.vm = (tid >> 6) * ZEST_TILE_BYTES + c * 16;
    r.ve = (tid >> 6) * ZEST_TILE_BYTES + ZEST_TILE_MANT + c * 2;
    return r;
}

__device__ inline unit_regs load_unit(const slab_reader & rd, int soff) {
    unit_regs r;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rd.rsrc, rd.vm, soff, 0);
    r.m = make_uint4(v[0], v[1], v[2], v[3]);
    r.e = __builtin_amdgcn_raw_buffer_load_b16(rd.rsrc, rd.ve, soff, 0);
    return r;
}

// Thread tid's units of one K-step are tid + i*NT: i*NT/64 tiles further on.
template <class C>
__device__ inline void load_step(unit_regs (&st)[C::U], const slab_reader & ra, int a_off, const slab_reader & rw,
                                 int w_off) {
    constexpr int STEP = C::NT / 64 * ZEST_TILE_BYTES;
#pragma unroll
    for (int i = 0; i < C::AU; i++) st[i] = load_unit(ra, a_off + i * STEP);
#pragma unroll
    for (int i = 0; i < C::BU; i++) st[C::AU + i] = load_unit(rw, w_off + i * STEP);
}

// LDS rows are 128 bytes = 8 chunks of 16 bytes (one bfp16 block as bf16
// each); chunk c of row r is stored at position c ^ swz(r), with
// swz(r) = (r % 8) ^ ((r / 8) % 2). Any 16 consecutive rows (from a multiple
// of 16) then put one chunk index in 16 different 16-byte slots of a 256-byte
// window, and any 8 consecutive rows in 8 slots of a 128-byte window: the
// fragment reads (16 lanes = 16 rows, one chunk) and the unit stores (16 lanes
// = 16 rows, one chunk) are free of bank conflicts, and swz is unchanged by
// the +32-row offsets of the MFMA tiles, which stay immediates.
__device__ inline int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Per-lane LDS byte offsets. Unit tid + i*NT is row (tid/64)*16 + tid%16 +
// i*NT/4 of its slab, chunks 2q, 2q+1 (q = (tid/16)%4).
struct lds_lanes {
    int st0, st1;      // unit-store chunks 2q and 2q+1 (A buffer 0; the rest as immediates)
    int fa[4], fw[4];  // fragment reads for sub-steps s = 0..3
};

template <class C>
__device__ inline lds_lanes make_lanes(int tid) {
    lds_lanes l;
    const int row = (tid >> 6) * 16 + (tid & 15), q = (tid >> 4) & 3, sw = swz(row);
    l.st0 = row * C::ROWB + ((2 * q) ^ sw) * 16;
    l.st1 = row * C::ROWB + ((2 * q + 1) ^ sw) * 16;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WGN, wn = wave % C::WGN, khalf = lane >> 5;
    const int ar = wm * C::WM + (lane & 31), wr = wn * C::WN + (lane & 31);
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int ch = 2 * s + khalf;
        l.fa[s] = ar * C::ROWB + (ch ^ swz(ar)) * 16;
        l.fw[s] = C::W_BASE + wr * C::ROWB + (ch ^ swz(wr)) * 16;
    }
    return l;
}

__device__ inline void lds_put(uint8_t * smem, int off, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *reinterpret_cast<uint4 *>(smem + off) = make_uint4(a, b, c, d);
}

__device__ inline bf16x8 lds_get(const uint8_t * smem, int off) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(smem + off));
}

// Expands units [first, last) of a step's staging registers into LDS buffer BUF.
template <class C, int BUF>
__device__ inline void store_units(const unit_regs (&st)[C::U], uint8_t * smem, const lds_lanes & ll, int first,
                                   int last) {
#pragma unroll
    for (int i = 0; i < C::U; i++) {
        if (i < first || i >= last) continue;
        const int base = i < C::AU ? BUF * C::A_BUF + i * C::UNIT_ROWS * C::ROWB
                                   : C::W_BASE + BUF * C::W_BUF + (i - C::AU) * C::UNIT_ROWS * C::ROWB;
        uint32_t b[8];  // prologue only: the general expansion
        zest::expand16(st[i].m, st[i].e, b);
        lds_put(smem, ll.st0 + base, b[0], b[1], b[2], b[3]);
        lds_put(smem, ll.st1 + base, b[4], b[5], b[6], b[7]);
    }
}

template <class C>
__device__ inline int unit_base(int i, int buf) {
    return i < C::AU ? buf * C::A_BUF + i * C::UNIT_ROWS * C::ROWB
                     : C::W_BASE + buf * C::W_BUF + (i - C::AU) * C::UNIT_ROWS * C::ROWB;
}

template <class C>
__device__ inline void read_frags(bf16x8 (&af)[C::TI], bf16x8 (&bfr)[C::TJ], const uint8_t * smem,
                                  const lds_lanes & ll, int s, int cur) {
#pragma unroll
    for (int i = 0; i < C::TI; i++) af[i] = lds_get(smem, ll.fa[s] + cur * C::A_BUF + i * 32 * C::ROWB);
#pragma unroll
    for (int j = 0; j < C::TJ; j++) bfr[j] = lds_get(smem, ll.fw[s] + cur * C::W_BUF + j * 32 * C::ROWB);
}

// One K-step on LDS buffer CUR: 4 sub-steps of 16 K. If LOAD, the next
// step's units are requested from memory first, into the staging registers
// `st`; they arrive while sub-steps 0..EXP_START-1 run and are expanded (fast
// path, branch-free) and stored to the other LDS buffer in between the MFMAs
// of the later sub-steps. The fragments of sub-step s+1 are read while
// sub-step s's TI*TJ MFMAs run. The scheduling pattern below interleaves
// MFMAs, VALU and LDS operations so the matrix core and the VALU work at the
// same time (one wave per SIMD, in-order issue). Units whose exponent bytes
// need the general expansion are redone after the MFMAs, behind a
// wave-uniform branch that real data almost never takes.
template <class C, int CUR, bool LOAD, bool EXPAND>
__device__ inline void mma_step(f32x16 (&acc)[C::TI][C::TJ], uint8_t * smem, const lds_lanes & ll,
                                unit_regs (&sl)[C::U], unit_regs (&st)[C::U], const slab_reader & ra, int a_off,
                                const slab_reader & rw, int w_off) {
    constexpr int EXP_START = C::EXP_START;
    constexpr int EXP_STEPS = 4 - EXP_START;
    if (LOAD) load_step<C>(sl, ra, a_off, rw, w_off);
    bf16x8 af[2][C::TI], bfr[2][C::TJ];
    read_frags<C>(af[0], bfr[0], smem, ll, 0, CUR);
    bool slow[C::U];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        if (s < 3) read_frags<C>(af[(s + 1) & 1], bfr[(s + 1) & 1], smem, ll, s + 1, CUR);
#pragma unroll
        for (int i = 0; i < C::TI; i++)
#pragma unroll
            for (int j = 0; j < C::TJ; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s & 1][i], bfr[s & 1][j], acc[i][j], 0, 0, 0);
        if (EXPAND && s >= EXP_START) {
#pragma unroll
            for (int u = (s - EXP_START) * C::U / EXP_STEPS; u < (s - EXP_START + 1) * C::U / EXP_STEPS; u++) {
                uint32_t b[8];
                slow[u] = zest::expand16_fast(st[u].m, st[u].e, b);
                const int base = unit_base<C>(u, CUR ^ 1);
                lds_put(smem, ll.st0 + base, b[0], b[1], b[2], b[3]);
                lds_put(smem, ll.st1 + base, b[4], b[5], b[6], b[7]);
            }
        }
    }
    // the scheduling pattern: per MFMA, VALU ops (expansion sub-steps only),
    // a fragment read every other MFMA, LDS stores spread over the expansion
    constexpr int PER = C::TI * C::TJ;  // MFMAs per sub-step
    constexpr int MFMAS = 4 * PER;
    constexpr int EXP_MFMAS = EXP_STEPS * PER;
    constexpr int VALU_PER = EXPAND ? (C::U * 34 + EXP_MFMAS - 1) / EXP_MFMAS : 0;
    constexpr int STORES = EXPAND ? 2 * C::U : 0;
    constexpr int READS = 3 * (C::TI + C::TJ);
    constexpr int LOADS = LOAD ? 2 * C::U : 0;
#ifndef ZEST_GEMM_SCHED
#define ZEST_GEMM_SCHED 1
#endif
    if (ZEST_GEMM_SCHED) __builtin_amdgcn_sched_group_barrier(0x100, C::TI + C::TJ, 0);  // sub-step 0's fragments
#pragma unroll
    for (int q = 0; q < (ZEST_GEMM_SCHED ? MFMAS : 0); q++) {
        if (q < LOADS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // next step's loads, early
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                // MFMA
        if (q * READS / MFMAS != (q + 1) * READS / MFMAS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (q >= MFMAS - EXP_MFMAS) {
            const int e = q - (MFMAS - EXP_MFMAS);
            if (VALU_PER) __builtin_amdgcn_sched_group_barrier(0x002, VALU_PER, 0);
            if (STORES && e * STORES / EXP_MFMAS != (e + 1) * STORES / EXP_MFMAS)
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
    }
    if (EXPAND) {
        bool any = false;
#pragma unroll
        for (int u = 0; u < C::U; u++) any |= slow[u];
        if (__builtin_expect(__any(any), 0)) {
#pragma unroll
            for (int u = 0; u < C::U; u++)
                if (slow[u]) {
                    uint32_t b[8];
                    zest::expand16(st[u].m, st[u].e, b);
                    const int base = unit_base<C>(u, CUR ^ 1);
                    lds_put(smem, ll.st0 + base, b[0], b[1], b[2], b[3]);
                    lds_put(smem, ll.st1 + base, b[4], b[5], b[6], b[7]);
                }
        }
    }
}

// The fp32 store. 32x32 accumulator layout: lane l, register v holds row
// (v/4)*8 + (l/32)*4 + v%4 and column l%32 of its MFMA tile. Stores go
// through a buffer resource covering rows [0, M) of C, so rows past M are
// dropped by the hardware range check on the vector offset (the whole byte
// offset is kept there); columns past N are masked per lane. Also ORs 1 into
// *nonfinite if any stored value is NaN or infinite.
template <class C>
__device__ inline void store_tile(const f32x16 (&acc)[C::TI][C::TJ], float * Cout, int64_t M, int64_t N, int64_t ldc,
                                  int64_t m0, int64_t n0, int wm, int wn, int lane, uint32_t * nonfinite) {
    const __amdgpu_buffer_rsrc_t rc =
        __builtin_amdgcn_make_buffer_rsrc(Cout, (short) 0, (int) (M * ldc * 4), 0x00020000);
    const int khalf = lane >> 5;
    const int row0 = (int) m0 + wm * C::WM;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < C::TJ; j++) {
        const int64_t col = n0 + wn * C::WN + j * 32 + (lane & 31);
        if (col < N) {
            const int voff = (int) (col * 4 + (int64_t) khalf * 4 * ldc * 4);
#pragma unroll
            for (int i = 0; i < C::TI; i++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const float x = acc[i][j][v];
                    bad |= !(__builtin_fabsf(x) <= 3.402823466e38f);
                    const int roff = (row0 + i * 32 + (v >> 2) * 8 + (v & 3)) * (int) ldc * 4;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rc, voff + roff, 0, 0);
                }
        }
    }
    if (nonfinite && __any(bad) && lane == 0) atomicOr(nonfinite, 1u);
}

template <class C>
__global__ __launch_bounds__(C::NT, 1) void gemm_kernel(const uint8_t * __restrict__ A, int64_t M_pad,
                                                        const uint8_t * __restrict__ W, int64_t N_pad, int nk,
                                                        float * __restrict__ Cout, int64_t M, int64_t N, int64_t ldc,
                                                        uint32_t * nonfinite) {
    extern __shared__ uint4 smem_u4[];
    uint8_t * smem = reinterpret_cast<uint8_t *>(smem_u4);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WGN, wn = wave % C::WGN;
    const int64_t m0 = (int64_t) blockIdx.y * C::BM, n0 = (int64_t) blockIdx.x * C::BN;

    // operands are < 2 GiB (checked by the host), so byte offsets fit an int
    const int a_kstride = (int) ((M_pad / ZEST_TILE_ROWS) * ZEST_TILE_BYTES);
    const int w_kstride = (int) ((N_pad / ZEST_TILE_ROWS) * ZEST_TILE_BYTES);
    const int a0 = (int) ((m0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES);
    const int w0 = (int) ((n0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES);
    const slab_reader ra = make_reader(A, (int64_t) a_kstride * nk, tid);
    const slab_reader rw = make_reader(W, (int64_t) w_kstride * nk, tid);
    const lds_lanes ll = make_lanes<C>(tid);

    f32x16 acc[C::TI][C::TJ];
#pragma unroll
    for (int i = 0; i < C::TI; i++)
#pragma unroll
        for (int j = 0; j < C::TJ; j++) acc[i][j] = f32x16{};
    if (C::DEPTH == 1) {
        // Step k computes on buffer k&1 and, unless it is the last, loads
        // step k+1 as it starts and expands it into the other buffer.
        unit_regs st[C::U];
        load_step<C>(st, ra, a0, rw, w0);
        store_units<C, 0>(st, smem, ll, 0, C::U);
        __syncthreads();
        int kc = 0;
        for (; kc + 2 < nk; kc += 2) {
            mma_step<C, 0, true, true>(acc, smem, ll, st, st, ra, a0 + (kc + 1) * a_kstride, rw, w0 + (kc + 1) * w_kstride);
            __syncthreads();
            mma_step<C, 1, true, true>(acc, smem, ll, st, st, ra, a0 + (kc + 2) * a_kstride, rw, w0 + (kc + 2) * w_kstride);
            __syncthreads();
        }
        if (kc + 1 < nk) {  // 2 left
            mma_step<C, 0, true, true>(acc, smem, ll, st, st, ra, a0 + (kc + 1) * a_kstride, rw, w0 + (kc + 1) * w_kstride);
            __syncthreads();
            mma_step<C, 1, false, false>(acc, smem, ll, st, st, ra, 0, rw, 0);
        } else {  // 1 left
            mma_step<C, 0, false, false>(acc, smem, ll, st, st, ra, 0, rw, 0);
        }
    } else {
        // Two staging sets: step k loads step k+2 into one while expanding
        // step k+1 (loaded during step k-1) from the other.
        unit_regs sa[C::U], sb[C::U];
        load_step<C>(sa, ra, a0, rw, w0);
        if (nk > 1) load_step<C>(sb, ra, a0 + a_kstride, rw, w0 + w_kstride);
        store_units<C, 0>(sa, smem, ll, 0, C::U);
        __syncthreads();
        int kc = 0;
        for (; kc + 3 < nk; kc += 2) {
            mma_step<C, 0, true, true>(acc, smem, ll, sa, sb, ra, a0 + (kc + 2) * a_kstride, rw, w0 + (kc + 2) * w_kstride);
            __syncthreads();
            mma_step<C, 1, true, true>(acc, smem, ll, sb, sa, ra, a0 + (kc + 3) * a_kstride, rw, w0 + (kc + 3) * w_kstride);
            __syncthreads();
        }
        if (kc + 2 < nk) {  // 3 left
            mma_step<C, 0, true, true>(acc, smem, ll, sa, sb, ra, a0 + (kc + 2) * a_kstride, rw, w0 + (kc + 2) * w_kstride);
            __syncthreads();
            mma_step<C, 1, false, true>(acc, smem, ll, sb, sa, ra, 0, rw, 0);
            __syncthreads();
            mma_step<C, 0, false, false>(acc, smem, ll, sa, sb, ra, 0, rw, 0);
        } else if (kc + 1 < nk) {  // 2 left
            mma_step<C, 0, false, true>(acc, smem, ll, sa, sb, ra, 0, rw, 0);
            __syncthreads();
            mma_step<C, 1, false, false>(acc, smem, ll, sa, sb, ra, 0, rw, 0);
        } else {  // 1 left
            mma_step<C, 0, false, false>(acc, smem, ll, sa, sb, ra, 0, rw, 0);
        }
    }

    store_tile<C>(acc, Cout, M, N, ldc, m0, n0, wm, wn, lane, nonfinite);
}

template <class C>
int launch(const void * a, int64_t M, const void * w, int64_t N, int64_t K, float * c, int64_t ldc, uint32_t * nf,
           hipStream_t s) {
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_kernel<C>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int) C::LDS_BYTES);
        if (e != hipSuccess) return zest::fail(ZEST_E_HIP, "zest_gemm: LDS attribute: %s", hipGetErrorString(e));
        attr_set = true;
    }
    const int64_t M_pad = zest_rows_padded(M), N_pad = zest_rows_padded(N), K_pad = zest_k_padded(K);
    const dim3 grid((unsigned) ((N + C::BN - 1) / C::BN), (unsigned) ((M + C::BM - 1) / C::BM));
    hipLaunchKernelGGL((gemm_kernel<C>), grid, dim3(C::NT), C::LDS_BYTES, s, (const uint8_t *) a, M_pad,
                       (const uint8_t *) w, N_pad, (int) (K_pad / ZEST_TILE_K), c, M, N, ldc, nf);
    return zest::check_launch("zest_gemm");
}

// Measured on MI355X over the BASELINE shapes: 256x128 tiles on 8 waves
// (128x32 each) with two staging sets lead wherever there are enough tiles;
// 128x128 on 4 waves for the narrow ones (K/V projections).
#ifndef ZEST_GEMM_BIG
#define ZEST_GEMM_BIG 256, 128, 2, 4, 2, 0
#endif
#ifndef ZEST_GEMM_SMALL
#define ZEST_GEMM_SMALL 128, 128, 2, 2, 2, 0
#endif
using cfg_big = gemm_cfg<ZEST_GEMM_BIG>;
using cfg_small = gemm_cfg<ZEST_GEMM_SMALL>;

} // namespace

extern "C" int zest_gemm(const void * a, int64_t M, const void * w, int64_t N, int64_t K, float * c, int64_t ldc,
                         uint32_t * nonfinite, void * stream) {
    ZEST_REQUIRE(a && w && c, "zest_gemm: null pointer");
    ZEST_REQUIRE(M > 0 && N > 0 && K > 0 && K % 8 == 0, "zest_gemm: M=%lld N=%lld K=%lld", (long long) M,
                 (long long) N, (long long) K);
    ZEST_REQUIRE(ldc >= N, "zest_gemm: ldc %lld < N %lld", (long long) ldc, (long long) N);
    ZEST_REQUIRE(zest_bfp16_bytes(M, K) < (1ull << 31) && zest_bfp16_bytes(N, K) < (1ull << 31) &&
                     (uint64_t) zest_rows_padded(M) * (uint64_t) ldc * 4 < (1ull << 31),
                 "zest_gemm: operands and output must be under 2 GiB (M=%lld N=%lld K=%lld ldc=%lld)", (long long) M,
                 (long long) N, (long long) K, (long long) ldc);
    hipStream_t s = zest::as_stream(stream);
    // 256x256 tiles when they give the GPU enough workgroups, else 128x128
#ifndef ZEST_GEMM_BIG_MIN_TILES
#define ZEST_GEMM_BIG_MIN_TILES 160
#endif
    const int64_t big_tiles = ((M + cfg_big::BM - 1) / cfg_big::BM) * ((N + cfg_big::BN - 1) / cfg_big::BN);
    if (big_tiles >= ZEST_GEMM_BIG_MIN_TILES) return launch<cfg_big>(a, M, w, N, K, c, ldc, nonfinite, s);
    return launch<cfg_small>(a, M, w, N, K, c, ldc, nonfinite, s);
}

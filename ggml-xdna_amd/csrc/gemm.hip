// The bfp16 GEMM: C[M][N] = A[M][K] . W[N][K]^T, A the expanded activation
// operand (the bfp16 pack stored decoded as bf16, zest_layout.h) and W a
// packed bfp16 weight from the resident cache.
//
// Per workgroup a BM x BN output tile, in K-steps of 64 (one tile-layout
// column chunk), by two kinds of waves:
//   * producer waves load the W slab (bfp16 units: 16 mantissas + their 2
//     exponent bytes) two steps ahead into registers, expand the units
//     losslessly to bf16 (zest::expand16) and store them into a ring of three
//     LDS stages; LDS rows are 64 bf16 with the 16-byte chunks XOR-swizzled by
//     row so the stores and the fragment reads are free of bank conflicts;
//   * consumer waves (CWM of them, each WM rows by all BN columns) load their
//     A fragments straight from memory into registers, two steps ahead (the
//     expanded layout holds each fragment as one contiguous 1 KB), read the W
//     fragments from LDS and run v_mfma_f32_32x32x16_bf16, each lane's eight
//     K values of an operand exactly one bfp16 block, accumulating in fp32.
// One consumer and one producer wave share each SIMD, so the producer's
// expansion and the consumer's MFMAs issue side by side. While the consumers
// work on step k, the producers fill step k+2, and step k+1 is complete, so
// the consumers read its first fragments before step k ends. One barrier per
// K-step. The store is fp32 row-major, as the reference's output mode 0
// (kernels/bfp16_gemm/aie_kernels/aie2p/mm_bfp_acc.cc:106-116, 258-278).
// A launch of several rounds of whole tiles runs as persistent workgroups,
// one a CU, each walking its XCD's tiles and fetching the next tile's first
// steps while it finishes the current one (gemm_kernel_tiles; mixed launches:
// gemm_kernel_mixed_tiles).
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "zest_common.h"
#include "zest_device.h"

#ifndef ZEST_GEMM_XCD
#define ZEST_GEMM_XCD 1  // XCD-aware workgroup -> tile order
#endif
#ifndef ZEST_GEMM_GROUP_M
#define ZEST_GEMM_GROUP_M 4  // tile rows per group of the tile order
#endif

// The split-K workspace of zest_gemm_group_noalloc: one static array per GPU
// (the code object's own copy on each device, held until the process ends),
// ZEST_NOALLOC_PARTIAL_BYTES of fp32 partial sums, then
// ZEST_NOALLOC_COUNTERS counters. Host code never passes `scratch` itself to
// a kernel (on the host it names a stand-in, not device memory): it uses the
// device address that scratch_address() looks up per device.
static __device__ __align__(256) uint8_t scratch[ZEST_NOALLOC_PARTIAL_BYTES + ZEST_NOALLOC_COUNTERS * 4];

namespace {

// Epilogues other than the GLU kinds (which are >= 0)
constexpr int EPI_PLAIN = -1, EPI_RESIDUAL = -2;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// BM x BN tile; CWM x CWN consumer waves, each a WM x WN block of 32x32 MFMA
// tiles (TI x TJ of them; consumer w takes row block w % CWM, column block
// w / CWM); NP/64 producer waves (as many as the consumers' row blocks by
// default). LDS holds the expanded W ring; after the K loop each consumer
// wave uses WM x WN floats of it for its epilogue. MINB workgroups a CU at
// least (the launch bound). KG K-groups: the workgroup holds KG copies of
// these waves, each with a ring of its own, and K-group g takes the g-th of
// KG equal runs of the tile's K-steps; the groups' sums are added in LDS,
// in group order (run_tile).
template <int BM_, int BN_, int CWM_, int NP_ = 64 * CWM_, int MINB_ = 1, int CWN_ = 1, int NP1_ = 0, int KG_ = 1>
struct gemm_cfg {
    static constexpr int BM = BM_, BN = BN_, CWM = CWM_, CWN = CWN_, MINB = MINB_, KG = KG_;
    static constexpr int NC = 64 * CWM * CWN;  // consumer threads
    static constexpr int NP = NP_;             // producer threads
    static constexpr int NP1 = NP1_;           // of them, the last NP1 take one W unit each, not two
    static constexpr int NW = (NC + NP) / 64;  // waves of a K-group
    static constexpr int NT = KG * (NC + NP);
    static constexpr int WM = BM / CWM, WN = BN / CWN;
    static constexpr int TI = WM / 32, TJ = WN / 32;
    static constexpr int NP2 = NP - NP1;    // producer threads of two W units (two blocks each) a K-step
    static constexpr int ROWB = 128;        // LDS bytes per row (64 bf16)
    static constexpr int STAGE = BN * ROWB;
    static constexpr int STAGES = 3;
    static constexpr size_t RING = (size_t) STAGES * STAGE;
    // K-group g's ring at g * RING; after the K loop, the epilogue regions
    // of group 0's waves in [0, BM*BN*4) and group g's sums at g * BM*BN*4
    static constexpr size_t LDS_BYTES = KG * (RING > (size_t) BM * BN * 4 ? RING : (size_t) BM * BN * 4);
    // a persistent launch: the GLU epilogue's staging (WM rows of 16 TJ + 4
    // floats a wave) above the ring
    static constexpr size_t LDS_APART = (size_t) STAGES * STAGE + (size_t) (NC / 64) * WM * (16 * TJ + 4) * 4;
    static constexpr size_t LDS_TILES = LDS_BYTES > LDS_APART ? LDS_BYTES : LDS_APART;
    static_assert(NP2 % 64 == 0 && NP1 % 64 == 0 && NP2 / 32 + NP1 / 64 == BN / 16,
                  "32 two-unit or 64 one-unit producer threads a 16-row W tile, whole waves of each");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
};

// LDS rows are 128 bytes = 8 chunks of 16 bytes (one block as bf16 each);
// chunk c of row r is stored at position c ^ swz(r), with
// swz(r) = (r % 8) ^ ((r / 8) % 2). Any 8 consecutive rows of one chunk
// index then fall in 8 different 16-byte bank groups, and swz depends only on
// r % 16, so the +32-row offsets of the MFMA tiles stay immediates.
__device__ inline int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ inline void lds_put(uint8_t * smem, int off, uint4 v) { *reinterpret_cast<uint4 *>(smem + off) = v; }

__device__ inline bf16x8 lds_get(const uint8_t * smem, int off) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(smem + off));
}

__device__ inline uint4 load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// A producer thread's registers for one K-step's U W units.
template <class C, int U = 2>
struct stage_regs {
    uint4 wm[U];
    uint32_t we;  // the units' exponent bytes: unit 0 in bits 0-15, unit 1 in bits 16-31
};

typedef __attribute__((address_space(3))) void * lds_ptr_t;

// The producer side. W loads go through a buffer resource: the slab's byte
// offset is wave-uniform (a scalar offset), the lane's place in it a fixed
// vector offset. The hardware range check covers the vector offset only, so
// every slab offset a load is given names a K-step of the operand (callers
// clamp the steps past the end to the last one). With U = 2, thread p takes
// two adjacent units of tile p/32 of the W slab: row p%16, column quarters 2h
// and 2h+1 with h = p/16%2, i.e. 32 contiguous mantissa bytes (two 16-byte
// loads) and 4 contiguous exponent bytes (one 4-byte load). With U = 1 (the
// slab's last tiles, after the NP2/32 of the two-unit threads), thread p
// takes one unit of tile NP2/32 + p/64: row p%16, quarter q = p/16%4 (16
// mantissa bytes, 2 exponent bytes). 16 consecutive lanes are 16 consecutive
// rows, for the swizzled stores.
template <class C, int U = 2>
struct producer {
    static_assert(U == 1 || U == 2, "one or two W units a thread");
    __amdgpu_buffer_rsrc_t rw;
    int vwm, vwe;          // lane offsets: W mantissas, W exponents
    int stw[U][2];         // LDS offsets of the W units' two chunks each

    __device__ producer(const uint8_t * W, int64_t w_bytes, int p) {
        rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W), (short) 0, (int) w_bytes, 0x00020000);
        const int t = U == 2 ? p >> 5 : C::NP2 / 32 + (p >> 6), row = p & 15;
        const int q0 = U == 2 ? 2 * ((p >> 4) & 1) : (p >> 4) & 3;  // the first unit's quarter
        vwm = t * ZEST_TILE_BYTES + row * ZEST_TILE_K + q0 * 16;
        vwe = t * ZEST_TILE_BYTES + ZEST_TILE_MANT + row * 8 + q0 * 2;
        const int wrow = t * 16 + row, sw = swz(wrow);
#pragma unroll
        for (int i = 0; i < U; i++) {
            stw[i][0] = wrow * C::ROWB + ((2 * (q0 + i)) ^ sw) * 16;
            stw[i][1] = wrow * C::ROWB + ((2 * (q0 + i) + 1) ^ sw) * 16;
        }
    }

    __device__ void load_w(stage_regs<C, U> & st, int w_off) const {
        st.wm[0] = load16(rw, vwm, w_off);
        if constexpr (U == 2) {
            st.wm[1] = load16(rw, vwm + 16, w_off);
            st.we = __builtin_amdgcn_raw_buffer_load_b32(rw, vwe, w_off, 0);
        } else {
            st.we = __builtin_amdgcn_raw_buffer_load_b16(rw, vwe, w_off, 0);
        }
    }

    // W unit i of a step, by the branch-free fast expansion, stored; true if
    // the unit needs the general expansion (store_w_general) instead.
    __device__ bool store_w_unit(const stage_regs<C, U> & st, int i, uint8_t * smem, int stage) const {
        uint32_t b[8];
        const bool slow = zest::expand16_fast(st.wm[i], i ? st.we >> 16 : st.we & 0xffffu, b);
        lds_put(smem, stw[i][0] + stage, make_uint4(b[0], b[1], b[2], b[3]));
        lds_put(smem, stw[i][1] + stage, make_uint4(b[4], b[5], b[6], b[7]));
        return slow;
    }

    // Every unit of the step by the general expansion, stored.
    __device__ void store_w_general(const stage_regs<C, U> & st, uint8_t * smem, int stage) const {
#pragma unroll
        for (int i = 0; i < U; i++) {
            uint32_t b[8];
            zest::expand16(st.wm[i], i ? st.we >> 16 : st.we & 0xffffu, b);
            lds_put(smem, stw[i][0] + stage, make_uint4(b[0], b[1], b[2], b[3]));
            lds_put(smem, stw[i][1] + stage, make_uint4(b[4], b[5], b[6], b[7]));
        }
    }

    // The units take the branch-free fast expansion; a unit whose exponent
    // bytes need the general one is redone behind a single wave-uniform
    // branch, which real weights almost never take.
    __device__ void store_w(const stage_regs<C, U> & st, uint8_t * smem, int stage) const {
        bool slow = false;
#pragma unroll
        for (int i = 0; i < U; i++) slow |= store_w_unit(st, i, smem, stage);
        if (__builtin_expect(__any(slow), 0)) store_w_general(st, smem, stage);
    }
};

// The consumers' A fragments come from memory straight into registers.
// Fragment i of sub-step s is sub-tile s of the 32-row group wm*WM/32 + i of
// the tile's K-step slab: lane l takes row l%32, chunk 2s + l/32 (one block
// as bf16, the MFMA's A operand), the 16 bytes at 32(l%32) + 16(l/32), so the
// wave's load covers one contiguous 1 KB. The K-step's offset is a scalar
// offset, which the range check does not cover: callers pass only steps of
// the operand.
template <class C>
struct a_loader {
    __amdgpu_buffer_rsrc_t ra;
    int va[C::TI];

    __device__ a_loader(const uint8_t * A, int64_t a_bytes, int wm, int lane) {
        ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(A), (short) 0, (int) a_bytes, 0x00020000);
#pragma unroll
        for (int i = 0; i < C::TI; i++)
            va[i] = (wm * C::WM / 32 + i) * ZEST_XGROUP_BYTES + (lane & 31) * 32 + (lane >> 5) * 16;
    }

    __device__ bf16x8 load(int i, int s, int a_off) const {
        return __builtin_bit_cast(bf16x8,
                                  __builtin_amdgcn_raw_buffer_load_b128(ra, va[i] + s * ZEST_XSUB_BYTES, a_off, 0));
    }

    // every fragment of a K-step
    __device__ void load_step(bf16x8 (&a)[4][C::TI], int a_off) const {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < C::TI; i++) a[s][i] = load(i, s, a_off);
    }
};

// One K-step of a consumer wave: A from registers `a` (this step's,
// loaded two steps ago), W fragments from the stage at `cur`, read a
// sub-step ahead (sub-step 0 of stage `nxt` during the last). As each
// sub-step's MFMAs are issued, its A registers are reloaded with the same
// fragments of the step at a_next (LOAD), two steps ahead, so a load has two
// steps to land. The scheduling groups interleave the W reads and A loads
// with the MFMAs.
template <class C, bool LOAD>
__device__ inline void consume(f32x16 (&acc)[C::TI][C::TJ], bf16x8 (&a)[4][C::TI], bf16x8 (&bw)[2][C::TJ],
                               const uint8_t * smem, const int (&fw)[4], int cur, int nxt, const a_loader<C> & al,
                               int a_next) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int off = s < 3 ? fw[s + 1] + cur : fw[0] + nxt;
#pragma unroll
        for (int j = 0; j < C::TJ; j++) bw[(s + 1) & 1][j] = lds_get(smem, off + j * 32 * C::ROWB);
#pragma unroll
        for (int i = 0; i < C::TI; i++)
#pragma unroll
            for (int j = 0; j < C::TJ; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s][i], bw[s & 1][j], acc[i][j], 0, 0, 0);
        if (LOAD) {
#pragma unroll
            for (int i = 0; i < C::TI; i++) a[s][i] = al.load(i, s, a_next);
        }
#pragma unroll
        for (int q = 0; q < C::TI * C::TJ; q++) {
            if (q < C::TJ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a W fragment read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // an MFMA
            if (LOAD && (q + 1) % C::TJ == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // an A load
        }
    }
}

// The fp32 store. 32x32 accumulator layout: lane l, register v holds row
// (v/4)*8 + (l/32)*4 + v%4 and column l%32 of its MFMA tile. Stores go
// through a buffer resource covering rows [0, M) of C, so rows past M are
// dropped by the hardware range check on the vector offset (the whole byte
// offset is kept there); columns past N are masked per lane. Also ORs 1 into
// *nonfinite if any stored value is NaN or infinite.
// With `res` (RES), the consumer wave's WM x WN block of the residual comes
// into the wave's own LDS region first (LDS DMA, every load in flight at
// once: the ring is free after the K loop), and each output is acc + res
// (res may be Cout itself: every element is read before it is written, by
// the lane that writes it).
template <class C, bool RES = false>
__device__ inline void store_tile(const f32x16 (&acc)[C::TI][C::TJ], float * Cout, int64_t M, int64_t N, int64_t ldc,
                                  int64_t m0, int64_t n0, int wm, int wn, int lane, uint32_t * nonfinite,
                                  const float * res = nullptr, int64_t ldr = 0, uint8_t * smem = nullptr,
                                  int wave = 0) {
    const __amdgpu_buffer_rsrc_t rc =
        __builtin_amdgcn_make_buffer_rsrc(Cout, (short) 0, (int) (M * ldc * 4), 0x00020000);
    const int khalf = lane >> 5;
    const int row0 = (int) m0 + wm * C::WM;
    const float * rl = nullptr;  // the residual block in LDS: WM rows of WN floats
    if constexpr (RES) {
        // the block row-major in the region: instruction q fills bytes
        // [1024q, 1024q + 1024), lane l the 16 at 1024q + 16l, i.e. floats
        // f = 256q + 4l, row f / WN and column f % WN (a lane's 4 floats never
        // straddle rows: WN % 4 == 0); the whole byte offset is in the vector
        // offset, so the range check turns rows past M into zeros instead of
        // reads past the residual
        static_assert(C::WM * C::WN % 256 == 0 && C::WN % 4 == 0, "whole DMA instructions");
        uint8_t * region = smem + wave * (C::WM * C::WN * 4);
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(res), (short) 0, (int) (M * ldr * 4), 0x00020000);
#pragma unroll
        for (int q = 0; q < C::WM * C::WN / 256; q++) {
            const int f = 256 * q + 4 * lane, r = f / C::WN, c = f - r * C::WN;
            const int voff = (int) ((row0 + r) * ldr * 4 + (n0 + wn * C::WN + c) * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_ptr_t) (region + q * 1024), 16, voff, 0, 0, 0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        rl = reinterpret_cast<const float *>(region);
    }
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
                    float x = acc[i][j][v];
                    const int rt = i * 32 + (v >> 2) * 8 + khalf * 4 + (v & 3);  // row in the wave's block
                    if constexpr (RES) x += rl[rt * C::WN + j * 32 + (lane & 31)];
                    // only rows that are stored count
                    bad |= row0 + rt < M && !(__builtin_fabsf(x) <= 3.402823466e38f);
                    const int roff = (row0 + i * 32 + (v >> 2) * 8 + (v & 3)) * (int) ldc * 4;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rc, voff + roff, 0, 0);
                }
        }
    }
    if (nonfinite && __any(bad) && lane == 0) atomicOr(nonfinite, 1u);
}

// The fused gate/up epilogue: the weight is a gate/up pair interleaved by
// 32-row groups (zest_convert_weight_gu), so accumulator tiles 2p and 2p+1 of
// a wave hold the gate and the up values of the same 32 output columns, lane
// l%32 = column. Computes h = glu(g, u) in fp32 (the GLU kernel's arithmetic)
// and optionally stores it. For the down projection's operand the wave stages
// its WM x HW block of h in LDS (the K loop is over and every stage consumed),
// then reads it back by rows: lane l takes 16 consecutive columns of one row,
// i.e. two whole bfp16 blocks, which it encodes and stores decoded as the
// activation packer does (store_expanded16: two 16-byte stores). Each wave
// has its own LDS region, so no barrier is needed: a wave's LDS operations
// complete in order. Rows and columns past M and F come from zero padding and
// store zeros, as the packer's padding is. With APART the regions lie above
// the W ring (a persistent workgroup's producers fill the next tile's first
// stages meanwhile); else each is the wave's region of the split-K fixup.
template <class C, int KIND, bool APART = false>
__device__ inline void store_glu(const f32x16 (&acc)[C::TI][C::TJ], uint8_t * smem, uint8_t * xout, float * h,
                                 int64_t ldh, int64_t M, int64_t F, int64_t m0, int64_t n0, int wave, int wm, int wn,
                                 int lane, uint32_t * nonfinite) {
    constexpr int NPAIR = C::TJ / 2, HW = 32 * NPAIR;  // gate/up pairs; h columns of the wave
    static_assert(C::TJ % 2 == 0 && HW <= ZEST_TILE_K, "the fused GLU needs whole gate/up pairs in one K chunk");
    // staged rows of HW + 4 floats: the 16-lane groups of the row reads below
    // (rows r..r+15, one 16-byte column chunk) then hit distinct banks
    constexpr int P = HW + 4;
    static_assert(P <= C::WN && (size_t) C::BM * C::BN * 4 <= C::LDS_BYTES, "staging must fit the wave's region");
    static_assert(P == 16 * C::TJ + 4 && C::LDS_APART <= C::LDS_TILES, "staging above the ring must fit");
    float * st = reinterpret_cast<float *>(APART ? smem + C::STAGES * C::STAGE + wave * (C::WM * P * 4)
                                                 : smem + wave * (C::WM * C::WN * 4));
    const int64_t c0 = n0 / 2 + wn * HW;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < C::TI; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int rw = i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);  // row in the wave tile
            const int64_t row = m0 + wm * C::WM + rw;
#pragma unroll
            for (int q = 0; q < NPAIR; q++) {
                const float g = acc[i][2 * q][v], u = acc[i][2 * q + 1][v];
                const float hv = zest::glu(KIND, g, u);
                const int64_t col = c0 + q * 32 + (lane & 31);
                bad |= !(__builtin_fabsf(g) <= 3.402823466e38f) || !(__builtin_fabsf(u) <= 3.402823466e38f) ||
                       !(__builtin_fabsf(hv) <= 3.402823466e38f);
                if (h && row < M && col < F) h[row * ldh + col] = hv;
                if (xout) st[rw * P + q * 32 + (lane & 31)] = hv;
            }
        }
    if (xout) {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const int64_t M_pad = zest_rows_padded(M);
        // a pass reads RPP rows, lane l taking row l%RPP and 16-column chunk l/RPP
        constexpr int QPR = HW / 16, RPP = 64 / QPR;
        const int q = lane / RPP;
#pragma unroll
        for (int j = 0; j < C::WM / RPP; j++) {
            const int rw = j * RPP + lane % RPP;
            const float4 * p = reinterpret_cast<const float4 *>(st + rw * P + q * 16);
            float v[16];
#pragma unroll
            for (int x = 0; x < 4; x++) {
                const float4 f = p[x];
                v[4 * x] = f.x;
                v[4 * x + 1] = f.y;
                v[4 * x + 2] = f.z;
                v[4 * x + 3] = f.w;
            }
            zest::store_expanded16(xout, M_pad, m0 + wm * C::WM + rw, c0 + q * 16, v);
        }
        // The last tile row also zeroes the operand's rows that no tile
        // reaches, [m0 + BM, M_pad): a row's HW columns are Z lanes of 16
        // bytes, so a wave covers 64/Z rows at a time.
        constexpr int Z = HW / 8, RZ = 64 / Z;
        if (m0 + C::BM >= M)
            for (int64_t row = m0 + C::BM + wm * RZ + lane / Z; row < M_pad; row += RZ * C::CWM)
                *reinterpret_cast<uint4 *>(xout + zest_xoffset(row, c0 + (lane % Z) * 8, M_pad)) = make_uint4(0, 0, 0, 0);
    }
    if (nonfinite && __any(bad) && lane == 0) atomicOr(nonfinite, 1u);
}

// One weight of a launch. Weights that share the activation operand (a
// group: q, k and v) run as one launch; their column tiles follow each other.
struct gemm_weight {
    const uint8_t * w;  // packed bfp16
    float * c;          // fp32 output (plain epilogue)
    int64_t n, ldc;
    int w_kstride;      // bytes between K-steps of the packed weight
    int tile0;          // its first column tile in the launch
};

struct gemm_params {
    const uint8_t * a;  // expanded activations
    int64_t M;
    int a_kstride;      // bytes between K-steps of the activation operand
    int nk;             // K-steps
    int mt, nt;         // tile rows; column tiles of all weights
    int nw;             // weights
    gemm_weight wt[ZEST_GEMM_MAX_GROUP];
    uint8_t * xout;     // fused GLU outputs (one weight)
    float * h;
    int64_t ldh;
    const float * res;  // residual added by the EPI_RESIDUAL epilogue (one weight)
    int64_t ldr;
    uint32_t * nonfinite;
    // Split-K: with splits S > 1, workgroup v takes unit v of the sequence
    // (split 0 of every tile, split 1 of every tile, ...): split s of a tile is
    // its K-steps [s*nk/S, (s+1)*nk/S). The workgroups running one split walk
    // K side by side, as whole tiles do, so they keep sharing A and W slabs in
    // L2. The splits of a tile are summed through `partial` (BM*BN floats per
    // unit) and `counters` (one per tile and consumer wave, zero between
    // launches).
    int splits;
    float * partial;
    uint32_t * counters;
    // Mixed launches (gemm_kernel_mixed): the first nbig tiles (mt x nt
    // tiles of the big shape) run whole, each of the others as two tiles of
    // half its rows (the small shape).
    int nbig;
};

// Byte offset of a consumer wave's float4 (i, j, quad q) in a unit's partial
// sums: [unit][wave][i][j][quad][lane], so each store and load instruction
// covers 1 KB contiguous.
template <class C>
__device__ inline int partial_off(int unit, int wave, int i, int j, int q, int lane) {
    return (((((unit * (C::NC / 64) + wave) * (C::TI * C::TJ) + i * C::TJ + j) * 4 + q) * 64) + lane) * 16;
}

// Cache policy of the partial sums' loads and stores: sc1, coherent at device
// scope (the writer and the reader may sit on different XCDs, whose L2s are
// not coherent with each other). No fence is used: a device-scope fence
// writes back and invalidates the XCD's whole L2, which would take the A and
// W slabs the other workgroups there are sharing.
#define ZEST_SC1 16

// Split-K fixup of one consumer wave's block of tile t, split `split` of
// p.splits. Writes this wave's sums to its unit's partial (sc1 stores), waits
// for them to be acknowledged, and counts itself in. The wave that arrives
// last forms ((p[S-1] + p[S-2]) + p[S-3]) + ... + p[0] and resets the
// counter. The order is fixed, so the result does not depend on arrival
// order; since a + b == b + a exactly, a last wave of split S-1 or S-2 (the
// usual case: splits run in that order) starts from its own sums in acc and
// reads one partial fewer, others read their own back like the rest. Each
// partial comes into the wave's own LDS region by LDS DMA (all of its loads
// in flight at once, no registers held), then is added from there. LDS is
// free: the K loop is over, and this workgroup has no other tile. Returns
// true for the last wave, whose acc then holds the tile's sums. No wave
// waits for another.
template <class C>
__device__ inline bool fixup(f32x16 (&acc)[C::TI][C::TJ], const gemm_params & p, uint8_t * smem, int t, int split,
                             int wave, int lane) {
    constexpr int PARTS = C::TI * C::TJ * 4;  // 1 KB pieces of a wave's share
    const int T = p.mt * p.nt, S = p.splits;
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        p.partial, (short) 0, (int) ((int64_t) T * S * C::BM * C::BN * 4), 0x00020000);
    const int me = split * T + t;
#pragma unroll
    for (int i = 0; i < C::TI; i++)
#pragma unroll
        for (int j = 0; j < C::TJ; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 x = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                             acc[i][j][4 * q + 3]);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rp,
                                                       partial_off<C>(me, wave, i, j, q, lane), 0, ZEST_SC1);
            }
    // the stores have reached the coherent level before the count goes up
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint32_t * counter = p.counters + (int64_t) t * (C::NC / 64) + wave;
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    asm volatile("" ::: "memory");
    if (old != (uint32_t) (S - 1)) return false;
    uint8_t * region = smem + wave * (C::WM * C::WN * 4);
    // acc already holds p[S-1] (split S-1) or its commuted first sum's other
    // operand (split S-2)
    const bool own = split >= S - 2;
    for (int v = own ? 1 : 0; v < S; v++) {
        // operand v of the sum is p[S-1-v], except that a split-S-2 wave's
        // second operand is p[S-1] (its own sums stand in for p[S-2]). u is
        // uniform but derived from the split, which the tile arithmetic can
        // leave in a vector register, and a DMA's scalar offset taken from
        // one costs a loop per load
        const int u = __builtin_amdgcn_readfirstlane(own && v == 1 ? (split == S - 1 ? S - 2 : S - 1) : S - 1 - v);
        const int base = partial_off<C>(u * T + t, wave, 0, 0, 0, 0);
#pragma unroll
        for (int x = 0; x < PARTS; x++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_ptr_t) (region + x * 1024), 16, lane * 16,
                                                     base + x * 1024, 0, ZEST_SC1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < C::TI; i++)
#pragma unroll
            for (int j = 0; j < C::TJ; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 x =
                        *reinterpret_cast<const float4 *>(region + ((i * C::TJ + j) * 4 + q) * 1024 + lane * 16);
                    if (v == 0) {
                        acc[i][j][4 * q] = x.x;
                        acc[i][j][4 * q + 1] = x.y;
                        acc[i][j][4 * q + 2] = x.z;
                        acc[i][j][4 * q + 3] = x.w;
                    } else {
                        acc[i][j][4 * q] += x.x;
                        acc[i][j][4 * q + 1] += x.y;
                        acc[i][j][4 * q + 2] += x.z;
                        acc[i][j][4 * q + 3] += x.w;
                    }
                }
        // the reads are done before the next partial's DMA overwrites them
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// The workgroup barrier without a fence: no wave writes global memory in the
// K loop, and a fence would make the compiler wait for every load in flight;
// the LDS waits a barrier needs are explicit before it.
__device__ inline void bare_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt lgkmcnt(0) alone: this wave's LDS stores done, loads left in flight
// (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// One steady-state producer step: step j's W units (loaded two steps ago)
// expanded and stored into `stage`, step j+2's requested into the same
// registers. A unit whose exponent bytes need the general expansion is
// redone behind one wave-uniform branch, which real weights almost never take.
template <class C, int U>
__device__ inline void produce_step(const producer<C, U> & pr, uint8_t * smem, int stage, stage_regs<C, U> & r,
                                   int w_off_next) {
    bool slow = false;
#pragma unroll
    for (int u = 0; u < U; u++) {
        slow |= pr.store_w_unit(r, u, smem, stage);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (__builtin_expect(__any(slow), 0)) pr.store_w_general(r, smem, stage);
    pr.load_w(r, w_off_next);
}

// The producer's part of one tile over K-steps [k0, k0 + ns), with steps 0
// and 1 already requested into r0 and r1: step j's W units are loaded during
// step j-4 and stored into stage j%3 during step j-2 (the consumers read step
// j+1's first fragments before the barrier that ends step j, so a stage must
// be complete a step before it is consumed, and it is free only after the
// step that last read it). Every load goes into registers and every LDS store
// is the compiler's own, so the compiler counts the loads in flight and waits
// for exactly those whose registers a store reads; before a barrier only the
// LDS stores are waited for. Steps 2-3 are requested whether or not this tile
// has them (a step past this split's steps reads the next split's slab; one
// past the operand's last step, `last` steps after w0, reads that last step
// again; neither is stored), so the steady state starts with an exact count;
// it runs without conditions, and the last steps do their remaining stores
// one by one. With `next` (ns even), the two requests that follow the tile's
// last step fetch steps 0 and 1 of the workgroup's next tile (producer pn, at
// wn0) into r0 and r1 instead. The barriers match the consumers', step for
// step.
template <class C, int U = 2>
__device__ inline void produce_tile(const producer<C, U> & pr, uint8_t * smem, int w0, int w_kstride, int ns,
                                    int last, stage_regs<C, U> & r0, stage_regs<C, U> & r1, const producer<C, U> & pn,
                                    int wn0, int wn_kstride, bool next) {
    pr.store_w(r0, smem, 0);
    pr.load_w(r0, w0 + min(2, last) * w_kstride);
    if (ns > 1) pr.store_w(r1, smem, C::STAGE);
    pr.load_w(r1, w0 + min(3, last) * w_kstride);
    wait_lgkm0();
    bare_barrier();
    // during step k: step k+2 stored into stage (k+2)%3, step k+4 requested
    int stage = 2 * C::STAGE, k = 0;
    for (; k + 5 < ns; k += 2) {
        produce_step<C, U>(pr, smem, stage, r0, w0 + (k + 4) * w_kstride);
        stage = stage == 2 * C::STAGE ? 0 : stage + C::STAGE;
        wait_lgkm0();
        bare_barrier();
        produce_step<C, U>(pr, smem, stage, r1, w0 + (k + 5) * w_kstride);
        stage = stage == 2 * C::STAGE ? 0 : stage + C::STAGE;
        wait_lgkm0();
        bare_barrier();
    }
    for (; k < ns; k += 2) {
        if (k + 2 < ns) {
            pr.store_w(r0, smem, stage);
            if (k + 4 < ns)
                pr.load_w(r0, w0 + (k + 4) * w_kstride);
            else if (next && k + 4 == ns)
                pn.load_w(r0, wn0);
        }
        stage = stage == 2 * C::STAGE ? 0 : stage + C::STAGE;
        wait_lgkm0();
        bare_barrier();
        if (k + 1 < ns) {
            if (k + 3 < ns) {
                pr.store_w(r1, smem, stage);
                if (k + 5 < ns)
                    pr.load_w(r1, w0 + (k + 5) * w_kstride);
                else if (next && k + 5 == ns + 1)
                    pn.load_w(r1, wn0 + wn_kstride);
            }
            stage = stage == 2 * C::STAGE ? 0 : stage + C::STAGE;
            wait_lgkm0();
            bare_barrier();
        }
    }
}

// The producer's part of a workgroup's only tile.
template <class C, int U>
__device__ inline void produce(const producer<C, U> & pr, uint8_t * smem, int w0, int w_kstride, int ns, int last) {
    stage_regs<C, U> r0, r1;
    pr.load_w(r0, w0);
    pr.load_w(r1, w0 + min(1, last) * w_kstride);
    produce_tile<C, U>(pr, smem, w0, w_kstride, ns, last, r0, r1, pr, 0, 0, false);
}

// The consumer's K loop over a tile's steps [0, ns), its A fragments of
// steps 0 and 1 requested into a0s and a1s: starts with the barrier that
// completes the first two W stages. Past the tile's last step, a load of
// step j reads step min(j, last) (the next split's slab or the operand's
// last step again, never used). Pairs of steps run without conditions.
template <class C>
__device__ inline void consume_tile(f32x16 (&acc)[C::TI][C::TJ], bf16x8 (&a0s)[4][C::TI], bf16x8 (&a1s)[4][C::TI],
                                    const uint8_t * smem, const int (&fw)[4], const a_loader<C> & al, int a0, int ks,
                                    int ns, int last) {
    bf16x8 bw[2][C::TJ];
    bare_barrier();
#pragma unroll
    for (int j = 0; j < C::TJ; j++) bw[0][j] = lds_get(smem, fw[0] + j * 32 * C::ROWB);
    int cur = 0, k = 0;
    for (; k + 1 < ns; k += 2) {
        int nxt = cur == 2 * C::STAGE ? 0 : cur + C::STAGE;
        consume<C, true>(acc, a0s, bw, smem, fw, cur, nxt, al, a0 + min(k + 2, last) * ks);
        cur = nxt;
        bare_barrier();
        nxt = cur == 2 * C::STAGE ? 0 : cur + C::STAGE;
        consume<C, true>(acc, a1s, bw, smem, fw, cur, nxt, al, a0 + min(k + 3, last) * ks);
        cur = nxt;
        bare_barrier();
    }
    if (k < ns) {
        const int nxt = cur == 2 * C::STAGE ? 0 : cur + C::STAGE;
        consume<C, false>(acc, a0s, bw, smem, fw, cur, nxt, al, 0);
        bare_barrier();
    }
}

// The consumer's epilogue of one tile; APART as for store_glu (the plain
// store uses no LDS).
template <class C, int EPI, bool APART = false>
__device__ inline void epilogue(const f32x16 (&acc)[C::TI][C::TJ], const gemm_params & p, uint8_t * smem,
                                const gemm_weight & W, int64_t m0, int64_t n0, int wave, int wm, int wn, int lane) {
    if constexpr (EPI == EPI_RESIDUAL)
        store_tile<C, true>(acc, W.c, p.M, W.n, W.ldc, m0, n0, wm, wn, lane, p.nonfinite, p.res, p.ldr, smem, wave);
    else if constexpr (EPI < 0)
        store_tile<C>(acc, W.c, p.M, W.n, W.ldc, m0, n0, wm, wn, lane, p.nonfinite);
    else
        store_glu<C, EPI, APART>(acc, smem, p.xout, p.h, p.ldh, p.M, W.n / 2, m0, n0, wave, wm, wn, lane,
                                 p.nonfinite);
}

// Tile t of a launch in the tile order: tiles go in groups of GROUP_M tile
// rows, M-fastest inside a group, so the ~32 workgroups resident on one XCD
// cover a compact block of about 4 x 8 tiles and share their A and W slabs in
// its L2. Returns the tile's weight (of a group launch) and its first row and
// column.
template <class C>
__device__ inline gemm_weight tile_of(const gemm_params & p, int t, int64_t & m0, int64_t & n0) {
    const int per_group = ZEST_GEMM_GROUP_M * p.nt, first_m = t / per_group * ZEST_GEMM_GROUP_M;
    const int gm = min(p.mt - first_m, ZEST_GEMM_GROUP_M), in = t % per_group;
    const int tm = first_m + in % gm, tn = in / gm;
    int g = 0;
#pragma unroll
    for (int i = 1; i < ZEST_GEMM_MAX_GROUP; i++)
        if (i < p.nw && tn >= p.wt[i].tile0) g = i;
    g = __builtin_amdgcn_readfirstlane(g);
    m0 = (int64_t) tm * C::BM;
    n0 = (int64_t) (tn - p.wt[g].tile0) * C::BN;
    return p.wt[g];
}

// Workgroups go to the 8 XCDs round-robin by linear id b; the n workgroups
// numbered by this map hold a contiguous run of it on each XCD.
__device__ inline int xcd_order(int b, int n) {
#if ZEST_GEMM_XCD
    return (b % 8) * (n / 8) + min(b % 8, n % 8) + b / 8;
#else
    return b;
#endif
}

// One output tile (rows m0.., columns n0.. of weight W), over K-steps
// [k0, k0 + ns); with SPLIT, unit `split` of tile t. With K-groups (C::KG >
// 1; ns a multiple of KG), group g runs steps [k0 + g*ns/KG, k0 +
// (g+1)*ns/KG) on its own ring, the groups meet the same barriers step for
// step, and after the K loop every wave meets one more: groups 1.. have left
// their sums in LDS, and group 0 adds them in group order (((s0 + s1) + s2)
// + ...) before the split-K fixup and the epilogue. A group's waves take
// their roles rotated by g * NC/64, so that with waves placed on SIMDs in
// turn each SIMD holds consumers and producers alike.
template <class C, int EPI, bool SPLIT>
__device__ inline void run_tile(const gemm_params & p, uint8_t * smem, const gemm_weight & W, int64_t m0, int64_t n0,
                                int k0, int ns, int t, int split) {
    int grp = 0, wave, tid;
    if constexpr (C::KG > 1) {
        grp = __builtin_amdgcn_readfirstlane((int) threadIdx.x / (C::NC + C::NP));
        const int wig = __builtin_amdgcn_readfirstlane(((int) threadIdx.x % (C::NC + C::NP)) >> 6);
        wave = (wig + grp * (C::NC / 64)) % C::NW;
        tid = wave * 64 + ((int) threadIdx.x & 63);
    } else {
        tid = threadIdx.x;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    }
    const int lane = tid & 63;
    const int nk = p.nk;
    uint8_t * const base = smem;
    if constexpr (C::KG > 1) {
        smem += grp * C::RING;
        ns /= C::KG;
        k0 += grp * ns;
    }
    if (wave >= C::NC / 64) {
        const int job = tid - C::NC;
        // uniform, but the tile arithmetic can leave it in a vector register,
        // and a load's scalar offset taken from one costs a loop per load
        const int w0 =
            __builtin_amdgcn_readfirstlane((int) ((n0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES) + k0 * W.w_kstride);
        if constexpr (C::NP1 > 0)
            if (job >= C::NP2) {  // whole waves: NP2 % 64 == 0
                const producer<C, 1> pr(W.w, (int64_t) W.w_kstride * nk, job - C::NP2);
                produce<C, 1>(pr, smem, w0, W.w_kstride, ns, nk - 1 - k0);
                if constexpr (C::KG > 1) bare_barrier();  // the K-groups' sums
                return;
            }
        const producer<C, 2> pr(W.w, (int64_t) W.w_kstride * nk, job);
        produce<C, 2>(pr, smem, w0, W.w_kstride, ns, nk - 1 - k0);
        if constexpr (C::KG > 1) bare_barrier();  // the K-groups' sums
        return;
    }

    // Consumer: rows wm*WM.. and columns wn*WN.. of the tile. swz depends
    // only on the row mod 16, so a column block's W rows keep rows wr's.
    const int wm = wave % C::CWM, wn = wave / C::CWM, khalf = lane >> 5, wr = lane & 31;
    int fw[4];
#pragma unroll
    for (int s = 0; s < 4; s++) fw[s] = (wn * C::WN + wr) * C::ROWB + ((2 * s + khalf) ^ swz(wr)) * 16;
    f32x16 acc[C::TI][C::TJ];
#pragma unroll
    for (int i = 0; i < C::TI; i++)
#pragma unroll
        for (int j = 0; j < C::TJ; j++) acc[i][j] = f32x16{};
    {
        // A two steps ahead in registers; no fence at the barriers, so the
        // loads stay in flight across them (consumers write no memory here)
        const a_loader<C> al(p.a, (int64_t) p.a_kstride * nk, wm, lane);
        const int ks = p.a_kstride;
        const int a0 =
            __builtin_amdgcn_readfirstlane((int) ((m0 / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES) + k0 * p.a_kstride);
        // the operand's last K-step, counted from a0: the steps loaded past
        // it load it again (the scalar offset is not range-checked)
        const int last = nk - 1 - k0;
        bf16x8 a0s[4][C::TI], a1s[4][C::TI];
        al.load_step(a0s, a0);
        al.load_step(a1s, a0 + min(1, last) * ks);
        consume_tile<C>(acc, a0s, a1s, smem, fw, al, a0, ks, ns, last);
        // the loads of steps past the end are still in flight
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    }
    smem = base;
    if constexpr (C::KG > 1) {
        // every group is past its K loop's last barrier, so no ring is read
        // or written any more except by a consumer's unused read ahead
        if (grp > 0) {
            uint8_t * sums = smem + (size_t) grp * C::BM * C::BN * 4 + wave * (C::WM * C::WN * 4);
#pragma unroll
            for (int i = 0; i < C::TI; i++)
#pragma unroll
                for (int j = 0; j < C::TJ; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        *reinterpret_cast<float4 *>(sums + ((i * C::TJ + j) * 4 + q) * 1024 + lane * 16) =
                            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                        acc[i][j][4 * q + 3]);
            wait_lgkm0();
            bare_barrier();
            return;
        }
        bare_barrier();
#pragma unroll
        for (int g = 1; g < C::KG; g++) {
            const uint8_t * sums = smem + (size_t) g * C::BM * C::BN * 4 + wave * (C::WM * C::WN * 4);
#pragma unroll
            for (int i = 0; i < C::TI; i++)
#pragma unroll
                for (int j = 0; j < C::TJ; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 x =
                            *reinterpret_cast<const float4 *>(sums + ((i * C::TJ + j) * 4 + q) * 1024 + lane * 16);
                        acc[i][j][4 * q] += x.x;
                        acc[i][j][4 * q + 1] += x.y;
                        acc[i][j][4 * q + 2] += x.z;
                        acc[i][j][4 * q + 3] += x.w;
                    }
        }
    }
    if (SPLIT && !fixup<C>(acc, p, smem, t, split, wave, lane)) return;
    epilogue<C, EPI>(acc, p, smem, W, m0, n0, wave, wm, wn, lane);
}

// EPI: EPI_PLAIN the fp32 store, EPI_RESIDUAL the fp32 store of acc + res,
// >= 0 the fused GLU of that kind.
// SPLIT: split-K (p.splits > 1), else one whole tile per workgroup.
template <class C, int EPI, bool SPLIT>
__global__ __launch_bounds__(C::NT, C::MINB) void gemm_kernel(const gemm_params p) {
    extern __shared__ uint4 smem_u4[];
    uint8_t * smem = reinterpret_cast<uint8_t *>(smem_u4);
    const int v = xcd_order((int) blockIdx.x, (int) gridDim.x), nk = p.nk;
    const int T = p.mt * p.nt;
    const int split = SPLIT ? v / T : 0, t = SPLIT ? v - split * T : v;
    const int k0 = SPLIT ? split * nk / p.splits : 0, ns = SPLIT ? (split + 1) * nk / p.splits - k0 : nk;
    int64_t m0, n0;
    const gemm_weight W = tile_of<C>(p, t, m0, n0);
    run_tile<C, EPI, SPLIT>(p, smem, W, m0, n0, k0, ns, t, split);
}

// The mixed launch: CB tiles (p.mt x p.nt of them) whose count is a whole
// number of rounds of the GPU plus a part of one; that part runs as tiles of
// half the rows (CS), twice as many workgroups of about half the time, so the
// last round ends sooner. On each XCD the whole tiles come first (the first
// workgroups it is given), then the halves.
template <class CB, class CS, int EPI>
__global__ __launch_bounds__(CB::NT, 1) void gemm_kernel_mixed(const gemm_params p) {
    static_assert(CB::NT == CS::NT && CS::BM * 2 == CB::BM && CS::BN == CB::BN && CB::KG == 1 && CS::KG == 1,
                  "halves of the big tiles");
    extern __shared__ uint4 smem_u4[];
    uint8_t * smem = reinterpret_cast<uint8_t *>(smem_u4);
    const int b = (int) blockIdx.x, per_xcd = p.nbig / 8, i = b / 8;
    int64_t m0, n0;
    if (i < per_xcd) {
        const int t = (b % 8) * per_xcd + i;
        const gemm_weight W = tile_of<CB>(p, t, m0, n0);
        run_tile<CB, EPI, false>(p, smem, W, m0, n0, 0, p.nk, t, 0);
    } else {
        const int nhalf = (int) gridDim.x - p.nbig;
        const int u = xcd_order(b - p.nbig, nhalf);  // b - nbig keeps b's XCD: nbig % 8 == 0
        const int t = p.nbig + u / 2;
        const gemm_weight W = tile_of<CB>(p, t, m0, n0);
        run_tile<CS, EPI, false>(p, smem, W, m0 + (u % 2) * CS::BM, n0, 0, p.nk, t, 0);
    }
}

// Persistent workgroups for a launch of more than one round of whole tiles
// (ns = nk, even, at least 4; not the residual epilogue). Workgroup b works on
// XCD b % 8 and takes the tiles of that XCD's run (the contiguous run
// xcd_order gives it) in turn: start + b/8, start + b/8 + G/8, ... for G
// workgroups, a multiple of 8. The producers' last two requests of a tile
// fetch the next tile's first two W steps, and once past the tile's last
// barrier they expand and store them into the first two stages while the
// consumers run the epilogue (which uses no LDS, or the GLU's staging above
// the ring; the only LDS read a consumer still has in flight there is its
// unused read ahead of a next stage). The consumers request the next tile's
// first two A steps after the epilogue (held through it they would not fit
// the registers).
template <class C, int EPI>
__global__ __launch_bounds__(C::NT, 1) void gemm_kernel_tiles(const gemm_params p) {
    static_assert(C::KG == 1, "one K-group");
    extern __shared__ uint4 smem_u4[];
    uint8_t * smem = reinterpret_cast<uint8_t *>(smem_u4);
    const int b = (int) blockIdx.x, g = (int) gridDim.x / 8, T = p.mt * p.nt, nk = p.nk;
    const int x = b % 8, end = (x + 1) * (T / 8) + min(x + 1, T % 8);
    int t = x * (T / 8) + min(x, T % 8) + b / 8;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t m0, n0;
    gemm_weight W = tile_of<C>(p, t, m0, n0);
    if (wave >= C::NC / 64) {
        const int job = tid - C::NC;
        producer<C> pr(W.w, (int64_t) W.w_kstride * nk, job);
        int w0 = __builtin_amdgcn_readfirstlane((int) ((n0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES));
        stage_regs<C> r0, r1;
        pr.load_w(r0, w0);
        pr.load_w(r1, w0 + W.w_kstride);
        for (;;) {
            const int tn = t + g;
            const bool next = tn < end;
            int64_t mn = m0, nn = n0;
            const gemm_weight Wn = next ? tile_of<C>(p, tn, mn, nn) : W;
            const producer<C> pn(Wn.w, (int64_t) Wn.w_kstride * nk, job);
            const int wn0 = __builtin_amdgcn_readfirstlane((int) ((nn / ZEST_TILE_ROWS) * ZEST_TILE_BYTES));
            produce_tile<C>(pr, smem, w0, W.w_kstride, nk, nk - 1, r0, r1, pn, wn0, Wn.w_kstride, next);
            if (!next) return;
            t = tn;
            W = Wn;
            pr = pn;
            w0 = wn0;
        }
    }
    const int wm = wave % C::CWM, wn = wave / C::CWM, khalf = lane >> 5, wr = lane & 31;
    int fw[4];
#pragma unroll
    for (int s = 0; s < 4; s++) fw[s] = (wn * C::WN + wr) * C::ROWB + ((2 * s + khalf) ^ swz(wr)) * 16;
    const a_loader<C> al(p.a, (int64_t) p.a_kstride * nk, wm, lane);
    const int ks = p.a_kstride;
    int a0 = __builtin_amdgcn_readfirstlane((int) ((m0 / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES));
    bf16x8 a0s[4][C::TI], a1s[4][C::TI];
    al.load_step(a0s, a0);
    al.load_step(a1s, a0 + ks);
    for (;;) {
        f32x16 acc[C::TI][C::TJ];
#pragma unroll
        for (int i = 0; i < C::TI; i++)
#pragma unroll
            for (int j = 0; j < C::TJ; j++) acc[i][j] = f32x16{};
        consume_tile<C>(acc, a0s, a1s, smem, fw, al, a0, ks, nk, nk - 1);
        // the loads of steps past the end are still in flight
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        epilogue<C, EPI, true>(acc, p, smem, W, m0, n0, wave, wm, wn, lane);
        t += g;
        if (t >= end) return;
        W = tile_of<C>(p, t, m0, n0);
        a0 = __builtin_amdgcn_readfirstlane((int) ((m0 / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES));
        al.load_step(a0s, a0);
        al.load_step(a1s, a0 + ks);
    }
}

// One item of a persistent mixed launch, a consumer wave's part: the K loop
// of a tile (its A fragments of steps 0 and 1 requested into a0s and a1s),
// then its epilogue (with no LDS of its own).
template <class C, int EPI>
__device__ inline void consume_item(const gemm_params & p, uint8_t * smem, const gemm_weight & W, int64_t m0,
                                    int64_t n0, int wave, int lane, bf16x8 (&a0s)[4][C::TI],
                                    bf16x8 (&a1s)[4][C::TI]) {
    const int wm = wave % C::CWM, wn = wave / C::CWM, khalf = lane >> 5, wr = lane & 31;
    int fw[4];
#pragma unroll
    for (int s = 0; s < 4; s++) fw[s] = (wn * C::WN + wr) * C::ROWB + ((2 * s + khalf) ^ swz(wr)) * 16;
    const a_loader<C> al(p.a, (int64_t) p.a_kstride * p.nk, wm, lane);
    const int a0 = __builtin_amdgcn_readfirstlane((int) ((m0 / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES));
    f32x16 acc[C::TI][C::TJ];
#pragma unroll
    for (int i = 0; i < C::TI; i++)
#pragma unroll
        for (int j = 0; j < C::TJ; j++) acc[i][j] = f32x16{};
    consume_tile<C>(acc, a0s, a1s, smem, fw, al, a0, p.a_kstride, p.nk, p.nk - 1);
    // the loads of steps past the end are still in flight
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    static_assert(EPI < 0 && EPI != EPI_RESIDUAL, "the plain store");
    epilogue<C, EPI>(acc, p, smem, W, m0, n0, wave, wm, wn, lane);
}

// A consumer wave's requests of a tile's first two A steps.
template <class C>
__device__ inline void load_item_a(const gemm_params & p, int64_t m0, int wave, int lane, bf16x8 (&a0s)[4][C::TI],
                                   bf16x8 (&a1s)[4][C::TI]) {
    const a_loader<C> al(p.a, (int64_t) p.a_kstride * p.nk, wave % C::CWM, lane);
    const int a0 = __builtin_amdgcn_readfirstlane((int) ((m0 / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES));
    al.load_step(a0s, a0);
    al.load_step(a1s, a0 + p.a_kstride);
}

// The mixed launch as persistent workgroups (nk even, at least 4), one a CU:
// workgroup b takes the whole tiles of XCD b % 8's run (the first nbig/8 of
// its tiles, as gemm_kernel_mixed's first nbig workgroups have them), then
// the half tiles of that XCD's run of halves, from b/8 in steps of G/8 (G
// workgroups, a multiple of 8, at most nbig). The producers request the next
// item's first two W steps during the current item's last ones (a half tile
// has its whole tile's W rows and the same producer layout) and store them
// into the first two stages while the consumers run the epilogue (the plain
// store, no LDS); the consumers request its first two A steps after it.
template <class CB, class CS, int EPI>
__global__ __launch_bounds__(CB::NT, 1) void gemm_kernel_mixed_tiles(const gemm_params p) {
    static_assert(CB::NT == CS::NT && CS::BM * 2 == CB::BM && CS::BN == CB::BN && CS::NP == CB::NP &&
                      CS::TI == CB::TI && CB::NP1 == 0 && CS::NP1 == 0 && CB::KG == 1 && CS::KG == 1,
                  "halves of the big tiles, with the same producers");
    extern __shared__ uint4 smem_u4[];
    uint8_t * smem = reinterpret_cast<uint8_t *>(smem_u4);
    const int b = (int) blockIdx.x, g = (int) gridDim.x / 8, x = b % 8, j = b / 8, nk = p.nk;
    const int T = p.mt * p.nt, per_xcd = p.nbig / 8, nhalf = 2 * (T - p.nbig);
    const int hs = x * (nhalf / 8) + min(x, nhalf % 8), he = (x + 1) * (nhalf / 8) + min(x + 1, nhalf % 8);
    const int n_whole = (per_xcd - j + g - 1) / g;
    const int n_items = n_whole + (hs + j < he ? (he - hs - j + g - 1) / g : 0);
    // item i: its tile, and the first row of its rows (a half's)
    auto item = [&](int i, int64_t & m0, int64_t & n0) {
        if (i < n_whole) return tile_of<CB>(p, x * per_xcd + j + i * g, m0, n0);
        const int u = hs + j + (i - n_whole) * g;
        const gemm_weight w = tile_of<CB>(p, p.nbig + u / 2, m0, n0);
        m0 += (u % 2) * CS::BM;
        return w;
    };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t m0, n0;
    gemm_weight W = item(0, m0, n0);
    if (wave >= CB::NC / 64) {
        const int job = tid - CB::NC;
        producer<CB> pr(W.w, (int64_t) W.w_kstride * nk, job);
        int w0 = __builtin_amdgcn_readfirstlane((int) ((n0 / ZEST_TILE_ROWS) * ZEST_TILE_BYTES));
        stage_regs<CB> r0, r1;
        pr.load_w(r0, w0);
        pr.load_w(r1, w0 + W.w_kstride);
        for (int i = 0;; i++) {
            const bool next = i + 1 < n_items;
            int64_t mn = m0, nn = n0;
            const gemm_weight Wn = next ? item(i + 1, mn, nn) : W;
            const producer<CB> pn(Wn.w, (int64_t) Wn.w_kstride * nk, job);
            const int wn0 = __builtin_amdgcn_readfirstlane((int) ((nn / ZEST_TILE_ROWS) * ZEST_TILE_BYTES));
            produce_tile<CB>(pr, smem, w0, W.w_kstride, nk, nk - 1, r0, r1, pn, wn0, Wn.w_kstride, next);
            if (!next) return;
            W = Wn;
            pr = pn;
            w0 = wn0;
        }
    }
    bf16x8 a0s[4][CB::TI], a1s[4][CB::TI];
    load_item_a<CB>(p, m0, wave, lane, a0s, a1s);
    for (int i = 0;; i++) {
        if (i < n_whole)
            consume_item<CB, EPI>(p, smem, W, m0, n0, wave, lane, a0s, a1s);
        else
            consume_item<CS, EPI>(p, smem, W, m0, n0, wave, lane, a0s, a1s);
        if (i + 1 >= n_items) return;
        W = item(i + 1, m0, n0);
        if (i + 1 < n_whole)
            load_item_a<CB>(p, m0, wave, lane, a0s, a1s);
        else
            load_item_a<CS>(p, m0, wave, lane, a0s, a1s);
    }
}

// 256x128 tiles (4 consumer waves of 64x128); 128x128 (4 of 32x128) where
// the cost model prefers them (few rows, or too few big tiles).
#ifndef ZEST_GEMM_BIG
#define ZEST_GEMM_BIG 256, 128, 4
#endif
#ifndef ZEST_GEMM_SMALL
#define ZEST_GEMM_SMALL 128, 128, 4
#endif
// Launch cost model, in K-steps of a 256x128 tile at full occupancy (about
// 0.85 us): T tiles on P CUs take ceil(T/P) rounds of nk steps, plus PROLOGUE
// steps per round to fill the pipeline. S K-splits take ceil(T*S/P) rounds of
// nk/S steps, plus the fixup: every split writes its fp32 tile and the last
// reads all S back through HBM, 2*T*S*BM*BN*4 bytes at about FIX_BW bytes
// per step, and FIX_LAT steps more: the fixup's round trips (store and
// acknowledge, count in, read back) that follow the K loop of every split
// launch, however little data they move. A 128x128 step costs SMALL_STEP of
// a 256x128 one (half the MFMA work, not half the waiting). The cheapest plan
// wins.
#ifndef ZEST_GEMM_PERSIST
#define ZEST_GEMM_PERSIST 1
#endif
#ifndef ZEST_GEMM_MAX_SPLIT
#define ZEST_GEMM_MAX_SPLIT 16
#endif
#ifndef ZEST_GEMM_PROLOGUE
#define ZEST_GEMM_PROLOGUE 2.0
#endif
#ifndef ZEST_GEMM_FIX_BW
#define ZEST_GEMM_FIX_BW 4.25e6  // bytes per step: ~5 TB/s x 0.85 us
#endif
#ifndef ZEST_GEMM_FIX_LAT
#define ZEST_GEMM_FIX_LAT 5.0  // ~4 us
#endif
#ifndef ZEST_GEMM_SMALL_STEP
#define ZEST_GEMM_SMALL_STEP 0.8
#endif
// 64x64 tiles (2 consumer waves of 32x64, 2 producers; two workgroups a CU)
// for launches too small to fill the GPU with bigger tiles: a step of one
// costs TINY_STEP of a 256x128 one, and two run on a CU side by side.
#ifndef ZEST_GEMM_TINY
#define ZEST_GEMM_TINY 64, 64, 2, 128, 2
#endif
#ifndef ZEST_GEMM_TINY_STEP
#define ZEST_GEMM_TINY_STEP 0.45  // measured: ~0.38 us a step in a launch of 16 or 64 steps
#endif
// The same tiles as two K-groups (eight waves a workgroup), alone or with K
// splits, for launches of at most one and a half such workgroups a CU: each
// CU has twice the loads in flight, and the groups' sums meet in LDS instead
// of through a split-K fixup in HBM (the down projection of a 1024-token
// chunk at hidden 1024, 1024 x 1024 x 4096: 17.3 us against 21.3 in two
// splits of single-group tiles; its O projection, K 1024: 8.1 against 9.2
// unsplit). A group's step costs TINY2_STEP of a 256x128 one in the cost
// model (fitted to the launch times of the hidden-1024 layer's four GEMMs at
// 256 to 4096 tokens).
#ifndef ZEST_GEMM_TINY2_STEP
#define ZEST_GEMM_TINY2_STEP 0.4
#endif
// 256x128 tiles with 8 consumer waves of 32x128 and 4 producer waves, two
// consumers on each SIMD: for the fused GLU (its long launches gain ~3% from
// the second consumer), the whole tiles of mixed launches, and launches of
// at most one round of whole tiles that 128x160 tiles cannot take (each CU
// has one tile to hide its latencies in: the O projection at 2048 tokens as
// 160 of these, 57.9 -> 55.7 us); other launches of several rounds lose what
// the second consumer gains to its doubled W fragment reads.
#ifndef ZEST_GEMM_GLU
#define ZEST_GEMM_GLU 256, 128, 8, 256
#endif
// 128x160 tiles (4 consumer waves of 32x160) for a launch that 256x128 tiles
// would run in one round, unsplit, when its weights are whole 160-row tiles
// and these fit one round too: the O projection at 2048 tokens (2048 x 2560)
// is 256 of them, one per CU, where 160 256x128 tiles leave 96 CUs idle
// (55.5 -> ~49 us). The producers are this launch's critical path: four
// waves take two W units a thread (tiles 0-7) and two waves one (tiles 8-9),
// so the two SIMDs that hold a second producer wave carry one and a half
// waves' expansion, not two (five waves of two units: 52.5 -> 48.6 us).
// Launches with long K take them unsplit too when they fill more than half
// the GPU (launch_any): the down projection (K 9728) at 2048 tokens, 96 us
// against 104.5 us in three splits of 256x128 tiles.
#ifndef ZEST_GEMM_O
#define ZEST_GEMM_O 128, 160, 4, 384, 1, 1, 128
#endif
using cfg_big = gemm_cfg<ZEST_GEMM_BIG>;
using cfg_o = gemm_cfg<ZEST_GEMM_O>;
using cfg_small = gemm_cfg<ZEST_GEMM_SMALL>;
using cfg_glu = gemm_cfg<ZEST_GEMM_GLU>;
using cfg_tiny = gemm_cfg<ZEST_GEMM_TINY>;
// Mixed launches run their whole tiles as cfg_glu's (two consumers per SIMD)
// and the halves as 128x128 tiles of 8 consumer waves of 32x64 (4 row blocks
// x 2 column blocks) and 4 producers, the same threads (the q/k/v group at
// 2048 tokens: 66.8 -> 65.6 us against one consumer per SIMD in both).
using cfg_half8 = gemm_cfg<128, 128, 4, 256, 1, 2>;
using cfg_tiny2 = gemm_cfg<ZEST_GEMM_TINY, 1, 0, 2>;

// Per device and stream: the split-K workspace (grown as needed; counters
// zeroed when allocated, and zero again after every launch).
struct sk_space {
    float * partial = nullptr;
    size_t partial_bytes = 0;
    uint32_t * counters = nullptr;
    size_t n_counters = 0;
};

// Clears n counters (a kernel, not a memset, so a captured graph replays it).
__global__ void clear_counters(uint32_t * c, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = 0;
}

// The device address of `scratch` on device `dev`, looked up once per device
// with that device current.
int scratch_address(int dev, uint8_t ** out) {
    static std::mutex mu;
    static uint8_t * addr[ZEST_MAX_DEVICES];  // no heap: the no-alloc entry point comes here on every call
    if (dev < 0 || dev >= ZEST_MAX_DEVICES) return zest::fail(ZEST_E_ARG, "device %d: at most %d", dev, ZEST_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return zest::fail(ZEST_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        addr[dev] = (uint8_t *) p;
    }
    *out = addr[dev];
    return ZEST_OK;
}

int cu_count(int dev) {
    static std::mutex mu;
    static int cus[ZEST_MAX_DEVICES];
    if (dev < 0 || dev >= ZEST_MAX_DEVICES) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (cus[dev] > 0) return cus[dev];
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
    return n;
}

// The split-K workspaces, by device and stream (until zest_release_stream).
std::mutex g_sk_mu;
std::map<std::pair<int, hipStream_t>, sk_space> g_sk_spaces;

int sk_reserve(hipStream_t s, size_t partial_bytes, size_t n_counters, sk_space & out, const char * name) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: hipGetDevice failed", name);
    std::lock_guard<std::mutex> lock(g_sk_mu);
    sk_space & sp = g_sk_spaces[{dev, s}];
    // a launch still running on the stream may use the buffers being replaced
    if ((sp.partial_bytes < partial_bytes || sp.n_counters < n_counters) && (sp.partial || sp.counters) &&
        hipStreamSynchronize(s) != hipSuccess)
        return zest::fail(ZEST_E_HIP, "%s: stream synchronize", name);
    if (sp.partial_bytes < partial_bytes) {
        if (sp.partial) (void) hipFree(sp.partial);
        sp.partial = nullptr;
        sp.partial_bytes = 0;
        if (hipMalloc(&sp.partial, partial_bytes) != hipSuccess)
            return zest::fail(ZEST_E_HIP, "%s: split-K workspace of %zu bytes", name, partial_bytes);
        sp.partial_bytes = partial_bytes;
    }
    if (sp.n_counters < n_counters) {
        if (sp.counters) (void) hipFree(sp.counters);
        sp.counters = nullptr;
        sp.n_counters = 0;
        const size_t n = std::max(n_counters, (size_t) 4096);
        if (hipMalloc(&sp.counters, n * 4) != hipSuccess || hipMemsetAsync(sp.counters, 0, n * 4, s) != hipSuccess)
            return zest::fail(ZEST_E_HIP, "%s: split-K counters", name);
        sp.n_counters = n;
    }
    out = sp;
    return ZEST_OK;
}

template <class C, int EPI, bool SPLIT>
int set_lds(const char * name) {
    // threads that launch a kernel for the first time at once may both set
    // the attribute: the same value, harmless
    static std::atomic<bool> attr_set{false};
    if (!attr_set.load(std::memory_order_acquire)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_kernel<C, EPI, SPLIT>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int) C::LDS_BYTES);
        if (e != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: LDS attribute: %s", name, hipGetErrorString(e));
        attr_set.store(true, std::memory_order_release);
    }
    return ZEST_OK;
}

template <class C, int EPI>
int set_lds_tiles(const char * name) {
    static std::atomic<bool> attr_set{false};
    if (!attr_set.load(std::memory_order_acquire)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_kernel_tiles<C, EPI>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int) C::LDS_TILES);
        if (e != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: LDS attribute: %s", name, hipGetErrorString(e));
        attr_set.store(true, std::memory_order_release);
    }
    return ZEST_OK;
}

template <class CB, class CS, int EPI>
int set_lds_mixed_tiles(const char * name) {
    static std::atomic<bool> attr_set{false};
    if (!attr_set.load(std::memory_order_acquire)) {
        const size_t bytes = std::max(CB::LDS_BYTES, CS::LDS_BYTES);
        const hipError_t e =
            hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_kernel_mixed_tiles<CB, CS, EPI>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes);
        if (e != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: LDS attribute: %s", name, hipGetErrorString(e));
        attr_set.store(true, std::memory_order_release);
    }
    return ZEST_OK;
}

template <class CB, class CS, int EPI>
int set_lds_mixed(const char * name) {
    static std::atomic<bool> attr_set{false};
    if (!attr_set.load(std::memory_order_acquire)) {
        const size_t bytes = std::max(CB::LDS_BYTES, CS::LDS_BYTES);
        const hipError_t e =
            hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_kernel_mixed<CB, CS, EPI>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes);
        if (e != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: LDS attribute: %s", name, hipGetErrorString(e));
        attr_set.store(true, std::memory_order_release);
    }
    return ZEST_OK;
}

struct gemm_plan {
    int splits = 1;
    double cost = 0;
};

// Tiles of a launch for one tile shape.
int64_t tiles_of(const gemm_params & p, const int64_t * N, int BM, int BN) {
    int64_t nt = 0;
    for (int i = 0; i < p.nw; i++) nt += (N[i] + BN - 1) / BN;
    return ((p.M + BM - 1) / BM) * nt;
}

// The modelled cost of T tiles of nk steps on P CUs split S ways, with tiles
// of tile_bytes fp32 and steps of `step` 256x128-steps.
double split_cost(int64_t T, int nk, int64_t P, double tile_bytes, double step, int S) {
    if (S == 1) return (double) ((T + P - 1) / P) * (nk + ZEST_GEMM_PROLOGUE) * step;
    return (double) ((T * S + P - 1) / P) * ((double) nk / S + ZEST_GEMM_PROLOGUE) * step +
           2.0 * T * S * tile_bytes / ZEST_GEMM_FIX_BW + ZEST_GEMM_FIX_LAT;
}

// The cheapest number of K splits for T tiles (as split_cost).
gemm_plan plan_splits(int64_t T, int nk, int64_t P, double tile_bytes, double step) {
    gemm_plan best;
    best.cost = split_cost(T, nk, P, tile_bytes, step, 1);
    for (int S = 2; S <= ZEST_GEMM_MAX_SPLIT && nk / S >= 4; S++) {
        const double cost = split_cost(T, nk, P, tile_bytes, step, S);
        if (cost < best.cost) {
            best.splits = S;
            best.cost = cost;
        }
    }
    return best;
}

// Plans and launches one GEMM (a group of weights, or the fused GLU). A
// split-K plan takes its workspace from `fixed` when given (no allocation:
// a plan that does not fit is rejected, and the counters it uses are cleared
// first), else from the per-stream workspace.
template <class C, int EPI>
int launch(gemm_params p, const int64_t * N, int splits, hipStream_t s, const char * name,
           const sk_space * fixed = nullptr) {
    p.mt = (int) ((p.M + C::BM - 1) / C::BM);
    int nt = 0;
    for (int i = 0; i < p.nw; i++) {
        p.wt[i].tile0 = nt;
        nt += (int) ((N[i] + C::BN - 1) / C::BN);
    }
    p.nt = nt;
    const int64_t T = (int64_t) p.mt * nt;
    p.splits = splits;
    if (C::KG > 1 && p.nk % (splits * C::KG))
        return zest::fail(ZEST_E_ARG, "%s: %d K-steps do not make %d splits of %d K-groups", name, p.nk, splits,
                          C::KG);
    const int64_t grid = T * p.splits;
    if (grid >= (1ll << 31) || (p.splits > 1 && grid * C::BM * C::BN * 4 >= (1ll << 31)))
        return zest::fail(ZEST_E_ARG, "%s: %lld tiles is too many", name, (long long) T);
    if (p.splits > 1) {
        const size_t partial_bytes = (size_t) grid * C::BM * C::BN * 4, n_counters = (size_t) T * (C::NC / 64);
        sk_space sp;
        if (fixed) {
            if (partial_bytes > fixed->partial_bytes || n_counters > fixed->n_counters)
                return zest::fail(ZEST_E_ARG,
                                  "%s: this shape's split-K plan needs %zu bytes of partial sums and %zu counters; "
                                  "the static workspace holds %zu bytes and %zu counters",
                                  name, partial_bytes, n_counters, fixed->partial_bytes, fixed->n_counters);
            sp = *fixed;
            hipLaunchKernelGGL(clear_counters, dim3((unsigned) ((n_counters + 255) / 256)), dim3(256), 0, s,
                               sp.counters, (int) n_counters);
        } else {
            const int st = sk_reserve(s, partial_bytes, n_counters, sp, name);
            if (st != ZEST_OK) return st;
        }
        p.partial = sp.partial;
        p.counters = sp.counters;
    }
#if ZEST_GEMM_PERSIST
    // more than one round: persistent workgroups, one a CU (not for the
    // residual epilogue, whose persistent form does not fit the registers)
    if constexpr (EPI != EPI_RESIDUAL && C::MINB == 1 && C::NP1 == 0 && C::KG == 1)
        if (p.splits == 1 && p.nk % 2 == 0 && p.nk >= 4) {
            int dev = 0;
            (void) hipGetDevice(&dev);
            const int64_t G = cu_count(dev) / 8 * 8;
            if (G >= 8 && T > G) {
                const int st = set_lds_tiles<C, EPI>(name);
                if (st != ZEST_OK) return st;
                hipLaunchKernelGGL((gemm_kernel_tiles<C, EPI>), dim3((unsigned) G), dim3(C::NT), C::LDS_TILES, s, p);
                return zest::check_launch(name);
            }
        }
#endif
    const int st = p.splits > 1 ? set_lds<C, EPI, true>(name) : set_lds<C, EPI, false>(name);
    if (st != ZEST_OK) return st;
    if (p.splits > 1)
        hipLaunchKernelGGL((gemm_kernel<C, EPI, true>), dim3((unsigned) grid), dim3(C::NT), C::LDS_BYTES, s, p);
    else
        hipLaunchKernelGGL((gemm_kernel<C, EPI, false>), dim3((unsigned) grid), dim3(C::NT), C::LDS_BYTES, s, p);
    return zest::check_launch(name);
}

// A mixed launch: the first nbig big tiles whole, the rest as halves.
template <class CB, class CS, int EPI>
int launch_mixed(gemm_params p, const int64_t * N, int64_t nbig, hipStream_t s, const char * name) {
    p.mt = (int) ((p.M + CB::BM - 1) / CB::BM);
    int nt = 0;
    for (int i = 0; i < p.nw; i++) {
        p.wt[i].tile0 = nt;
        nt += (int) ((N[i] + CB::BN - 1) / CB::BN);
    }
    p.nt = nt;
    const int64_t T = (int64_t) p.mt * nt, grid = nbig + 2 * (T - nbig);
    if (grid >= (1ll << 31) || nbig % 8 || nbig >= T)
        return zest::fail(ZEST_E_ARG, "%s: mixed launch of %lld tiles", name, (long long) T);
    p.splits = 1;
    p.nbig = (int) nbig;
#if ZEST_GEMM_PERSIST
    // persistent workgroups, one a CU (not for the residual epilogue, whose
    // persistent form does not fit the registers)
    if constexpr (EPI != EPI_RESIDUAL)
        if (p.nk % 2 == 0 && p.nk >= 4) {
            int dev = 0;
            (void) hipGetDevice(&dev);
            const int64_t G = std::min<int64_t>(nbig, cu_count(dev) / 8 * 8);
            if (G >= 8) {
                const int st = set_lds_mixed_tiles<CB, CS, EPI>(name);
                if (st != ZEST_OK) return st;
                hipLaunchKernelGGL((gemm_kernel_mixed_tiles<CB, CS, EPI>), dim3((unsigned) G), dim3(CB::NT),
                                   std::max(CB::LDS_BYTES, CS::LDS_BYTES), s, p);
                return zest::check_launch(name);
            }
        }
#endif
    const int st = set_lds_mixed<CB, CS, EPI>(name);
    if (st != ZEST_OK) return st;
    hipLaunchKernelGGL((gemm_kernel_mixed<CB, CS, EPI>), dim3((unsigned) grid), dim3(CB::NT),
                       std::max(CB::LDS_BYTES, CS::LDS_BYTES), s, p);
    return zest::check_launch(name);
}

// The plan of a plain (or residual) launch: its tile shape and K splits.
enum class shape_kind { o_round, mixed, tiny, small, o_one, glu_one, big };
struct plain_plan {
    shape_kind kind;
    int splits;
    int64_t nbig;  // mixed: the whole tiles
    int kg = 1;    // tiny: K-groups
};

// The cost model above, applied: the cheapest of one round of 128x160 tiles
// (long K), a mixed launch, 64x64 tiles (with their best K split, alone or as
// two K-groups), 128x128 or 256x128 tiles (each with its best K split), and,
// for one unsplit round, 128x160 or two-consumer 256x128 tiles.
plain_plan plan_plain(const gemm_params & p, const int64_t * N, int64_t P) {
    const gemm_plan big =
        plan_splits(tiles_of(p, N, cfg_big::BM, cfg_big::BN), p.nk, P, (double) cfg_big::BM * cfg_big::BN * 4, 1.0);
    const gemm_plan small = plan_splits(tiles_of(p, N, cfg_small::BM, cfg_small::BN), p.nk, P,
                                        (double) cfg_small::BM * cfg_small::BN * 4, ZEST_GEMM_SMALL_STEP);
    bool whole = true;  // every weight whole 160-row tiles
    for (int i = 0; i < p.nw; i++) whole &= N[i] % cfg_o::BN == 0;
    const int64_t To = tiles_of(p, N, cfg_o::BM, cfg_o::BN);
    // one round of 128x160 tiles, unsplit, when every weight is whole
    // 160-row tiles, they fill more than half the GPU and K is long enough
    // for the prologue not to matter: no split-K fixup traffic, and the
    // tile's producers keep up with its consumers (the down projection at
    // 2048 tokens, K 9728: 104.5 us in three splits, 96 us so)
    if (whole && To <= P && 2 * To > P && p.nk >= 16) return {shape_kind::o_round, 1, 0};
    // mixed: whole rounds of big tiles, the part-round left as half tiles
    const int64_t Tb = tiles_of(p, N, cfg_big::BM, cfg_big::BN), R = Tb / P, rem = Tb - R * P;
    if (R >= 1 && rem > 0 && R * P % 8 == 0) {
        const double mixed =
            ((double) R + (double) ((2 * rem + P - 1) / P) * ZEST_GEMM_SMALL_STEP) * (p.nk + ZEST_GEMM_PROLOGUE);
        if (mixed < big.cost && mixed < small.cost) return {shape_kind::mixed, 1, R * P};
    }
    // tiny tiles, cfg_tiny::MINB of them a CU
    const int64_t Tt = tiles_of(p, N, cfg_tiny::BM, cfg_tiny::BN);
    const gemm_plan tiny =
        plan_splits(Tt, p.nk, P * cfg_tiny::MINB, (double) cfg_tiny::BM * cfg_tiny::BN * 4, ZEST_GEMM_TINY_STEP);
    // as two K-groups: the launch's nk/2 group steps in S splits
    gemm_plan tiny2;
    tiny2.splits = 0;
    for (int S = 1; S <= 8; S *= 2) {
        if (p.nk % (2 * S) || p.nk / (2 * S) < 4 || 2 * Tt * S > 3 * P) continue;
        const double cost = split_cost(Tt, p.nk / 2, P, (double) cfg_tiny::BM * cfg_tiny::BN * 4,
                                       ZEST_GEMM_TINY2_STEP, S);
        if (tiny2.splits == 0 || cost < tiny2.cost) tiny2 = {S, cost};
    }
    if (tiny2.splits > 0 && tiny2.cost < tiny.cost && tiny2.cost < big.cost && tiny2.cost < small.cost)
        return {shape_kind::tiny, tiny2.splits, 0, 2};
    if (tiny.cost < big.cost && tiny.cost < small.cost) return {shape_kind::tiny, tiny.splits, 0};
    if (small.cost < big.cost) return {shape_kind::small, small.splits, 0};
    if (big.splits == 1 && Tb <= P) {
        // one round of whole tiles: as 128x160 tiles where the weights are
        // whole 160-row tiles (the tiles then read only rows each packed
        // weight holds) and they fit one round too, else with two consumers
        // per SIMD
        if (whole && To <= P) return {shape_kind::o_one, 1, 0};
        return {shape_kind::glu_one, 1, 0};
    }
    return {shape_kind::big, big.splits, 0};
}

// Plans and launches a GEMM; `fixed` as for launch(). A fused GLU launch
// splits K as the plain launch of its 2F columns would, in as many K-groups
// (so its gate and up sums are that launch's, bit for bit: a sum depends on
// the K-steps' partition and order, not on the tile shape), and takes the
// cheaper of 256x128 and 128x128 tiles at that split (64x64 tiles for
// K-groups).
template <int EPI>
int launch_any(gemm_params p, const int64_t * N, hipStream_t s, const char * name,
               const sk_space * fixed = nullptr) {
    int dev = 0;
    (void) hipGetDevice(&dev);
    const int64_t P = cu_count(dev);
    const plain_plan pp = plan_plain(p, N, P);
    if constexpr (EPI >= 0) {
        const int S = pp.splits;
        // The tiles cover the output operand's K padding too: the columns of
        // 2F rounded up to 128 rows of the gate/up pair, whose rows past 2F
        // are zero blocks, so the h columns past F store the packer's zeros
        // (with 64-column tiles and F % 64 == 32 the last tile would end at F).
        const int64_t Nt = (N[0] + 127) / 128 * 128;
        if (pp.kg == 2) return launch<cfg_tiny2, EPI>(p, &Nt, S, s, name, fixed);
        const double big = split_cost(tiles_of(p, N, cfg_glu::BM, cfg_glu::BN), p.nk, P,
                                      (double) cfg_glu::BM * cfg_glu::BN * 4, 1.0, S);
        const double small = split_cost(tiles_of(p, N, cfg_small::BM, cfg_small::BN), p.nk, P,
                                        (double) cfg_small::BM * cfg_small::BN * 4, ZEST_GEMM_SMALL_STEP, S);
        if (small < big) return launch<cfg_small, EPI>(p, &Nt, S, s, name, fixed);
        return launch<cfg_glu, EPI>(p, &Nt, S, s, name, fixed);
    } else {
        switch (pp.kind) {
            case shape_kind::o_round:
            case shape_kind::o_one: return launch<cfg_o, EPI>(p, N, 1, s, name, fixed);
            case shape_kind::mixed: return launch_mixed<cfg_glu, cfg_half8, EPI>(p, N, pp.nbig, s, name);
            case shape_kind::tiny:
                if (pp.kg == 2) return launch<cfg_tiny2, EPI>(p, N, pp.splits, s, name, fixed);
                return launch<cfg_tiny, EPI>(p, N, pp.splits, s, name, fixed);
            case shape_kind::small: return launch<cfg_small, EPI>(p, N, pp.splits, s, name, fixed);
            case shape_kind::glu_one: return launch<cfg_glu, EPI>(p, N, 1, s, name, fixed);
            case shape_kind::big: break;
        }
        return launch<cfg_big, EPI>(p, N, pp.splits, s, name, fixed);
    }
}

// The parts of a launch's parameters common to every kind.
gemm_params base_params(const void * a, int64_t M, int64_t K, uint32_t * nonfinite) {
    gemm_params p{};
    p.a = (const uint8_t *) a;
    p.M = M;
    p.a_kstride = (int) ((zest_rows_padded(M) / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES);
    p.nk = (int) (zest_k_padded(K) / ZEST_TILE_K);
    p.nonfinite = nonfinite;
    return p;
}

gemm_weight weight_of(const void * w, int64_t N, float * c, int64_t ldc) {
    gemm_weight g{};
    g.w = (const uint8_t *) w;
    g.c = c;
    g.n = N;
    g.ldc = ldc;
    g.w_kstride = (int) ((zest_rows_padded(N) / ZEST_TILE_ROWS) * ZEST_TILE_BYTES);
    return g;
}

// The rows of one launch's band. A launch reaches its output (and a
// residual) through buffer resources whose byte ranges are 32-bit, so an
// output of rows `ld` floats apart runs as bands of whole 256-row tiles, each
// under 2 GiB, one launch a band (the reference likewise cuts a claimed
// matmul into NPU calls of at most 1024 rows, src/xdna-npu.cpp:392-420).
// 0 when not even 256 rows fit.
int64_t band_rows(int64_t ld) {
    const int64_t rows = ((1ll << 31) - 1) / (ld * 4);
    return rows / ZEST_ROW_ALIGN * ZEST_ROW_ALIGN;
}

// The launch parameters of the band of rows [r0, r0 + rows): the activation
// operand from row r0 on (whole 32-row groups; the K-step stride stays the
// whole operand's) and each weight's output from its row r0.
gemm_params band_of(const gemm_params & p, int64_t r0, int64_t rows) {
    gemm_params q = p;
    q.M = rows;
    q.a = p.a + r0 / ZEST_XGROUP_ROWS * ZEST_XGROUP_BYTES;
    for (int i = 0; i < p.nw; i++)
        if (q.wt[i].c) q.wt[i].c += r0 * q.wt[i].ldc;
    if (q.res) q.res += r0 * q.ldr;
    return q;
}

bool aligned_to(const void * p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// zest_gemm_group's checks and launches. A no-alloc call takes its split-K
// workspace from the device's static array (looked up once the arguments
// pass), else from the per-stream workspace.
int gemm_group(const void * a, int64_t M, int64_t K, int n, const void * const * w, const int64_t * N,
               float * const * c, const int64_t * ldc, uint32_t * nonfinite, void * stream, const char * name,
               bool noalloc) {
    ZEST_REQUIRE(a && w && N && c && ldc, "%s: null pointer", name);
    ZEST_REQUIRE(n >= 1 && n <= ZEST_GEMM_MAX_GROUP, "%s: %d weights (1..%d)", name, n, ZEST_GEMM_MAX_GROUP);
    ZEST_REQUIRE(M > 0 && K > 0 && K % 8 == 0, "%s: M=%lld K=%lld", name, (long long) M, (long long) K);
    ZEST_REQUIRE(zest_act_bytes(M, K) < (1ull << 31), "%s: activations must be under 2 GiB", name);
    ZEST_REQUIRE(aligned_to(a, 16) && aligned_to(nonfinite, 4), "%s: a must be 16-byte aligned, nonfinite 4", name);
    gemm_params p = base_params(a, M, K, nonfinite);
    p.nw = n;
    int64_t ld_max = 0;
    for (int i = 0; i < n; i++) {
        ZEST_REQUIRE(w[i] && c[i], "%s: null weight or output %d", name, i);
        ZEST_REQUIRE(aligned_to(w[i], 16) && aligned_to(c[i], 4),
                     "%s: weight %d must be 16-byte aligned and its output 4", name, i);
        ZEST_REQUIRE(N[i] > 0 && ldc[i] >= N[i], "%s: weight %d: N=%lld ldc=%lld", name, i, (long long) N[i],
                     (long long) ldc[i]);
        ZEST_REQUIRE(zest_bfp16_bytes(N[i], K) < (1ull << 31), "%s: weight %d must be under 2 GiB (N=%lld K=%lld)",
                     name, i, (long long) N[i], (long long) K);
        p.wt[i] = weight_of(w[i], N[i], c[i], ldc[i]);
        ld_max = std::max(ld_max, ldc[i]);
    }
    const int64_t band = band_rows(ld_max);
    ZEST_REQUIRE(band > 0, "%s: 256 output rows of %lld floats must be under 2 GiB", name, (long long) ld_max);
    sk_space ws;
    const sk_space * fixed = nullptr;
    if (noalloc) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return zest::fail(ZEST_E_HIP, "%s: hipGetDevice failed", name);
        uint8_t * base = nullptr;
        const int st = scratch_address(dev, &base);
        if (st != ZEST_OK) return st;
        ws.partial = reinterpret_cast<float *>(base);
        ws.partial_bytes = ZEST_NOALLOC_PARTIAL_BYTES;
        ws.counters = reinterpret_cast<uint32_t *>(base + ZEST_NOALLOC_PARTIAL_BYTES);
        ws.n_counters = ZEST_NOALLOC_COUNTERS;
        fixed = &ws;
    }
    const hipStream_t s = zest::as_stream(stream);
    for (int64_t r0 = 0; r0 < M; r0 += band) {
        const int st = launch_any<EPI_PLAIN>(band_of(p, r0, std::min(band, M - r0)), N, s, name, fixed);
        if (st != ZEST_OK) return st;
    }
    return ZEST_OK;
}

} // namespace

namespace zest {

int scratch_setup(int dev) {
    uint8_t * p = nullptr;
    return scratch_address(dev, &p);
}

} // namespace zest

extern "C" int zest_gemm_group(const void * a, int64_t M, int64_t K, int n, const void * const * w, const int64_t * N,
                               float * const * c, const int64_t * ldc, uint32_t * nonfinite, void * stream) {
    return gemm_group(a, M, K, n, w, N, c, ldc, nonfinite, stream, "zest_gemm", false);
}

extern "C" int zest_gemm_group_noalloc(const void * a, int64_t M, int64_t K, int n, const void * const * w,
                                       const int64_t * N, float * const * c, const int64_t * ldc,
                                       uint32_t * nonfinite, void * stream) {
    return gemm_group(a, M, K, n, w, N, c, ldc, nonfinite, stream, "zest_gemm_group_noalloc", true);
}

extern "C" int zest_release_stream(void * stream) {
    const hipStream_t s = zest::as_stream(stream);
    std::lock_guard<std::mutex> lock(g_sk_mu);
    bool synced = false;
    for (auto it = g_sk_spaces.begin(); it != g_sk_spaces.end();) {
        if (it->first.second != s) {
            ++it;
            continue;
        }
        // launches still queued on the stream may use the workspace
        if (!synced && hipStreamSynchronize(s) != hipSuccess)
            return zest::fail(ZEST_E_HIP, "zest_release_stream: stream synchronize");
        synced = true;
        if (it->second.partial) (void) hipFree(it->second.partial);
        if (it->second.counters) (void) hipFree(it->second.counters);
        it = g_sk_spaces.erase(it);
    }
    return ZEST_OK;
}

extern "C" int zest_gemm(const void * a, int64_t M, const void * w, int64_t N, int64_t K, float * c, int64_t ldc,
                         uint32_t * nonfinite, void * stream) {
    return zest_gemm_group(a, M, K, 1, &w, &N, &c, &ldc, nonfinite, stream);
}

extern "C" int zest_gemm_residual(const void * a, int64_t M, const void * w, int64_t N, int64_t K, const float * res,
                                  int64_t ldr, float * c, int64_t ldc, uint32_t * nonfinite, void * stream) {
    ZEST_REQUIRE(a && w && c && res, "zest_gemm_residual: null pointer");
    ZEST_REQUIRE(M > 0 && N > 0 && K > 0 && K % 8 == 0, "zest_gemm_residual: M=%lld N=%lld K=%lld", (long long) M,
                 (long long) N, (long long) K);
    ZEST_REQUIRE(ldc >= N && ldr >= N, "zest_gemm_residual: ldc %lld / ldr %lld < N %lld", (long long) ldc,
                 (long long) ldr, (long long) N);
    ZEST_REQUIRE((reinterpret_cast<uintptr_t>(res) & 15) == 0 && ldr % 4 == 0,
                 "zest_gemm_residual: the residual's rows must be 16-byte aligned");
    ZEST_REQUIRE(aligned_to(a, 16) && aligned_to(w, 16) && aligned_to(c, 4) && aligned_to(nonfinite, 4),
                 "zest_gemm_residual: a and w must be 16-byte aligned, c and nonfinite 4");
    ZEST_REQUIRE(zest_act_bytes(M, K) < (1ull << 31) && zest_bfp16_bytes(N, K) < (1ull << 31),
                 "zest_gemm_residual: operands must be under 2 GiB");
    const int64_t band = band_rows(std::max(ldc, ldr));
    ZEST_REQUIRE(band > 0, "zest_gemm_residual: 256 rows of the output and residual must be under 2 GiB");
    gemm_params p = base_params(a, M, K, nonfinite);
    p.nw = 1;
    p.wt[0] = weight_of(w, N, c, ldc);
    p.res = res;
    p.ldr = ldr;
    const hipStream_t s = zest::as_stream(stream);
    for (int64_t r0 = 0; r0 < M; r0 += band) {
        const int st = launch_any<EPI_RESIDUAL>(band_of(p, r0, std::min(band, M - r0)), &N, s, "zest_gemm_residual");
        if (st != ZEST_OK) return st;
    }
    return ZEST_OK;
}

extern "C" int zest_gemm_glu(int kind, const void * a, int64_t M, const void * w_gu, int64_t F, int64_t K,
                             void * xout, float * h, int64_t ldh, uint32_t * nonfinite, void * stream) {
    ZEST_REQUIRE(a && w_gu && (xout || h), "zest_gemm_glu: null pointer");
    ZEST_REQUIRE(M > 0 && F > 0 && F % 32 == 0 && K > 0 && K % 8 == 0, "zest_gemm_glu: M=%lld F=%lld K=%lld",
                 (long long) M, (long long) F, (long long) K);
    ZEST_REQUIRE(!h || ldh >= F, "zest_gemm_glu: ldh %lld < F %lld", (long long) ldh, (long long) F);
    ZEST_REQUIRE(aligned_to(a, 16) && aligned_to(w_gu, 16) && aligned_to(xout, 16) && aligned_to(h, 4) &&
                     aligned_to(nonfinite, 4),
                 "zest_gemm_glu: a, w_gu and xout must be 16-byte aligned, h and nonfinite 4");
    ZEST_REQUIRE(zest_act_bytes(M, K) < (1ull << 31) && zest_bfp16_bytes(2 * F, K) < (1ull << 31) &&
                     zest_act_bytes(M, F) < (1ull << 31),
                 "zest_gemm_glu: operands must be under 2 GiB (M=%lld F=%lld K=%lld)", (long long) M, (long long) F,
                 (long long) K);
    gemm_params p = base_params(a, M, K, nonfinite);
    const int64_t N = 2 * F;
    p.nw = 1;
    p.wt[0] = weight_of(w_gu, N, nullptr, 0);
    p.xout = (uint8_t *) xout;
    p.h = h;
    p.ldh = ldh;
    hipStream_t s = zest::as_stream(stream);
    const char * name = "zest_gemm_glu";
    switch (kind) {
        case ZEST_GLU_SWIGLU: return launch_any<ZEST_GLU_SWIGLU>(p, &N, s, name);
        case ZEST_GLU_GEGLU: return launch_any<ZEST_GLU_GEGLU>(p, &N, s, name);
        case ZEST_GLU_GEGLU_ERF: return launch_any<ZEST_GLU_GEGLU_ERF>(p, &N, s, name);
        case ZEST_GLU_GEGLU_QUICK: return launch_any<ZEST_GLU_GEGLU_QUICK>(p, &N, s, name);
        case ZEST_GLU_REGLU: return launch_any<ZEST_GLU_REGLU>(p, &N, s, name);
        default: return zest::fail(ZEST_E_UNSUPPORTED, "zest_gemm_glu: GLU kind %d", kind);
    }
}

// The bfp16 operand layout in HBM ("tile layout"), shared by the packers, the
// weight converter and the GEMM.
//
// The block format is the reference's: eight values along K share one
// exponent byte e (the largest biased exponent field of the eight), and each
// value is a signed 8-bit mantissa q = RNE(x * 2^(133 - e)) saturated to
// [-128, 127]; the value it stands for is q * 2^(e - 133)
// (src/npu/bfp16_pack.h:28-35). 9 bytes per 8 values, as in the reference.
//
// Only the byte ORDER differs from the reference's NPU order, for 128-bit
// coalesced access on the GPU:
//   * An operand of R rows x K columns (K along a row: activations [M][K], or
//     a GGUF weight [N][K]) is padded to R_pad = roundup(R, 256) rows and
//     K_pad = roundup(K, 64) columns with zero blocks.
//   * It is cut into tiles of 16 rows x 64 columns. Tile (rt, kc) starts at
//     byte (kc * R_pad/16 + rt) * 1152: all row tiles of one 64-column chunk
//     are contiguous, so a GEMM K-step over 256 rows reads one 18 KB run.
//   * Inside a tile: the 16 x 64 mantissas row-major (1024 bytes), then the
//     16 x 8 exponent bytes row-major (128 bytes). 1152 = 9 x 128: every tile
//     is a whole number of 128-byte lines.
// The bijection to the reference's row-major blocks is zest_block_offsets();
// tests map our bytes through it and compare with the reference packer's.
//
// The GEMM's activation operand ("expanded" layout) holds the same bfp16
// blocks already decoded, each value q * 2^(e-133) as the bf16 it is exactly
// (a signed 8-bit mantissa times a power of two fits a bf16 significand):
// rows padded to 256 and columns to 64 as above, cut into sub-tiles of 32
// rows x 16 columns (1 KB; a row's 16 values, two blocks, are 32 contiguous
// bytes), ordered [64-column chunk][32-row group][16-column quarter]:
// element (r, c) is at byte
//   ((c/64 * R_pad/32 + r/32) * 4 + (c%64)/16) * 1024 + (r%32) * 32 + (c%16) * 2.
// A sub-tile is exactly the A operand of one 32x32x16 MFMA (lane l: row l%32,
// columns 8(l/32)..8(l/32)+7, the 16 bytes at 32(l%32) + 16(l/32)), so a wave
// loads it with one instruction covering 1 KB contiguous, and a K-step (64
// columns) of 256 rows is one contiguous 32 KB run. The activation packers write it directly, so
// every activation value is expanded once rather than once per output tile
// of the GEMM.
#pragma once

#include <stdint.h>

#define ZEST_TILE_ROWS 16
#define ZEST_TILE_K 64
#define ZEST_TILE_MANT 1024
#define ZEST_TILE_BYTES 1152
#define ZEST_ROW_ALIGN 256
#define ZEST_XGROUP_ROWS 32    // rows of an expanded sub-tile
#define ZEST_XSUB_BYTES 1024   // an expanded sub-tile: 32 rows x 16 columns
#define ZEST_XGROUP_BYTES 4096 // the four sub-tiles of a 32-row group in one 64-column chunk

#ifdef __HIPCC__
#define ZEST_HD __host__ __device__ inline
#else
#define ZEST_HD static inline
#endif

ZEST_HD int64_t zest_round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
ZEST_HD int64_t zest_rows_padded(int64_t rows) { return zest_round_up(rows, ZEST_ROW_ALIGN); }
ZEST_HD int64_t zest_k_padded(int64_t K) { return zest_round_up(K, ZEST_TILE_K); }

// Byte offset of tile (rt, kc) in an operand of R_pad rows.
ZEST_HD int64_t zest_tile_offset(int64_t rt, int64_t kc, int64_t R_pad) {
    return (kc * (R_pad / ZEST_TILE_ROWS) + rt) * ZEST_TILE_BYTES;
}

// Byte offset of element (r, c) of an expanded operand of R_pad rows.
ZEST_HD int64_t zest_xoffset(int64_t r, int64_t c, int64_t R_pad) {
    return ((c / ZEST_TILE_K) * (R_pad / ZEST_XGROUP_ROWS) + r / ZEST_XGROUP_ROWS) * ZEST_XGROUP_BYTES +
           ((c % ZEST_TILE_K) / 16) * ZEST_XSUB_BYTES + (r % ZEST_XGROUP_ROWS) * 32 + (c % 16) * 2;
}

// Where block cb (columns 8cb..8cb+7) of row r lives: its exponent byte and
// its first mantissa byte (the eight mantissas are contiguous).
ZEST_HD void zest_block_offsets(int64_t r, int64_t cb, int64_t R_pad, int64_t * exp_off, int64_t * mant_off) {
    const int64_t t = zest_tile_offset(r / ZEST_TILE_ROWS, cb / 8, R_pad);
    const int64_t rr = r % ZEST_TILE_ROWS, bb = cb % 8;
    *mant_off = t + rr * ZEST_TILE_K + bb * 8;
    *exp_off = t + ZEST_TILE_MANT + rr * 8 + bb;
}

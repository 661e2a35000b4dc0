// Host-visible launch interface of the affine quantized-projection kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

// Largest number of quantization groups one workgroup of the small-row kernel covers (bounds
// the scales and biases it stages in LDS). The host splits K so that this holds.
constexpr int kMaxGroupsPerSplit = 64;

struct QmvParams {
  const uint16_t* x;         // [M, K] activations
  const uint32_t* w[2];      // [N, K*bits/32] packed codes (gate, up for SwiGLU)
  const uint16_t* s[2];      // [N, K/G] scales
  const uint16_t* b[2];      // [N, K/G] biases
  const uint16_t* residual;  // [M, N] or null (single projection only)
  uint16_t* y;               // [M, N] output
  float* partial;            // [ksplit][nproj][M][N] split-K partial sums
  uint32_t* counters;        // [N/32] split-K arrival counters, zero between calls
  int M, K, N, G;
  int group_shift;           // log2(G / 64)
  int ksplit;
  int steps_per_split;
  int strips;                // column strips; the staged kernels take strips of N / strips
                             // (16..32) columns, the register kernel N / 32 (grid x = strips)
  int tiles;                 // staged kernels: strips per workgroup (1 or 2; grid x =
                             // strips / tiles)
  // Code layout, as byte strides of a column's codes and of one 64-wide K step: MLX rows
  // (column stride K * bits / 8, step stride 8 * bits) or the step-major repack (column stride
  // 8 * bits, step stride N * 8 * bits; see launch_affine_repack).
  uint32_t col_stride;
  uint32_t step_stride;
  int col_align;             // staged kernels: strip boundaries at multiples of this many
                             // columns (1, or a 128-byte line of repacked codes)
  int strip_cols;            // staged kernels: the width of every strip when all are equal
                             // (strip s = columns [s strip_cols, (s + 1) strip_cols)), else 0
  int groups_per_row;        // K / G
  int order;                 // GEMV kernel: 1 = column groups dealt out XCD by XCD
  int gemv_groups;           // GEMV kernel: column groups per workgroup (affine_gemv_groups)
  int gemv_groups_per_wave;  // GEMV kernel, whole groups in every wave: groups per wave
  int gemv_dealt;            // GEMV kernel: workgroups dealt out XCD by XCD (order 1: the grid
                             // rounded down to a multiple of 8; order 0: none)
  int wave_steps;            // block kernel: K steps per wave (steps_per_split / waves, up)
  int sb_words;              // block kernel: 32-bit words of one staged scale or bias row
};

// Step-major repack of MLX affine codes: the 8 * bits bytes of column n and K step t (codes
// [64 t, 64 t + 64) of row n) move to byte (t * N + n) * 8 * bits, so the codes every column of
// a strip needs for one K step are contiguous.
hipError_t launch_affine_repack(const uint32_t* w, uint32_t* out, int N, int K, int bits,
                                hipStream_t stream);

hipError_t launch_affine_qmv(const QmvParams& p, int bits, int dtype, int nproj,
                             hipStream_t stream);

// LDS row (in 32-bit words) of one column's scales or biases over a split's groups.
constexpr int kSbRowWords = kMaxGroupsPerSplit / 2 + 2;

// ---- activation-staged small-row kernels (M <= 32; 16 for groups of 32) -----------------
// Eight waves per strip ("tile"), one or two tiles per workgroup; the workgroup's activation
// rows for its K range live in LDS, shared by its tiles.
constexpr int kQmvLdsWaves = 8;
constexpr int kQmvLdsMaxRows = 32;        // groups of 64 or more
constexpr int kQmvLdsMaxRowsHalf = 16;    // groups of 32 (two MFMA chains per step)
// Dynamic LDS bound of one workgroup: two one-tile workgroups share a CU's 160 KiB, a two-tile
// workgroup has the CU to itself (less room for the kernel's static shared variables).
__host__ __device__ constexpr uint32_t qmv_lds_max_bytes(int tiles) {
  return tiles == 1 ? 80u * 1024u : 152u * 1024u;
}

// 16-byte activation chunks each thread stages (M * steps_per_split * 8 chunks in all, over
// 512 * tiles threads).
__host__ __device__ constexpr int qmv_lds_chunk_iters(int mrows, int tiles) {
  return ((mrows <= 8 ? 5 : mrows <= 16 ? 8 : 12) + tiles - 1) / tiles;
}

// Dynamic LDS of one workgroup, byte offsets: scales and biases [tiles][2 nproj][32]
// [kSbRowWords] (32-bit words), activation rows [M + 1][steps_per_split * 64 + 8] (16-bit; row M is all
// zeros and stands in for rows M..31 of the MFMA tile), per-step row sums
// [steps_per_split * halves][mrows] (fp32; halves = 2 for groups of 32, one sum per group).
// After the K loop the cross-wave reduction buffer
// [tiles][waves][nproj][mrows][33] (fp32) reuses the space from offset 0.
struct QmvLdsLayout {
  uint32_t x;
  uint32_t zero;
  uint32_t xsum;
  uint32_t bytes;
};

__host__ __device__ inline QmvLdsLayout qmv_lds_layout(int M, int steps_per_split, int mrows,
                                                       int nproj, int halves, int tiles) {
  QmvLdsLayout l;
  const uint32_t row = (uint32_t)(steps_per_split * 64 + 8) * 2u;
  l.x = (uint32_t)(tiles * 2 * nproj * 32 * kSbRowWords) * 4u;
  l.zero = l.x + (uint32_t)M * row;
  l.xsum = l.zero + row;
  const uint32_t staged = l.xsum + (uint32_t)(steps_per_split * halves * mrows) * 4u;
  const uint32_t red = (uint32_t)(tiles * kQmvLdsWaves * nproj * mrows * 33) * 4u;
  l.bytes = staged > red ? staged : red;
  return l;
}

// Whether the activation-staged kernels take M rows split into K ranges of steps_per_split
// 64-wide steps with `tiles` strips per workgroup (the staging must fit the per-thread chunk
// budget, the scale rows and qmv_lds_max_bytes). They are the only small-row kernels for
// groups of 32.
bool affine_qmv_lds_fits(int M, int steps_per_split, int nproj, int group_size, int tiles);

hipError_t launch_affine_qmv_lds(const QmvParams& p, int bits, int dtype, int nproj,
                                 hipStream_t stream);

// ---- GEMV kernel (M <= 4, no K split) ----------------------------------------------------
// Workgroups of `waves` waves (1 to kGemvMaxWaves) each own `cols` output columns (2, 4 or 8)
// per column group and all of K; reads x, w, s, b, residual, y, M, K, N, G and the code layout
// of p.
constexpr int kGemvMaxRows = 4;
constexpr int kGemvMaxWaves = 8;
// Whether a workgroup holds `cols` columns of `nproj` projections at `rows` rows (rounded up to
// 1, 2 or 4) in registers without spilling: always when every lane has one chunk per column
// (`one_pass`: one pass of loads in registers), else (two passes) when nproj * cols * rows <= 8.
__host__ __device__ constexpr int affine_gemv_row_bucket(int rows) {
  return rows <= 1 ? 1 : rows <= 2 ? 2 : 4;
}
__host__ __device__ constexpr bool affine_gemv_fits(int rows, int nproj, int cols,
                                                    bool one_pass) {
  return rows >= 1 && rows <= kGemvMaxRows &&
         (cols == 2 || cols == 4 || (cols == 8 && one_pass && nproj == 1 && rows <= 2)) &&
         (one_pass || nproj * cols * affine_gemv_row_bucket(rows) <= 8);
}
// Whether a dispatch of K codes per column takes one pass with `waves` waves.
__host__ __device__ constexpr bool affine_gemv_one_pass(int K, int bits, int waves) {
  return K * bits / 128 <= 64 * waves;
}
// Column groups (of `cols` columns each) one workgroup covers. When a column's chunks fit in one
// wave (at most 64), every wave holds whole groups: 64 / chunks of them when the chunks fill
// whole rows of 16 lanes (so DPP row sums never mix groups), else one. Otherwise, in one pass,
// when the chunks fill whole rows of 16 lanes, as many groups as the workgroup's lanes hold
// (lane t: group t / chunks, chunk t % chunks), and else one. Grid: N / (cols * groups)
// workgroups.
__host__ __device__ constexpr int affine_gemv_groups(int K, int bits, int waves) {
  return K * bits / 128 <= 64
             ? waves * ((K * bits / 128) % 16 == 0 ? 64 / (K * bits / 128) : 1)
         : affine_gemv_one_pass(K, bits, waves) && (K * bits / 128) % 16 == 0
             ? 64 * waves / (K * bits / 128)
             : 1;
}
hipError_t launch_affine_gemv(const QmvParams& p, int bits, int dtype, int nproj, int waves,
                              int cols, hipStream_t stream);

// ---- column-block kernel (M <= 32, groups of 64 or more) ----------------------------------
// A workgroup owns a block of at most kBlockMaxCols columns (block b = columns [b N / strips,
// (b + 1) N / strips), in units of col_align) over the K range of its split (grid strips x
// ksplit); its `waves` waves (1 to kBlockMaxWaves) take consecutive runs of wave_steps steps of
// that range, each over every column of the block, with v_mfma_f32_16x16x32 (16-column tiles,
// one or two 16-row tiles).
constexpr int kBlockMaxWaves = 8;
constexpr int kBlockMaxCols = 64;
constexpr int kBlockMaxRows = 32;
// Scale rows are staged for at most this many groups per split.
constexpr int kBlockMaxGroups = 160;
// Whether a wave's accumulators (tiles x projections x row tiles f32x4, and as many MFMA
// results) leave room for its load ring in 256 registers.
__host__ __device__ constexpr bool block_fits_registers(int tiles, int nproj, int row_tiles) {
  return tiles * nproj * row_tiles <= 12;
}
// 16-column tiles of a block of `cols` columns.
__host__ __device__ constexpr int block_tiles(int cols) { return (cols + 15) / 16; }
// 32-bit words of one staged scale row covering `groups` groups (one more element for a row
// that starts on an odd element, in whole words), rounded up to a power of two of at least 4.
__host__ __device__ constexpr int block_sb_words(int groups) {
  int w = 4;
  while (w < (groups + 2) / 2) w *= 2;
  return w;
}
// Dynamic LDS of one workgroup: the staged scale and bias rows, reused after the K loop by the
// cross-wave reduction [waves][tiles][nproj][row tiles][64 lanes][4] (fp32).
__host__ __device__ constexpr uint32_t block_lds_bytes(int waves, int tiles, int nproj,
                                                       int row_tiles, int sb_words) {
  const uint32_t sb = (uint32_t)(2 * nproj * 16 * tiles * sb_words) * 4u;
  const uint32_t red = (uint32_t)(waves * tiles * nproj * row_tiles) * 1024u;
  return sb > red ? sb : red;
}
constexpr uint32_t kBlockMaxLds = 160u * 1024u - 256u;
hipError_t launch_affine_block(const QmvParams& p, int bits, int dtype, int nproj, int waves,
                               int tiles, hipStream_t stream);


// ---- 4x4x4-MFMA GEMV kernel (M <= 4, 4-bit codes, groups of 32 or more) ----------------------
// A workgroup owns `cg` groups of 4 columns (of each projection; cg 1, 2 or 4) and all of K
// (grid N / (4 cg)); its `waves` waves take consecutive runs of 512-wide K rounds, at most four
// rounds each, and a wave's loads of all its rounds stay in flight together (below the 64 loads
// a wave can count).
constexpr int kGemv4MaxWaves = 8;
__host__ __device__ constexpr int gemv4_loads_per_round(int nproj, int cg) {
  return 4 + 3 * nproj * cg;
}
__host__ __device__ constexpr bool affine_gemv4_fits(int K, int waves, int nproj, int cg) {
  return waves >= 1 && waves <= kGemv4MaxWaves && (cg == 1 || cg == 2 || cg == 4) &&
         waves <= (K + 511) / 512 && ((K + 511) / 512 + waves - 1) / waves <= 4 &&
         ((K + 511) / 512 + waves - 1) / waves * gemv4_loads_per_round(nproj, cg) < 64;
}
hipError_t launch_affine_gemv4(const QmvParams& p, int dtype, int nproj, int waves, int cg,
                               hipStream_t stream);

hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                    float* out, int N, int K, int G, int bits, int dtype,
                                    hipStream_t stream);

}  // namespace mt

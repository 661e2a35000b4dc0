// Host-visible launch interface of the prefill affine GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mt {

struct GemmParams {
  const uint16_t* x;   // [M, K] activations
  const uint32_t* w;   // [N, K/8] packed 4-bit codes
  const uint16_t* s;   // [N, K/G] scales
  const uint16_t* b;   // [N, K/G] biases
  uint16_t* y;         // [M, N] output
  float* partial;      // split-K partial sums: [ksplit][M][N] (register-staged kernel) or
                       // [ksplit][tile][128 x tile_n] in register layout (ring kernel)
  uint32_t* counters;  // one per output tile, zero between calls
  int M, K, N, G;
  int tile;            // register-staged kernel: 2: 128 x 128 output tiles, 1: 64 x 64
  int tile_n;          // ring kernel: output tiles of 128 x tile_n (64, 96, 128, 160, 192, 256)
  int ksplit;
  int steps_per_split;
  int sb_words;        // ring kernel: dwords of scales (and of biases) staged per column
  int order;           // ring kernel: 0 grid order; 1, 2: each XCD a contiguous run of tiles,
                       // column tiles (1) or row blocks (2) fastest
};

// Register-staged kernel (affine_gemm.hip).
hipError_t launch_affine_gemm(const GemmParams& p, int dtype, hipStream_t stream);

// Ring kernel (affine_gemm_ring.hip): G a power of two of 64 or more, N a multiple of 8,
// steps_per_split a multiple of 3, ksplit <= kGemmMaxSplits, and the LDS of
// gemm_ring_static_lds + gemm_ring_dynamic_lds within kGemmRingLdsBytes.
hipError_t launch_affine_gemm_ring(const GemmParams& p, int dtype, hipStream_t stream);

constexpr int kGemmMaxSplits = 8;
constexpr size_t kGemmRingLdsBytes = 160 * 1024;  // LDS of a gfx950 CU

// Workgroup waves of the ring kernel at a tile width: eight (four along N) for 128, 192 and 256,
// else four.
constexpr int gemm_ring_waves(int tile_n) {
  return tile_n == 128 || tile_n == 192 || tile_n == 256 ? 8 : 4;
}

// One code stage of the ring kernel: 32 bytes per column, plus a spare kilobyte when the waves do
// not share the 1 KiB code loads evenly.
constexpr int gemm_ring_code_stage(int tile_n, int waves) {
  return tile_n * 32 + ((tile_n / 32) % waves ? 1024 : 0);
}

// Static LDS of the ring kernel: three activation stages of 16 KiB and three code stages.
constexpr size_t gemm_ring_static_lds(int tile_n) {
  return 3 * (size_t)(128 * 128) +
         3 * (size_t)gemm_ring_code_stage(tile_n, gemm_ring_waves(tile_n)) + 16;
}

// Dynamic LDS: the staged scales and biases (sb_words dwords each per column), or the output
// tile of 16-bit values, whichever is larger.
constexpr size_t gemm_ring_dynamic_lds(int tile_n, int sb_words) {
  const size_t sb = (size_t)2 * tile_n * sb_words * 4;
  const size_t out = (size_t)128 * tile_n * 2;
  return sb > out ? sb : out;
}

}  // namespace mt

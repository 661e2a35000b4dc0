// Host-visible launch interface of the prefill affine GEMM.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

struct GemmParams {
  const uint16_t* x;   // [M, K] activations
  const uint32_t* w;   // [N, K/8] packed 4-bit codes
  const uint16_t* s;   // [N, K/G] scales
  const uint16_t* b;   // [N, K/G] biases
  uint16_t* y;         // [M, N] output
  float* partial;      // [ksplit][M][N] split-K partial sums
  uint32_t* counters;  // one per output tile, zero between calls
  int M, K, N, G;
  int tile;            // 2: 128 x 128 output tiles, 1: 64 x 64
  int ksplit;
  int steps_per_split;
};

hipError_t launch_affine_gemm(const GemmParams& p, int dtype, hipStream_t stream);

}  // namespace mt

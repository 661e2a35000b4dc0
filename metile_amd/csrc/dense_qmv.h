// Host-visible launch interface of the dense 16-bit small-batch projection kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

struct DenseParams {
  const uint16_t* x;         // [M, K] activations (M <= 128 per launch)
  const uint16_t* w[2];      // [N, K] weights (gate, up for SwiGLU)
  const uint16_t* residual;  // [M, N] or null (single projection only)
  uint16_t* y;               // [M, N] output
  float* partial;            // [chunks][ksplit][nproj][row_chunk or M][N] split-K partial sums
  uint32_t* counters;        // [chunks][N/32] split-K arrival counters, zero between calls
  int M, K, N;
  int ksplit;
  int steps_per_split;
  int row_chunk;             // rows per grid z index (rows [z row_chunk, ...) of this launch,
                             // each with its own partials and counters); 0: one chunk of M rows
};

hipError_t launch_dense_qmv(const DenseParams& p, int dtype, int nproj, hipStream_t stream);

}  // namespace mt

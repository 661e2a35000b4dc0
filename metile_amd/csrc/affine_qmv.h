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
};

hipError_t launch_affine_qmv(const QmvParams& p, int bits, int dtype, int nproj,
                             hipStream_t stream);

hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                    float* out, int N, int K, int G, int bits, int dtype,
                                    hipStream_t stream);

}  // namespace mt

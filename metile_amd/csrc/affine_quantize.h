// Host-visible launch interface of the affine group quantizer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

// Dense 16-bit weights [N, K] -> MLX affine codes [N, K * bits / 32], scales and biases
// [N, K / G] in the weights' type (see affine_quantize.hip for the algorithm).
hipError_t launch_affine_quantize(const uint16_t* w, uint32_t* w_q, uint16_t* scales,
                                  uint16_t* biases, int N, int K, int G, int bits, int dtype,
                                  hipStream_t stream);

}  // namespace mt

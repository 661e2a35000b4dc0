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

// ---- activation-staged small-row variant (M <= 16) -------------------------------------
// Eight waves per workgroup; the workgroup's activation rows for its K range live in LDS.
constexpr int kQmvLdsWaves = 8;
constexpr int kQmvLdsMaxRows = 16;

// 16-byte activation chunks each thread stages (M * steps_per_split * 8 chunks in all).
__host__ __device__ constexpr int qmv_lds_chunk_iters(int mrows) { return mrows <= 8 ? 5 : 8; }

// Dynamic LDS of one workgroup, in bytes: activation rows [M + 1][steps_per_split * 64 + 8]
// (row M is all zeros and stands in for rows M..31 of the MFMA tile), per-step row sums
// [steps_per_split][mrows] (fp32). The cross-wave reduction buffer [waves][nproj][mrows][33]
// (fp32) reuses the same space after the K loop.
struct QmvLdsLayout {
  uint32_t zero;
  uint32_t xsum;
  uint32_t bytes;
};

__host__ __device__ inline QmvLdsLayout qmv_lds_layout(int M, int steps_per_split, int mrows,
                                                       int nproj) {
  QmvLdsLayout l;
  const uint32_t row = (uint32_t)(steps_per_split * 64 + 8) * 2u;
  l.zero = (uint32_t)M * row;
  l.xsum = l.zero + row;
  const uint32_t staged = l.xsum + (uint32_t)(steps_per_split * mrows) * 4u;
  const uint32_t red = (uint32_t)(kQmvLdsWaves * nproj * mrows * 33) * 4u;
  l.bytes = staged > red ? staged : red;
  return l;
}

// Whether the activation-staged variant takes a call of M rows split into K ranges of
// steps_per_split 64-wide steps (its staging must fit in the per-thread chunk budget and in
// 64 KiB of dynamic LDS).
bool affine_qmv_lds_fits(int M, int steps_per_split, int nproj);

hipError_t launch_affine_qmv_lds(const QmvParams& p, int bits, int dtype, int nproj,
                                 hipStream_t stream);

hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                    float* out, int N, int K, int G, int bits, int dtype,
                                    hipStream_t stream);

}  // namespace mt

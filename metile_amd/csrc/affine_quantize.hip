// Affine group quantization of dense 16-bit weights into MLX's packed format, for gfx950.
//
// Restates the published algorithm of MLX's affine quantize (mlx.core.quantize with
// mode="affine", mlx 0.32; the call sites are metile/backends/mlx_compressed_down.py:41-48 and
// the tests of metile/backends): per group of G consecutive elements of a row, with
// n = 2^bits - 1 and all arithmetic in fp32,
//   scale = max((max - min) / n, 1e-7), negated unless |min| > |max|;
//   edge  = min if |min| > |max| else max  (the extreme of larger magnitude);
//   q0    = rint(edge / scale); if q0 != 0: scale = edge / q0, bias = edge; else bias = 0,
// so the edge value maps to a code exactly. Scale and bias are rounded to the weights' 16-bit
// type; codes are rint((w - bias) / scale) with those rounded values, clamped to [0, n], and
// packed low bits first (code k of a row in word k / (32 / bits)).
#include "common.h"
#include "affine_quantize.h"

namespace mt {

namespace {

// One thread per (row, group).
template <int BITS, int DT>
__global__ __launch_bounds__(256) void affine_quantize_kernel(const uint16_t* __restrict__ w,
                                                              uint32_t* __restrict__ w_q,
                                                              uint16_t* __restrict__ scales,
                                                              uint16_t* __restrict__ biases,
                                                              int N, int K, int G) {
  constexpr int kPer = 32 / BITS;
  constexpr float kBins = (float)((1 << BITS) - 1);
  const int groups = K / G;
  const size_t total = (size_t)N * groups;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const int n = (int)(t / groups);
    const int g = (int)(t - (size_t)n * groups);
    const uint16_t* src = w + (size_t)n * K + (size_t)g * G;
    float w_max = act_to_f32<DT>(src[0]), w_min = w_max;
    for (int e = 1; e < G; ++e) {
      const float v = act_to_f32<DT>(src[e]);
      w_max = fmaxf(w_max, v);
      w_min = fminf(w_min, v);
    }
    const bool low_edge = fabsf(w_min) > fabsf(w_max);
    float scale = fmaxf((w_max - w_min) / kBins, 1e-7f);
    if (!low_edge) scale = -scale;
    const float edge = low_edge ? w_min : w_max;
    const float q0 = rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
      scale = edge / q0;
      bias = edge;
    }
    const uint16_t s16 = f32_to_act<DT>(scale);
    const uint16_t b16 = f32_to_act<DT>(bias);
    scales[t] = s16;
    biases[t] = b16;
    const float s = act_to_f32<DT>(s16);
    const float b = act_to_f32<DT>(b16);
    uint32_t* dst = w_q + ((size_t)n * K + (size_t)g * G) / kPer;
    for (int wd = 0; wd < G / kPer; ++wd) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const float v = act_to_f32<DT>(src[wd * kPer + e]);
        const float q = fminf(fmaxf(rintf((v - b) / s), 0.0f), kBins);
        word |= (uint32_t)q << (e * BITS);
      }
      dst[wd] = word;
    }
  }
}

}  // namespace

hipError_t launch_affine_quantize(const uint16_t* w, uint32_t* w_q, uint16_t* scales,
                                  uint16_t* biases, int N, int K, int G, int bits, int dtype,
                                  hipStream_t stream) {
  const size_t total = (size_t)N * (K / G);
  const size_t want = (total + 255) / 256;
  const int blocks = (int)(want < 8192 ? want : 8192);
  if (blocks == 0) return hipSuccess;
  auto kernel = bits == 4 ? (dtype == kBF16 ? affine_quantize_kernel<4, kBF16>
                                            : affine_quantize_kernel<4, kF16>)
                          : (dtype == kBF16 ? affine_quantize_kernel<8, kBF16>
                                            : affine_quantize_kernel<8, kF16>);
  kernel<<<blocks, 256, 0, stream>>>(w, w_q, scales, biases, N, K, G);
  return hipGetLastError();
}

}  // namespace mt

// Small-row affine quantized projection (M = 1..32) for gfx950.
//
// Computes y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/G] + b[n, k/G]) for MLX affine packed
// weights (reference semantics: kernels/affine_qmv.py:4-54 and the residual / SwiGLU epilogues
// of kernels/affine_qmv.py:124-132,204-214), reading every packed weight byte from HBM once
// per dispatch whatever the row count.
//
// Design (wave64, MFMA 32x32x16):
//  * A workgroup owns a strip of 32 output columns (32 gate + 32 up columns for SwiGLU) and a
//    contiguous range of 64-wide K steps; its four waves split that range.
//  * Per K step a lane (j, h) = (lane % 32, lane / 32) loads 32 consecutive K of column j
//    (16 B of 4-bit codes or 32 B of 8-bit codes) and 32 consecutive activations of row j.
//    Codes are turned into exact 16-bit floats (offset + q) in registers and multiplied by the
//    activations on the matrix cores; rows >= M read as zero (buffer range check).
//  * The per-group affine terms are applied to each step's fp32 MFMA result:
//      acc += s * sum_k x_k (offset + q_k) + (b - offset * s) * sum_k x_k,
//    which equals sum_k x_k (q_k s + b) exactly in real arithmetic. The per-row activation
//    sums of each step are computed once per workgroup into LDS.
//  * Cross-wave partials are reduced in LDS in a fixed order. When K is split across
//    workgroups, fp32 partials go to a caller-provided workspace and the last workgroup of a
//    strip (detected with a device-scope counter that it resets) sums them in split order and
//    runs the epilogue, so results are deterministic.
#include "common.h"
#include "affine_qmv.h"

namespace mt {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kUnroll = 4;  // K steps in flight per wave

template <int BITS, int DT, int MROWS, int NPROJ>
__global__ __launch_bounds__(kThreads) void affine_qmv_kernel(const QmvParams p) {
  constexpr int kRegs = MROWS / 2;                  // valid accumulator registers per lane
  constexpr int kWV = (BITS == 4) ? 1 : 2;          // 16-byte weight vectors per lane per step
  constexpr float kOff = CodeOffset<BITS, DT>::value;

  __shared__ __attribute__((aligned(16))) float xsum[kMaxStepsPerSplit][MROWS];
  __shared__ float red[kWaves][NPROJ][MROWS][33];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = lane & 31;
  const int h = lane >> 5;
  const int strip = blockIdx.x;
  const int split = blockIdx.y;
  const int M = p.M, K = p.K, N = p.N;
  const int col = strip * 32 + j;
  const int steps_total = K >> 6;
  const int s_beg = split * p.steps_per_split;
  const int s_end = min(steps_total, s_beg + p.steps_per_split);
  const int ns = s_end - s_beg;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2u);

  // ---- per-row activation sums of every K step of this split --------------------------
  for (int pp = tid; pp < ns * MROWS; pp += kThreads) {
    const int sl = pp / MROWS;
    const int m = pp - sl * MROWS;
    float acc = 0.0f;
    if (m < M) {
      const uint32_t base = ((uint32_t)m * K + (uint32_t)(s_beg + sl) * 64u) * 2u;
#pragma unroll
      for (int v = 0; v < 8; ++v) acc = sum8<DT>(load16(rx, base + 16u * v), acc);
    }
    xsum[sl][m] = acc;
  }
  __syncthreads();

  // ---- main loop --------------------------------------------------------------------------
  const int per_wave = (ns + kWaves - 1) / kWaves;
  const int w_beg = s_beg + wave * per_wave;
  const int w_end = min(s_end, w_beg + per_wave);

  const int words_per_row = K * BITS / 32;
  const int groups_per_row = K / p.G;
  __amdgpu_buffer_rsrc_t rw[NPROJ], rs[NPROJ], rb[NPROJ];
#pragma unroll
  for (int q = 0; q < NPROJ; ++q) {
    rw[q] = make_rsrc(p.w[q], (uint32_t)N * words_per_row * 4u);
    rs[q] = make_rsrc(p.s[q], (uint32_t)N * groups_per_row * 2u);
    rb[q] = make_rsrc(p.b[q], (uint32_t)N * groups_per_row * 2u);
  }
  const uint32_t w_row = (uint32_t)col * words_per_row * 4u;       // byte offset of the row
  const uint32_t g_row = (uint32_t)col * groups_per_row * 2u;
  const uint32_t x_row = (j < M) ? (uint32_t)j * K * 2u : kOOB;
  const int steps_per_group = p.G >> 6;

  f32x16 acc[NPROJ];
#pragma unroll
  for (int q = 0; q < NPROJ; ++q) acc[q] = (f32x16){0};

  for (int s0 = w_beg; s0 < w_end; s0 += kUnroll) {
    u32x4 wv[kUnroll][NPROJ][kWV];
    uint32_t sv[kUnroll][NPROJ], bv[kUnroll][NPROJ];
    u32x4 xa[kUnroll][4];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int st = s0 + u;
      const bool ok = st < w_end;
      // 32 K of this lane's half-step: byte offset (64*st + 32*h) * BITS / 8.
      const uint32_t woff = ok ? w_row + (uint32_t)(st * 64 + 32 * h) * BITS / 8u : kOOB;
      const uint32_t goff = ok ? g_row + (uint32_t)(st / steps_per_group) * 2u : kOOB;
#pragma unroll
      for (int q = 0; q < NPROJ; ++q) {
#pragma unroll
        for (int v = 0; v < kWV; ++v) wv[u][q][v] = load16(rw[q], woff + 16u * v);
        sv[u][q] = load2(rs[q], goff);
        bv[u][q] = load2(rb[q], goff);
      }
      const uint32_t xoff = (ok && x_row != kOOB) ? x_row + (uint32_t)(st * 64 + 32 * h) * 2u
                                                  : kOOB;
#pragma unroll
      for (int e = 0; e < 4; ++e) xa[u][e] = load16(rx, xoff == kOOB ? kOOB : xoff + 16u * e);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int sl = s0 + u - s_beg;
      float xs[kRegs];
      if (s0 + u < w_end) {
#pragma unroll
        for (int r4 = 0; r4 < kRegs / 4; ++r4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(&xsum[sl][8 * r4 + 4 * h]);
          xs[4 * r4 + 0] = v.x;
          xs[4 * r4 + 1] = v.y;
          xs[4 * r4 + 2] = v.z;
          xs[4 * r4 + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int r = 0; r < kRegs; ++r) xs[r] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < NPROJ; ++q) {
        f32x16 t = (f32x16){0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          u32x4 bfrag;
          if constexpr (BITS == 4) {
            const uint32_t word = (e == 0)   ? wv[u][q][0].x
                                  : (e == 1) ? wv[u][q][0].y
                                  : (e == 2) ? wv[u][q][0].z
                                             : wv[u][q][0].w;
            bfrag = unpack_u4<DT>(word);
          } else {
            const u32x4 src = wv[u][q][e >> 1];
            const uint32_t w0 = (e & 1) ? src.z : src.x;
            const uint32_t w1 = (e & 1) ? src.w : src.y;
            const u32x2 lo = unpack_u8<DT>(w0);
            const u32x2 hi = unpack_u8<DT>(w1);
            bfrag = (u32x4){lo.x, lo.y, hi.x, hi.y};
          }
          t = mfma32<DT>(xa[u][e], bfrag, t);
        }
        const float sf = act_to_f32<DT>(sv[u][q]);
        const float bf = act_to_f32<DT>(bv[u][q]);
        const float bp = __builtin_fmaf(-kOff, sf, bf);
#pragma unroll
        for (int r = 0; r < kRegs; ++r) {
          acc[q][r] = __builtin_fmaf(sf, t[r], acc[q][r]);
          acc[q][r] = __builtin_fmaf(bp, xs[r], acc[q][r]);
        }
      }
    }
  }

  // ---- cross-wave reduction (fixed order) --------------------------------------------------
#pragma unroll
  for (int q = 0; q < NPROJ; ++q) {
#pragma unroll
    for (int r = 0; r < kRegs; ++r) red[wave][q][mfma32_row(r, h)][j] = acc[q][r];
  }
  __syncthreads();

  const int outs = M * 32;
  if (p.ksplit == 1) {
    for (int o = tid; o < outs; o += kThreads) {
      const int i = o >> 5, c = o & 31;
      float v[NPROJ];
#pragma unroll
      for (int q = 0; q < NPROJ; ++q)
        v[q] = ((red[0][q][i][c] + red[1][q][i][c]) + red[2][q][i][c]) + red[3][q][i][c];
      const size_t oi = (size_t)i * N + strip * 32 + c;
      float out;
      if constexpr (NPROJ == 2) {
        out = silu_mul(v[0], v[1]);
      } else {
        out = v[0];
        if (p.residual) out += act_to_f32<DT>(p.residual[oi]);
      }
      p.y[oi] = f32_to_act<DT>(out);
    }
    return;
  }

  // ---- split-K: publish partials, last workgroup of the strip finishes -------------------
  // Partials are written and read with device-scope relaxed atomic accesses, which the gfx950
  // memory model makes coherent across the chip's L2 slices without any cache-wide writeback
  // or invalidate. Each wave waits for its stores to complete before the barrier, so every
  // partial of this workgroup is visible before the arrival counter moves.
  const size_t plane = (size_t)M * N;
  for (int o = tid; o < outs; o += kThreads) {
    const int i = o >> 5, c = o & 31;
#pragma unroll
    for (int q = 0; q < NPROJ; ++q) {
      const float v = ((red[0][q][i][c] + red[1][q][i][c]) + red[2][q][i][c]) + red[3][q][i][c];
      __hip_atomic_store(&p.partial[(size_t)(split * NPROJ + q) * plane + (size_t)i * N +
                                    strip * 32 + c],
                         v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&p.counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (prev == (unsigned)(p.ksplit - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  for (int o = tid; o < outs; o += kThreads) {
    const int i = o >> 5, c = o & 31;
    const size_t oi = (size_t)i * N + strip * 32 + c;
    float v[NPROJ];
#pragma unroll
    for (int q = 0; q < NPROJ; ++q) {
      float sacc = 0.0f;
      for (int sp = 0; sp < p.ksplit; ++sp)
        sacc += __hip_atomic_load(&p.partial[(size_t)(sp * NPROJ + q) * plane + oi],
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[q] = sacc;
    }
    float out;
    if constexpr (NPROJ == 2) {
      out = silu_mul(v[0], v[1]);
    } else {
      out = v[0];
      if (p.residual) out += act_to_f32<DT>(p.residual[oi]);
    }
    p.y[oi] = f32_to_act<DT>(out);
  }
  if (tid == 0)
    __hip_atomic_store(&p.counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int BITS, int DT, int NPROJ>
hipError_t launch_rows(const QmvParams& p, hipStream_t stream) {
  const dim3 grid(p.N / 32, p.ksplit);
  const dim3 block(kThreads);
  if (p.M <= 8) {
    affine_qmv_kernel<BITS, DT, 8, NPROJ><<<grid, block, 0, stream>>>(p);
  } else if (p.M <= 16) {
    affine_qmv_kernel<BITS, DT, 16, NPROJ><<<grid, block, 0, stream>>>(p);
  } else {
    affine_qmv_kernel<BITS, DT, 32, NPROJ><<<grid, block, 0, stream>>>(p);
  }
  return hipGetLastError();
}

template <int BITS, int DT>
hipError_t launch_bits_dt(const QmvParams& p, int nproj, hipStream_t stream) {
  return nproj == 2 ? launch_rows<BITS, DT, 2>(p, stream) : launch_rows<BITS, DT, 1>(p, stream);
}

}  // namespace

hipError_t launch_affine_qmv(const QmvParams& p, int bits, int dtype, int nproj,
                             hipStream_t stream) {
  if (bits == 4) {
    return dtype == kBF16 ? launch_bits_dt<4, kBF16>(p, nproj, stream)
                          : launch_bits_dt<4, kF16>(p, nproj, stream);
  }
  return dtype == kBF16 ? launch_bits_dt<8, kBF16>(p, nproj, stream)
                        : launch_bits_dt<8, kF16>(p, nproj, stream);
}

// ---- dequantize (bit-exact fp32) --------------------------------------------------------

namespace {

template <int BITS, int DT>
__global__ __launch_bounds__(256) void affine_dequantize_kernel(const uint32_t* __restrict__ w,
                                                                const uint16_t* __restrict__ s,
                                                                const uint16_t* __restrict__ b,
                                                                float* __restrict__ out, int N,
                                                                int K, int G) {
  constexpr int kPer = 32 / BITS;
  const int words_per_row = K / kPer;
  const size_t total = (size_t)N * words_per_row;
  for (size_t wi = (size_t)blockIdx.x * blockDim.x + threadIdx.x; wi < total;
       wi += (size_t)gridDim.x * blockDim.x) {
    const int n = (int)(wi / words_per_row);
    const int kw = (int)(wi - (size_t)n * words_per_row);
    const uint32_t word = w[wi];
    const int k0 = kw * kPer;
    const size_t gi = (size_t)n * (K / G) + k0 / G;
    const float sf = act_to_f32<DT>(s[gi]);
    const float bf = act_to_f32<DT>(b[gi]);
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const float q = (float)((word >> (e * BITS)) & ((1u << BITS) - 1u));
      out[(size_t)n * K + k0 + e] = __builtin_fmaf(q, sf, bf);
    }
  }
}

}  // namespace

hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                    float* out, int N, int K, int G, int bits, int dtype,
                                    hipStream_t stream) {
  const size_t words = (size_t)N * K * bits / 32;
  const int blocks = (int)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
  if (blocks == 0) return hipSuccess;
  if (bits == 4) {
    if (dtype == kBF16)
      affine_dequantize_kernel<4, kBF16><<<blocks, 256, 0, stream>>>(w, s, b, out, N, K, G);
    else
      affine_dequantize_kernel<4, kF16><<<blocks, 256, 0, stream>>>(w, s, b, out, N, K, G);
  } else {
    if (dtype == kBF16)
      affine_dequantize_kernel<8, kBF16><<<blocks, 256, 0, stream>>>(w, s, b, out, N, K, G);
    else
      affine_dequantize_kernel<8, kF16><<<blocks, 256, 0, stream>>>(w, s, b, out, N, K, G);
  }
  return hipGetLastError();
}

}  // namespace mt

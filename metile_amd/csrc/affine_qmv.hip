// Small-row affine quantized projection (M = 1..32) for gfx950.
//
// Computes y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/G] + b[n, k/G]) for MLX affine packed
// weights (reference semantics: kernels/affine_qmv.py:4-54 and the residual / SwiGLU epilogues
// of kernels/affine_qmv.py:124-132,204-214), reading every packed weight byte from HBM once
// per dispatch whatever the row count.
//
// Design (wave64, MFMA 32x32x16, streaming):
//  * A workgroup owns a strip of 32 output columns (for SwiGLU the same 32 gate and 32 up
//    columns) and a range of 64-wide K steps; its four waves split the range into contiguous
//    sub-ranges.
//  * Per K step a lane (j, h) = (lane % 32, lane / 32) needs 32 consecutive K of column j
//    (one 16-byte load of 4-bit codes, two of 8-bit codes; the two halves of a wave read the
//    step's 32 or 64 contiguous bytes of each column) and 32 consecutive activations of row j.
//    One step's loads form a pipeline stage; each wave keeps kStages stages in flight in
//    registers and refills a stage as soon as it is consumed. A stage's loads are issued
//    together, so waiting for one stage never waits for a later one (vector loads complete in
//    issue order).
//  * The group scales and biases of the workgroup's strip and K range are staged once into LDS
//    with coalesced loads (issued before the weight prefetch) and read from there per step.
//  * Codes are turned into exact 16-bit floats (offset + q) in registers and multiplied by the
//    activations on the matrix cores. The per-group affine terms are applied to each step's
//    fp32 MFMA result:  acc += s * sum_k x_k (offset + q_k) + (b - offset * s) * sum_k x_k.
//    The per-row activation sums come from four more MFMAs of the same activations against a
//    matrix of ones, which lands them in the accumulator layout directly.
//  * Rows >= M and steps past the range read as zero through the buffer range check.
//  * Cross-wave partials are reduced in LDS in a fixed order. When K is split across
//    workgroups, fp32 partials go to a caller-provided workspace and the last workgroup of a
//    strip (detected with a device-scope counter that it resets) sums them in split order and
//    runs the epilogue, so results are deterministic.
#include "common.h"
#include "affine_qmv.h"

namespace mt {

namespace {

template <int DT>
__device__ __forceinline__ u32x4 ones8() {
  constexpr uint32_t one2 = (DT == kBF16) ? 0x3F803F80u : 0x3C003C00u;
  return (u32x4){one2, one2, one2, one2};
}

// One pipeline stage: the codes (16 B per 32 K of 4-bit, 32 B of 8-bit) of every projection
// and the four 16-byte activation fragments of one K step.
template <int BITS, int NPROJ>
struct Stage {
  u32x4 w[NPROJ][BITS / 4];
  u32x4 x[4];
};


template <int BITS, int DT, int MROWS, int NPROJ, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void affine_qmv_kernel(const QmvParams args) {
  const QmvParams p = preload_args(args);  // all arguments in one batch of scalar loads
  constexpr int kThreads = WAVES * 64;
  constexpr float kOff = SumOffset<BITS, DT>::value;
  constexpr int kRegs = MROWS / 2;  // accumulator registers holding rows < MROWS
  constexpr int kArrays = 2 * NPROJ;  // scales and biases of each projection

  __shared__ float red[WAVES][NPROJ][MROWS][33];
  __shared__ uint32_t sb[kArrays][32][kSbRowWords];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;
  const int h = lane >> 5;
  const int strip = blockIdx.x;
  const int split = blockIdx.y;
  const int M = p.M, K = p.K, N = p.N;
  const int steps_total = K >> 6;
  const int s_beg = split * p.steps_per_split;
  const int s_end = min(steps_total, s_beg + p.steps_per_split);
  const int per_wave = (s_end - s_beg + WAVES - 1) / WAVES;
  const int w_beg = s_beg + wave * per_wave;
  const int w_end = min(s_end, w_beg + per_wave);
  const int gshift = p.group_shift;  // log2(G / 64)
  // Scale rows are staged from the 32-bit word holding group g_beg; a row whose element
  // index (row * groups_per_row + g_beg) is odd starts one 16-bit element into its segment.
  const int g_beg = s_beg >> gshift;
  const int g_last = (s_end - 1) >> gshift;
  const int nwords = (g_last - g_beg + 1) / 2 + 1;  // 32-bit words per staged row segment

  const uint32_t row_bytes = (uint32_t)K * BITS / 8u;
  const int groups_per_row = p.groups_per_row;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr) rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * row_bytes);

  // ---- scales and biases of this strip and K range: issued first, parked in LDS below -----
  // For each array (unrolled, so the buffer descriptor stays wave-uniform) thread t copies
  // 16-byte quads q = t / 32 + k * (kThreads / 32) of row t % 32.
  constexpr int kQuadsPerRow = (kSbRowWords + 3) / 4;
  constexpr int kSbIters = (kQuadsPerRow + kThreads / 32 - 1) / (kThreads / 32);
  const int sb_row = tid & 31;
  const int sb_q0 = tid >> 5;
  u32x4 sbv[kArrays][kSbIters];
#pragma unroll
  for (int a = 0; a < kArrays; ++a) {
    const uint16_t* src = (a & 1) ? p.b[a >> 1] : p.s[a >> 1];
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (uint32_t)N * groups_per_row * 2u);
    const uint32_t base = (((uint32_t)(strip * 32 + sb_row) * groups_per_row + g_beg) * 2u) & ~3u;
#pragma unroll
    for (int k = 0; k < kSbIters; ++k) {
      const int q = sb_q0 + k * (kThreads / 32);
      sbv[a][k] = load16(r, 4 * q < nwords ? base + 16u * q : kOOB);
    }
  }

  // ---- weight and activation pipeline ----------------------------------------------------
  const uint32_t w_row = (uint32_t)(strip * 32 + j) * p.col_stride + (uint32_t)h * 4u * BITS;
  const uint32_t x_row = j < M ? ((uint32_t)j * K + 32u * h) * 2u : kOOB;

  Stage<BITS, NPROJ> ring[STAGES];
  // Steps past this wave's range load nothing (range-checked offsets), so the refills below
  // need no branch and every wait stays exact.
  auto load_stage = [&](Stage<BITS, NPROJ>& S, int st) {
    const bool ok = st < w_end;
    const uint32_t woff = ok ? w_row + (uint32_t)st * p.step_stride : kOOB;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int v = 0; v < BITS / 4; ++v)
        S.w[pr][v] = load16_nt(rw[pr], ok ? woff + 16u * v : kOOB);
    const bool xok = ok && x_row != kOOB;
    const uint32_t xoff = x_row + (uint32_t)st * 128u;
#pragma unroll
    for (int e = 0; e < 4; ++e) S.x[e] = load16(rx, xok ? xoff + 16u * e : kOOB);
  };
#pragma unroll
  for (int d = 0; d < STAGES; ++d) load_stage(ring[d], w_beg + d);

#pragma unroll
  for (int a = 0; a < kArrays; ++a)
#pragma unroll
    for (int k = 0; k < kSbIters; ++k) {
      const int q = sb_q0 + k * (kThreads / 32);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (4 * q + c < kSbRowWords) sb[a][sb_row][4 * q + c] = sbv[a][k][c];
    }
  __syncthreads();

  float acc[NPROJ][kRegs];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int r = 0; r < kRegs; ++r) acc[pr][r] = 0.0f;

  const u32x4 ones = ones8<DT>();
  const f32x16 zero16 = (f32x16){0};
  const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(&sb[0][0][0]);
  const int sb_shift = ((strip * 32 + j) * groups_per_row + g_beg) & 1;
  for (int s0 = w_beg; s0 < w_end; s0 += STAGES) {
#pragma unroll
    for (int d = 0; d < STAGES; ++d) {
      Stage<BITS, NPROJ>& S = ring[d];
      const int st = s0 + d;
      if (st < w_end) {
        f32x16 xs = mfma32<DT>(S.x[0], ones, zero16);
#pragma unroll
        for (int e = 1; e < 4; ++e) xs = mfma32<DT>(S.x[e], ones, xs);
        const int gl = (st >> gshift) - g_beg + sb_shift;
#pragma unroll
        for (int pr = 0; pr < NPROJ; ++pr) {
          f32x16 t = mfma32<DT>(S.x[0], codes_for_sum<DT>(code_frag<BITS, DT>(S.w[pr], 0)), zero16);
#pragma unroll
          for (int e = 1; e < 4; ++e)
            t = mfma32<DT>(S.x[e], codes_for_sum<DT>(code_frag<BITS, DT>(S.w[pr], e)), t);
          const float sf = act_to_f32<DT>(sb16[((2 * pr) * 32 + j) * 2 * kSbRowWords + gl]);
          const float bf = act_to_f32<DT>(sb16[((2 * pr + 1) * 32 + j) * 2 * kSbRowWords + gl]);
          const float bp = __builtin_fmaf(-kOff, sf, bf);
#pragma unroll
          for (int r = 0; r < kRegs; ++r) {
            acc[pr][r] = __builtin_fmaf(sf, t[r], acc[pr][r]);
            acc[pr][r] = __builtin_fmaf(bp, xs[r], acc[pr][r]);
          }
        }
      }
      load_stage(S, st + STAGES);
    }
  }

  // ---- cross-wave reduction (fixed order) --------------------------------------------------
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int r = 0; r < kRegs; ++r) red[wave][pr][mfma32_row(r, h)][j] = acc[pr][r];
  __syncthreads();

  auto reduce = [&](int pr, int i, int c) {
    float v = red[0][pr][i][c];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[w][pr][i][c];
    return v;
  };

  const int outs = M * 32;
  if (p.ksplit == 1) {
    for (int o = tid; o < outs; o += kThreads) {
      const int i = o >> 5, c = o & 31;
      float v[NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) v[pr] = reduce(pr, i, c);
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
    for (int pr = 0; pr < NPROJ; ++pr) {
      const float v = reduce(pr, i, c);
      __hip_atomic_store(&p.partial[(size_t)(split * NPROJ + pr) * plane + (size_t)i * N +
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
    for (int pr = 0; pr < NPROJ; ++pr) {
      v[pr] = sum_partials(p.partial + (size_t)pr * plane + oi, (size_t)NPROJ * plane, p.ksplit);
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

// Pipeline depth: as many K steps in flight per wave as fit in about 128 registers.
template <int BITS, int NPROJ, int MROWS>
constexpr int stages() {
  constexpr int per_stage = NPROJ * BITS + 16;  // registers of one stage
  constexpr int s = 128 / per_stage - (MROWS == 32 ? 1 : 0);
  return s < 2 ? 2 : s;
}

template <int BITS, int DT, int MROWS, int NPROJ>
hipError_t launch_waves(const QmvParams& p, hipStream_t stream) {
  // Four waves per workgroup, so that two or three workgroups fit on a CU and a grid of a
  // few hundred workgroups is resident at once (a workgroup that waits for a free CU doubles
  // the kernel time of a weight-streaming launch).
  constexpr int kW = 4;
  const dim3 grid(p.N / 32, p.ksplit);
  affine_qmv_kernel<BITS, DT, MROWS, NPROJ, kW, stages<BITS, NPROJ, MROWS>()>
      <<<grid, dim3(kW * 64), 0, stream>>>(p);
  return hipGetLastError();
}

template <int BITS, int DT, int NPROJ>
hipError_t launch_rows(const QmvParams& p, hipStream_t stream) {
  if (p.M <= 8) return launch_waves<BITS, DT, 8, NPROJ>(p, stream);
  if (p.M <= 16) return launch_waves<BITS, DT, 16, NPROJ>(p, stream);
  return launch_waves<BITS, DT, 32, NPROJ>(p, stream);
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

// ---- step-major repack ---------------------------------------------------------------------

namespace {

// Thread i writes 16-byte piece i of the repacked buffer: piece q of the chunk of column n and
// K step t, where chunk c = t * N + n holds `pieces` pieces.
__global__ __launch_bounds__(256) void affine_repack_kernel(const u32x4* __restrict__ w,
                                                            u32x4* __restrict__ out, int N,
                                                            int steps, int pieces) {
  const size_t total = (size_t)N * steps * pieces;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t c = i / pieces;
    const int q = (int)(i - c * pieces);
    const int t = (int)(c / N);
    const int n = (int)(c - (size_t)t * N);
    out[i] = w[((size_t)n * steps + t) * pieces + q];
  }
}

}  // namespace

hipError_t launch_affine_repack(const uint32_t* w, uint32_t* out, int N, int K, int bits,
                                hipStream_t stream) {
  const int steps = K / 64;
  const int pieces = bits / 2;  // a chunk is 8 * bits bytes
  const size_t total = (size_t)N * steps * pieces;
  const size_t want = (total + 255) / 256;
  const int blocks = (int)(want < 8192 ? want : 8192);
  if (blocks == 0) return hipSuccess;
  affine_repack_kernel<<<blocks, 256, 0, stream>>>(reinterpret_cast<const u32x4*>(w),
                                                   reinterpret_cast<u32x4*>(out), N, steps,
                                                   pieces);
  return hipGetLastError();
}

}  // namespace mt

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

// B operand of MFMA e (K slice [8e, 8e+8) of the lane's 32 K) as 8 exact 16-bit floats.
template <int BITS, int DT>
__device__ __forceinline__ u32x4 bfrag(const u32x4 (&w)[BITS / 4], int e) {
  if constexpr (BITS == 4) {
    return unpack_u4<DT>(w[0][e]);
  } else {
    const u32x4 src = w[e >> 1];
    const u32x2 lo = unpack_u8<DT>((e & 1) ? src.z : src.x);
    const u32x2 hi = unpack_u8<DT>((e & 1) ? src.w : src.y);
    return (u32x4){lo.x, lo.y, hi.x, hi.y};
  }
}

// LDS row (in 32-bit words) of one column's scales or biases over a split's groups.
constexpr int kSbRowWords = kMaxGroupsPerSplit / 2 + 2;

template <int BITS, int DT, int MROWS, int NPROJ, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void affine_qmv_kernel(const QmvParams p) {
  constexpr int kThreads = WAVES * 64;
  constexpr float kOff = CodeOffset<BITS, DT>::value;
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
  const int groups_per_row = K / p.G;
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
  const uint32_t w_row = (uint32_t)(strip * 32 + j) * row_bytes + (uint32_t)h * 4u * BITS;
  const uint32_t x_row = j < M ? ((uint32_t)j * K + 32u * h) * 2u : kOOB;

  Stage<BITS, NPROJ> ring[STAGES];
  // Steps past this wave's range load nothing (range-checked offsets), so the refills below
  // need no branch and every wait stays exact.
  auto load_stage = [&](Stage<BITS, NPROJ>& S, int st) {
    const bool ok = st < w_end;
    const uint32_t woff = ok ? w_row + (uint32_t)st * 8u * BITS : kOOB;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int v = 0; v < BITS / 4; ++v)
        S.w[pr][v] = load16(rw[pr], ok ? woff + 16u * v : kOOB);
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
          f32x16 t = mfma32<DT>(S.x[0], bfrag<BITS, DT>(S.w[pr], 0), zero16);
#pragma unroll
          for (int e = 1; e < 4; ++e) t = mfma32<DT>(S.x[e], bfrag<BITS, DT>(S.w[pr], e), t);
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
      float sacc = 0.0f;
      for (int sp = 0; sp < p.ksplit; ++sp)
        sacc += __hip_atomic_load(&p.partial[(size_t)(sp * NPROJ + pr) * plane + oi],
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[pr] = sacc;
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


// ---- activation-staged variant (M <= 16) -------------------------------------------------
// Same work split, scale staging, reduction and split-K protocol as affine_qmv_kernel. The
// differences:
//  * The workgroup's activation rows for its K range are loaded once and parked in LDS. For
//    4-bit codes each group of 8 elements is stored in the paired order (0,4,1,5,2,6,3,7), so
//    a word of codes unpacks with one AND-OR per pair of codes (unpack_u4_paired) and the MFMA
//    A operand of a K slice is one 16-byte LDS read. Lanes of rows >= M read a zero block.
//  * The per-row activation sum of every K step (the factor of the bias term) is summed once
//    while staging: eight lanes hold the eight 16-byte chunks of one (row, step) and combine
//    their sums with three lane exchanges.
//  * The register ring holds codes only, so a wave needs about half the registers of
//    affine_qmv_kernel and a workgroup runs eight waves of a few K steps each.
template <int BITS, int DT, int MROWS, int NPROJ, int STAGES>
// At most 128 registers, so that two eight-wave workgroups share a CU.
__global__ __launch_bounds__(kQmvLdsWaves * 64) __attribute__((amdgpu_waves_per_eu(4)))
void affine_qmv_lds_kernel(const QmvParams p) {
  constexpr int WAVES = kQmvLdsWaves;
  constexpr int kThreads = WAVES * 64;
  constexpr float kOff = CodeOffset<BITS, DT>::value;
  constexpr int kRegs = MROWS / 2;
  constexpr int kArrays = 2 * NPROJ;
  constexpr int kXIters = qmv_lds_chunk_iters(MROWS);

  extern __shared__ __align__(16) unsigned char dyn[];
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
  const int steps_here = s_end - s_beg;
  const int per_wave = (steps_here + WAVES - 1) / WAVES;
  const int w_beg = s_beg + wave * per_wave;
  const int w_end = min(s_end, w_beg + per_wave);
  const int gshift = p.group_shift;
  const int g_beg = s_beg >> gshift;
  const int g_last = (s_end - 1) >> gshift;
  const int nwords = (g_last - g_beg + 1) / 2 + 1;
  const QmvLdsLayout lay = qmv_lds_layout(M, p.steps_per_split, MROWS, NPROJ);
  const int xstride = p.steps_per_split * 64 + 8;  // staged row stride, elements

  const uint32_t row_bytes = (uint32_t)K * BITS / 8u;
  const int groups_per_row = K / p.G;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr) rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * row_bytes);

  // ---- scales and biases (first), then activation chunks, then the code prefetch --------
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

  // Chunk c = row * cpr + cc covers elements [8 cc, 8 cc + 8) of the row's K range.
  const int cpr = steps_here * 8;
  const int nchunks = M * cpr;
  const float inv_cpr = 1.0f / (float)cpr;
  u32x4 xv[kXIters];
#pragma unroll
  for (int i = 0; i < kXIters; ++i) {
    const int c = tid + i * kThreads;
    const int row = (int)(((float)c + 0.5f) * inv_cpr);
    const int cc = c - row * cpr;
    xv[i] = load16(rx, c < nchunks ? ((uint32_t)row * K + (uint32_t)(s_beg * 64 + cc * 8)) * 2u
                                   : kOOB);
  }

  const uint32_t w_row = (uint32_t)(strip * 32 + j) * row_bytes + (uint32_t)h * 4u * BITS;
  typedef u32x4 StageW[NPROJ][BITS / 4];
  StageW ring[STAGES];
  auto load_stage = [&](StageW& S, int st) {
    const bool ok = st < w_end;
    const uint32_t woff = ok ? w_row + (uint32_t)st * 8u * BITS : kOOB;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int v = 0; v < BITS / 4; ++v) S[pr][v] = load16(rw[pr], ok ? woff + 16u * v : kOOB);
  };
#pragma unroll
  for (int d = 0; d < STAGES; ++d) load_stage(ring[d], w_beg + d);

  // ---- park scales, biases and activations in LDS; per-step row sums ----------------------
#pragma unroll
  for (int a = 0; a < kArrays; ++a)
#pragma unroll
    for (int k = 0; k < kSbIters; ++k) {
      const int q = sb_q0 + k * (kThreads / 32);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (4 * q + c < kSbRowWords) sb[a][sb_row][4 * q + c] = sbv[a][k][c];
    }
  float* xsum = reinterpret_cast<float*>(dyn + lay.xsum);  // [steps_per_split][MROWS]
#pragma unroll
  for (int i = 0; i < kXIters; ++i) {
    const int c = tid + i * kThreads;
    // Every chunk group of 8 (one row and step) is either wholly below nchunks or wholly
    // above, so the lane exchanges below stay inside active groups.
    if (i * kThreads < nchunks) {
      const bool ok = c < nchunks;
      const int row = (int)(((float)c + 0.5f) * inv_cpr);
      const int cc = c - row * cpr;
      float s = sum8<DT>(xv[i], 0.0f);
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      if (ok) {
        const u32x4 v = (BITS == 4) ? pair_order(xv[i]) : xv[i];
        *reinterpret_cast<u32x4*>(dyn + ((uint32_t)row * xstride + cc * 8) * 2u) = v;
        if ((cc & 7) == 0) xsum[(cc >> 3) * MROWS + row] = s;
      }
    }
  }
  // Row sums of rows M..MROWS-1 and the zero row.
  for (int idx = tid; idx < steps_here * MROWS; idx += kThreads)
    if ((idx % MROWS) >= M) xsum[idx] = 0.0f;
  for (int q = tid; q < xstride / 8; q += kThreads)
    *reinterpret_cast<u32x4*>(dyn + lay.zero + 16u * q) = (u32x4){0u, 0u, 0u, 0u};
  __syncthreads();

  float acc[NPROJ][kRegs];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int r = 0; r < kRegs; ++r) acc[pr][r] = 0.0f;

  const f32x16 zero16 = (f32x16){0};
  const PairedConsts pc = paired_consts<DT>();
  const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(&sb[0][0][0]);
  const int sb_shift = ((strip * 32 + j) * groups_per_row + g_beg) & 1;
  // A operand of lane (j, h): row j (the zero row for j >= M), elements [32 h, 32 h + 32) of
  // each step's 64.
  const uint32_t a_base = ((uint32_t)min(j, M) * xstride + 32u * h) * 2u;
  for (int s0 = w_beg; s0 < w_end; s0 += STAGES) {
#pragma unroll
    for (int d = 0; d < STAGES; ++d) {
      StageW& S = ring[d];
      const int st = s0 + d;
      if (st < w_end) {
        const int sl = st - s_beg;
        const unsigned char* ap = dyn + a_base + (uint32_t)sl * 128u;
        u32x4 a[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = *reinterpret_cast<const u32x4*>(ap + 16 * e);
        float xs[kRegs];
#pragma unroll
        for (int q = 0; q < kRegs / 4; ++q) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(&xsum[sl * MROWS + 8 * q + 4 * h]);
#pragma unroll
          for (int r = 0; r < 4; ++r) xs[4 * q + r] = v[r];
        }
        const int gl = (st >> gshift) - g_beg + sb_shift;
#pragma unroll
        for (int pr = 0; pr < NPROJ; ++pr) {
          f32x16 t;
          if constexpr (BITS == 4) {
            t = mfma32<DT>(a[0], unpack_u4_paired(S[pr][0][0], pc), zero16);
#pragma unroll
            for (int e = 1; e < 4; ++e) t = mfma32<DT>(a[e], unpack_u4_paired(S[pr][0][e], pc), t);
          } else {
            t = mfma32<DT>(a[0], bfrag<BITS, DT>(S[pr], 0), zero16);
#pragma unroll
            for (int e = 1; e < 4; ++e) t = mfma32<DT>(a[e], bfrag<BITS, DT>(S[pr], e), t);
          }
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

  // ---- cross-wave reduction (fixed order); the buffer reuses the staged activations ------
  __syncthreads();
  float* red = reinterpret_cast<float*>(dyn);  // [WAVES][NPROJ][MROWS][33]
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
      red[((wave * NPROJ + pr) * MROWS + mfma32_row(r, h)) * 33 + j] = acc[pr][r];
  __syncthreads();

  auto reduce = [&](int pr, int i, int c) {
    float v = red[(pr * MROWS + i) * 33 + c];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[((w * NPROJ + pr) * MROWS + i) * 33 + c];
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

  // ---- split-K: publish partials, last workgroup of the strip finishes (as above) --------
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
      float sacc = 0.0f;
      for (int sp = 0; sp < p.ksplit; ++sp)
        sacc += __hip_atomic_load(&p.partial[(size_t)(sp * NPROJ + pr) * plane + oi],
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[pr] = sacc;
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

template <int BITS, int DT, int MROWS, int NPROJ>
hipError_t launch_lds_rows(const QmvParams& p, hipStream_t stream) {
  constexpr int kStages = BITS == 4 ? 6 : (NPROJ == 2 ? 3 : 4);
  const QmvLdsLayout lay = qmv_lds_layout(p.M, p.steps_per_split, MROWS, NPROJ);
  const dim3 grid(p.N / 32, p.ksplit);
  affine_qmv_lds_kernel<BITS, DT, MROWS, NPROJ, kStages>
      <<<grid, dim3(kQmvLdsWaves * 64), lay.bytes, stream>>>(p);
  return hipGetLastError();
}

template <int BITS, int DT, int NPROJ>
hipError_t launch_lds_bits_dt_nproj(const QmvParams& p, hipStream_t stream) {
  return p.M <= 8 ? launch_lds_rows<BITS, DT, 8, NPROJ>(p, stream)
                  : launch_lds_rows<BITS, DT, 16, NPROJ>(p, stream);
}

template <int BITS, int DT>
hipError_t launch_lds_bits_dt(const QmvParams& p, int nproj, hipStream_t stream) {
  return nproj == 2 ? launch_lds_bits_dt_nproj<BITS, DT, 2>(p, stream)
                    : launch_lds_bits_dt_nproj<BITS, DT, 1>(p, stream);
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

bool affine_qmv_lds_fits(int M, int steps_per_split, int nproj) {
  if (M < 1 || M > kQmvLdsMaxRows) return false;
  const int mrows = M <= 8 ? 8 : 16;
  if (M * steps_per_split * 8 > qmv_lds_chunk_iters(mrows) * kQmvLdsWaves * 64) return false;
  return qmv_lds_layout(M, steps_per_split, mrows, nproj).bytes <= 64u * 1024u;
}

hipError_t launch_affine_qmv_lds(const QmvParams& p, int bits, int dtype, int nproj,
                                 hipStream_t stream) {
  if (bits == 4) {
    return dtype == kBF16 ? launch_lds_bits_dt<4, kBF16>(p, nproj, stream)
                          : launch_lds_bits_dt<4, kF16>(p, nproj, stream);
  }
  return dtype == kBF16 ? launch_lds_bits_dt<8, kBF16>(p, nproj, stream)
                        : launch_lds_bits_dt<8, kF16>(p, nproj, stream);
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

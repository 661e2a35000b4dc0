// Activation-staged small-row affine projections (M <= 32) for gfx950.
//
// Same contract as affine_qmv.hip: y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/G] + b[n, k/G])
// (reference semantics kernels/affine_qmv.py:4-54; residual and SwiGLU epilogues
// kernels/affine_qmv.py:124-132,204-214), with the same work split (32-column strips x
// K splits, four to eight K steps per wave), scale staging, fixed-order cross-wave reduction and
// deterministic split-K protocol. What differs from affine_qmv_kernel:
//  * The workgroup's activation rows for its K range are loaded once and parked in LDS. For
//    4-bit codes each group of 8 elements is stored in the paired order (0,4,1,5,2,6,3,7), so
//    a word of codes unpacks with one AND-OR per pair of codes (unpack_u4_paired) and the MFMA
//    A operand of a K slice is one 16-byte LDS read. Lanes of rows >= M read a zero row.
//  * The per-row activation sum of every K step (the factor of the bias term) is summed once
//    while staging: eight lanes hold the eight 16-byte chunks of one (row, step) and combine
//    their sums with three lane exchanges.
//  * The register ring holds codes only, so a wave needs about half the registers and a
//    workgroup runs eight waves.
#include "common.h"
#include "affine_qmv.h"

namespace mt {
namespace {

// Code stages each wave requests before the workgroup parks its scales and activations: one for
// the three-stage 4-bit ring of a one-split short K (its waves have at most three steps, and
// every code request ahead of the activations delays the staging all steps wait for: config-1
// SwiGLU at M=16 8.55 -> 8.31 us, one projection 6.26 -> 6.03 us against two), else two (the
// six-stage ring of a long K split: the down projection at M=16 8.14 us, 8.37 with one).
template <int BITS, int STAGES, bool HALF>
constexpr int qmv_early_stages() { return BITS == 4 && STAGES == 3 && !HALF ? 1 : 2; }

// One workgroup's share: TILES consecutive output strips (strip s = columns [s N / strips,
// (s + 1) N / strips), at most 32), strips [group TILES, group TILES + TILES), over K split
// `split`. Each strip is computed by its own eight waves (a tile); the activations of the K
// split are staged once for all tiles. Lanes and rows past a strip's width load nothing and
// store nothing.
// HALF: groups of 32, two per 64-wide K step. Each projection then runs two MFMA chains per
// step, one per group: lanes of the other K half (h) read the zero row, so each chain sums one
// group only and gets its own scale, bias and row sum.
template <int BITS, int DT, int MROWS, int NPROJ, int STAGES, int EARLY, bool HALF, int TILES>
__device__ __forceinline__ void lds_task(const QmvParams& p, const int group, const int split,
                                         unsigned char* __restrict__ dyn, int* flag) {
  constexpr int WAVES = kQmvLdsWaves;  // per tile
  constexpr int kTileThreads = WAVES * 64;
  constexpr int kThreads = kTileThreads * TILES;
  constexpr float kOff = SumOffset<BITS, DT>::value;
  constexpr int kRegs = MROWS / 2;
  constexpr int kArrays = 2 * NPROJ;
  constexpr int kXIters = qmv_lds_chunk_iters(MROWS, TILES);
  constexpr int kHalves = HALF ? 2 : 1;  // row sums (groups) per K step

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_wg = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wave_wg / WAVES;
  const int wave = wave_wg % WAVES;     // within the tile
  const int ttid = tid % kTileThreads;  // thread within the tile
  const int strip = group * TILES + tile;
  const int j = lane & 31;
  const int h = lane >> 5;
  const int M = p.M, K = p.K, N = p.N;
  // Strip boundaries fall on multiples of p.col_align columns (whole cache lines of the
  // repacked codes, so no line is fetched by two strips). Equal strips (the host's strip_cols)
  // skip the two divisions.
  int col0, width;
  if (p.strip_cols) {
    col0 = strip * p.strip_cols;
    width = p.strip_cols;
  } else {
    const int units = N / p.col_align;
    col0 = (int)(((int64_t)strip * units) / p.strips) * p.col_align;
    width = (int)(((int64_t)(strip + 1) * units) / p.strips) * p.col_align - col0;
  }
  const int steps_total = K >> 6;
  const int s_beg = split * p.steps_per_split;
  const int s_end = min(steps_total, s_beg + p.steps_per_split);
  const int steps_here = s_end - s_beg;
  const int per_wave = (steps_here + WAVES - 1) / WAVES;
  const int w_beg = s_beg + wave * per_wave;
  const int w_end = min(s_end, w_beg + per_wave);
  const int gshift = p.group_shift;
  // Scale rows are staged from the 32-bit word holding group g_beg; a row whose element
  // index (row * groups_per_row + g_beg) is odd starts one 16-bit element into its segment.
  const int g_beg = HALF ? 2 * s_beg : s_beg >> gshift;
  const int g_last = HALF ? 2 * s_end - 1 : (s_end - 1) >> gshift;
  const int nwords = (g_last - g_beg + 1) / 2 + 1;
  const QmvLdsLayout lay = qmv_lds_layout(M, p.steps_per_split, MROWS, NPROJ, kHalves, TILES);
  const int xstride = p.steps_per_split * 64 + 8;  // staged row stride, elements
  // [kArrays][32][kSbRowWords] of this tile
  uint32_t* sb = reinterpret_cast<uint32_t*>(dyn) + tile * (kArrays * 32 * kSbRowWords);
  float* xsum = reinterpret_cast<float*>(dyn + lay.xsum);  // [steps_per_split * kHalves][MROWS]

  const uint32_t row_bytes = (uint32_t)K * BITS / 8u;
  const int groups_per_row = p.groups_per_row;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr) rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * row_bytes);

  // ---- scales and biases: thread t copies 16-byte quads of row t % 32 of every array -----
  constexpr int kQuadsPerRow = (kSbRowWords + 3) / 4;
  constexpr int kSbIters = (kQuadsPerRow + kTileThreads / 32 - 1) / (kTileThreads / 32);
  const int sb_row = ttid & 31;
  const int sb_q0 = ttid >> 5;
  u32x4 sbv[kArrays][kSbIters];
#pragma unroll
  for (int a = 0; a < kArrays; ++a) {
    const uint16_t* src = (a & 1) ? p.b[a >> 1] : p.s[a >> 1];
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (uint32_t)N * groups_per_row * 2u);
    const uint32_t base = (((uint32_t)(col0 + sb_row) * groups_per_row + g_beg) * 2u) & ~3u;
#pragma unroll
    for (int k = 0; k < kSbIters; ++k) {
      const int q = sb_q0 + k * (kTileThreads / 32);
      sbv[a][k] = load16(r, (4 * q < nwords && sb_row < width) ? base + 16u * q : kOOB);
    }
  }

  // ---- the residual this thread's output (row tid / 32, column tid % 32) adds, requested now
  // so that the workgroup finishing the strip does not wait for it at the end --------------
  // Outputs per thread in the epilogue (output o = ttid + kTileThreads r): one up to 16 rows,
  // two at 32.
  constexpr int kResPer = (MROWS * 32 + kTileThreads - 1) / kTileThreads;
  uint16_t res_pre[kResPer];
#pragma unroll
  for (int r = 0; r < kResPer; ++r) res_pre[r] = 0;
  if constexpr (NPROJ == 1) {
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(p.residual, p.residual ? (uint32_t)M * N * 2u : 0u);
#pragma unroll
    for (int r = 0; r < kResPer; ++r) {
      const int o = ttid + kTileThreads * r;
      const int ri = o >> 5, rc = o & 31;
      res_pre[r] = load2(rr, oob_unless(ri < M && rc < width, ((uint32_t)ri * N + col0 + rc) * 2u));
    }
  }

  // ---- activation chunks: chunk c = row * cpr + cc holds elements [8 cc, 8 cc + 8) --------
  const int cpr = steps_here * 8;
  const int nchunks = M * cpr;
  // (c + 1/2) / cpr stays at least 1 / (2 cpr) >= 1/1008 from an integer for c < 32 cpr, far
  // beyond the hardware reciprocal's error, so the truncated product is the exact row.
  const float inv_cpr = __builtin_amdgcn_rcpf((float)cpr);
  u32x4 xv[kXIters];
  auto issue_x = [&]() {
#pragma unroll
    for (int i = 0; i < kXIters; ++i) {
      const int c = tid + i * kThreads;
      const int row = (int)(((float)c + 0.5f) * inv_cpr);
      const int cc = c - row * cpr;
      const uint32_t off =
          c < nchunks ? ((uint32_t)row * K + (uint32_t)(s_beg * 64 + cc * 8)) * 2u : kOOB;
      xv[i] = load16(rx, off);
    }
  };
  issue_x();

  // ---- code ring ---------------------------------------------------------------------------
  const uint32_t w_row =
      j < width ? (uint32_t)(col0 + j) * p.col_stride + (uint32_t)h * 4u * BITS : kOOB;
  typedef u32x4 StageW[NPROJ][BITS / 4];
  StageW ring[STAGES];
  auto load_stage = [&](StageW& S, int st) {
    const bool ok = st < w_end;
    const uint32_t woff = (ok && w_row != kOOB) ? w_row + (uint32_t)st * p.step_stride : kOOB;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int v = 0; v < BITS / 4; ++v) S[pr][v] = load16_nt(rw[pr], ok ? woff + 16u * v : kOOB);
  };
  // The first EARLY stages are requested before the scales and activations are parked, the
  // rest after: requests behind the bulk of the grid's code stream would otherwise hold up
  // the data every K step depends on.
  constexpr int kEarly = EARLY > STAGES ? STAGES : EARLY;
#pragma unroll
  for (int d = 0; d < kEarly; ++d) load_stage(ring[d], w_beg + d);

  // ---- park scales, biases and activations in LDS; per-step row sums ----------------------
#pragma unroll
  for (int a = 0; a < kArrays; ++a)
#pragma unroll
    for (int k = 0; k < kSbIters; ++k) {
      const int q = sb_q0 + k * (kTileThreads / 32);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (4 * q + c < kSbRowWords) sb[(a * 32 + sb_row) * kSbRowWords + 4 * q + c] = sbv[a][k][c];
    }
#pragma unroll
  for (int i = 0; i < kXIters; ++i) {
    const int c = tid + i * kThreads;
    // Every aligned group of 8 chunks (one row and step) is wholly below nchunks or wholly
    // above, so the lane exchanges stay inside active groups.
    if (i * kThreads < nchunks) {
      const int row = (int)(((float)c + 0.5f) * inv_cpr);
      const int cc = c - row * cpr;
      // Sum over the chunks of one group: 8 (a whole step) or 4 (a half step).
      float s = sum8<DT>(xv[i], 0.0f);
      s = HALF ? group_sum4(s) : group_sum8(s);
      if (c < nchunks) {
        const u32x4 v = (BITS == 4) ? pair_order(xv[i]) : xv[i];
        *reinterpret_cast<u32x4*>(dyn + lay.x + ((uint32_t)row * xstride + cc * 8) * 2u) = v;
        constexpr int kChunksPerSum = HALF ? 4 : 8;
        if ((cc & (kChunksPerSum - 1)) == 0) xsum[(cc / kChunksPerSum) * MROWS + row] = s;
      }
    }
  }
  // Row sums of rows M..MROWS-1 and the zero row.
  for (int idx = tid; idx < steps_here * kHalves * MROWS; idx += kThreads)
    if ((idx % MROWS) >= M) xsum[idx] = 0.0f;
  for (int q = tid; q < xstride / 8; q += kThreads)
    *reinterpret_cast<u32x4*>(dyn + lay.zero + 16u * q) = (u32x4){0u, 0u, 0u, 0u};
  __syncthreads();
#pragma unroll
  for (int d = kEarly; d < STAGES; ++d) load_stage(ring[d], w_beg + d);

  // ---- K loop --------------------------------------------------------------------------------
  float acc[NPROJ][kRegs];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int r = 0; r < kRegs; ++r) acc[pr][r] = 0.0f;

  const f32x16 zero16 = (f32x16){0};
  const PairedConsts pc = paired_consts<DT>();
  const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(sb);
  const int sb_shift = ((col0 + j) * groups_per_row + g_beg) & 1;
  // A operand of lane (j, h): row j (the zero row for j >= M), elements [32 h, 32 h + 32) of
  // each step's 64.
  const uint32_t a_base = lay.x + ((uint32_t)min(j, M) * xstride + 32u * h) * 2u;
  const uint32_t z_base = lay.x + ((uint32_t)M * xstride + 32u * h) * 2u;
  for (int s0 = w_beg; s0 < w_end; s0 += STAGES) {
#pragma unroll
    for (int d = 0; d < STAGES; ++d) {
      StageW& S = ring[d];
      const int st = s0 + d;
      if (st < w_end) {
        const int sl = st - s_beg;
        // A operands of each chain: chain g takes the real row in lanes of K half h == g (all
        // lanes when the step is one group) and the zero row elsewhere.
        u32x4 a[kHalves][4];
#pragma unroll
        for (int g = 0; g < kHalves; ++g) {
          const uint32_t base = (!HALF || h == g) ? a_base : z_base;
          const unsigned char* ap = dyn + base + (uint32_t)sl * 128u;
#pragma unroll
          for (int e = 0; e < 4; ++e) a[g][e] = *reinterpret_cast<const u32x4*>(ap + 16 * e);
        }
        float xs[kHalves][kRegs];
#pragma unroll
        for (int g = 0; g < kHalves; ++g)
#pragma unroll
          for (int q = 0; q < kRegs / 4; ++q) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(
                &xsum[(sl * kHalves + g) * MROWS + 8 * q + 4 * h]);
#pragma unroll
            for (int r = 0; r < 4; ++r) xs[g][4 * q + r] = v[r];
          }
        const int gl = (HALF ? 2 * st : (st >> gshift)) - g_beg + sb_shift;
#pragma unroll
        for (int pr = 0; pr < NPROJ; ++pr) {
          u32x4 b[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (BITS == 4) b[e] = codes_for_sum<DT>(unpack_u4_paired(S[pr][0][e], pc));
            else b[e] = codes_for_sum<DT>(code_frag<BITS, DT>(S[pr], e));
          }
#pragma unroll
          for (int g = 0; g < kHalves; ++g) {
            f32x16 t = mfma32<DT>(a[g][0], b[0], zero16);
#pragma unroll
            for (int e = 1; e < 4; ++e) t = mfma32<DT>(a[g][e], b[e], t);
            const int gg = gl + g;
            const float sf = act_to_f32<DT>(sb16[((2 * pr) * 32 + j) * 2 * kSbRowWords + gg]);
            const float bf =
                act_to_f32<DT>(sb16[((2 * pr + 1) * 32 + j) * 2 * kSbRowWords + gg]);
            const float bp = __builtin_fmaf(-kOff, sf, bf);
#pragma unroll
            for (int r = 0; r < kRegs; ++r) {
              acc[pr][r] = __builtin_fmaf(sf, t[r], acc[pr][r]);
              acc[pr][r] = __builtin_fmaf(bp, xs[g][r], acc[pr][r]);
            }
          }
        }
      }
      load_stage(S, st + STAGES);
    }
  }

  // ---- cross-wave reduction (fixed order); the buffer reuses the staged data -------------
  __syncthreads();
  // [WAVES][NPROJ][MROWS][33] of this tile
  float* red = reinterpret_cast<float*>(dyn) + tile * (WAVES * NPROJ * MROWS * 33);
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

  // Final value of output (i, c) of this strip from its K sums v[].
  auto finish = [&](int i, int c, const float (&v)[NPROJ]) {
    const size_t oi = (size_t)i * N + col0 + c;
    float out;
    if constexpr (NPROJ == 2) {
      out = silu_mul(v[0], v[1]);
    } else {
      out = v[0];
      // output i * 32 + c is this thread's output (i * 32 + c - ttid) / kTileThreads
      if (p.residual) out += act_to_f32<DT>(res_pre[(i * 32 + c - ttid) / kTileThreads]);
    }
    p.y[oi] = f32_to_act<DT>(out);
  };

  const int outs = M * 32;
  if (p.ksplit == 1) {
    for (int o = ttid; o < outs; o += kTileThreads) {
      if ((o & 31) >= width) continue;
      float v[NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) v[pr] = reduce(pr, o >> 5, o & 31);
      finish(o >> 5, o & 31, v);
    }
    return;
  }

  // ---- split-K: publish partials, last workgroup of the strip finishes -------------------
  // Partials are written and read with device-scope relaxed atomic accesses, which the gfx950
  // memory model makes coherent across the chip's L2 slices without any cache-wide writeback
  // or invalidate. Each wave waits for its stores to complete before the barrier, so every
  // partial of this workgroup is visible before the arrival counter moves.
  const size_t plane = (size_t)M * N;
  for (int o = ttid; o < outs; o += kTileThreads) {
    const int i = o >> 5, c = o & 31;
    if (c >= width) continue;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
      __hip_atomic_store(&p.partial[(size_t)(split * NPROJ + pr) * plane + (size_t)i * N +
                                    col0 + c],
                         reduce(pr, i, c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (ttid == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&p.counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flag[tile] = (prev == (unsigned)(p.ksplit - 1));
  }
  __syncthreads();
  // No workgroup barrier follows: one tile may return while the other finishes its strip.
  if (!flag[tile]) return;
  // A thread's outputs (one, two at 32 rows) over every split, requested in batches.
  constexpr int kOuts = (MROWS * 32 + kTileThreads - 1) / kTileThreads;
  const float* src[kOuts * NPROJ];
  float sum[kOuts * NPROJ];
#pragma unroll
  for (int u = 0; u < kOuts; ++u) {
    const int o = ttid + u * kTileThreads;
    const bool ok = o < outs && (o & 31) < width;
    const size_t oi = (size_t)(o >> 5) * N + col0 + (o & 31);
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
      src[u * NPROJ + pr] = ok ? p.partial + (size_t)pr * plane + oi : nullptr;
  }
  sum_partials_multi<kOuts * NPROJ>(src, (size_t)NPROJ * plane, p.ksplit, sum);
#pragma unroll
  for (int u = 0; u < kOuts; ++u) {
    const int o = ttid + u * kTileThreads;
    if (o >= outs || (o & 31) >= width) continue;
    float v[NPROJ];
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr) v[pr] = sum[u * NPROJ + pr];
    finish(o >> 5, o & 31, v);
  }
  if (ttid == 0)
    __hip_atomic_store(&p.counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// At most 128 registers, so that sixteen waves (two one-tile workgroups or one two-tile
// workgroup) share a CU.
template <int BITS, int DT, int MROWS, int NPROJ, int STAGES, bool HALF, int TILES>
__global__ __launch_bounds__(kQmvLdsWaves * 64 * TILES) __attribute__((amdgpu_waves_per_eu(4)))
void affine_qmv_lds_kernel(const QmvParams args) {
  const QmvParams p = preload_args(args);  // all arguments in one batch of scalar loads
  extern __shared__ __align__(16) unsigned char dyn_plain[];
  __shared__ int flag[TILES];
  lds_task<BITS, DT, MROWS, NPROJ, STAGES, qmv_early_stages<BITS, STAGES, HALF>(), HALF, TILES>(
      p, blockIdx.x, blockIdx.y, dyn_plain, flag);
}

// Raises a kernel's dynamic LDS limit (64 KiB by default) to what a workgroup of `tiles`
// strips may use. The launchers call it once per kernel instantiation (a function-local static
// in each launcher template).
hipError_t allow_lds(const void* kernel, int tiles) {
  return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)qmv_lds_max_bytes(tiles));
}

template <int BITS, int DT, int MROWS, int NPROJ, int STAGES, bool HALF, int TILES>
hipError_t launch_lds_stages(const QmvParams& p, hipStream_t stream) {
  const QmvLdsLayout lay =
      qmv_lds_layout(p.M, p.steps_per_split, MROWS, NPROJ, HALF ? 2 : 1, TILES);
  const dim3 grid(p.strips / TILES, p.ksplit);
  auto kernel = affine_qmv_lds_kernel<BITS, DT, MROWS, NPROJ, STAGES, HALF, TILES>;
  static const hipError_t attr = allow_lds(reinterpret_cast<const void*>(kernel), TILES);
  if (attr != hipSuccess) return attr;
  kernel<<<grid, dim3(kQmvLdsWaves * 64 * TILES), lay.bytes, stream>>>(p);
  return hipGetLastError();
}

// Code ring depth: for 4-bit codes six stages, or three when no wave has more than three K
// steps (the common one-split K = 1536): every stage past a wave's last step is still issued
// as an out-of-range load, and those measured about 0.9 us per launch at that shape. Groups
// of 32 hold two A operand sets per step, so their ring is shallower.
template <int BITS, int DT, int MROWS, int NPROJ, bool HALF, int TILES>
hipError_t launch_lds_tiles(const QmvParams& p, hipStream_t stream) {
  if constexpr (HALF) {
    return launch_lds_stages<BITS, DT, MROWS, NPROJ, BITS == 4 ? 3 : 2, HALF, TILES>(p, stream);
  } else if constexpr (MROWS == 32 && NPROJ == 2) {
    // 32 rows of gate and up accumulators: a shallower ring keeps within 128 registers.
    return launch_lds_stages<BITS, DT, MROWS, NPROJ, BITS == 4 ? 3 : 2, HALF, TILES>(p, stream);
  } else if constexpr (BITS == 8) {
    return launch_lds_stages<BITS, DT, MROWS, NPROJ, NPROJ == 2 ? 3 : 4, HALF, TILES>(p, stream);
  } else {
    const int steps = min(p.steps_per_split, p.K / 64);
    const int per_wave = (steps + kQmvLdsWaves - 1) / kQmvLdsWaves;
    return per_wave <= 3 ? launch_lds_stages<BITS, DT, MROWS, NPROJ, 3, HALF, TILES>(p, stream)
                         : launch_lds_stages<BITS, DT, MROWS, NPROJ, 6, HALF, TILES>(p, stream);
  }
}

template <int BITS, int DT, int MROWS, int NPROJ, bool HALF>
hipError_t launch_lds_rows(const QmvParams& p, hipStream_t stream) {
  return p.tiles == 2 ? launch_lds_tiles<BITS, DT, MROWS, NPROJ, HALF, 2>(p, stream)
                      : launch_lds_tiles<BITS, DT, MROWS, NPROJ, HALF, 1>(p, stream);
}

template <int BITS, int DT, int NPROJ, bool HALF>
hipError_t launch_lds_half(const QmvParams& p, hipStream_t stream) {
  if (p.M <= 8) return launch_lds_rows<BITS, DT, 8, NPROJ, HALF>(p, stream);
  if (p.M <= 16 || HALF) return launch_lds_rows<BITS, DT, 16, NPROJ, HALF>(p, stream);
  if constexpr (!HALF) return launch_lds_rows<BITS, DT, 32, NPROJ, HALF>(p, stream);
  return hipErrorInvalidValue;
}

template <int BITS, int DT, int NPROJ>
hipError_t launch_lds_nproj(const QmvParams& p, hipStream_t stream) {
  return p.G == 32 ? launch_lds_half<BITS, DT, NPROJ, true>(p, stream)
                   : launch_lds_half<BITS, DT, NPROJ, false>(p, stream);
}

template <int BITS, int DT>
hipError_t launch_lds_bits_dt(const QmvParams& p, int nproj, hipStream_t stream) {
  return nproj == 2 ? launch_lds_nproj<BITS, DT, 2>(p, stream)
                    : launch_lds_nproj<BITS, DT, 1>(p, stream);
}

}  // namespace

bool affine_qmv_lds_fits(int M, int steps_per_split, int nproj, int group_size, int tiles) {
  if (M < 1 || M > (group_size == 32 ? kQmvLdsMaxRowsHalf : kQmvLdsMaxRows) ||
      (tiles != 1 && tiles != 2))
    return false;
  const int mrows = M <= 8 ? 8 : M <= 16 ? 16 : 32;
  if (M * steps_per_split * 8 > qmv_lds_chunk_iters(mrows, tiles) * kQmvLdsWaves * 64 * tiles)
    return false;
  // Groups staged per split (one more may straddle) within the scale rows.
  const int groups = group_size == 32 ? 2 * steps_per_split : steps_per_split;
  if (groups > kMaxGroupsPerSplit - 1) return false;
  const int halves = group_size == 32 ? 2 : 1;
  return qmv_lds_layout(M, steps_per_split, mrows, nproj, halves, tiles).bytes <=
         qmv_lds_max_bytes(tiles);
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

}  // namespace mt

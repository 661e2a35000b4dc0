// Dense 16-bit small-batch projections for gfx950: the gate/up SwiGLU and the down projection
// with a residual epilogue (reference: metile/compiler/dense.py:193-381 with the typed
// epilogues of metile/codegen/msl_emitter.py:1098-1120,1218-1252).
//
// Weights are the native output-major [N, K] matrices. The kernel streams them exactly like
// the affine kernel (32-column strips, 64-wide K steps split over four waves, a register
// pipeline of whole K steps, 16-byte buffer loads), but the codes are already 16-bit floats,
// so each step is four MFMAs chained into the same accumulator and there is no per-step
// fix-up.
//
// Row invariance: the value of every output depends only on its own activation row and on an
// accumulation order fixed by (K, N): the K partition among splits and waves comes from
// (K, N) alone, every wave accumulates its steps in order through one MFMA chain, and the
// cross-wave and split-K sums run in a fixed order. Running a row alone or inside a batch
// therefore gives the same bits. A launch covers up to 64 rows per grid z index (row chunks,
// each with its own partial sums and counters); the host dispatches up to 128 rows at a time.
#include "common.h"
#include "dense_qmv.h"

namespace mt {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <int NPROJ, int MT>
struct DStage {
  u32x4 w[NPROJ][4];  // 4 x 8 K of column j for each projection
  u32x4 x[MT][4];     // 4 x 8 K of row j of each 32-row tile
};

// The reference's typed SwiGLU epilogue: gate and up rounded to the activation type, then
// y = 1/(1+exp(|g|)), sig = g < 0 ? y : 1 - y, act = g*sig, out = act*u, each operation
// computed in fp32 and rounded to the activation type.
template <int DT>
__device__ __forceinline__ float round_act(float v) {
  return act_to_f32<DT>(f32_to_act<DT>(v));
}

template <int DT>
__device__ __forceinline__ uint16_t typed_swiglu(float g, float u) {
  const float left = round_act<DT>(g);
  const float right = round_act<DT>(u);
  const float e = round_act<DT>(expf(fabsf(left)));
  const float y = round_act<DT>(1.0f / round_act<DT>(1.0f + e));
  const float sig = left < 0.0f ? y : round_act<DT>(1.0f - y);
  const float act = round_act<DT>(left * sig);
  return f32_to_act<DT>(act * right);
}

// Workgroups per CU the kernel is built for: two (up to 64 rows, MT <= 2; larger batches run
// as 64-row chunks, which measured faster than 128-row tiles at one workgroup per CU).
template <int MT>
constexpr int dense_occupancy() { return 2; }

// Activation tiles above 8 rows go through LDS (XLDS): lane j of an MFMA operand needs row
// j, so loading the operand directly touches 32 rows (32 cache lines, 32 bytes of each) per
// instruction; loaded 8 lanes per row instead, every instruction reads 8 whole 128-byte lines
// (config 2 at M = 128: gate/up 35.5 -> 29.2 us, down 40.0 -> 30.7 us in a probe with the same
// loads). Each wave stages its own tile of the step (wave-private, no barrier) and reads it back
// in the MFMA layout; the 16-byte chunk c of staged row r sits at slot c ^ (r % 8), so that the
// eight lanes of a read phase (rows r..r+7, one chunk) hit distinct banks. The operands, and so
// every MFMA and sum, are the same as with direct loads.

// LDS of one workgroup, 16-byte units: during the K loop each wave's staged activation tile
// (XLDS) and weight tile ([NPROJ][32 columns][8 chunks], the same swizzle); after it the
// cross-wave reduction buffer [kWaves][NPROJ][32][33] (fp32), in the same space.
template <int MT, int NPROJ, bool XLDS>
constexpr int dense_lds_units() {
  constexpr int per_wave = (XLDS ? MT * 32 * 8 : 0) + NPROJ * 32 * 8;
  constexpr int loop = kWaves * per_wave;
  constexpr int red = (kWaves * NPROJ * 32 * 33 + 3) / 4;
  return loop > red ? loop : red;
}

// NT: weights read with the non-temporal hint. One row chunk reads each weight line once (M=1
// MLP 25.0 -> 22.5 us, M=64 36.5 -> 34.4 us); with two chunks the second reads the lines the
// first left in L2 (M=128 48.6 -> 54.0 us with the hint), so those launches go without it.
template <int DT, int MT, int NPROJ, int STAGES, bool XLDS, bool NT>
__global__ __launch_bounds__(kThreads, dense_occupancy<MT>()) void dense_qmv_kernel(
    const DenseParams args) {
  const DenseParams p = preload_args(args);  // all arguments in one batch of scalar loads
  constexpr int kXUnits = XLDS ? MT * 32 * 8 : 0;  // per wave
  constexpr int kWUnits = NPROJ * 32 * 8;          // per wave
  __shared__ __attribute__((aligned(16))) u32x4 smem[dense_lds_units<MT, NPROJ, XLDS>()];
  __shared__ int last_flag;
  auto red = reinterpret_cast<float (*)[NPROJ][32][33]>(smem);  // [kWaves][NPROJ][32][33]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;
  const int h = lane >> 5;
  const int strip = blockIdx.x;
  const int split = blockIdx.y;
  const int K = p.K, N = p.N;
  // Row chunk z of the launch: its rows, outputs, partial sums and counters.
  const int rc = p.row_chunk;
  const int r0 = rc ? (int)blockIdx.z * rc : 0;
  const int M = rc ? min(rc, p.M - r0) : p.M;
  const uint16_t* const xg = p.x + (size_t)r0 * K;
  uint16_t* const yg = p.y + (size_t)r0 * N;
  const uint16_t* const resg = p.residual ? p.residual + (size_t)r0 * N : nullptr;
  float* const partg =
      p.partial ? p.partial + (size_t)blockIdx.z * p.ksplit * NPROJ * (size_t)(rc ? rc : p.M) * N
                : nullptr;
  uint32_t* const cntg = p.counters ? p.counters + (size_t)blockIdx.z * (N / 32) : nullptr;
  const int steps_total = K >> 6;
  const int s_beg = split * p.steps_per_split;
  const int s_end = min(steps_total, s_beg + p.steps_per_split);
  const int per_wave = (s_end - s_beg + kWaves - 1) / kWaves;
  const int w_beg = s_beg + wave * per_wave;
  const int w_end = min(s_end, w_beg + per_wave);

  const uint32_t row_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xg, (uint32_t)M * K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr) rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * row_bytes);
  // Weights are loaded 8 lanes per column like the staged activations: instruction e of a
  // projection reads columns 8 e + lane / 8 of the strip, chunk lane % 8 of each step, and the
  // wave reads them back from LDS as the MFMA B operand (column j, chunks 4 h + e).
  const uint32_t w_row = (uint32_t)(strip * 32 + (lane >> 3)) * row_bytes + 16u * (lane & 7);
  const uint32_t w_step8 = 8u * row_bytes;
  u32x4* const xs = smem + wave * (kXUnits + kWUnits);  // [MT * 32 rows][8]
  u32x4* const ws = xs + kXUnits;                        // [NPROJ][32 columns][8]
  // Direct operand loads: lane (j, h) reads row 32 rt + j, K [32 h, 32 h + 32) of each step.
  // Staged loads (XLDS): instruction e of row tile rt reads rows 32 rt + 8 e + lane / 8, chunk
  // lane % 8 (K [8 (lane % 8), +8)) of each step.
  uint32_t x_row[MT];
#pragma unroll
  for (int rt = 0; rt < MT; ++rt) {
    const int row = XLDS ? 32 * rt + (lane >> 3) : 32 * rt + j;
    x_row[rt] = row < M ? (XLDS ? ((uint32_t)row * K + 8u * (lane & 7)) * 2u
                                : ((uint32_t)row * K + 32u * h) * 2u)
                        : kOOB;
  }
  // XLDS: rows 8 e + lane / 8 of a tile are 8 apart per instruction, whatever M is.
  const uint32_t x_step8 = 8u * (uint32_t)K * 2u;

  DStage<NPROJ, MT> ring[STAGES];
  // Out-of-range offsets are set with oob_unless (x_row of a row past M already is), not
  // with selects: with selects the compiler could no longer count the ring's loads and waited
  // for nearly all of them before every step.
  auto load_stage = [&](DStage<NPROJ, MT>& S, int st) {
    const bool ok = st < w_end;
    const uint32_t woff = w_row + (uint32_t)st * 128u;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t off = oob_unless(ok, woff + e * w_step8);
        S.w[pr][e] = NT ? load16_nt(rw[pr], off) : load16(rw[pr], off);
      }
#pragma unroll
    for (int rt = 0; rt < MT; ++rt) {
      const uint32_t xoff = x_row[rt] + (uint32_t)st * 128u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (XLDS) {
          // rows past M read zero: their offset is already out of range, and rows 8 e apart
          // past the end of x stay beyond the buffer's range
          const bool row_ok = 32 * rt + 8 * e + (lane >> 3) < M;
          S.x[rt][e] = load16(rx, oob_unless(ok && row_ok, xoff + (uint32_t)e * x_step8));
        } else {
          S.x[rt][e] = load16(rx, oob_unless(ok, xoff + 16u * e));
        }
      }
    }
  };
  // The ring is filled in stage order: the scheduler may not issue a later stage's loads
  // first, or the first step would wait for all of them (and the loop, whose wait counts also
  // cover its entry, for nearly every load in flight).
#pragma unroll
  for (int d = 0; d < STAGES; ++d) {
    load_stage(ring[d], w_beg + d);
    __builtin_amdgcn_sched_barrier(0);
  }

  f32x16 acc[NPROJ][MT];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int rt = 0; rt < MT; ++rt) acc[pr][rt] = (f32x16){0};

  for (int s0 = w_beg; s0 < w_end; s0 += STAGES) {
#pragma unroll
    for (int d = 0; d < STAGES; ++d) {
      DStage<NPROJ, MT>& S = ring[d];
      if (s0 + d < w_end) {
        // Stage the step's tiles (slot of chunk c of row or column r: c ^ (r % 8)), then read
        // row or column j, chunks 4 h + e, back; the waits keep this step's reads after its
        // writes and ahead of the next step's writes.
        const int wr = lane >> 3, wc = lane & 7;
#pragma unroll
        for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
          for (int e = 0; e < 4; ++e) ws[(pr * 32 + 8 * e + wr) * 8 + (wc ^ wr)] = S.w[pr][e];
        if constexpr (XLDS) {
#pragma unroll
          for (int rt = 0; rt < MT; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) xs[(32 * rt + 8 * e + wr) * 8 + (wc ^ wr)] = S.x[rt][e];
        }
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        u32x4 b[NPROJ][4];
#pragma unroll
        for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
          for (int e = 0; e < 4; ++e) b[pr][e] = ws[(pr * 32 + j) * 8 + ((4 * h + e) ^ (j & 7))];
#pragma unroll
        for (int rt = 0; rt < MT; ++rt) {
          u32x4 a[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            a[e] = XLDS ? xs[(32 * rt + j) * 8 + ((4 * h + e) ^ (j & 7))] : S.x[rt][e];
#pragma unroll
          for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[pr][rt] = mfma32<DT>(a[e], b[pr][e], acc[pr][rt]);
        }
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
      load_stage(S, s0 + d + STAGES);
    }
  }

  // ---- per row tile: cross-wave reduction (fixed order), then epilogue or split-K -------
  const size_t plane = (size_t)M * N;
  __syncthreads();  // the reduction buffer reuses the other waves' staging space
#pragma unroll
  for (int rt = 0; rt < MT; ++rt) {
    if (rt > 0) __syncthreads();
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[wave][pr][mfma32_row(r, h)][j] = acc[pr][rt][r];
    __syncthreads();
    const int rows = min(32, M - 32 * rt);
    for (int o = tid; o < rows * 32; o += kThreads) {
      const int i = o >> 5, c = o & 31;
      const size_t oi = (size_t)(32 * rt + i) * N + strip * 32 + c;
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const float v = ((red[0][pr][i][c] + red[1][pr][i][c]) + red[2][pr][i][c]) +
                        red[3][pr][i][c];
        if (p.ksplit == 1) {
          // stash the full sum for the epilogue below
          red[0][pr][i][c] = v;
        } else {
          __hip_atomic_store(&partg[(size_t)(split * NPROJ + pr) * plane + oi], v,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (p.ksplit == 1) {
        if constexpr (NPROJ == 2) {
          yg[oi] = typed_swiglu<DT>(red[0][0][i][c], red[0][1][i][c]);
        } else {
          float out = round_act<DT>(red[0][0][i][c]);
          if (resg) out = out + act_to_f32<DT>(resg[oi]);
          yg[oi] = f32_to_act<DT>(out);
        }
      }
    }
  }
  if (p.ksplit == 1) return;

  // ---- split-K handoff: see the affine kernel; partials and counter are agent-coherent ----
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&cntg[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (prev == (unsigned)(p.ksplit - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  // A thread's outputs over every split, their loads requested in batches (sum_partials_multi)
  // rather than one round trip per output: one output at up to 8 rows (the instances without
  // staged activations), else up to 32 MT rows x 32 columns over the workgroup's threads.
  constexpr int kOuts = XLDS ? 32 * 32 * MT / kThreads : 1;
  const float* src[kOuts * NPROJ];
  float sum[kOuts * NPROJ];
#pragma unroll
  for (int u = 0; u < kOuts; ++u) {
    const int o = tid + u * kThreads;
    const size_t oi = (size_t)(o >> 5) * N + strip * 32 + (o & 31);
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
      src[u * NPROJ + pr] = o < M * 32 ? partg + (size_t)pr * plane + oi : nullptr;
  }
  sum_partials_multi<kOuts * NPROJ>(src, (size_t)NPROJ * plane, p.ksplit, sum);
#pragma unroll
  for (int u = 0; u < kOuts; ++u) {
    const int o = tid + u * kThreads;
    if (o >= M * 32) break;
    const size_t oi = (size_t)(o >> 5) * N + strip * 32 + (o & 31);
    const float* v = sum + u * NPROJ;
    if constexpr (NPROJ == 2) {
      yg[oi] = typed_swiglu<DT>(v[0], v[1]);
    } else {
      float out = round_act<DT>(v[0]);
      if (resg) out = out + act_to_f32<DT>(resg[oi]);
      yg[oi] = f32_to_act<DT>(out);
    }
  }
  if (tid == 0)
    __hip_atomic_store(&cntg[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Register ring depth: the stages that fit beside the accumulators in the registers of one
// wave (256 at two workgroups per CU), with at most 60 loads in flight: the
// hardware counts at most 63 outstanding loads per wave, and a ring deeper than that count
// makes the compiler wait for almost every load before each step.
template <int NPROJ, int MT>
constexpr int dense_stages() {
  constexpr int per_stage = 16 * NPROJ + 16 * MT;
  constexpr int loads = 4 * NPROJ + 4 * MT;
  constexpr int budget = 112;  // ring registers beside the accumulators at two workgroups per CU
  constexpr int s = budget / per_stage < 60 / loads ? budget / per_stage : 60 / loads;
  return s < 1 ? 1 : (s > 4 ? 4 : s);
}

template <int DT, int NPROJ, bool NT>
hipError_t launch_dense_rows(const DenseParams& p, int rows, dim3 grid, hipStream_t stream) {
  // Activations staged through LDS above 8 rows (at fewer rows most operand lanes read zero
  // and the direct loads touch few lines).
  if (rows <= 8) {
    dense_qmv_kernel<DT, 1, NPROJ, dense_stages<NPROJ, 1>(), false, NT>
        <<<grid, kThreads, 0, stream>>>(p);
  } else if (rows <= 32) {
    dense_qmv_kernel<DT, 1, NPROJ, dense_stages<NPROJ, 1>(), true, NT>
        <<<grid, kThreads, 0, stream>>>(p);
  } else if (rows <= 64) {
    dense_qmv_kernel<DT, 2, NPROJ, dense_stages<NPROJ, 2>(), true, NT>
        <<<grid, kThreads, 0, stream>>>(p);
  } else {
    return hipErrorInvalidValue;  // more than 64 rows run as row chunks (row_chunk)
  }
  return hipGetLastError();
}

template <int DT, int NPROJ>
hipError_t launch_dense_dt(const DenseParams& p, hipStream_t stream) {
  // Rows per chunk (grid z): the instance is chosen by the rows of one chunk.
  const int rows = p.row_chunk ? p.row_chunk : p.M;
  const int chunks = p.row_chunk ? (p.M + p.row_chunk - 1) / p.row_chunk : 1;
  const dim3 grid(p.N / 32, p.ksplit, chunks);
  return chunks == 1 ? launch_dense_rows<DT, NPROJ, true>(p, rows, grid, stream)
                     : launch_dense_rows<DT, NPROJ, false>(p, rows, grid, stream);
}

}  // namespace

hipError_t launch_dense_qmv(const DenseParams& p, int dtype, int nproj, hipStream_t stream) {
  if (dtype == kBF16)
    return nproj == 2 ? launch_dense_dt<kBF16, 2>(p, stream) : launch_dense_dt<kBF16, 1>(p, stream);
  return nproj == 2 ? launch_dense_dt<kF16, 2>(p, stream) : launch_dense_dt<kF16, 1>(p, stream);
}

}  // namespace mt

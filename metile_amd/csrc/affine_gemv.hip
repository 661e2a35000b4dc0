// Small-row affine QMV / SwiGLU without a split-K hand-off (gfx950), for projections whose K
// is long and N short (the down projection: K = 8960, N = 1536): the same semantics as the
// staged kernel (kernels/affine_qmv.py:57-214; mlx_affine_qmv, mlx_affine_swiglu,
// metile/backends/mlx_quantized.py:691-751,1645-1720).
//
// A workgroup owns COLS output columns (2, 4, or 8 for one projection of one or two rows) and
// all of K, so no partial sum leaves it. Its
// lanes (1 to 8 waves; the plan picks the fewest that cover K in a given number of passes) split
// K into 16-byte code chunks (32 codes at 4 bits, 16 at 8 bits): lane t takes the chunks t,
// t + lanes, t + 2 lanes, ... of every one of the workgroup's columns, and loads the activations
// of a chunk once for all COLS columns. When K is short enough for one pass and a column's
// chunks fill whole rows of 16 lanes, a workgroup covers several groups of COLS columns, lane t
// taking chunk t % chunks of group t / chunks (K = 1536 at 4 bits: 48 chunks, three waves serve
// four groups with no idle lane). A chunk's codes are unpacked to exact
// 16-bit floats offset + q (4-bit codes in the paired order of each word, the activations
// re-ordered to match) and dotted with the activations two at a time (fp32
// accumulate), together with the activations' sum; the group's affine terms are applied in
// fp32 as in the staged kernel: acc += s * sum_k x_k (offset + q_k) + (b - offset * s) sum_k x_k.
// Chunks never straddle a group (groups are 32 codes or more and chunk-aligned).
// The lanes' partial sums are added by DPP moves within rows of 16 lanes, then across rows and
// waves in LDS, always in the same order, so a row's result depends only on the plan (and not
// on M or the code layout).
#include "common.h"
#include "affine_qmv.h"

namespace mt {

namespace {

// Column group of workgroup b under plan order 1: consecutive workgroups are dispatched to the
// 8 XCDs in turn, so the groups are dealt out XCD by XCD (workgroups b, b + 8, b + 16, ... take
// adjacent column groups), and neighbouring columns share their XCD's L2 for the cache lines
// they have in common (scale and bias rows do not start on line boundaries). Any order is
// correct; which is faster depends on the shape (measured: the one-row down projection 4.41 ->
// 4.30 us with this order, the one-row SwiGLU 6.99 -> 7.14 us), so the plan picks it. `whole`
// (from the host: the grid rounded down to a multiple of 8, or 0 under order 0) workgroups are
// dealt out; the rest keep their index. Branch-free, with no read of the grid size: a branch
// here had split the kernel's argument loads into three dependent rounds before the first
// memory request.
__device__ __forceinline__ int gemv_column_group(int b, int whole) {
  constexpr int kXcds = 8;
  const int dealt = (b % kXcds) * (whole / kXcds) + b / kXcds;
  return b < whole ? dealt : b;
}

// How a one-pass workgroup lays its column groups over its lanes.
//  * kOneGroup: one group of COLS columns; its chunks span the waves (cross-wave sums in LDS).
//  * kStraddle: several groups, lane t taking group t / chunks, chunk t % chunks; groups may
//    span two waves (cross-wave sums in LDS).
//  * kWaveGroups (a column's chunks fit in one wave): every wave holds whole groups (64 / chunks
//    of them when chunks is a multiple of 16, else one), so each group's sums stay inside its
//    wave: DPP within rows of 16 lanes, then the group's row sums read with readlane and added
//    in row order. No wave waits for another (no LDS, no barrier); the order of every addition
//    is the same as the LDS path's, so the results are the same bit for bit.
enum GemvLayout : int { kOneGroup = 0, kStraddle = 1, kWaveGroups = 2 };

// ONE_PASS: every lane has at most one chunk per column (K / chunk <= lanes), so no second
// pass is held in registers (more waves fit on a CU). LAYOUT: see GemvLayout (one pass only
// for kStraddle and kWaveGroups); separate instances, so that one-group workgroups keep their
// columns wave-uniform and issue their loads without the per-lane group arithmetic.
template <int BITS, int DT, int ROWS, int NPROJ, int COLS, bool ONE_PASS, int LAYOUT>
__global__ __launch_bounds__(64 * kGemvMaxWaves) void affine_gemv_kernel(const QmvParams args) {
  // All arguments in one batch of scalar loads: left to itself the compiler fetched them in
  // three dependent rounds (a full scalar-memory wait each) before the first load was issued.
  const QmvParams p = preload_args(args);
  constexpr int kChunks = BITS / 2;        // 16-byte chunks per column and 64-wide K step
  constexpr int kCodes = 128 / BITS;       // codes per chunk
  constexpr int kXLoads = kCodes / 8;      // 16-byte activation loads per chunk and row
  constexpr int kOut = NPROJ * COLS * ROWS;
  constexpr float kOff = SumOffset<BITS, DT>::value;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int waves = blockDim.x >> 6;
  const int lanes = blockDim.x;
  const int M = p.M, K = p.K, N = p.N;
  const int chunks = K / kCodes;
  // One pass over short K: the workgroup covers `groups` column groups, lane t group t / chunks
  // and chunk t % chunks (lanes past the last group load nothing). Otherwise one group. The
  // quotient comes from a float reciprocal: (t + 1/2) / chunks stays at least 1 / (2 chunks)
  // from an integer, far beyond the reciprocal's error for t and chunks below 512.
  static_assert(ONE_PASS || LAYOUT == kOneGroup, "column groups need one pass");
  constexpr bool GROUPS = LAYOUT != kOneGroup;
  const int groups = GROUPS ? p.gemv_groups : 1;
  // kWaveGroups: groups per wave (from the host), and lane t of wave w takes group
  // w * gpw + lane / chunks.
  const int gpw = LAYOUT == kWaveGroups ? p.gemv_groups_per_wave : 0;
  const int lt = LAYOUT == kWaveGroups ? lane : tid;  // position counted within the wave
  const int gq = GROUPS ? (int)(((float)lt + 0.5f) * __builtin_amdgcn_rcpf((float)chunks)) : 0;
  const int gi = LAYOUT == kWaveGroups ? wave * gpw + gq : gq;
  const int kc0 = GROUPS ? lt - gq * chunks : tid;
  const bool lane_on = !GROUPS || (LAYOUT == kWaveGroups ? gq < gpw : gi < groups);
  const int wg = gemv_column_group(blockIdx.x, p.gemv_dealt);
  const int col0 = (wg * groups + gi) * COLS;  // this lane's first column
  const int gshift = __builtin_ctz((unsigned)p.G);
  const int groups_per_row = K >> gshift;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ], rs[NPROJ], rb[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr) {
    rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * (uint32_t)(K * BITS / 8));
    rs[pr] = make_rsrc(p.s[pr], (uint32_t)N * groups_per_row * 2u);
    rb[pr] = make_rsrc(p.b[pr], (uint32_t)N * groups_per_row * 2u);
  }

  struct Stage {
    u32x4 q[NPROJ][COLS];
    u32x4 x[ROWS][kXLoads];
    uint32_t s[NPROJ][COLS], b[NPROJ][COLS];
  };
  auto load = [&](Stage& S, int kc) {
    const bool ok = lane_on && kc < chunks;
    const int st = kc / kChunks;
    const uint32_t wo = (uint32_t)st * p.step_stride + 16u * (uint32_t)(kc % kChunks);
    const int k0 = kc * kCodes;
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int j = 0; j < COLS; ++j) {
        const uint32_t col = (uint32_t)(col0 + j);
        S.q[pr][j] = load16_nt(rw[pr], oob_unless(ok, col * p.col_stride + wo));
        const uint32_t go =
            oob_unless(ok, (col * (uint32_t)groups_per_row + (uint32_t)(k0 >> gshift)) * 2u);
        S.s[pr][j] = load2_nt(rs[pr], go);
        S.b[pr][j] = load2_nt(rb[pr], go);
      }
#pragma unroll
    for (int m = 0; m < ROWS; ++m)
#pragma unroll
      for (int v = 0; v < kXLoads; ++v)
        S.x[m][v] = load16(rx, oob_unless(ok && m < M, ((uint32_t)m * K + k0 + 8 * v) * 2u));
  };

  float acc[NPROJ][COLS][ROWS];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
    for (int j = 0; j < COLS; ++j)
#pragma unroll
      for (int m = 0; m < ROWS; ++m) acc[pr][j][m] = 0.0f;

  // 4-bit codes are unpacked in the paired order (0,4,1,5,2,6,3,7) of each word, one AND-OR per
  // pair of codes (unpack_u4_paired), and the activations are put in the same order once per
  // lane (pair_order), for all of its columns.
  const PairedConsts pc = paired_consts<DT>();
  auto compute = [&](const Stage& S) {
    float xs[ROWS];
    u32x4 xp[ROWS][kXLoads];
#pragma unroll
    for (int m = 0; m < ROWS; ++m) {
      xs[m] = 0.0f;
#pragma unroll
      for (int v = 0; v < kXLoads; ++v) {
        xs[m] = sum8<DT>(S.x[m][v], xs[m]);
        xp[m][v] = BITS == 4 ? pair_order(S.x[m][v]) : S.x[m][v];
      }
    }
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int j = 0; j < COLS; ++j) {
        u32x4 cw[kXLoads];
#pragma unroll
        for (int v = 0; v < kXLoads; ++v) {
          if constexpr (BITS == 4) {
            cw[v] = codes_for_sum<DT>(unpack_u4_paired(S.q[pr][j][v], pc));
          } else {
            const u32x2 lo = unpack_u8<DT>(S.q[pr][j][2 * v]);
            const u32x2 hi = unpack_u8<DT>(S.q[pr][j][2 * v + 1]);
            cw[v] = codes_for_sum<DT>((u32x4){lo.x, lo.y, hi.x, hi.y});
          }
        }
        const float sf = act_to_f32<DT>(S.s[pr][j]);
        const float bp = __builtin_fmaf(-kOff, sf, act_to_f32<DT>(S.b[pr][j]));
#pragma unroll
        for (int m = 0; m < ROWS; ++m) {
          float t = 0.0f;
#pragma unroll
          for (int v = 0; v < kXLoads; ++v) {
            const u32x4 xv = xp[m][v];
            const u32x4 cv = cw[v];
            t = dot2<DT>(xv.x, cv.x, t);
            t = dot2<DT>(xv.y, cv.y, t);
            t = dot2<DT>(xv.z, cv.z, t);
            t = dot2<DT>(xv.w, cv.w, t);
          }
          acc[pr][j][m] = __builtin_fmaf(sf, t, acc[pr][j][m]);
          acc[pr][j][m] = __builtin_fmaf(bp, xs[m], acc[pr][j][m]);
        }
      }
  };

  // Passes of one chunk per lane, two in registers: the next pass's loads are issued before
  // this one's math, so a workgroup with one or two passes waits for memory once. The pass
  // count is the same for every lane (lanes past K load zeros), so the branches are uniform.
  if constexpr (ONE_PASS) {
    Stage cur;
    load(cur, kc0);
    compute(cur);
  } else {
    Stage cur, nxt;
    load(cur, tid);
    for (int base = 0; base < chunks; base += lanes) {
      const bool more = base + lanes < chunks;
      if (more) load(nxt, base + lanes + tid);
      compute(cur);
      if (more) cur = nxt;
    }
  }

  // Rows of 16 lanes by DPP (each lane ends with its row's sum; a row never spans two groups),
  // then a group's rows: by row broadcasts within the wave (kWaveGroups; kOneGroup, whose
  // waves' sums then meet in LDS), or in row order through LDS (kStraddle).
  if constexpr (LAYOUT == kWaveGroups) {
    // A group fills 1, 2 or 4 rows of 16 lanes (4, 2 or 1 groups per wave; with one group per
    // wave, rows past its chunks hold +0, which leaves a sum unchanged). Each row's sum is
    // taken within the row, then row broadcasts add the rows of a group: rows 1 and 3 add
    // rows 0 and 2, and row 3 adds row 1, so group g's totals land in every lane of row
    // (g + 1) * slot - 1, slot = 4 / gpw, summed as (S0 + S1) + (S2 + S3). Lane j * ROWS + m
    // of that row stores output (m, column j).
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int j = 0; j < COLS; ++j)
#pragma unroll
        for (int m = 0; m < ROWS; ++m) {
          const float v = group_sum8(acc[pr][j][m]);
          acc[pr][j][m] = v + dpp_read<kDppRowRor8>(v);
        }
    // One wave-uniform branch per group shape; within it the slot is a constant.
    auto finish = [&](auto slot_c) {
      constexpr int SLOT = decltype(slot_c)::value;
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
        for (int j = 0; j < COLS; ++j)
#pragma unroll
          for (int m = 0; m < ROWS; ++m) {
            float v = acc[pr][j][m];
            if constexpr (SLOT >= 2) v += dpp_read_rows<kDppRowBcast15, 0xA>(v);
            if constexpr (SLOT == 4) v += dpp_read_rows<kDppRowBcast31, 0x8>(v);
            acc[pr][j][m] = v;
          }
      const int r = lane >> 4, i = lane & 15;
      const int j = i / ROWS, m = i % ROWS;
      if (((r + 1) & (SLOT - 1)) != 0 || i >= COLS * ROWS || m >= M) return;
      // Lane i picks output i by a chain of selects over register values (made opaque, so
      // that the compiler does not turn the chain into an indexed access of a private array,
      // which it places in LDS).
      float mine[NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) mine[pr] = opaque(acc[pr][0][0]);
#pragma unroll
      for (int k = 1; k < COLS * ROWS; ++k)
#pragma unroll
        for (int pr = 0; pr < NPROJ; ++pr) {
          const float v = opaque(acc[pr][k / ROWS][k % ROWS]);
          mine[pr] = i == k ? v : mine[pr];
        }
      const int g = r / SLOT;
      const size_t o = (size_t)m * N + (wg * groups + wave * gpw + g) * COLS + j;
      float out;
      if constexpr (NPROJ == 2) {
        out = silu_mul(mine[0], mine[1]);
      } else {
        out = mine[0];
        if (p.residual) out += act_to_f32<DT>(p.residual[o]);
      }
      p.y[o] = f32_to_act<DT>(out);
    };
    if (gpw >= 4)
      finish(IntConst<1>{});
    else if (gpw == 2)
      finish(IntConst<2>{});
    else
      finish(IntConst<4>{});
  } else if constexpr (LAYOUT == kOneGroup) {
    // One group over all the workgroup's lanes: each wave adds its rows by row broadcasts
    // ((S0 + S1) + (S2 + S3), rows past K hold +0) and its last lane leaves the wave's sum
    // in LDS; the waves' sums are then added in wave order.
    __shared__ float red[kGemvMaxWaves][kOut];
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int j = 0; j < COLS; ++j)
#pragma unroll
        for (int m = 0; m < ROWS; ++m) {
          float v = group_sum8(acc[pr][j][m]);
          v += dpp_read<kDppRowRor8>(v);
          v += dpp_read_rows<kDppRowBcast15, 0xA>(v);
          v += dpp_read_rows<kDppRowBcast31, 0x8>(v);
          if (lane == 63) red[wave][(pr * COLS + j) * ROWS + m] = v;
        }
    __syncthreads();
    if (tid < COLS * ROWS) {
      const int j = tid / ROWS, m = tid % ROWS;
      float v[NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const int o = (pr * COLS + j) * ROWS + m;
        float s = red[0][o];
#pragma unroll
        for (int w = 1; w < kGemvMaxWaves; ++w)
          if (w < waves) s += red[w][o];
        v[pr] = s;
      }
      if (m < M) {
        const size_t o = (size_t)m * N + wg * COLS + j;
        float out;
        if constexpr (NPROJ == 2) {
          out = silu_mul(v[0], v[1]);
        } else {
          out = v[0];
          if (p.residual) out += act_to_f32<DT>(p.residual[o]);
        }
        p.y[o] = f32_to_act<DT>(out);
      }
    }
  } else {
    // Groups straddling waves (kStraddle): row sums through LDS, a group's rows in row order.
    __shared__ float red[kGemvMaxWaves][kOut][4];  // per wave, output and row of 16 lanes
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int j = 0; j < COLS; ++j)
#pragma unroll
        for (int m = 0; m < ROWS; ++m) {
          float v = group_sum8(acc[pr][j][m]);
          v += dpp_read<kDppRowRor8>(v);
          if ((lane & 15) == 0) red[wave][(pr * COLS + j) * ROWS + m][lane >> 4] = v;
        }
    __syncthreads();
    if (tid < groups * COLS * ROWS) {
      const int g = tid / (COLS * ROWS), j = (tid / ROWS) % COLS, m = tid % ROWS;
      const int r0 = g * (chunks / 16);
      const int r1 = r0 + chunks / 16;
      float v[NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        float s = 0.0f;
        for (int r = r0; r < r1; ++r) s += red[r >> 2][(pr * COLS + j) * ROWS + m][r & 3];
        v[pr] = s;
      }
      if (m < M) {
        const size_t o = (size_t)m * N + (wg * groups + g) * COLS + j;
        float out;
        if constexpr (NPROJ == 2) {
          out = silu_mul(v[0], v[1]);
        } else {
          out = v[0];
          if (p.residual) out += act_to_f32<DT>(p.residual[o]);
        }
        p.y[o] = f32_to_act<DT>(out);
      }
    }
  }
}

template <int BITS, int DT, int ROWS, int NPROJ, int COLS>
hipError_t launch_waves(const QmvParams& p, int waves, hipStream_t stream) {
  if (affine_gemv_one_pass(p.K, BITS, waves)) {
    const int groups = affine_gemv_groups(p.K, BITS, waves);
    if (p.K * BITS / 128 <= 64)
      affine_gemv_kernel<BITS, DT, ROWS, NPROJ, COLS, true, kWaveGroups>
          <<<p.N / (COLS * groups), 64 * waves, 0, stream>>>(p);
    else if (groups > 1)
      affine_gemv_kernel<BITS, DT, ROWS, NPROJ, COLS, true, kStraddle>
          <<<p.N / (COLS * groups), 64 * waves, 0, stream>>>(p);
    else
      affine_gemv_kernel<BITS, DT, ROWS, NPROJ, COLS, true, kOneGroup>
          <<<p.N / COLS, 64 * waves, 0, stream>>>(p);
    return hipGetLastError();
  }
  if constexpr (affine_gemv_fits(ROWS, NPROJ, COLS, false)) {
    affine_gemv_kernel<BITS, DT, ROWS, NPROJ, COLS, false, kOneGroup>
        <<<p.N / COLS, 64 * waves, 0, stream>>>(p);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

template <int BITS, int DT, int ROWS, int NPROJ>
hipError_t launch_cols(const QmvParams& p, int waves, int cols, hipStream_t stream) {
  if (cols == 2) return launch_waves<BITS, DT, ROWS, NPROJ, 2>(p, waves, stream);
  if (cols == 4) return launch_waves<BITS, DT, ROWS, NPROJ, 4>(p, waves, stream);
  if constexpr (NPROJ == 1 && ROWS <= 2) {
    if (cols == 8) return launch_waves<BITS, DT, ROWS, NPROJ, 8>(p, waves, stream);
  }
  return hipErrorInvalidValue;
}

template <int BITS, int DT, int NPROJ>
hipError_t launch_rows(const QmvParams& p, int waves, int cols, hipStream_t stream) {
  if (p.M <= 1) return launch_cols<BITS, DT, 1, NPROJ>(p, waves, cols, stream);
  if (p.M <= 2) return launch_cols<BITS, DT, 2, NPROJ>(p, waves, cols, stream);
  if (p.M <= 4) return launch_cols<BITS, DT, 4, NPROJ>(p, waves, cols, stream);
  return hipErrorInvalidValue;
}

template <int BITS, int DT>
hipError_t launch_bits_dt(const QmvParams& p, int nproj, int waves, int cols,
                          hipStream_t stream) {
  return nproj == 2 ? launch_rows<BITS, DT, 2>(p, waves, cols, stream)
                    : launch_rows<BITS, DT, 1>(p, waves, cols, stream);
}

}  // namespace

hipError_t launch_affine_gemv(const QmvParams& p, int bits, int dtype, int nproj, int waves,
                              int cols, hipStream_t stream) {
  if (p.K % 64 || p.G < 32 || waves < 1 || waves > kGemvMaxWaves ||
      p.N % (cols * affine_gemv_groups(p.K, bits, waves)) ||
      !affine_gemv_fits(p.M, nproj, cols, affine_gemv_one_pass(p.K, bits, waves)))
    return hipErrorInvalidValue;
  if (bits == 4) {
    return dtype == kBF16 ? launch_bits_dt<4, kBF16>(p, nproj, waves, cols, stream)
                          : launch_bits_dt<4, kF16>(p, nproj, waves, cols, stream);
  }
  return dtype == kBF16 ? launch_bits_dt<8, kBF16>(p, nproj, waves, cols, stream)
                        : launch_bits_dt<8, kF16>(p, nproj, waves, cols, stream);
}

}  // namespace mt

// Prefill affine quantized GEMM for gfx950: y[M, N] = x[M, K] @ dequantize(w_q)[N, K]^T for
// many rows (reference: lower_affine_matmul, metile/compiler/affine_quantized.py:7-99, and its
// dispatcher mlx_affine_matmul, metile/backends/mlx_affine.py:359-406).
//
// Design: a workgroup of WM x WN waves computes a (32 TM WM) x (32 TN WN) output tile; each
// wave owns TM x TN tiles of MFMA 32x32x16 (fp32 accumulate). The K loop runs in 64-wide steps
// through a double-buffered LDS pipeline with one barrier per step: the next step's activation
// tile and packed codes are loaded into registers while the current step's MFMAs run from LDS,
// then stored to the other buffer: the codes as exact 16-bit floats (offset + q), the
// activations as loaded, and each column's scale.
// Dequantization stays exact: each step's MFMA partial t = sum_k x_k (offset + q_k) gets its
// group's affine terms in fp32, acc += s * t + (b - offset * s) * X with X = sum_k x_k, as in
// the small-row kernel. X is summed while staging: eight lanes hold a row's eight 16-byte
// chunks (dot products with ones) and combine with DPP moves. Rows beyond M and columns beyond
// N read zero through the buffer range check and are not stored.
#include "common.h"
#include "affine_gemm.h"

namespace mt {

namespace {

constexpr int kBK = 64;        // K per pipeline step
constexpr int kPad = 8;        // LDS row padding, in 16-bit elements
constexpr int kLdsRow = kBK + kPad;

template <int DT, int WM, int WN, int TM, int TN>
__global__ __launch_bounds__(64 * WM * WN, 2) void affine_gemm_kernel(const GemmParams p) {
  constexpr int kThreads = 64 * WM * WN;
  constexpr int BM = 32 * TM * WM;
  constexpr int BN = 32 * TN * WN;
  constexpr int kAChunks = BM * kBK * 2 / 16 / kThreads;  // 16-byte activation chunks/thread
  constexpr float kOff = CodeOffset<4, DT>::value;
  static_assert(kAChunks >= 1 && BM * kBK * 2 / 16 % kThreads == 0, "tile too small");
  static_assert(2 * BN <= kThreads, "one thread per half column of codes");

  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][kLdsRow];
  __shared__ __attribute__((aligned(16))) float Xs[2][BM];   // per-row sums of the step
  __shared__ float Ss[2][BN], Bp[2][BN];                     // scale, bias - offset*scale

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int j = lane & 31, h = lane >> 5;
  const int M = p.M, K = p.K, N = p.N;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int steps = K / kBK;
  const int s_beg = blockIdx.z * p.steps_per_split;
  const int s_end = min(steps, s_beg + p.steps_per_split);

  const uint32_t row_bytes = (uint32_t)K / 2u;
  const int gshift = __builtin_ctz((unsigned)p.G);  // groups are powers of two
  const int groups_per_row = K >> gshift;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, (uint32_t)N * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.s, (uint32_t)N * groups_per_row * 2u);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, (uint32_t)N * groups_per_row * 2u);

  // Activation tile: chunk c = tid + kThreads i covers row c / 8, 16 bytes (c % 8) of the step;
  // the eight chunks of a row sit in eight consecutive lanes (kThreads is a multiple of 8).
  uint32_t a_off[kAChunks];
  int a_row[kAChunks], a_col[kAChunks];
#pragma unroll
  for (int i = 0; i < kAChunks; ++i) {
    const int c = tid + kThreads * i;
    a_row[i] = c >> 3;
    a_col[i] = (c & 7) * 8;
    const int gr = m0 + a_row[i];
    a_off[i] = gr < M ? ((uint32_t)gr * K + a_col[i]) * 2u : kOOB;
  }
  // Codes: thread t < 2*BN loads K half (t & 1) of column t >> 1 (16 bytes = 32 codes).
  const bool b_active = tid < 2 * BN;
  const int b_col = tid >> 1, b_half = tid & 1;
  const int gcol = n0 + b_col;
  const bool col_ok = b_active && gcol < N;
  const uint32_t b_off = col_ok ? (uint32_t)gcol * row_bytes + 16u * b_half : kOOB;
  const uint32_t g_off = col_ok ? (uint32_t)gcol * groups_per_row * 2u : kOOB;

  u32x4 ra[kAChunks];
  u32x4 rc;
  uint32_t rsv, rbv;
  auto load_step = [&](int st) {
#pragma unroll
    for (int i = 0; i < kAChunks; ++i)
      ra[i] = load16(rx, a_off[i] == kOOB ? kOOB : a_off[i] + (uint32_t)st * 128u);
    rc = load16(rw, b_off == kOOB ? kOOB : b_off + (uint32_t)st * 32u);
    const uint32_t go = g_off == kOOB ? kOOB : g_off + (uint32_t)((st * kBK) >> gshift) * 2u;
    rsv = load2(rs, go);
    rbv = load2(rb, go);
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kAChunks; ++i) {
      *reinterpret_cast<u32x4*>(&As[buf][a_row[i]][a_col[i]]) = ra[i];
      // Row sum of the step: this lane's eight elements, then the row's eight lanes.
      const float sum = group_sum8(sum8<DT>(ra[i], 0.0f));
      if ((tid & 7) == 0) Xs[buf][a_row[i]] = sum;
    }
    if (b_active) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x4*>(&Bs[buf][b_col][32 * b_half + 8 * q]) = unpack_u4<DT>(rc[q]);
      if (b_half == 0) {
        const float sf = act_to_f32<DT>(rsv);
        Ss[buf][b_col] = sf;
        Bp[buf][b_col] = __builtin_fmaf(-kOff, sf, act_to_f32<DT>(rbv));
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = (f32x16){0};

  if (s_beg < s_end) {
    load_step(s_beg);
    store_step(0);
  }
  __syncthreads();
  const f32x16 zero16 = (f32x16){0};
  for (int st = s_beg; st < s_end; ++st) {
    const int buf = (st - s_beg) & 1;
    const bool more = st + 1 < s_end;
    if (more) load_step(st + 1);
    f32x16 t[TM][TN];
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      u32x4 af[TM], bfr[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a)
        af[a] = *reinterpret_cast<const u32x4*>(
            &As[buf][wm * 32 * TM + 32 * a + j][16 * kk + 8 * h]);
#pragma unroll
      for (int b = 0; b < TN; ++b)
        bfr[b] = *reinterpret_cast<const u32x4*>(
            &Bs[buf][wn * 32 * TN + 32 * b + j][16 * kk + 8 * h]);
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          t[a][b] = mfma32<DT>(af[a], bfr[b], kk == 0 ? zero16 : t[a][b]);
    }
    // Affine terms of the step's group, per column (lane) and row (register).
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int col = wn * 32 * TN + 32 * b + j;
      const float sf = Ss[buf][col];
      const float bp = Bp[buf][col];
#pragma unroll
      for (int a = 0; a < TM; ++a) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 xs = *reinterpret_cast<const f32x4*>(
              &Xs[buf][wm * 32 * TM + 32 * a + 8 * r4 + 4 * h]);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 4 * r4 + v;
            acc[a][b][r] = __builtin_fmaf(sf, t[a][b][r], acc[a][b][r]);
            acc[a][b][r] = __builtin_fmaf(bp, xs[v], acc[a][b][r]);
          }
        }
      }
    }
    // The other buffer was last read in the previous step, before that step's barrier.
    if (more) store_step(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: fp32 tile -> activation type (or split-K fp32 partials) -----------------
  // Partials go out as device-coherent buffer stores (cache policy sc1), all in flight at once;
  // one wait below covers them before the arrival counter moves. (As relaxed atomic stores each
  // had waited for the one before it: 16 to 64 serialized stores per lane.)
  const __amdgpu_buffer_rsrc_t rp =
      make_rsrc(p.partial, p.ksplit > 1 ? (uint32_t)p.ksplit * (uint32_t)M * (uint32_t)N * 4u : 0u);
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 32 * TM + 32 * a + mfma32_row(r, h);
        const int col = n0 + wn * 32 * TN + 32 * b + j;
        if (row < M && col < N) {
          if (p.ksplit == 1) {
            p.y[(size_t)row * N + col] = f32_to_act<DT>(acc[a][b][r]);
          } else {
            // (__float_as_uint: __builtin_bit_cast of a vector element reads its first word.)
            __builtin_amdgcn_raw_buffer_store_b32(
                __float_as_uint(acc[a][b][r]), rp,
                (((uint32_t)blockIdx.z * M + row) * (uint32_t)N + col) * 4u, 0, kDeviceScope);
          }
        }
      }
  if (p.ksplit == 1) return;

  // Split-K: the last workgroup of an output tile sums the partials in split order.
  __shared__ int last_flag;
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  if (tid == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (prev == (unsigned)(p.ksplit - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  for (int o = tid; o < BM * BN; o += kThreads) {
    const int row = m0 + o / BN, col = n0 + o % BN;
    if (row >= M || col >= N) continue;
    const float v = sum_partials(p.partial + (size_t)row * N + col, (size_t)M * N, p.ksplit);
    p.y[(size_t)row * N + col] = f32_to_act<DT>(v);
  }
  if (tid == 0)
    __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int WM, int WN, int TM, int TN>
hipError_t launch_tile(const GemmParams& p, hipStream_t stream) {
  constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
  const dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, p.ksplit);
  affine_gemm_kernel<DT, WM, WN, TM, TN><<<grid, 64 * WM * WN, 0, stream>>>(p);
  return hipGetLastError();
}

// 128 x 128 tiles: four waves of 64 x 64; 64 x 64 tiles: four waves of 32 x 32.
template <int DT>
hipError_t launch_dt(const GemmParams& p, hipStream_t stream) {
  if (p.tile == 2) return launch_tile<DT, 2, 2, 2, 2>(p, stream);
  return launch_tile<DT, 2, 2, 1, 1>(p, stream);
}

}  // namespace

hipError_t launch_affine_gemm(const GemmParams& p, int dtype, hipStream_t stream) {
  return dtype == kBF16 ? launch_dt<kBF16>(p, stream) : launch_dt<kF16>(p, stream);
}

}  // namespace mt

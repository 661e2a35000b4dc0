// Column-block small-row affine projections (M <= 32, groups of 64 or more) for gfx950.
//
// Same contract as the other small-row kernels: y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/G] +
// b[n, k/G]) in fp32 (kernels/affine_qmv.py:4-54), with the residual (:124-132) or SwiGLU
// (:204-214) epilogue (mlx_affine_qmv, mlx_affine_residual_qmv, mlx_affine_swiglu,
// metile/backends/mlx_quantized.py:691-751,1538-1720).
//
// A workgroup owns a block of up to 64 output columns over the K range of its split. Its waves
// take consecutive runs of K steps (64 wide), each over EVERY column of the block, so that the
// activations of a step are read once per workgroup, straight from global memory into the MFMA
// operand layout, and serve all of the block's 16-column tiles and both projections. The cost of
// a K step is then the same at 1 and at 16 rows: per 16-column tile and projection one 8-byte
// (4-bit) or 16-byte (8-bit) code load per lane and two v_mfma_f32_16x16x32, whatever M is.
// Layout of a step on the matrix cores (lane l: i = l % 16, g = l / 16):
//  * A = activations: lane l holds row 16 rt + i, K slice [16 g + 8 kk, + 8) for MFMA kk;
//  * B = codes: lane l holds column 16 t + i, the same K slices (codes [16 g, 16 g + 16) of the
//    step: one 8-byte load at 4 bits, 16 bytes at 8 bits), unpacked to exact offset + q floats
//    (4-bit words in the paired order, the activations permuted alike);
//  * result: lane l holds rows 16 rt + 4 g + r (r = 0..3) of column 16 t + i.
// An MFMA of the activations against a constant operand (-offset, or 1 where the codes carry no
// offset) gives -offset X (or X), X the step's row sums, already in the result layout. Each
// tile's chain starts from -offset X, so it sums x * q exactly inside the fp32 accumulation; the
// group's affine terms follow in fp32: acc += s t + (b / -offset) (-offset X).
// Scales and biases of the block and split are staged in LDS once (buffer_load...lds). After the
// K loop the waves' sums meet in LDS and are added in wave order; a split-K dispatch then follows
// the deterministic partial-sum protocol of the staged kernel.
#include <type_traits>

#include "common.h"
#include "affine_qmv.h"

namespace mt {
namespace {

// Steps of code and activation loads each wave keeps in flight: as many as about 128 registers
// hold (at most 8, at least 2). A wave's loads of a step wait behind one HBM round trip; a ring
// shorter than the wave's run of steps pays another round trip per refill.
__host__ __device__ constexpr int block_ring(int bits, int nproj, int row_tiles, int tiles) {
  const int per_step = 8 * row_tiles + tiles * nproj * (bits / 2);  // VGPRs of one stage
  const int d = (128 - 4 * tiles * nproj * row_tiles) / per_step;
  return d < 2 ? 2 : d > 3 ? 3 : d;
}

template <int BITS, int DT, int NPROJ, int RT, int TPB>
__global__ __launch_bounds__(64 * kBlockMaxWaves) void affine_block_kernel(const QmvParams args) {
  const QmvParams p = preload_args(args);
  constexpr int D = block_ring(BITS, NPROJ, RT, TPB);
  constexpr int kCols = 16 * TPB;
  constexpr float kOff = SumOffset<BITS, DT>::value;
  // B operand of the row-sum MFMA: -offset (two 16-bit floats per word), or 1 when the codes
  // multiplied are the integers themselves (8-bit bf16, f16); the bias then multiplies by
  // kXScale of it.
  constexpr uint32_t kXB = kOff == 0.0f ? (DT == kBF16 ? 0x3F803F80u : 0x3C003C00u)
                                        : (DT == kBF16 ? (BITS == 4 ? 0xC300C300u : 0u)
                                                       : 0xE400E400u);
  static_assert(kOff == 0.0f || kOff == 128.0f || kOff == 1024.0f, "code offset");
  constexpr float kXScale = kOff == 0.0f ? 1.0f : -1.0f / kOff;  // exact: a power of two
  constexpr int kCodeLoads = TPB * NPROJ;
  constexpr int kLoadsPerStage = 2 * RT + kCodeLoads;
  static_assert(D * kLoadsPerStage < 64, "loads in flight exceed the vmcnt range");
  typedef typename std::conditional<BITS == 4, u32x2, u32x4>::type CodeT;

  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ int last_flag;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  const int M = p.M, K = p.K, N = p.N;
  int col0, width;
  if (p.strip_cols) {
    col0 = blockIdx.x * p.strip_cols;
    width = p.strip_cols;
  } else {
    const int units = N / p.col_align;
    col0 = (int)(((int64_t)blockIdx.x * units) / p.strips) * p.col_align;
    width = (int)(((int64_t)(blockIdx.x + 1) * units) / p.strips) * p.col_align - col0;
  }
  const int steps = K >> 6;
  const int split = blockIdx.y;
  const int s_beg = split * p.steps_per_split;
  const int s_end = min(steps, s_beg + p.steps_per_split);
  const int w_beg = s_beg + wave * p.wave_steps;
  const int w_end = min(s_end, w_beg + p.wave_steps);
  const int gshift = p.group_shift;
  const int gpr = p.groups_per_row;
  const int g_beg = s_beg >> gshift;
  const int sbw = p.sb_words;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr)
    rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * (uint32_t)(K * BITS / 8));

  // ---- scales and biases of the block and split: LDS row (2 pr + a) * kCols + c holds sbw
  // dwords (a power of two, at least 4) of column col0 + c's array a (0 scales, 1 biases), from
  // the even element at or below group g_beg. Load d fills LDS words [64 d, 64 d + 64): rows of
  // one array only (64 / sbw rows, or a part of one row, and kCols is a multiple of 16), so its
  // buffer descriptor is wave-uniform.
  {
    const int sh = __builtin_ctz((unsigned)sbw);
    const int loads = (2 * NPROJ * kCols * sbw) >> 6;
    for (int d = wave; d < loads; d += waves) {
      const int q = d * 64 + lane;
      const int row = q >> sh;
      const int wd = q & (sbw - 1);
      const int arr = __builtin_amdgcn_readfirstlane(((d * 64) >> sh) / kCols);  // 2 pr + a
      const int c = row - arr * kCols;
      const uint32_t first = ((uint32_t)(col0 + c) * (uint32_t)gpr + (uint32_t)g_beg) & ~1u;
      const uint32_t off = oob_unless(c < width, (first + 2u * (uint32_t)wd) * 2u);
      // Selected with constant indices only: an index into the argument block would move it to
      // scratch and make every buffer descriptor per-lane.
      const uint16_t* src = arr == 0 ? p.s[0] : arr == 1 ? p.b[0] : arr == 2 ? p.s[NPROJ - 1]
                                                                             : p.b[NPROJ - 1];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(src, (uint32_t)N * (uint32_t)gpr * 2u),
                                               (lds_ptr_t)(dyn + d * 256), 4, off, 0, 0, 0);
    }
  }

  // ---- the code and activation ring -------------------------------------------------------
  struct Stage {
    u32x4 a[RT][2];
    CodeT c[TPB][NPROJ];
  };
  uint32_t a_off[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = 16 * rt + i16;
    a_off[rt] = oob_unless(row < M, ((uint32_t)row * (uint32_t)K + 16u * (uint32_t)g) * 2u);
  }
  uint32_t c_off[TPB];
#pragma unroll
  for (int t = 0; t < TPB; ++t) {
    const int c = 16 * t + i16;
    c_off[t] = oob_unless(c < width, (uint32_t)(col0 + c) * p.col_stride +
                                         (uint32_t)g * (uint32_t)(2 * BITS));
  }
  auto issue = [&](Stage& S, int st) {
    const bool ok = st < w_end;
    const uint32_t xo = (uint32_t)st * 128u;
    const uint32_t co = (uint32_t)st * p.step_stride;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        S.a[rt][kk] = load16(rx, oob_unless(ok, a_off[rt] + xo + 16u * kk));
#pragma unroll
    for (int t = 0; t < TPB; ++t)
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        if constexpr (BITS == 4)
          S.c[t][pr] = load8_nt(rw[pr], oob_unless(ok, c_off[t] + co));
        else
          S.c[t][pr] = load16_nt(rw[pr], oob_unless(ok, c_off[t] + co));
      }
  };

  Stage ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d) issue(ring[d], w_beg + d);
  // The staged scales: this wave's loads done (only the ring's are younger), then everyone's.
  wait_vmcnt<D * kLoadsPerStage>();
  __syncthreads();

  f32x4 acc[TPB][NPROJ][RT];
#pragma unroll
  for (int t = 0; t < TPB; ++t)
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[t][pr][rt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const f32x4 zero4 = (f32x4){0.f, 0.f, 0.f, 0.f};
  const u32x4 xb = (u32x4){kXB, kXB, kXB, kXB};
  const PairedConsts pc = paired_consts<DT>();
  const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(dyn);
  // Element of (array row, group) of this lane's column: the row's first dword starts at the
  // even element at or below g_beg, so groups start at element sh0 (16 t more columns of gpr
  // groups keep the parity).
  const int sh0 = ((col0 + i16) * gpr + g_beg) & 1;
  const int srow = i16 * 2 * sbw + sh0;  // u16 index of column i16's row, array 0

  auto compute = [&](const Stage& S, int st) {
    // Scales and biases first (their LDS latency hides behind the MFMAs), then every MFMA chain
    // of the step, then the fix-ups: a chain's fix-up waits for its MFMA results, and with the
    // chains issued back to back only the first wait is exposed.
    const int gl = (st >> gshift) - g_beg;
    uint32_t sv[TPB][NPROJ], bv[TPB][NPROJ];
#pragma unroll
    for (int t = 0; t < TPB; ++t)
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const int e = ((2 * pr) * kCols + 16 * t) * 2 * sbw + srow + gl;
        sv[t][pr] = sb16[e];
        bv[t][pr] = sb16[e + kCols * 2 * sbw];
      }
    u32x4 a[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) a[rt][kk] = BITS == 4 ? pair_order(S.a[rt][kk]) : S.a[rt][kk];
    f32x4 tx[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      tx[rt] = mfma16<DT>(a[rt][0], xb, zero4);
      tx[rt] = mfma16<DT>(a[rt][1], xb, tx[rt]);
    }
    f32x4 tt[TPB][NPROJ][RT];
#pragma unroll
    for (int t = 0; t < TPB; ++t)
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        u32x4 b0, b1;
        if constexpr (BITS == 4) {
          b0 = codes_for_sum<DT>(unpack_u4_paired(S.c[t][pr].x, pc));
          b1 = codes_for_sum<DT>(unpack_u4_paired(S.c[t][pr].y, pc));
        } else {
          const CodeT w = S.c[t][pr];
          const u32x2 l0 = unpack_u8<DT>(w.x), l1 = unpack_u8<DT>(w.y);
          const u32x2 h0 = unpack_u8<DT>(w.z), h1 = unpack_u8<DT>(w.w);
          b0 = codes_for_sum<DT>((u32x4){l0.x, l0.y, l1.x, l1.y});
          b1 = codes_for_sum<DT>((u32x4){h0.x, h0.y, h1.x, h1.y});
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          tt[t][pr][rt] = mfma16<DT>(a[rt][0], b0, kOff == 0.0f ? zero4 : tx[rt]);
          tt[t][pr][rt] = mfma16<DT>(a[rt][1], b1, tt[t][pr][rt]);
        }
      }
#pragma unroll
    for (int t = 0; t < TPB; ++t)
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const float sf = act_to_f32<DT>(sv[t][pr]);
        const float bq = act_to_f32<DT>(bv[t][pr]) * kXScale;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[t][pr][rt][r] = __builtin_fmaf(sf, tt[t][pr][rt][r], acc[t][pr][rt][r]);
            acc[t][pr][rt][r] = __builtin_fmaf(bq, tx[rt][r], acc[t][pr][rt][r]);
          }
      }
  };

  // Rounds of D steps; a round with steps after it refills every stage (a refill past the
  // wave's last step reads nothing), so wait counts are exact; the last round refills nothing.
  int s0 = w_beg;
  for (; s0 + D < w_end; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      compute(ring[d], s0 + d);
      issue(ring[d], s0 + d + D);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (s0 + d < w_end) compute(ring[d], s0 + d);

  // ---- cross-wave reduction in wave order (the buffer reuses the staged scales) ------------
  // Wave w leaves its accumulators at red4[(w kSlots + slot) 64 + lane], slot = (t NPROJ + pr)
  // RT + rt. Thread (t, rt, lane) then adds its four outputs (rows 16 rt + 4 g + r of column
  // 16 t + i) over the waves, both projections at once.
  constexpr int kSlots = TPB * NPROJ * RT;  // f32x4 per lane
  __syncthreads();
  f32x4* red4 = reinterpret_cast<f32x4*>(dyn);
#pragma unroll
  for (int t = 0; t < TPB; ++t)
#pragma unroll
    for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        red4[(wave * kSlots + (t * NPROJ + pr) * RT + rt) * 64 + lane] = acc[t][pr][rt];
  __syncthreads();
  constexpr int kJobs = TPB * RT * 64;  // (t, rt, lane)
  const int threads = blockDim.x;
  const size_t plane = (size_t)M * N;
  if (p.ksplit > 1) {
    // Split-K: partials as device-scope stores; the last workgroup of the block adds them in
    // split order (the staged kernel's protocol).
    for (int j = tid; j < kJobs; j += threads) {
      const int l = j & 63, tr = j >> 6, t = tr / RT, rt = tr - t * RT;
      const int c = 16 * t + (l & 15), m0 = 16 * rt + 4 * (l >> 4);
      if (c >= width || m0 >= M) continue;
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const int slot = (t * NPROJ + pr) * RT + rt;
        f32x4 v = red4[slot * 64 + l];
        for (int w = 1; w < waves; ++w) v += red4[(w * kSlots + slot) * 64 + l];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (m0 + r < M)
            __hip_atomic_store(&p.partial[(size_t)(split * NPROJ + pr) * plane +
                                          (size_t)(m0 + r) * N + col0 + c],
                               v[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&p.counters[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      last_flag = (prev == (unsigned)(p.ksplit - 1));
    }
    __syncthreads();
    if (!last_flag) return;
  }
  for (int j = tid; j < kJobs; j += threads) {
    const int l = j & 63, tr = j >> 6, t = tr / RT, rt = tr - t * RT;
    const int c = 16 * t + (l & 15), m0 = 16 * rt + 4 * (l >> 4);
    if (c >= width || m0 >= M) continue;
    f32x4 v[NPROJ];
    if (p.ksplit == 1) {
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const int slot = (t * NPROJ + pr) * RT + rt;
        v[pr] = red4[slot * 64 + l];
        for (int w = 1; w < waves; ++w) v[pr] += red4[(w * kSlots + slot) * 64 + l];
      }
    } else {
      // the job's 4 NPROJ outputs over all splits, their loads in flight together
      const float* src[4 * NPROJ];
      float sum[4 * NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          src[pr * 4 + r] = m0 + r < M ? p.partial + (size_t)pr * plane +
                                             (size_t)(m0 + r) * N + col0 + c
                                       : nullptr;
      sum_partials_multi<4 * NPROJ>(src, (size_t)NPROJ * plane, p.ksplit, sum);
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr)
#pragma unroll
        for (int r = 0; r < 4; ++r) v[pr][r] = sum[pr * 4 + r];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (m0 + r >= M) break;
      const size_t o = (size_t)(m0 + r) * N + col0 + c;
      float out;
      if constexpr (NPROJ == 2) {
        out = silu_mul(v[0][r], v[1][r]);
      } else {
        out = v[0][r];
        if (p.residual) out += act_to_f32<DT>(p.residual[o]);
      }
      p.y[o] = f32_to_act<DT>(out);
    }
  }
  if (p.ksplit > 1 && tid == 0)
    __hip_atomic_store(&p.counters[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int BITS, int DT, int NPROJ, int RT, int TPB>
hipError_t launch_block_tpb(const QmvParams& p, int waves, hipStream_t stream) {
  if constexpr (!block_fits_registers(TPB, NPROJ, RT)) {
    return hipErrorInvalidValue;
  } else {
  auto kernel = affine_block_kernel<BITS, DT, NPROJ, RT, TPB>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
      (int)kBlockMaxLds);
  if (attr != hipSuccess) return attr;
  const uint32_t lds = block_lds_bytes(waves, TPB, NPROJ, RT, p.sb_words);
  if (lds > kBlockMaxLds) return hipErrorInvalidValue;
  kernel<<<dim3(p.strips, p.ksplit), dim3(64 * waves), lds, stream>>>(p);
  return hipGetLastError();
  }
}

template <int BITS, int DT, int NPROJ, int RT>
hipError_t launch_block_rt(const QmvParams& p, int waves, int tiles, hipStream_t stream) {
  switch (tiles) {
    case 1: return launch_block_tpb<BITS, DT, NPROJ, RT, 1>(p, waves, stream);
    case 2: return launch_block_tpb<BITS, DT, NPROJ, RT, 2>(p, waves, stream);
    case 3: return launch_block_tpb<BITS, DT, NPROJ, RT, 3>(p, waves, stream);
    case 4: return launch_block_tpb<BITS, DT, NPROJ, RT, 4>(p, waves, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int BITS, int DT, int NPROJ>
hipError_t launch_block_nproj(const QmvParams& p, int waves, int tiles, hipStream_t stream) {
  return p.M <= 16 ? launch_block_rt<BITS, DT, NPROJ, 1>(p, waves, tiles, stream)
                   : launch_block_rt<BITS, DT, NPROJ, 2>(p, waves, tiles, stream);
}

template <int BITS, int DT>
hipError_t launch_block_bits_dt(const QmvParams& p, int nproj, int waves, int tiles,
                                hipStream_t stream) {
  return nproj == 2 ? launch_block_nproj<BITS, DT, 2>(p, waves, tiles, stream)
                    : launch_block_nproj<BITS, DT, 1>(p, waves, tiles, stream);
}

}  // namespace

hipError_t launch_affine_block(const QmvParams& p, int bits, int dtype, int nproj, int waves,
                               int tiles, hipStream_t stream) {
  if (p.M < 1 || p.M > kBlockMaxRows || p.G < 64 || waves < 1 || waves > kBlockMaxWaves ||
      p.wave_steps < 1 || (int64_t)p.wave_steps * waves < p.steps_per_split)
    return hipErrorInvalidValue;
  if (bits == 4)
    return dtype == kBF16 ? launch_block_bits_dt<4, kBF16>(p, nproj, waves, tiles, stream)
                          : launch_block_bits_dt<4, kF16>(p, nproj, waves, tiles, stream);
  return dtype == kBF16 ? launch_block_bits_dt<8, kBF16>(p, nproj, waves, tiles, stream)
                        : launch_block_bits_dt<8, kF16>(p, nproj, waves, tiles, stream);
}

}  // namespace mt

// One-to-four-row affine QMV / SwiGLU on v_mfma_f32_4x4x4 (gfx950), 4-bit codes: the same
// semantics as the other small-row kernels (kernels/affine_qmv.py:4-54 with the residual and
// SwiGLU epilogues :124-132, :204-214; mlx_affine_qmv, mlx_affine_residual_qmv,
// mlx_affine_swiglu, metile/backends/mlx_quantized.py:691-751,1538-1720).
//
// A workgroup owns 4, 8 or 16 output columns (CG groups of 4, of each projection) and all of K;
// its waves split K into rounds of 512. In a round, the 16 blocks of the 4x4x4 MFMA take 16 segments of 32 K (block b:
// K0 + 32 b): lane l = 4 b + q supplies activation row q (A) and code column q (B), four K of its
// segment per MFMA, eight MFMAs per segment, so one 16-byte code load per lane and column group
// feeds a whole round and every code is multiplied once by all four rows. Codes are unpacked to
// exact 16-bit floats offset + q in the paired order of each word (the activations permuted
// alike). bf16: an MFMA chain of the activations against -offset gives -offset times each
// segment's row sums, and every column's chain starts from it, so it sums x * q in fp32; f16
// (offset 1024) subtracts the offset from the codes first (packed 16-bit, exact) and takes the
// row sums against 1. A segment lies in one group (groups of 32 or more), so each block applies
// its group's affine terms to its own chain: acc += s t + b X. After the K loop the 16 blocks of a lane
// column are added by lane exchanges within rows of 16 lanes and in LDS across rows and waves,
// in a fixed order, then the epilogue.
#include "common.h"
#include "affine_qmv.h"

namespace mt {
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// 4x4x4 MFMA of 16 blocks: a and b hold four 16-bit floats each (two per word).
template <int DT>
__device__ __forceinline__ f32x4 mfma4(u32x2 a, u32x2 b, f32x4 c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a),
                                                  __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, a),
                                              __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

constexpr int kRoundK = 512;  // K per round: 16 blocks x 32
constexpr int kDppRowRor4 = 0x124;  // row_ror:4 (lane i reads lane i + 4 of its row)
constexpr int kDppRowRor8x = 0x128;  // row_ror:8

// ROWS: activation rows the instance holds (1, 2 or 4; lanes of rows >= M read zeros).
// CG: groups of 4 columns per workgroup (of each projection), sharing the activation operands and
// their row sums. RPW: rounds per wave (the wave's loads for all of them are issued at once).
template <int DT, int ROWS, int NPROJ, int CG, int RPW>
__global__ __launch_bounds__(64 * kGemv4MaxWaves) void affine_gemv4_kernel(const QmvParams args) {
  const QmvParams p = preload_args(args);
  constexpr float kOff = CodeOffset<4, DT>::value;
  // B operand of the row-sum chain: -offset (bf16), or 1 (f16, whose codes lose the offset
  // before the MFMA: 1024 + q against an offset of 1024 would cost the fp32 chain 7 more bits
  // than bf16's 128 + q).
  constexpr uint32_t kXB2 = DT == kBF16 ? 0xC300C300u : 0x3C003C00u;
  constexpr int kSlots = NPROJ * CG;  // column groups of the workgroup, projection-major
  static_assert(RPW * gemv4_loads_per_round(NPROJ, CG) < 64, "loads in flight exceed vmcnt");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int b = lane >> 2, q = lane & 3;
  const int M = p.M, K = p.K, N = p.N;
  const int c0 = blockIdx.x * 4 * CG;
  const int rounds = (K + kRoundK - 1) / kRoundK;
  const int r_beg = wave * RPW;
  const int gshift = __builtin_ctz((unsigned)p.G);
  const int gpr = p.groups_per_row;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
  __amdgpu_buffer_rsrc_t rw[NPROJ], rs[NPROJ], rb[NPROJ];
#pragma unroll
  for (int pr = 0; pr < NPROJ; ++pr) {
    rw[pr] = make_rsrc(p.w[pr], (uint32_t)N * (uint32_t)(K / 2));
    rs[pr] = make_rsrc(p.s[pr], (uint32_t)N * (uint32_t)gpr * 2u);
    rb[pr] = make_rsrc(p.b[pr], (uint32_t)N * (uint32_t)gpr * 2u);
  }

  // ---- every load of the wave's rounds, in round order ------------------------------------
  struct Round {
    u32x4 x[4];           // row q, K [32 b, 32 b + 32) of the round: 8 values per load
    u32x4 w[kSlots];      // column c0 + 4 cg + q of each projection, the same 32 codes
    uint32_t s[kSlots], bias[kSlots];
  };
  Round R[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int k = (r_beg + r) * kRoundK + 32 * b;  // the lane's segment
    const bool ok = r_beg + r < rounds && k < K;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      R[r].x[v] = load16(rx, oob_unless(ok && q < M, ((uint32_t)q * K + k + 8 * v) * 2u));
    const uint32_t wk = (uint32_t)(k >> 6) * p.step_stride + 16u * (uint32_t)((k >> 5) & 1);
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      const uint32_t col = (uint32_t)(c0 + 4 * cg + q);
      const uint32_t go = (col * (uint32_t)gpr + (uint32_t)(k >> gshift)) * 2u;
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        R[r].w[pr * CG + cg] = load16_nt(rw[pr], oob_unless(ok, col * p.col_stride + wk));
        R[r].s[pr * CG + cg] = load2(rs[pr], oob_unless(ok, go));
        R[r].bias[pr * CG + cg] = load2(rb[pr], oob_unless(ok, go));
      }
    }
  }

  f32x4 acc[kSlots];
#pragma unroll
  for (int c = 0; c < kSlots; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const PairedConsts pc = paired_consts<DT>();
  const u32x2 xb = (u32x2){kXB2, kXB2};
  const f32x4 zero4 = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto round = [&](const Round& S) {
    // A operands in the paired order: word u of the codes (K 8u .. 8u + 7) feeds MFMAs 2u
    // (pairs (0,4), (1,5)) and 2u + 1 (pairs (2,6), (3,7)).
    u32x4 a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = pair_order(S.x[u]);
    // tx: -offset X (bf16) or X (f16), X the segment's row sums
    f32x4 tx = zero4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      tx = mfma4<DT>((u32x2){a[u].x, a[u].y}, xb, tx);
      tx = mfma4<DT>((u32x2){a[u].z, a[u].w}, xb, tx);
    }
    f32x4 t[kSlots];
#pragma unroll
    for (int c = 0; c < kSlots; ++c) t[c] = DT == kBF16 ? tx : zero4;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < kSlots; ++c) {
        const u32x4 cw = codes_for_sum<DT>(unpack_u4_paired(S.w[c][u], pc));
        t[c] = mfma4<DT>((u32x2){a[u].x, a[u].y}, (u32x2){cw.x, cw.y}, t[c]);
        t[c] = mfma4<DT>((u32x2){a[u].z, a[u].w}, (u32x2){cw.z, cw.w}, t[c]);
      }
#pragma unroll
    for (int c = 0; c < kSlots; ++c) {
      const float sf = act_to_f32<DT>(S.s[c]);
      // exact: a power of two (bf16), or 1
      const float bq = act_to_f32<DT>(S.bias[c]) * (DT == kBF16 ? -1.0f / kOff : 1.0f);
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        acc[c][r] = __builtin_fmaf(sf, t[c][r], acc[c][r]);
        acc[c][r] = __builtin_fmaf(bq, tx[r], acc[c][r]);
      }
    }
  };
  // (the compiler's wait counts let round r start once its own loads have arrived)
#pragma unroll
  for (int r = 0; r < RPW; ++r) round(R[r]);

  // ---- the 16 blocks of each lane column: rows of 16 lanes (4 blocks each) by DPP, then the
  // four rows and the waves in LDS, in a fixed order ------------------------------------------
  __shared__ float red[kGemv4MaxWaves][4][kSlots * ROWS][4];  // [wave][lane row][value][column]
#pragma unroll
  for (int c = 0; c < kSlots; ++c)
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float v = acc[c][r];
      v += dpp_read<kDppRowRor4>(v);
      v += dpp_read<kDppRowRor8x>(v);
      if ((lane & 15) < 4) red[wave][lane >> 4][c * ROWS + r][q] = v;
    }
  __syncthreads();
  // thread (r, cg, j): row r of column c0 + 4 cg + j
  if (tid < 4 * CG * ROWS) {
    const int j = tid & 3, cg = (tid >> 2) % CG, r = tid / (4 * CG);
    if (r < M) {
      float v[NPROJ];
#pragma unroll
      for (int pr = 0; pr < NPROJ; ++pr) {
        const int e = (pr * CG + cg) * ROWS + r;
        float s = 0.0f;
        for (int w = 0; w < waves; ++w)
#pragma unroll
          for (int lr = 0; lr < 4; ++lr) s += red[w][lr][e][j];
        v[pr] = s;
      }
      const size_t o = (size_t)r * N + c0 + 4 * cg + j;
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

template <int DT, int ROWS, int NPROJ, int CG>
hipError_t launch_cg(const QmvParams& p, int waves, hipStream_t stream) {
  const int rounds = (p.K + kRoundK - 1) / kRoundK;
  const int rpw = (rounds + waves - 1) / waves;
  const dim3 grid(p.N / (4 * CG)), block(64 * waves);
  constexpr int kLoads = gemv4_loads_per_round(NPROJ, CG);
  switch (rpw) {
    case 1: affine_gemv4_kernel<DT, ROWS, NPROJ, CG, 1><<<grid, block, 0, stream>>>(p); break;
    case 2:
      if constexpr (2 * kLoads < 64) {
        affine_gemv4_kernel<DT, ROWS, NPROJ, CG, 2><<<grid, block, 0, stream>>>(p);
        break;
      }
      return hipErrorInvalidValue;
    case 3:
      if constexpr (3 * kLoads < 64) {
        affine_gemv4_kernel<DT, ROWS, NPROJ, CG, 3><<<grid, block, 0, stream>>>(p);
        break;
      }
      return hipErrorInvalidValue;
    case 4:
      if constexpr (4 * kLoads < 64) {
        affine_gemv4_kernel<DT, ROWS, NPROJ, CG, 4><<<grid, block, 0, stream>>>(p);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DT, int ROWS, int NPROJ>
hipError_t launch_rows(const QmvParams& p, int waves, int cg, hipStream_t stream) {
  switch (cg) {
    case 1: return launch_cg<DT, ROWS, NPROJ, 1>(p, waves, stream);
    case 2: return launch_cg<DT, ROWS, NPROJ, 2>(p, waves, stream);
    case 4: return launch_cg<DT, ROWS, NPROJ, 4>(p, waves, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT, int NPROJ>
hipError_t launch_nproj(const QmvParams& p, int waves, int cg, hipStream_t stream) {
  if (p.M <= 1) return launch_rows<DT, 1, NPROJ>(p, waves, cg, stream);
  if (p.M <= 2) return launch_rows<DT, 2, NPROJ>(p, waves, cg, stream);
  return launch_rows<DT, 4, NPROJ>(p, waves, cg, stream);
}

}  // namespace

hipError_t launch_affine_gemv4(const QmvParams& p, int dtype, int nproj, int waves, int cg,
                               hipStream_t stream) {
  if (p.M < 1 || p.M > 4 || p.G < 32 || p.N % (4 * cg) ||
      !affine_gemv4_fits(p.K, waves, nproj, cg))
    return hipErrorInvalidValue;
  if (dtype == kBF16)
    return nproj == 2 ? launch_nproj<kBF16, 2>(p, waves, cg, stream)
                      : launch_nproj<kBF16, 1>(p, waves, cg, stream);
  return nproj == 2 ? launch_nproj<kF16, 2>(p, waves, cg, stream)
                    : launch_nproj<kF16, 1>(p, waves, cg, stream);
}

}  // namespace mt

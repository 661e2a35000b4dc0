// Prefill affine quantized GEMM, ring kernel (gfx950): y[M, N] = x[M, K] @ dequantize(w_q)[N, K]^T
// for many rows (reference: lower_affine_matmul, metile/compiler/affine_quantized.py:7-99, and its
// dispatcher mlx_affine_matmul, metile/backends/mlx_affine.py:359-406). The plan picks it or the
// register-staged kernel of affine_gemm.hip.
//
// A workgroup of four waves (2 x 2) computes a 128 x BN output tile (BN = 32 TN); each wave owns
// 64 x 16 TN of it as 4 x TN tiles of v_mfma_f32_16x16x32. The K loop runs in 64-wide steps:
//  * the step's activations (128 rows x 64) and codes (BN columns x 32 bytes) reach LDS through
//    buffer_load...lds, three steps in flight in a ring of three stages, one barrier per step;
//    no VGPR staging and no VALU on the way in. Each stage is its own LDS array, so the compiler
//    sees that a step's reads do not touch the stage being filled and does not wait for it;
//  * the scales and biases of the whole K range are staged once, before the loop;
//  * a lane's B operand is two code words of one column read straight from the staged codes
//    (k slices permuted alike in A and B: lane group g takes K 16 g .. 16 g + 15 of the step,
//    8 per MFMA), unpacked to exact offset + q 16-bit floats;
//  * an MFMA of the activations against -offset gives -offset * (row sum) in the output layout;
//    each column block's chain starts from it, so the chain sums x * q exactly (the offset term
//    cancels inside the fp32 accumulation, not in the output accumulator);
//  * the group's affine terms are applied in fp32: acc += s t + b (-1/offset)(-offset X).
// The MFMAs of column block c + 1 are issued ahead of the fix-up of block c, interleaved with it.
// Output tiles leave through LDS as 16-byte stores. With K split, the last workgroup of a tile
// to arrive adds the other splits' accumulators, stored in register layout, to its own.
#include "common.h"
#include "affine_gemm.h"

namespace mt {

namespace {

constexpr int kABytes = 128 * 128;  // one stage of activations: 128 rows x 64 K x 2 bytes

// The 16-byte chunk c of LDS row r sits in slot c ^ swz(r): the A reads of 8 or 16 lanes
// (consecutive rows, one chunk) hit distinct banks.
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// One step's loads by one of NW waves: 16 / NW activation loads of 1 KiB (rows
// 128 / NW * wave ..) and the wave's share of the code loads (1 KiB = 32 columns each, load d
// by wave d % NW). Every wave issues the same number of code loads, branch-free: a surplus one
// reads nothing (out of range) into the spare kilobyte at the end of the code stage.
template <int NW, int CODE_LOADS>
__device__ __forceinline__ void ring_issue(__amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rw,
                                           const uint32_t* a_src, const uint32_t* c_src, int wave,
                                           uint32_t st, bool ok, unsigned char* as,
                                           unsigned char* bs) {
#pragma unroll
  for (int d = 0; d < 16 / NW; ++d)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rx, (lds_ptr_t)(as + (128 / NW * wave + 8 * d) * 128), 16,
        oob_unless(ok, a_src[d] + st * 128u), 0, 0, 0);
#pragma unroll
  for (int i = 0; i < (CODE_LOADS + NW - 1) / NW; ++i) {
    const int d = wave + NW * i;
    const int dd = d < CODE_LOADS ? d : CODE_LOADS;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rw, (lds_ptr_t)(bs + dd * 1024), 16,
        oob_unless(ok && d < CODE_LOADS, c_src[i] + st * 32u), 0, 0, 0);
  }
}

// TN column blocks of 16 per wave, WN waves along N (2 or 4) and two along M: tiles of
// 128 x 16 TN WN, workgroups of 2 WN waves.
template <int DT, int TN, int WN>
__global__ __launch_bounds__(128 * WN) void affine_gemm_ring_kernel(const GemmParams args) {
  const GemmParams p = preload_args(args);
  constexpr int NW = 2 * WN;
  constexpr int kThreads = 64 * NW;
  constexpr int BN = 16 * TN * WN;
  constexpr int kCodeTotal = BN / 32;  // 1 KiB code loads per step
  constexpr int kCodeLoads = (kCodeTotal + NW - 1) / NW;  // per wave and step
  constexpr int kBBytes = gemm_ring_code_stage(BN, NW);
  constexpr float kOff = CodeOffset<4, DT>::value;
  constexpr uint32_t kNegOff2 = DT == kBF16 ? 0xC300C300u : 0xE400E400u;  // -offset, twice
  // Ops a wave has in flight past the current step's at the start of a step: the next step's.
  constexpr int kAhead = 16 / NW + kCodeLoads;
  __shared__ __attribute__((aligned(1024))) unsigned char A0[kABytes];
  __shared__ __attribute__((aligned(1024))) unsigned char A1[kABytes];
  __shared__ __attribute__((aligned(1024))) unsigned char A2[kABytes];
  __shared__ __attribute__((aligned(1024))) unsigned char B0[kBBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char B1[kBBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char B2[kBBytes];
  extern __shared__ __align__(16) unsigned char dyn[];  // scales and biases, then the output
  auto a_stage = [&](auto sc) -> unsigned char* {
    constexpr int S = decltype(sc)::value;
    if constexpr (S == 0) return A0;
    else if constexpr (S == 1) return A1;
    else return A2;
  };
  auto b_stage = [&](auto sc) -> unsigned char* {
    constexpr int S = decltype(sc)::value;
    if constexpr (S == 0) return B0;
    else if constexpr (S == 1) return B1;
    else return B2;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int i16 = lane & 15, g = lane >> 4;
  const int M = p.M, K = p.K, N = p.N;
  // Workgroup -> (column tile bx, row block by, split bz). Order 0: as launched. Orders 1 and 2:
  // workgroups go to the 8 XCDs in turn (XCD = linear index % 8), so workgroup L takes item
  // k T/8 + min(k, T%8) + L/8 (k = L % 8) of the sequence of T tiles, in which column tiles (1)
  // or row blocks (2) vary fastest: each XCD gets a contiguous run of it.
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  if (p.order) {
    const int gx = gridDim.x, gy = gridDim.y, total = gx * gy * gridDim.z;
    const int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int k = lin & 7;
    const int item = k * (total >> 3) + min(k, total & 7) + (lin >> 3);
    if (p.order == 1) {
      bx = item % gx;
      by = (item / gx) % gy;
    } else {
      by = item % gy;
      bx = (item / gy) % gx;
    }
    bz = item / (gx * gy);
  }
  const int m0 = by * 128, n0 = bx * BN;
  const int steps = K >> 6;
  const int s_beg = bz * p.steps_per_split;
  const int s_end = min(steps, s_beg + p.steps_per_split);
  const int gshift = __builtin_ctz((unsigned)p.G);
  const int gpr = K >> gshift;
  const int g_beg = (s_beg * 64) >> gshift;
  const uint32_t row_bytes = (uint32_t)K / 2u;
  const int W = p.sb_words;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, (uint32_t)N * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.s, (uint32_t)N * (uint32_t)gpr * 2u);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, (uint32_t)N * (uint32_t)gpr * 2u);

  // ---- scales and biases of the K range: dword q of [array][column][W] ----------------------
  // Row q / W from a float reciprocal: (q + 1/2) / W stays 1 / (2 W) from an integer, far beyond
  // the reciprocal's error for the sizes the host admits. A column's dwords start at the even
  // element at or below its first group, so its groups start at element sh0 (0 or 1).
  {
    const int total = 2 * BN * W;
    const float inv_w = __builtin_amdgcn_rcpf((float)W);
    for (int d = wave; d * 64 < total; d += NW) {
      const int q = d * 64 + lane;
      const int rowq = (int)(((float)q + 0.5f) * inv_w);  // array * BN + column
      const int wd = q - rowq * W;
      const int arr = rowq >= BN;
      const int n = n0 + rowq - arr * BN;
      const uint32_t first = ((uint32_t)n * (uint32_t)gpr + (uint32_t)g_beg) & ~1u;
      const uint32_t off = oob_unless(q < total && n < N, (first + 2u * wd) * 2u);
      if (arr)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(dyn + d * 256), 4, off, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(dyn + d * 256), 4, off, 0, 0, 0);
    }
  }

  // Activations: load d of a wave fills LDS rows 128 / NW * wave + 8 d .. + 7, lane l the slot
  // l % 8 of row l / 8, with the chunk that slot holds (rows past M read zero).
  uint32_t a_src[16 / NW];
#pragma unroll
  for (int d = 0; d < 16 / NW; ++d) {
    const int r = 128 / NW * wave + 8 * d + (lane >> 3);
    const int c = (lane & 7) ^ swz(r);
    a_src[d] = oob_unless(m0 + r < M, ((uint32_t)(m0 + r) * (uint32_t)K + 8u * c) * 2u);
  }
  // Codes: load d covers columns 32 d .. 32 d + 31, two lanes (16 bytes each) per column.
  uint32_t c_src[kCodeLoads];
#pragma unroll
  for (int i = 0; i < kCodeLoads; ++i) {
    const int n = n0 + 32 * (wave + NW * i) + (lane >> 1);
    c_src[i] = oob_unless(n < N, (uint32_t)n * row_bytes + 16u * (lane & 1));
  }
  auto issue = [&](int st, auto sc) {
    ring_issue<NW, kCodeTotal>(rx, rw, a_src, c_src, wave, (uint32_t)st, st < s_end, a_stage(sc),
                               b_stage(sc));
  };

  f32x4 acc[4][TN];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < TN; ++c) acc[a][c] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Column of block c within the tile: lc0 + 16 c. Its staged scale row starts at parity sh0
  // (16 c more columns of gpr groups each keep the parity of column lc0).
  const int lc0 = wn * 16 * TN + i16;  // (also with four waves along N)
  const int sh0 = ((n0 + lc0) * gpr + g_beg) & 1;
  const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(dyn);
  const u32x4 negoff = (u32x4){kNegOff2, kNegOff2, kNegOff2, kNegOff2};
  const f32x4 zero4 = (f32x4){0.f, 0.f, 0.f, 0.f};

  // A step's operands as a lane holds them: A fragments of its 4 row blocks (two K halves),
  // two code words of each of its TN column blocks.
  struct Frag {
    u32x4 af[4][2];
    u32x2 cw[TN];
  };
  auto read_frags = [&](auto sc, Frag& f) {
    const unsigned char* as = a_stage(sc);
    const unsigned char* bs = b_stage(sc);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int row = wm * 64 + 16 * a + i16;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        f.af[a][kk] = *reinterpret_cast<const u32x4*>(as + row * 128 +
                                                      16 * ((2 * g + kk) ^ swz(row)));
    }
#pragma unroll
    for (int c = 0; c < TN; ++c)
      f.cw[c] = *reinterpret_cast<const u32x2*>(bs + (lc0 + 16 * c) * 32 + 8 * g);
  };
  auto sync = [&]() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Steps s_beg .. s_beg + 2 in flight, then the first step's operands.
  issue(s_beg, IntConst<0>{});
  issue(s_beg + 1, IntConst<1>{});
  issue(s_beg + 2, IntConst<2>{});
  wait_vmcnt<2 * kAhead>();
  sync();
  Frag f0, f1, f2;
  read_frags(IntConst<0>{}, f0);

  // Step st (stage S = (st - s_beg) % 3) computes from operands already in registers. Halfway
  // through its column blocks it waits for step st + 1's loads (every wave's, at the barrier),
  // refills stage S (every wave holds step st's operands by then) with step st + 3, and reads
  // step st + 1's operands, whose LDS latency the remaining blocks hide.
  auto step = [&](auto sc, int st, Frag& cur, Frag& nxt) {
    constexpr int S = decltype(sc)::value;
    constexpr int kMid = TN / 2;
    const int gl = ((st * 64) >> gshift) - g_beg;
    f32x4 tx[4], t[2][4];
    u32x4 bw[2][2];
    float sf[2], bq[2];
    auto prep = [&](int c, int slot) {
      bw[slot][0] = unpack_u4<DT>(cur.cw[c].x);
      bw[slot][1] = unpack_u4<DT>(cur.cw[c].y);
      const int e = (lc0 + 16 * c) * 2 * W + gl + sh0;
      sf[slot] = act_to_f32<DT>(sb16[e]);
      bq[slot] = act_to_f32<DT>(sb16[2 * BN * W + e]) * (-1.0f / kOff);  // exact: 2^-k
    };
    auto mm = [&](int slot) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        t[slot][a] = mfma16<DT>(cur.af[a][0], bw[slot][0], tx[a]);
        t[slot][a] = mfma16<DT>(cur.af[a][1], bw[slot][1], t[slot][a]);
      }
    };
    auto fix = [&](int c, int slot) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[a][c][r] = __builtin_fmaf(sf[slot], t[slot][a][r], acc[a][c][r]);
          acc[a][c][r] = __builtin_fmaf(bq[slot], tx[a][r], acc[a][c][r]);
        }
    };
    prep(0, 0);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      tx[a] = mfma16<DT>(cur.af[a][0], negoff, zero4);
      tx[a] = mfma16<DT>(cur.af[a][1], negoff, tx[a]);
    }
    mm(0);
    if (TN > 1) prep(1, 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < TN; ++c) {
      if (c == kMid) {
        wait_vmcnt<kAhead>();
        sync();
        issue(st + 3, IntConst<S>{});
        read_frags(IntConst<(S + 1) % 3>{}, nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (c + 1 < TN) mm((c + 1) & 1);
      fix(c, c & 1);
      if (c + 2 < TN) prep(c + 2, c & 1);
      if (c + 1 < TN) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA,
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // then six VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Steps in threes (the stages are compile-time): a split whose length is not a multiple of
  // three runs one or two steps more over out-of-range loads (zero codes and activations; their
  // scales are real), which add exact zeros.
  for (int st = s_beg; st < s_end; st += 3) {
    step(IntConst<0>{}, st, f0, f1);
    step(IntConst<1>{}, st + 1, f1, f2);
    step(IntConst<2>{}, st + 2, f2, f0);
  }

  if (p.ksplit > 1) {
    // ---- split K: each workgroup leaves its accumulators as they lie in its registers
    // (thread t's f32x4 j at 16 (j kThreads + t) bytes of its part: each wave store 1 KiB
    // contiguous, device-coherent); the last to arrive adds the other splits' parts to its own
    // in split order (so the sum does not depend on which arrived last) and stores the tile.
    // Parts are [split][tile][128 BN] fp32.
    const int tile = by * gridDim.x + bx;
    const int tiles = gridDim.x * gridDim.y;
    const int split = bz, parts = p.ksplit;
    constexpr uint32_t kPartBytes = 128u * BN * 4u;
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(p.partial, (uint32_t)parts * (uint32_t)tiles * kPartBytes);
    auto part_off = [&](int sp, int j) {
      return ((uint32_t)sp * tiles + tile) * kPartBytes + ((uint32_t)j * kThreads + tid) * 16u;
    };
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < TN; ++c)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[a][c]), rp,
                                               part_off(split, a * TN + c), 0, kDeviceScope);
    __shared__ int last_flag;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      last_flag = (prev == (unsigned)(parts - 1));
    }
    __syncthreads();
    if (!last_flag) return;
    if (tid == 0)
      __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Two parts in flight at a time (one for the widest tiles, for registers); the own part
    // from registers.
    constexpr int kBufs = TN >= 4 ? 1 : 2;
    f32x4 tot[4][TN];
    u32x4 v[kBufs][4][TN];
    auto fetch = [&](int sp, u32x4 (&d)[4][TN]) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < TN; ++c)
          d[a][c] = load16_device(
              rp, oob_unless(sp < parts && sp != split, part_off(sp, a * TN + c)));
    };
    if (kBufs == 2) fetch(0, v[0]);
#pragma unroll
    for (int sp = 0; sp < kGemmMaxSplits; ++sp) {
      if (sp >= parts) break;
      if (kBufs == 1) fetch(sp, v[0]);
      else if (sp + 1 < parts) fetch(sp + 1, v[(sp + 1) % kBufs]);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < TN; ++c) {
          const f32x4 x =
              sp == split ? acc[a][c] : __builtin_bit_cast(f32x4, v[sp % kBufs][a][c]);
          tot[a][c] = sp == 0 ? x : tot[a][c] + x;
        }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < TN; ++c) acc[a][c] = tot[a][c];
  }

  // ---- the output tile through LDS (the scale region, free once every wave is past its last
  // step), then 16-byte row stores ------------------------------------------------------------
  __syncthreads();
  uint16_t* ot = reinterpret_cast<uint16_t*>(dyn);
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < TN; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ot[(wm * 64 + 16 * a + 4 * g + r) * BN + lc0 + 16 * c] = f32_to_act<DT>(acc[a][c][r]);
  __syncthreads();
  constexpr int kChunks = 128 * BN / 8;
  for (int q = tid; q < kChunks; q += kThreads) {
    const int row = q / (BN / 8), c8 = (q - row * (BN / 8)) * 8;
    if (m0 + row < M && n0 + c8 < N)  // N is a multiple of 8: a chunk is wholly inside
      *reinterpret_cast<u32x4*>(p.y + (size_t)(m0 + row) * N + n0 + c8) =
          *reinterpret_cast<const u32x4*>(ot + row * BN + c8);
  }
}

template <int DT, int TN, int WN>
hipError_t launch_tn(const GemmParams& p, hipStream_t stream) {
  constexpr int BN = 16 * TN * WN;
  const size_t dyn = gemm_ring_dynamic_lds(BN, p.sb_words);
  // The kernel's dynamic LDS limit, raised once per instantiation to what the shapes the host
  // admits may use.
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&affine_gemm_ring_kernel<DT, TN, WN>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)(kGemmRingLdsBytes - gemm_ring_static_lds(BN)));
  if (attr != hipSuccess) return attr;
  const dim3 grid((p.N + BN - 1) / BN, (p.M + 127) / 128, p.ksplit);
  affine_gemm_ring_kernel<DT, TN, WN><<<grid, 128 * WN, dyn, stream>>>(p);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_dt(const GemmParams& p, hipStream_t stream) {
  switch (p.tile_n) {
    case 64: return launch_tn<DT, 2, 2>(p, stream);
    case 96: return launch_tn<DT, 3, 2>(p, stream);
    case 128: return launch_tn<DT, 2, 4>(p, stream);
    case 160: return launch_tn<DT, 5, 2>(p, stream);
    case 192: return launch_tn<DT, 3, 4>(p, stream);
    case 256: return launch_tn<DT, 4, 4>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_affine_gemm_ring(const GemmParams& p, int dtype, hipStream_t stream) {
  return dtype == kBF16 ? launch_dt<kBF16>(p, stream) : launch_dt<kF16>(p, stream);
}

}  // namespace mt

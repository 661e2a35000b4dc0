// Shared device helpers for the gfx950 (CDNA4) kernels of metile_amd.
//
// Conventions used by every kernel in this directory:
//  * activations, scales, biases and outputs are 16-bit floats (bf16 or f16) carried as
//    uint16_t bit patterns; accumulation is fp32;
//  * packed affine weights are MLX's output-major uint32 words, code k of a row at word
//    k / (32/bits), shift (k % (32/bits)) * bits (low bits first along K);
//  * all global reads go through raw buffer loads, whose hardware range check returns zero
//    for any offset at or beyond the buffer size; kOOB is used to switch a lane's load off.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

enum Dtype : int { kBF16 = 0, kF16 = 1 };

// Offsets at or above every buffer size used here read as zero.
constexpr uint32_t kOOB = 0x80000000u;

// `off`, or an offset at or past kOOB (reads zero) when the lane has nothing to load. Written as
// a bit operation rather than a select: with a select the compiler split loads into two branch
// arms writing the same registers, and the second arm then waited for every load in flight
// (s_waitcnt vmcnt(0)) before issuing. Every buffer here is below 2 GiB, so bit 31 suffices.
__device__ __forceinline__ uint32_t oob_unless(bool ok, uint32_t off) {
  return off | ((uint32_t)!ok << 31);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // Word 3 = 0x00020000: raw (unswizzled, untyped) dword access on gfx9-family parts.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}

constexpr int kCachePolicyNt = 2;  // the buffer instructions' nt bit on gfx950
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
// Streaming forms (non-temporal hint, `nt`) for data each launch reads once: the small-row
// kernels' packed codes (measured, one-row GEMV over weights 2.5x the MALL: SwiGLU 5.54 -> 5.19
// us, down 4.35 -> 4.14 us), the GEMV's scales and biases (down 4.17 -> 4.10 us; the staged
// kernel's scale staging measured slower with it) and dense weights of one-chunk launches.
__device__ __forceinline__ u32x4 load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCachePolicyNt);
}
__device__ __forceinline__ u32x2 load8_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCachePolicyNt);
}
__device__ __forceinline__ uint16_t load2_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kCachePolicyNt);
}
__device__ __forceinline__ u32x2 load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint16_t load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Device-coherent forms (cache policy sc1, device scope: the same accesses that device-scope
// relaxed atomics compile to), for data written by other workgroups of the same launch, which
// may run on another XCD with its own L2.
constexpr int kDeviceScope = 16;
__device__ __forceinline__ u32x4 load16_device(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kDeviceScope);
}
__device__ __forceinline__ void store2_device(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                              uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kDeviceScope);
}

// A kernel's argument block copied into scalar registers at once: every dword is read, then all
// are pinned in SGPRs together, so the compiler issues the scalar loads in one batch with one
// wait instead of fetching each field at its first use (which it did in several dependent
// rounds, each a full scalar-memory latency before the kernel's first memory request).
template <typename T>
__device__ __forceinline__ T preload_args(const T& a) {
  static_assert(sizeof(T) % 4 == 0, "argument block of whole dwords");
  constexpr int kWords = sizeof(T) / 4;
  uint32_t w[kWords];
  __builtin_memcpy(w, &a, sizeof(T));
#pragma unroll
  for (int i = 0; i < kWords; ++i) __asm__ volatile("" : "+s"(w[i]));
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}

// ---- 16-bit float conversions ----------------------------------------------------------

template <int DT>
__device__ __forceinline__ float act_to_f32(uint32_t bits16) {
  if constexpr (DT == kBF16) {
    return __uint_as_float(bits16 << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  }
}

// Round-to-nearest-even conversion of fp32 to the activation type.
template <int DT>
__device__ __forceinline__ uint16_t f32_to_act(float f) {
  if constexpr (DT == kBF16) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// ---- MFMA 32x32x16 (fp32 accumulate) -----------------------------------------------------
// Lane l supplies A[i = l%32][k = 8*(l/32) + 0..7] and B[k = 8*(l/32) + 0..7][j = l%32];
// the result element (i, j) lives in lane j + 32*((i/4)%2), register 4*(i/8) + i%4.

template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kBF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Row of the 32x32 output tile held in register r of a lane in half h (= lane / 32).
__device__ __forceinline__ constexpr int mfma32_row(int r, int h) {
  return 8 * (r / 4) + 4 * h + (r % 4);
}

// ---- MFMA 16x16x32 (fp32 accumulate) -----------------------------------------------------
// Lane l supplies A[i = l%16][k = 8*(l/16) + 0..7] and B[k = 8*(l/16) + 0..7][j = l%16]; the
// result element (i, j) lives in lane j + 16*(i/4), register i%4.
template <int DT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// LDS address space, for buffer_load...lds destinations.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// ---- code -> 16-bit float unpack (exact) -------------------------------------------------
// A 4-bit code q is written into the low mantissa bits of a 16-bit float whose exponent makes
// the mantissa step exactly 1: bf16 0x4300|q == 128 + q, f16 0x6400|q == 1024 + q. 8-bit
// codes use f16 0x6400|q == 1024 + q, or for bf16 an exact int -> fp32 -> bf16 conversion
// (integers below 256 have at most 8 significant bits). kCodeOffset is the constant added.

template <int BITS, int DT>
struct CodeOffset {
  static constexpr float value = (DT == kF16) ? 1024.0f : (BITS == 4 ? 128.0f : 0.0f);
};

// 8 nibbles of one word -> 8 values in K order, packed two per uint32.
template <int DT>
__device__ __forceinline__ u32x4 unpack_u4(uint32_t w) {
  constexpr uint32_t kMagic = (DT == kBF16) ? 0x43434343u : 0x64646464u;
  const uint32_t a = w & 0x0F0F0F0Fu;          // codes 0, 2, 4, 6 (one per byte)
  const uint32_t b = (w >> 4) & 0x0F0F0F0Fu;   // codes 1, 3, 5, 7
  const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // codes 0 1 2 3
  const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // codes 4 5 6 7
  u32x4 out;
  out.x = __builtin_amdgcn_perm(kMagic, lo, 0x04010400u);
  out.y = __builtin_amdgcn_perm(kMagic, lo, 0x04030402u);
  out.z = __builtin_amdgcn_perm(kMagic, hi, 0x04010400u);
  out.w = __builtin_amdgcn_perm(kMagic, hi, 0x04030402u);
  return out;
}

// 8 nibbles of one word -> 8 values in the paired order (0,4,1,5,2,6,3,7): element pair i of
// the result holds codes i and i + 4, which one AND-OR per pair produces (a shift and an
// AND-OR for i > 0). The other MFMA operand must be supplied in the same order.
// The mask and the exponent pattern are held in registers (see paired_consts) so that each
// AND-OR is one v_and_or_b32, which as a three-operand instruction takes no literals here.
struct PairedConsts {
  uint32_t mask;
  uint32_t magic;
};

template <int DT>
__device__ __forceinline__ PairedConsts paired_consts() {
  PairedConsts c{0x000F000Fu, (DT == kBF16) ? 0x43004300u : 0x64006400u};
  __asm__("" : "+v"(c.mask));
  __asm__("" : "+v"(c.magic));
  return c;
}

__device__ __forceinline__ u32x4 unpack_u4_paired(uint32_t w, PairedConsts c) {
  u32x4 out;
  out.x = (w & c.mask) | c.magic;
  out.y = ((w >> 4) & c.mask) | c.magic;
  out.z = ((w >> 8) & c.mask) | c.magic;
  out.w = ((w >> 12) & c.mask) | c.magic;
  return out;
}

// Eight 16-bit values in K order (two per uint32) -> the paired order (0,4,1,5,2,6,3,7).
__device__ __forceinline__ u32x4 pair_order(u32x4 v) {
  u32x4 out;
  out.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  out.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  out.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  out.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return out;
}

// 4 bytes of one word -> 4 values in K order, packed two per uint32.
template <int DT>
__device__ __forceinline__ u32x2 unpack_u8(uint32_t w) {
  u32x2 out;
  if constexpr (DT == kF16) {
    out.x = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    out.y = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
  } else {
    const uint32_t f0 = __float_as_uint((float)(w & 0xFFu));
    const uint32_t f1 = __float_as_uint((float)((w >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((w >> 16) & 0xFFu));
    const uint32_t f3 = __float_as_uint((float)(w >> 24));
    out.x = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    out.y = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
  }
  return out;
}

// B operand of MFMA e (K slice [8e, 8e+8) of a lane's 32 K, natural order) as 8 exact 16-bit
// floats, from the lane's 16 (4-bit) or 32 (8-bit) bytes of codes.
template <int BITS, int DT>
__device__ __forceinline__ u32x4 code_frag(const u32x4 (&w)[BITS / 4], int e) {
  if constexpr (BITS == 4) {
    return unpack_u4<DT>(w[0][e]);
  } else {
    const u32x4 src = w[e >> 1];
    const u32x2 lo = unpack_u8<DT>((e & 1) ? src.z : src.x);
    const u32x2 hi = unpack_u8<DT>((e & 1) ? src.w : src.y);
    return (u32x4){lo.x, lo.y, hi.x, hi.y};
  }
}

// f16 codes without their offset: 1024 + q minus 1024 is exact in f16 (one packed subtraction
// per word of two codes). The small-row kernels multiply q itself, so that their fp32 sums do not
// carry 1024 times the activation sums (seven bits more rounding than bf16's 128 + q);
// SumOffset is the offset the codes they multiply still hold. The word arrives as a scalar: a
// bit cast applied to an element of a vector value read the vector's first word.
__device__ __forceinline__ uint32_t f16_minus_offset(uint32_t w) {
  const f16x2 off = (f16x2){(_Float16)1024.0f, (_Float16)1024.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, w) - off);
}

template <int DT>
__device__ __forceinline__ u32x4 codes_for_sum(u32x4 v) {
  if constexpr (DT == kF16) {
    const uint32_t x = v.x, y = v.y, z = v.z, w = v.w;
    return (u32x4){f16_minus_offset(x), f16_minus_offset(y), f16_minus_offset(z),
                   f16_minus_offset(w)};
  } else {
    return v;
  }
}

template <int BITS, int DT>
struct SumOffset {
  static constexpr float value = DT == kF16 ? 0.0f : CodeOffset<BITS, DT>::value;
};

// The two 16-bit floats of a packed pair, widened to fp32 (element 0 is the low half).
template <int DT>
__device__ __forceinline__ float lo16(uint32_t w) {
  if constexpr (DT == kBF16) return __uint_as_float(w << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
template <int DT>
__device__ __forceinline__ float hi16(uint32_t w) {
  if constexpr (DT == kBF16) return __uint_as_float(w & 0xFFFF0000u);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// acc + a.lo * b.lo + a.hi * b.hi for words holding two 16-bit floats each, fp32 accumulate
// (one dot-product instruction). The words must arrive as scalars: with this compiler,
// __builtin_bit_cast applied directly to an element of a vector value read the vector's first
// word instead (which is what made dot products fed that way return wrong sums).
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b),
                                  acc, false);
}

// acc + a.lo + a.hi: the dot product with (1, 1).
template <int DT>
__device__ __forceinline__ float pair_sum(uint32_t a, float acc) {
  return dot2<DT>(a, DT == kBF16 ? 0x3f803f80u : 0x3c003c00u, acc);
}

// Sum of the 8 16-bit floats held in a u32x4, added to acc in fp32, two per instruction.
template <int DT>
__device__ __forceinline__ float sum8(u32x4 v, float acc) {
  return pair_sum<DT>(v.w, pair_sum<DT>(v.z, pair_sum<DT>(v.y, pair_sum<DT>(v.x, acc))));
}

// ---- lane exchanges within a row of 16 lanes (DPP: one VALU instruction, no LDS trip) ----
// kDppXor1 / kDppXor2: lane i reads lane i ^ 1 / i ^ 2 of its quad; kDppHalfMirror: lane i
// reads lane 7 - i of its group of eight.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppRowRor8 = 0x128;     // row_ror:8 (lane i reads lane i ^ 8 of its row)

template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// ---- across rows of 16 lanes: row broadcasts (rows outside ROW_MASK read +0) ----
// kDppRowBcast15: a row reads lane 15 of the row before it; kDppRowBcast31: rows 2 and 3 read
// lane 31.
constexpr int kDppRowBcast15 = 0x142;  // row_bcast:15
constexpr int kDppRowBcast31 = 0x143;  // row_bcast:31

// The value unchanged, opaque to the optimizer (an empty asm that may rewrite the register).
__device__ __forceinline__ float opaque(float v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}

// A compile-time int carried as a type (to instantiate a generic lambda per value).
template <int V>
struct IntConst {
  static constexpr int value = V;
};

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_read_rows(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xF, false));
}

// Sum over each aligned group of 4 (or 8) lanes; every lane of the group receives it. The
// additions pair the same operands as xor exchanges over 1, 2 (and 4) would: lanes of a quad
// hold the same quad sum, so the half mirror's partner quad is the xor-4 one.
__device__ __forceinline__ float group_sum4(float s) {
  s += dpp_read<kDppXor1>(s);
  s += dpp_read<kDppXor2>(s);
  return s;
}
__device__ __forceinline__ float group_sum8(float s) {
  s = group_sum4(s);
  s += dpp_read<kDppHalfMirror>(s);
  return s;
}

// Sum over sp = 0 .. n - 1 of the device-coherent floats p[sp * stride], added in sp order
// (split-K partials written by other workgroups). The loads of a batch are issued together, so
// a batch costs one memory round trip rather than one per term; indices past n re-read the
// last term and are not added.
__device__ __forceinline__ float sum_partials(const float* p, size_t stride, int n) {
  constexpr int kBatch = 8;
  float acc = 0.0f;
  for (int b = 0; b < n; b += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int sp = b + u < n ? b + u : n - 1;
      v[u] = __hip_atomic_load(p + (size_t)sp * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (b + u < n) acc += v[u];
  }
  return acc;
}

// NV such sums at once: out[v] = ((0 + q[v][0]) + q[v][1]) + ... over n splits of ptr[v] (split
// stride `stride` floats; a null pointer sums to 0), every load of a batch of splits (16 loads)
// requested before any is added, so a batch costs one memory round trip.
template <int NV>
__device__ __forceinline__ void sum_partials_multi(const float* const (&ptr)[NV], size_t stride,
                                                   int n, float (&out)[NV]) {
  constexpr int kBatch = NV >= 16 ? 1 : 16 / NV;
#pragma unroll
  for (int v = 0; v < NV; ++v) out[v] = 0.0f;
  for (int b = 0; b < n; b += kBatch) {
    float q[kBatch][NV];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int v = 0; v < NV; ++v)
        q[u][v] = b + u < n && ptr[v] ? __hip_atomic_load(ptr[v] + (size_t)(b + u) * stride,
                                                          __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                      : 0.0f;
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (b + u < n) {
#pragma unroll
        for (int v = 0; v < NV; ++v) out[v] += q[u][v];
      }
  }
}

// silu(g) * u with the hardware reciprocal (1 ulp in fp32, far below the 16-bit rounding of the
// result) instead of an IEEE division sequence. Large negative g: exp(-g) = inf, rcp(inf) = 0.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

}  // namespace mt

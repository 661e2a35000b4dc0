// extern "C" boundary of libmetile_amd.so: argument validation, workspace layout, split-K
// planning and error reporting. No allocation, no synchronisation, no exceptions across the ABI.
#include "../../include/metile_amd.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "affine_qmv.h"
#include "capi_internal.h"
#include "dense_qmv.h"
#include "affine_gemm.h"
#include "affine_quantize.h"
#include "stream_read.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(MT_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

constexpr int kRowChunk = 32;  // rows per small-row dispatch

// Every workspace starts with a fixed region of split-K arrival counters (one per 32-column
// strip), shared by all shapes so that each counter is always found at the same place; every
// call leaves the counters it used at zero. Partial sums follow the counter region.
constexpr size_t kCounterBytes = mt::kWorkspaceCounterBytes;
constexpr int kMaxStrips = (int)(kCounterBytes / 4);

// Split-K plan of the streaming kernels for one (K, N): about one workgroup per CU (splitting
// further costs more in partial-sum traffic and reduction than it gains in parallelism), with
// at least 16 K steps in each split. Depends only on K and N. `strips` = N / 32.
struct Plan {
  int ksplit;
  int steps_per_split;
  int strips;   // column strips (GEMV kernel: N / columns per workgroup)
  int kernel;   // mt_qmv_kernel
  int tiles;    // staged kernel: strips per workgroup; GEMV kernel: waves per workgroup
  int order;    // GEMV kernel: workgroup order (mt_qmv_plan.order)
};

Plan plan_split(int K, int N) {
  const int steps = K / 64;
  const int strips = N / 32;
  int ksplit = (256 + strips / 2) / strips;
  const int max_split = steps / 16 > 0 ? steps / 16 : 1;
  if (ksplit > max_split) ksplit = max_split;
  // Each split covers at most kMaxGroupsPerSplit - 1 groups of 64 (one more may straddle).
  const int min_split = (steps + mt::kMaxGroupsPerSplit - 2) / (mt::kMaxGroupsPerSplit - 1);
  if (ksplit < min_split) ksplit = min_split;
  if (ksplit < 1) ksplit = 1;
  Plan p;
  p.steps_per_split = (steps + ksplit - 1) / ksplit;
  p.ksplit = (steps + p.steps_per_split - 1) / p.steps_per_split;
  p.strips = strips;
  p.kernel = MT_QMV_REGISTER;
  p.tiles = 1;
  p.order = 0;
  return p;
}

// Activation-staged small-row kernel where it fits (M <= 16 and a bounded K range per split).
bool use_lds_path(int rows, int steps_per_split, int nproj, int group_size) {
  return mt::affine_qmv_lds_fits(rows, steps_per_split, nproj, group_size, 1);
}

// Compute units of the current device (hipDeviceProp_t::multiProcessorCount; 256 on an
// MI355X), read once per device. Plans depend on it through the workgroups per CU.
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Largest K split the tuner's candidate lists go to.
constexpr int kMaxCandidateSplits = 32;

// Code ring depth of the staged kernel for a shape (the stage counts its launcher picks; the
// 4-bit ring is six stages deep, or three when every wave has at most three K steps).
int staged_ring(int bits, int nproj, int group_size) {
  if (group_size == 32) return bits == 4 ? 3 : 2;
  if (bits == 8) return nproj == 2 ? 3 : 4;
  return 6;
}

// Plan of one small-row call chunk of `rows` rows: the split plan, and for the staged kernel
// a strip count that evens out the CUs. Its column strips need not be 32 wide: a workgroup
// takes columns [s N / strips, (s + 1) N / strips) (16 to 32 of them; the MFMA tile masks
// the rest). The fused gate/up kernel at one or two rows, when there are more 32-column
// strips than CUs, takes the smallest strip count that is a whole number of workgroups per CU,
// if it lowers the columns the busiest CU streams: with N / 32 = 280 strips on 256 CUs, 24 CUs
// would otherwise stream two full strips and set the kernel's time (SwiGLU 1536 -> 8960 at
// M = 1: 512 strips 7.75 us, 280 strips 8.0 us). Elsewhere the narrower strips measured
// slower: one projection of that shape (512 strips 5.86 us, 280 strips 5.60 us), four rows or
// more (two-strip workgroups below), fewer strips than CUs (SwiGLU 896 -> 4864: 256 strips
// 5.16 us, 152 strips 4.99 us). Only grids that are resident at once (two eight-wave
// workgroups per CU) are rebalanced: a grid of several rounds evens out as workgroups
// retire. (Changing the K split instead also measured slower: every split adds a partial-sum
// hand-off.)
Plan planner_qmv(int rows, int K, int N, int nproj, int group_size, int bits) {
  Plan plan = plan_split(K, N);
  if (group_size == 32) {
    // Two groups per K step: split K until the staged kernel's scale rows and LDS take it.
    const int steps = K / 64;
    for (int ks = plan.ksplit; ks <= steps; ++ks) {
      Plan c = plan;
      c.steps_per_split = (steps + ks - 1) / ks;
      c.ksplit = (steps + c.steps_per_split - 1) / c.steps_per_split;
      if (mt::affine_qmv_lds_fits(rows, c.steps_per_split, nproj, group_size, 1)) {
        plan = c;
        break;
      }
    }
  }
  // Split K further where that puts the rows on the staged kernel (its activation staging
  // holds M * steps_per_split * 8 chunks), at most to twice the planned split, except for the
  // fused gate/up kernel above 8 rows (there the register kernel unsplit measured faster:
  // SwiGLU 2048 -> 8192 at M = 16, 9.5 us against 11.6 us for the staged kernel over two
  // splits; one 8-bit projection 5120 -> 17408 at M = 16 is fastest staged over three); and in
  // grids of
  // several rounds of workgroups anyway, until every wave's K steps fit its code ring (a ring
  // that refills costs more than the extra split: K = 5120, N = 17408 at 8 bits measured
  // 30.3 us with 3 splits against 32.7 us with 2).
  const int kCus = device_cus();
  if (group_size != 32) {
    const int steps = K / 64;
    auto split_into = [&](int ks) {
      Plan c = plan;
      c.steps_per_split = (steps + ks - 1) / ks;
      c.ksplit = (steps + c.steps_per_split - 1) / c.steps_per_split;
      return c;
    };
    // A two-strip workgroup (the CU's LDS to itself) is taken before another K split: every
    // split adds a partial-sum hand-off (one projection 1536 -> 8960 at M = 32: two strips
    // unsplit 7.9 us against one strip over two splits 13.6 us; the down projection
    // 8960 -> 1536 at M = 32: two strips over 6 splits 11.5 us against 9 splits 12.7 us).
    auto staged_fits = [&](int steps_per_split) {
      return mt::affine_qmv_lds_fits(rows, steps_per_split, nproj, group_size, 1) ||
             (plan.strips % 2 == 0 &&
              mt::affine_qmv_lds_fits(rows, steps_per_split, nproj, group_size, 2));
    };
    if ((rows <= 8 || nproj == 1) && !staged_fits(plan.steps_per_split)) {
      for (int ks = plan.ksplit + 1; ks <= 2 * plan.ksplit && ks <= steps; ++ks) {
        const Plan c = split_into(ks);
        if (staged_fits(c.steps_per_split)) {
          plan = c;
          break;
        }
      }
    }
    const int ring = staged_ring(bits, nproj, group_size);
    for (int ks = plan.ksplit; (long)(N / 32) * ks > 2L * kCus && ks < steps; ++ks) {
      const Plan c = split_into(ks);
      if (c.ksplit < plan.ksplit) continue;
      if (!mt::affine_qmv_lds_fits(rows, c.steps_per_split, nproj, group_size, 1)) break;
      plan = c;
      if ((c.steps_per_split + mt::kQmvLdsWaves - 1) / mt::kQmvLdsWaves <= ring) break;
    }
  }
  // Up to 32 rows the staged kernel takes the call when its staging fits one workgroup of one
  // strip, or (more rows over a long split) of two strips, which has the CU's LDS to itself.
  const bool one_tile = use_lds_path(rows, plan.steps_per_split, nproj, group_size);
  if (!one_tile &&
      !(plan.strips % 2 == 0 &&
        mt::affine_qmv_lds_fits(rows, plan.steps_per_split, nproj, group_size, 2)))
    return plan;
  plan.kernel = MT_QMV_STAGED;
  const long base = N / 32, ks = plan.ksplit;
  const long per_cu_base = (base * ks + kCus - 1) / kCus;  // workgroups on the busiest CU
  const bool rebalance = nproj == 2 && rows <= 2 && base * ks > kCus;
  for (long rounds = per_cu_base; rebalance && rounds <= per_cu_base + 1; ++rounds) {
    if ((rounds * kCus) % ks) continue;
    const long strips = rounds * kCus / ks;
    if (strips <= base || strips > 2 * base || strips > kMaxStrips) continue;
    if (strips * ks > 2L * kCus) break;
    // Columns the busiest CU streams: rounds strips of N / strips columns against
    // per_cu_base strips of 32.
    if (rounds * N < per_cu_base * 32 * strips) {
      plan.strips = (int)strips;
      break;
    }
  }
  // Two strips per workgroup when the grid is one to two workgroups per CU and there are 4
  // rows or more: the two strips then share one staging of the activations (half the
  // activation reads through each CU's memory pipeline; SwiGLU 1536 -> 8960 at M = 8: 8.06 us
  // against 8.45 us). At fewer rows that staging is small and the 16-wave workgroup measured
  // slower (repacked SwiGLU at M = 1: 8.4 against 7.9 us).
  const long wgs = (long)plan.strips * plan.ksplit;
  int tiles = (!one_tile || (rows >= 4 && plan.strips % 2 == 0 && wgs > kCus &&
                             wgs <= 2L * kCus)) ? 2 : 1;
  if (tiles == 2 && !mt::affine_qmv_lds_fits(rows, plan.steps_per_split, nproj, group_size, 2))
    tiles = 1;
  plan.tiles = tiles;
  return plan;
}

// Rows per small-row dispatch: 32 (the register kernel's tile), 16 for groups of 32 (the
// staged kernel's largest row bucket).
int row_chunk(int group_size) { return group_size == 32 ? mt::kQmvLdsMaxRowsHalf : kRowChunk; }

// ---- installed plans -----------------------------------------------------------------------
// A tuner measures the plans mt_affine_qmv_plan_candidates lists and installs the fastest for a
// shape with mt_affine_qmv_plan_set; calls of that shape then take it instead of the planner's.
// Keys hold the rows of one dispatch rounded up to a power of two (a plan is validated at the
// bucket's largest row count, and every resource it needs grows with the rows), the shape and
// the dtype. Both code layouts take the same plan, so that their results stay bit-identical.
// The table is per process; lookups take a shared lock only once a plan has been installed.

int row_bucket(int rows) {
  int b = 1;
  while (b < rows) b <<= 1;
  return b;
}

struct PlanKey {
  int op, rows, K, N, nproj, G, bits, dtype;
  bool operator==(const PlanKey& o) const {
    return op == o.op && rows == o.rows && K == o.K && N == o.N && nproj == o.nproj &&
           G == o.G && bits == o.bits && dtype == o.dtype;
  }
};

struct PlanKeyHash {
  size_t operator()(const PlanKey& k) const {
    uint64_t h = 1469598103934665603ull;
    for (int v : {k.op, k.rows, k.K, k.N, k.nproj, k.G, k.bits, k.dtype}) {
      h ^= (uint64_t)(uint32_t)v;
      h *= 1099511628211ull;
    }
    return (size_t)h;
  }
};

enum PlanOp : int { kOpQmv = 0, kOpGemm = 1, kOpDense = 2 };

std::shared_mutex g_plans_mu;
std::unordered_map<PlanKey, mt_qmv_plan, PlanKeyHash> g_qmv_plans;
std::unordered_map<PlanKey, mt_gemm_plan, PlanKeyHash> g_gemm_plans;
std::unordered_map<PlanKey, mt_dense_plan, PlanKeyHash> g_dense_plans;

int installed_plans() {
  return (int)(g_qmv_plans.size() + g_gemm_plans.size() + g_dense_plans.size());
}
std::atomic<int> g_plans_installed{0};

PlanKey qmv_key(int rows, int K, int N, int nproj, int group_size, int bits, int dtype) {
  return PlanKey{kOpQmv, row_bucket(rows), K, N, nproj, group_size, bits, dtype};
}

bool find_qmv_plan(const PlanKey& key, mt_qmv_plan* out) {
  if (g_plans_installed.load(std::memory_order_acquire) == 0) return false;
  std::shared_lock<std::shared_mutex> lock(g_plans_mu);
  const auto it = g_qmv_plans.find(key);
  if (it == g_qmv_plans.end()) return false;
  *out = it->second;
  return true;
}

Plan split_plan(int steps, int ksplit) {
  Plan p{};
  p.steps_per_split = (steps + ksplit - 1) / ksplit;
  p.ksplit = (steps + p.steps_per_split - 1) / p.steps_per_split;
  return p;
}

Plan from_public(const mt_qmv_plan& q, int K) {
  Plan p = split_plan(K / 64, q.ksplit);
  p.strips = q.strips;
  p.kernel = q.kernel;
  p.tiles = q.kernel == MT_QMV_REGISTER ? 1 : q.tiles;
  p.order = q.kernel == MT_QMV_GEMV ? q.order : 0;
  return p;
}

mt_qmv_plan to_public(const Plan& p) {
  mt_qmv_plan q{};
  q.kernel = p.kernel;
  q.ksplit = p.ksplit;
  q.strips = p.strips;
  q.tiles = p.kernel == MT_QMV_REGISTER ? 1 : p.tiles;
  q.order = p.kernel == MT_QMV_GEMV ? p.order : 0;
  return q;
}

// Widest block of a column-block plan of `strips` workgroups per split, over both code layouts
// (repacked blocks start on whole 128-byte lines: units of 16 / bits columns).
int block_max_cols(int N, int strips, int bits) {
  const int align = 16 / bits;
  const int plain = (N + strips - 1) / strips;
  const int lined = (N / align + strips - 1) / strips * align;
  return plain > lined ? plain : lined;
}

// Staged scale-row words of a column-block split of `steps_per_split` K steps: the groups it
// spans, one more when it does not start on a group boundary.
int block_sb_words_for(int steps_per_split, int group_size) {
  const int per_group = group_size / 64;
  return mt::block_sb_words((steps_per_split + per_group - 1) / per_group + 1);
}

int block_groups_for(int steps_per_split, int group_size) {
  const int per_group = group_size / 64;
  return (steps_per_split + per_group - 1) / per_group + 1;
}

// Why `q` cannot run dispatches of up to `rows` rows at this shape ("" when it can): the
// register kernel covers 32-column strips of up to 32 rows and groups of 64 or more; the staged
// kernel up to 16 rows, N / 32 to 2 N / 32 strips (16 to 32 columns each) in workgroups of one or
// two strips, within its LDS; every split holds at most kMaxGroupsPerSplit - 1 groups. The GEMV
// kernel takes up to 4 rows, no K split, 2, 4 or 8 columns per column group (8: one projection
// of up to 2 rows; strips = N / (columns x column groups per workgroup)),
// 1 to 8 waves (tiles), and when a lane has more than one chunk per column, at most 8 of
// projections x columns x rows (more would spill registers).
std::string qmv_plan_problem(int rows, int K, int N, int nproj, int group_size, int bits,
                             const mt_qmv_plan& q) {
  const int steps = K / 64, base = N / 32;
  if (q.kernel == MT_QMV_GEMV) {
    if (rows > mt::kGemvMaxRows) return "more rows than the GEMV kernel takes";
    if (q.ksplit != 1) return "the GEMV kernel does not split K";
    if (q.tiles < 1 || q.tiles > mt::kGemvMaxWaves)
      return "GEMV tiles (waves per workgroup) must be in 1..8";
    const int groups = mt::affine_gemv_groups(K, bits, q.tiles);
    const int cols = q.strips >= 1 ? N / q.strips / groups : 0;
    if (q.strips < 1 || N % (q.strips * groups) || (cols != 2 && cols != 4 && cols != 8))
      return "GEMV strips must be N/(2, 4 or 8 columns x groups)";
    if (q.order != 0 && q.order != 1) return "GEMV order must be 0 or 1";
    if (!mt::affine_gemv_fits(rows, nproj, N / q.strips / groups,
                              mt::affine_gemv_one_pass(K, bits, q.tiles)))
      return "the GEMV kernel does not hold this many columns and rows in registers";
    return "";
  }
  if (q.kernel == MT_QMV_GEMV4) {
    if (rows > 4) return "more rows than the 4x4x4-MFMA GEMV kernel takes";
    if (bits != 4) return "the 4x4x4-MFMA GEMV kernel takes 4-bit codes";
    if (q.ksplit != 1) return "the 4x4x4-MFMA GEMV kernel does not split K";
    if (q.order != 0) return "order is a GEMV plan field (0 for the other kernels)";
    const int cg = q.strips >= 1 && N % q.strips == 0 ? N / q.strips / 4 : 0;
    if (cg * 4 * q.strips != N || (cg != 1 && cg != 2 && cg != 4))
      return "the 4x4x4-MFMA GEMV kernel runs N/4, N/8 or N/16 workgroups";
    if (!mt::affine_gemv4_fits(K, q.tiles, nproj, cg))
      return "4x4x4-MFMA GEMV tiles (waves) must be in 1..8, at most the 512-wide K rounds, "
             "with at most four rounds each and their loads within 64";
    return "";
  }
  if (q.kernel == MT_QMV_BLOCK) {
    if (group_size < 64) return "the block kernel takes groups of 64 or more";
    if (rows > mt::kBlockMaxRows) return "more rows than the block kernel takes";
    if (q.order != 0) return "order is a GEMV plan field (0 for the other kernels)";
    if (q.ksplit < 1 || q.ksplit > steps) return "ksplit must be in 1..K/64";
    const Plan p = split_plan(steps, q.ksplit);
    if (p.ksplit != q.ksplit) return "ksplit does not divide K/64 into equal-length splits";
    if (q.tiles < 1 || q.tiles > mt::kBlockMaxWaves || q.tiles > p.steps_per_split)
      return "block tiles (waves per workgroup) must be in 1..min(8, K steps per split)";
    if (q.strips < 1 || q.strips > kMaxStrips || q.strips > N / (16 / bits))
      return "block strips must be in 1..N/(16/bits)";
    const int cols = block_max_cols(N, q.strips, bits);
    if (cols > mt::kBlockMaxCols) return "blocks wider than 64 columns";
    if (!mt::block_fits_registers(mt::block_tiles(cols), nproj, rows <= 16 ? 1 : 2))
      return "the block kernel does not hold this many columns and rows in registers";
    if (block_groups_for(p.steps_per_split, group_size) > mt::kBlockMaxGroups)
      return "too many groups per split";
    const uint32_t lds = mt::block_lds_bytes(q.tiles, mt::block_tiles(cols), nproj,
                                             rows <= 16 ? 1 : 2,
                                             block_sb_words_for(p.steps_per_split, group_size));
    if (lds > mt::kBlockMaxLds) return "the block kernel's LDS does not hold this plan";
    return "";
  }
  if (q.kernel != MT_QMV_STAGED && q.kernel != MT_QMV_REGISTER) return "unknown kernel";
  if (q.order != 0) return "order is a GEMV plan field (0 for the other kernels)";
  if (q.ksplit < 1 || q.ksplit > steps) return "ksplit must be in 1..K/64";
  const Plan p = split_plan(steps, q.ksplit);
  if (p.ksplit != q.ksplit) return "ksplit does not divide K/64 into equal-length splits";
  const int groups = group_size == 32 ? 2 * p.steps_per_split : p.steps_per_split;
  if (groups > mt::kMaxGroupsPerSplit - 1) return "too many groups per split";
  if (q.kernel == MT_QMV_REGISTER) {
    if (group_size == 32) return "the register kernel takes groups of 64 or more";
    if (rows > kRowChunk) return "more rows than the register kernel takes";
    if (q.strips != base || q.tiles != 1)
      return "the register kernel runs N/32 strips, one per workgroup";
    return "";
  }
  if (rows > (group_size == 32 ? mt::kQmvLdsMaxRowsHalf : mt::kQmvLdsMaxRows))
    return "more rows than the staged kernel takes";
  if (q.strips < base || q.strips > 2 * base || q.strips > kMaxStrips)
    return "staged strips must be in N/32..2N/32";
  if (q.tiles != 1 && q.tiles != 2) return "tiles must be 1 or 2";
  if (q.strips % q.tiles) return "strips must be a multiple of tiles";
  if (!mt::affine_qmv_lds_fits(rows, p.steps_per_split, nproj, group_size, q.tiles))
    return "the staged kernel's LDS does not hold this split at these rows";
  return "";
}

// The plan dispatches of `rows` rows take: the installed one for the shape, else the planner's.
Plan plan_qmv(int rows, int K, int N, int nproj, int group_size, int bits, int dtype) {
  mt_qmv_plan q;
  if (find_qmv_plan(qmv_key(rows, K, N, nproj, group_size, bits, dtype), &q))
    return from_public(q, K);
  return planner_qmv(rows, K, N, nproj, group_size, bits);
}

// Staged strip counts worth measuring at a K split: N / 32, and the counts that put a whole
// number of workgroups on every CU within one round above the busiest CU's share.
std::vector<int> strip_options(int N, int ksplit) {
  std::vector<int> out{N / 32};
  const int kCus = device_cus();
  const long base = N / 32, per_cu = (base * ksplit + kCus - 1) / kCus;
  for (long rounds = per_cu; rounds <= per_cu + 1; ++rounds) {
    if ((rounds * kCus) % ksplit) continue;
    const long strips = rounds * kCus / ksplit;
    if (strips <= base || strips > 2 * base || strips > kMaxStrips) continue;
    bool seen = false;
    for (int v : out) seen |= v == strips;
    if (!seen) out.push_back((int)strips);
  }
  return out;
}

std::vector<mt_qmv_plan> qmv_candidates(int rows, int K, int N, int nproj, int group_size,
                                        int bits) {
  std::vector<mt_qmv_plan> out;
  const int steps = K / 64;
  int last = 0;
  for (int ks = 1; ks <= steps && ks <= kMaxCandidateSplits; ++ks) {
    const Plan p = split_plan(steps, ks);
    if (p.ksplit == last) continue;
    last = p.ksplit;
    const mt_qmv_plan reg{MT_QMV_REGISTER, p.ksplit, N / 32, 1, 0};
    if (qmv_plan_problem(rows, K, N, nproj, group_size, bits, reg).empty()) out.push_back(reg);
    for (int strips : strip_options(N, p.ksplit))
      for (int tiles : {1, 2}) {
        const mt_qmv_plan st{MT_QMV_STAGED, p.ksplit, strips, tiles, 0};
        if (qmv_plan_problem(rows, K, N, nproj, group_size, bits, st).empty()) out.push_back(st);
      }
  }
  // GEMV: when a column's chunks fit in one wave (each wave then holds whole column groups),
  // every wave count; otherwise, for each number of passes over K (one 16-byte chunk of codes
  // per lane and pass), the fewest waves that make it, and in one pass also the wave counts
  // whose lanes hold two or more whole column groups with no lane idle.
  const int chunks = K * bits / 128;
  std::vector<int> waves;
  if (chunks <= 64) {
    for (int w = 1; w <= mt::kGemvMaxWaves; ++w) waves.push_back(w);
  } else {
    for (int passes = 1; passes <= 2 * mt::kGemvMaxWaves; ++passes) {
      const int w = (chunks + 64 * passes - 1) / (64 * passes);
      if (w <= mt::kGemvMaxWaves && (waves.empty() || waves.back() != w)) waves.push_back(w);
      if (w == 1) break;
    }
    for (int w = 1; w <= mt::kGemvMaxWaves; ++w)
      if (mt::affine_gemv_groups(K, bits, w) >= 2 && (64 * w) % chunks == 0 &&
          std::find(waves.begin(), waves.end(), w) == waves.end())
        waves.push_back(w);
  }
  for (int cols : {8, 4, 2})
    for (int w : waves)
      for (int order : {1, 0}) {
        const int per_wg = cols * mt::affine_gemv_groups(K, bits, w);
        if (N % per_wg) continue;
        const mt_qmv_plan g{MT_QMV_GEMV, 1, N / per_wg, w, order};
        if (qmv_plan_problem(rows, K, N, nproj, group_size, bits, g).empty()) out.push_back(g);
      }
  // 4x4x4-MFMA GEMV: 1, 2 or 4 groups of 4 columns per workgroup, every wave count that fits.
  for (int cg : {1, 2, 4})
    for (int w = 1; w <= mt::kGemv4MaxWaves; ++w) {
      if (N % (4 * cg)) continue;
      const mt_qmv_plan g{MT_QMV_GEMV4, 1, N / (4 * cg), w, 0};
      if (qmv_plan_problem(rows, K, N, nproj, group_size, bits, g).empty()) out.push_back(g);
    }
  // Column blocks: one or two workgroups per CU, or blocks of 16 or 32 columns; 4, 6 or 8 waves
  // (six: config 3 at 16 rows 25.6 -> 25.2 us); K unsplit or in 4 splits.
  {
    const int kCus = device_cus();
    std::vector<int> strips;
    for (int s : {kCus, 2 * kCus, N / 16, N / 32})
      if (s >= 1 && std::find(strips.begin(), strips.end(), s) == strips.end()) strips.push_back(s);
    for (int ks : {1, 4}) {
      const Plan p = split_plan(steps, ks);
      if (p.ksplit != ks) continue;
      for (int s : strips)
        for (int w : {8, 6, 4}) {
          const mt_qmv_plan b{MT_QMV_BLOCK, ks, s, w, 0};
          if (qmv_plan_problem(rows, K, N, nproj, group_size, bits, b).empty()) out.push_back(b);
        }
    }
  }
  return out;
}

size_t qmv_workspace(int M, int K, int N, int nproj, int group_size, int bits) {
  // Row chunks and one remainder chunk may plan differently, and so may each dtype: the size
  // covers every plan a call of this shape can take.
  const int chunk = row_chunk(group_size);
  size_t need = 0;
  for (int rows : {M < chunk ? M : chunk, M % chunk}) {
    if (rows < 1) continue;
    std::vector<Plan> plans{planner_qmv(rows, K, N, nproj, group_size, bits)};
    for (int dtype : {MT_BF16, MT_F16}) {
      mt_qmv_plan q;
      if (find_qmv_plan(qmv_key(rows, K, N, nproj, group_size, bits, dtype), &q))
        plans.push_back(from_public(q, K));
    }
    for (const Plan& plan : plans) {
      if (plan.ksplit <= 1) continue;
      const size_t b = kCounterBytes + (size_t)plan.ksplit * nproj * rows * N * 4;
      if (b > need) need = b;
    }
  }
  return need;
}

int check_affine(const char* op, int M, int K, int N, int group_size, int bits, int dtype) {
  if (bits != 4 && bits != 8)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": bits must be 4 or 8");
  if (dtype != MT_BF16 && dtype != MT_F16)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": dtype must be MT_BF16 or MT_F16");
  if (M < 1 || K < 1 || N < 1)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": M, K and N must be positive");
  if (group_size < 32 || (group_size & (group_size - 1)) || K % group_size)
    return fail(MT_ERR_INVALID_ARGUMENT,
                std::string(op) + ": group_size must be a power of two >= 32 that divides K");
  if (K % 64 || N % 32)
    return fail(MT_ERR_INVALID_ARGUMENT,
                std::string(op) + ": K must be a multiple of 64 and N a multiple of 32");
  if (N / 32 > kMaxStrips)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": N larger than " +
                                             std::to_string(kMaxStrips * 32) + " is unsupported");
  const size_t wbytes = (size_t)N * K * bits / 8;
  const size_t xbytes = (size_t)(M < kRowChunk ? M : kRowChunk) * K * 2;
  if (wbytes >= (1ull << 31) || xbytes >= (1ull << 31) || (size_t)M * N >= (1ull << 31))
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": tensor larger than 2 GiB");
  return MT_OK;
}

// Code layouts the small-row kernels read: MLX's output-major words, or the step-major repack
// of mt_affine_repack.
enum CodeLayout : int { kLayoutMlx = 0, kLayoutStepMajor = 1 };

void set_layout(mt::QmvParams& p, int layout, int bits) {
  if (layout == kLayoutStepMajor) {
    p.col_stride = 8u * (uint32_t)bits;
    p.step_stride = (uint32_t)p.N * 8u * (uint32_t)bits;
    // A 128-byte line of repacked codes holds 128 / (8 bits) columns of one K step; strips
    // that split a line would each fetch it (balanced SwiGLU strips: 1.18x the algorithmic
    // bytes).
    p.col_align = 16 / bits;
  } else {
    p.col_stride = (uint32_t)p.K * (uint32_t)bits / 8u;
    p.step_stride = 8u * (uint32_t)bits;
    p.col_align = 1;
  }
}

int run_qmv(const char* op, int nproj, const void* x, const uint32_t* const w[2],
            const void* const s[2], const void* const b[2], const void* residual, void* y,
            int M, int K, int N, int group_size, int bits, int dtype, void* workspace,
            size_t workspace_bytes, void* stream, int layout) {
  int st = check_affine(op, M, K, N, group_size, bits, dtype);
  if (st) return st;
  if (!x || !y) return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": null x or output");
  for (int q = 0; q < nproj; ++q)
    if (!w[q] || !s[q] || !b[q])
      return fail(MT_ERR_INVALID_ARGUMENT,
                  std::string(op) + ": null packed weight, scales or biases");
  const size_t need = qmv_workspace(M, K, N, nproj, group_size, bits);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MT_ERR_WORKSPACE, std::string(op) + ": workspace of " + std::to_string(need) +
                                      " bytes required, got " + std::to_string(workspace_bytes));
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const int chunk = row_chunk(group_size);
  for (int r0 = 0; r0 < M; r0 += chunk) {
    const int rows = (M - r0) < chunk ? (M - r0) : chunk;
    const Plan plan = plan_qmv(rows, K, N, nproj, group_size, bits, dtype);
    if (group_size == 32 && plan.kernel == MT_QMV_REGISTER)
      return fail(MT_ERR_INVALID_ARGUMENT,
                  std::string(op) + ": no staged plan fits groups of 32 at this shape");
    mt::QmvParams p{};
    p.x = static_cast<const uint16_t*>(x) + (size_t)r0 * K;
    for (int q = 0; q < nproj; ++q) {
      p.w[q] = w[q];
      p.s[q] = static_cast<const uint16_t*>(s[q]);
      p.b[q] = static_cast<const uint16_t*>(b[q]);
    }
    p.residual = residual ? static_cast<const uint16_t*>(residual) + (size_t)r0 * N : nullptr;
    p.y = static_cast<uint16_t*>(y) + (size_t)r0 * N;
    if (plan.ksplit > 1) {
      p.counters = static_cast<uint32_t*>(workspace);
      p.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    }
    p.M = rows;
    p.K = K;
    p.N = N;
    p.G = group_size;
    p.group_shift = group_size >= 64 ? __builtin_ctz((unsigned)(group_size / 64)) : 0;
    p.ksplit = plan.ksplit;
    p.steps_per_split = plan.steps_per_split;
    p.strips = plan.strips;
    p.tiles = plan.kernel == MT_QMV_STAGED ? plan.tiles : 1;
    p.order = plan.order;
    p.gemv_groups = plan.kernel == MT_QMV_GEMV ? mt::affine_gemv_groups(K, bits, plan.tiles) : 1;
    p.gemv_groups_per_wave = plan.kernel == MT_QMV_GEMV ? p.gemv_groups / plan.tiles : 0;
    p.gemv_dealt = plan.kernel == MT_QMV_GEMV && plan.order ? plan.strips - plan.strips % 8 : 0;
    set_layout(p, layout, bits);
    const int units = N / p.col_align;
    p.strip_cols = units % p.strips == 0 ? units / p.strips * p.col_align : 0;
    p.groups_per_row = K / group_size;
    if (plan.kernel == MT_QMV_BLOCK) {
      p.wave_steps = (plan.steps_per_split + plan.tiles - 1) / plan.tiles;
      p.sb_words = block_sb_words_for(plan.steps_per_split, group_size);
    }
    hipError_t e;
    if (plan.kernel == MT_QMV_BLOCK)
      e = mt::launch_affine_block(
          p, bits, dtype, nproj, plan.tiles,
          mt::block_tiles((units + plan.strips - 1) / plan.strips * p.col_align), hs);
    else if (plan.kernel == MT_QMV_GEMV4)
      e = mt::launch_affine_gemv4(p, dtype, nproj, plan.tiles, N / plan.strips / 4, hs);
    else if (plan.kernel == MT_QMV_GEMV)
      e = mt::launch_affine_gemv(p, bits, dtype, nproj, plan.tiles,
                                 N / plan.strips / mt::affine_gemv_groups(K, bits, plan.tiles),
                                 hs);
    else if (plan.kernel == MT_QMV_STAGED)
      e = mt::launch_affine_qmv_lds(p, bits, dtype, nproj, hs);
    else
      e = mt::launch_affine_qmv(p, bits, dtype, nproj, hs);
    if (e != hipSuccess) return hip_fail(e, op);
  }
  return MT_OK;
}

constexpr int kDenseRowChunk = 128;  // rows per dense dispatch
// Within a dispatch, more than kDenseSubChunk rows run as grid chunks of kDenseSubChunk rows
// (two workgroups per CU instead of one with 128-row tiles); each chunk has its own partial
// sums (kDenseSubChunk rows) and counters.
constexpr int kDenseSubChunk = 64;

int dense_row_chunk(int rows) { return rows > kDenseSubChunk ? kDenseSubChunk : 0; }

// Dense plans: the K split of every dispatch of a (K, N) shape. Keyed without the rows, so that
// one plan serves every row count and each row keeps its summation order whatever M is (the
// per-row bit identity). The planner's is plan_split's; a tuner may install another.
PlanKey dense_key(int K, int N, int nproj, int dtype) {
  return PlanKey{kOpDense, 0, K, N, nproj, 0, 16, dtype};
}

Plan plan_dense(int K, int N, int nproj, int dtype) {
  if (g_plans_installed.load(std::memory_order_acquire) != 0) {
    std::shared_lock<std::shared_mutex> lock(g_plans_mu);
    const auto it = g_dense_plans.find(dense_key(K, N, nproj, dtype));
    if (it != g_dense_plans.end()) return split_plan(K / 64, it->second.ksplit);
  }
  return plan_split(K, N);
}

// Why `q` cannot run a dense dispatch of this shape ("" when it can): K split into equal-length
// splits of at least 4 steps (the four waves of a strip each take a contiguous quarter), at most
// kMaxCandidateSplits.
std::string dense_plan_problem(int K, const mt_dense_plan& q) {
  const int steps = K / 64;
  if (q.ksplit < 1 || q.ksplit > steps || q.ksplit > kMaxCandidateSplits)
    return "ksplit must be in 1..min(K/64, 32)";
  const Plan p = split_plan(steps, q.ksplit);
  if (p.ksplit != q.ksplit) return "ksplit does not divide K/64 into equal-length splits";
  if (p.steps_per_split < 4) return "each split needs at least 4 K steps (one per wave)";
  return "";
}

std::vector<mt_dense_plan> dense_candidates(int K) {
  std::vector<mt_dense_plan> out;
  int last = 0;
  for (int ks = 1; ks <= kMaxCandidateSplits / 2; ++ks) {
    const Plan p = split_plan(K / 64, ks);
    if (p.ksplit == last) continue;
    last = p.ksplit;
    const mt_dense_plan q{p.ksplit};
    if (dense_plan_problem(K, q).empty()) out.push_back(q);
  }
  return out;
}

size_t dense_workspace(int M, int K, int N, int nproj) {
  // The largest need of the planner's plan and of either dtype's installed plan.
  int ksplit = plan_split(K, N).ksplit;
  for (int dtype : {MT_BF16, MT_F16}) {
    const int ks = plan_dense(K, N, nproj, dtype).ksplit;
    if (ks > ksplit) ksplit = ks;
  }
  if (ksplit <= 1) return 0;
  const int rows = M < kDenseRowChunk ? M : kDenseRowChunk;
  const int sub = dense_row_chunk(rows);
  const int ws_rows = sub ? (rows + sub - 1) / sub * sub : rows;
  return kCounterBytes + (size_t)ksplit * nproj * ws_rows * N * 4;
}

int check_dense(const char* op, int M, int K, int N, int dtype) {
  if (dtype != MT_BF16 && dtype != MT_F16)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": dtype must be MT_BF16 or MT_F16");
  if (M < 1 || K < 1 || N < 1)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": M, K and N must be positive");
  if (K % 64 || N % 32)
    return fail(MT_ERR_INVALID_ARGUMENT,
                std::string(op) + ": K must be a multiple of 64 and N a multiple of 32");
  // Counters for two row chunks of up to kDenseSubChunk rows each.
  if (N / 32 > kMaxStrips / 2)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": N larger than " +
                                             std::to_string(kMaxStrips / 2 * 32) +
                                             " is unsupported");
  if ((size_t)N * K * 2 >= (1ull << 31) || (size_t)kDenseRowChunk * K * 2 >= (1ull << 31))
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": tensor larger than 2 GiB");
  return MT_OK;
}

int run_dense(const char* op, int nproj, const void* x, const void* const w[2],
              const void* residual, void* y, int M, int K, int N, int dtype, void* workspace,
              size_t workspace_bytes, void* stream) {
  int st = check_dense(op, M, K, N, dtype);
  if (st) return st;
  if (!x || !y) return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": null x or output");
  for (int q = 0; q < nproj; ++q)
    if (!w[q]) return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": null weight");
  const size_t need = dense_workspace(M, K, N, nproj);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MT_ERR_WORKSPACE, std::string(op) + ": workspace of " + std::to_string(need) +
                                      " bytes required, got " + std::to_string(workspace_bytes));
  const Plan plan = plan_dense(K, N, nproj, dtype);
  for (int r0 = 0; r0 < M; r0 += kDenseRowChunk) {
    const int rows = (M - r0) < kDenseRowChunk ? (M - r0) : kDenseRowChunk;
    mt::DenseParams p{};
    p.x = static_cast<const uint16_t*>(x) + (size_t)r0 * K;
    for (int q = 0; q < nproj; ++q) p.w[q] = static_cast<const uint16_t*>(w[q]);
    p.residual = residual ? static_cast<const uint16_t*>(residual) + (size_t)r0 * N : nullptr;
    p.y = static_cast<uint16_t*>(y) + (size_t)r0 * N;
    if (plan.ksplit > 1) {
      p.counters = static_cast<uint32_t*>(workspace);
      p.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    }
    p.M = rows;
    p.K = K;
    p.N = N;
    p.ksplit = plan.ksplit;
    p.steps_per_split = plan.steps_per_split;
    p.row_chunk = dense_row_chunk(rows);
    const hipError_t e = mt::launch_dense_qmv(p, dtype, nproj, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, op);
  }
  return MT_OK;
}

// Prefill GEMM plans. Kernel 0 (register-staged, affine_gemm.hip): square tiles of 64 or 128.
// Kernel 1 (ring, affine_gemm_ring.hip): tiles of 128 x tile_n, tile_n 64, 96, 128, 160, 192 or
// 256 (workgroups of eight waves for 128, 192 and 256, else four), N a multiple of 8, splits of
// a multiple of three K steps, at most kGemmMaxSplits of them.
struct GemmPlan {
  int kernel;  // 0: register-staged, 1: ring
  int tile;    // kernel 0: 2 (128 x 128) or 1 (64 x 64)
  int tile_n;  // kernel 1
  int tiles;
  int ksplit;
  int steps_per_split;
  int sb_words;  // kernel 1: scale (and bias) dwords staged per column
  int order;     // kernel 1: tile order (MT_GEMM_ORDER_*)
};

int gemm_tiles(int M, int N, int tile) {
  const int t = tile == 2 ? 128 : 64;
  return ((M + t - 1) / t) * ((N + t - 1) / t);
}

int ring_tiles(int M, int N, int tile_n) {
  return ((M + 127) / 128) * ((N + tile_n - 1) / tile_n);
}

bool ring_tile_ok(int tile_n) {
  return tile_n == 64 || tile_n == 96 || tile_n == 128 || tile_n == 160 || tile_n == 192 ||
         tile_n == 256;
}

// Ring splits: equal lengths rounded up to whole loop iterations (three steps).
Plan ring_split(int steps, int ksplit) {
  Plan p{};
  const int len = (steps + ksplit - 1) / ksplit;
  p.steps_per_split = (len + 2) / 3 * 3;
  p.ksplit = (steps + p.steps_per_split - 1) / p.steps_per_split;
  return p;
}

// Scale dwords a ring split stages per column: the groups it spans at the smallest group size
// (64; larger groups need fewer), one more for a start inside a dword.
int ring_sb_words(int steps_per_split) { return steps_per_split / 2 + 1; }

bool ring_lds_ok(int tile_n, int steps_per_split) {
  return mt::gemm_ring_static_lds(tile_n) +
             mt::gemm_ring_dynamic_lds(tile_n, ring_sb_words(steps_per_split)) <=
         mt::kGemmRingLdsBytes;
}

GemmPlan make_ring(int M, int K, int N, int tile_n, int ksplit) {
  GemmPlan g{};
  g.kernel = 1;
  g.tile_n = tile_n;
  g.tiles = ring_tiles(M, N, tile_n);
  const Plan p = ring_split(K / 64, ksplit);
  g.ksplit = p.ksplit;
  g.steps_per_split = p.steps_per_split;
  g.sb_words = ring_sb_words(p.steps_per_split);
  return g;
}

GemmPlan make_staged(int M, int K, int N, int tile, int ksplit) {
  GemmPlan g{};
  g.kernel = 0;
  g.tile = tile;
  g.tiles = gemm_tiles(M, N, tile);
  const Plan p = split_plan(K / 64, ksplit);
  g.ksplit = p.ksplit;
  g.steps_per_split = p.steps_per_split;
  return g;
}

// Why `q` cannot run the prefill GEMM at this shape for up to `M` rows ("" when it can); with a
// split, one arrival counter per output tile.
std::string gemm_plan_problem(int M, int K, int N, const mt_gemm_plan& q) {
  const int steps = K / 64;
  if (q.ksplit < 1 || q.ksplit > steps) return "ksplit must be in 1..K/64";
  if (q.order < 0 || q.order > 2) return "order must be 0, 1 or 2";
  if (q.kernel == 0 && q.order != 0) return "kernel 0 takes order 0";
  if (q.kernel == 0) {
    if (q.tile_m != q.tile_n || (q.tile_m != 64 && q.tile_m != 128))
      return "kernel 0 takes square tiles of 64 or 128";
    const Plan p = split_plan(steps, q.ksplit);
    if (p.ksplit != q.ksplit) return "ksplit does not divide K/64 into equal-length splits";
    if (q.ksplit > 1 && gemm_tiles(M, N, q.tile_m == 128 ? 2 : 1) > kMaxStrips)
      return "too many output tiles to split K";
    return "";
  }
  if (q.kernel != 1) return "kernel must be 0 (register-staged) or 1 (ring)";
  if (q.tile_m != 128 || !ring_tile_ok(q.tile_n))
    return "kernel 1 takes tiles of 128 x 64, 96, 128, 160, 192 or 256";
  if (N % 8) return "kernel 1 needs N to be a multiple of 8";
  if (q.ksplit > mt::kGemmMaxSplits) return "kernel 1 takes at most 8 K splits";
  const Plan p = ring_split(steps, q.ksplit);
  if (p.ksplit != q.ksplit)
    return "ksplit does not divide K/64 into splits of whole three-step iterations";
  if (!ring_lds_ok(q.tile_n, p.steps_per_split))
    return "the split's scales and biases do not fit in LDS (split K further)";
  if (q.ksplit > 1 && ring_tiles(M, N, q.tile_n) > kMaxStrips)
    return "too many output tiles to split K";
  if (q.ksplit > 1 && (size_t)q.ksplit * ring_tiles(M, N, q.tile_n) * 128 * q.tile_n * 4 >=
                          (1ull << 32))
    return "the partial sums would exceed 4 GiB";
  return "";
}

// The planner (measured on MI355X at the Qwen2.5-1.5B prefill shapes, M = 512): the ring kernel
// when N allows it, with 128 x 192 tiles (eight-wave workgroups) unsplit when they give at
// least half a workgroup per CU (up projection 1536 x 8960: 188 workgroups, 31.0 us; 128 x 160
// four-wave tiles 31.3 us; the best register-staged plan 42.4 us), in the XCD-contiguous order
// with row blocks fastest, which fetches each column tile's codes into one L2 (HBM bytes 2.86x
// -> 1.63x the algorithmic, time unchanged), else 128 x 96 tiles with K
// split to about one workgroup per CU (down projection 8960 x 1536: four splits, 33.9 us;
// 128 x 128 in five splits 35.0 us; register-staged 47.0 us); the register-staged kernel
// otherwise: 128 x 128 tiles when they give about one workgroup per CU, else 64 x 64, K split
// to about three workgroups per CU keeping 24 steps per split.
GemmPlan planner_gemm(int M, int K, int N) {
  const int steps = K / 64;
  if (N % 8 == 0) {
    for (int tile_n : {192, 96}) {
      const int tiles = ring_tiles(M, N, tile_n);
      if (tile_n == 192 && tiles < 128) continue;
      int ks = tile_n == 192 ? 1 : (256 + tiles / 2) / tiles;
      ks = ks < 1 ? 1 : ks > mt::kGemmMaxSplits ? mt::kGemmMaxSplits : ks;
      for (; ks <= mt::kGemmMaxSplits && ks <= steps; ++ks) {
        const mt_gemm_plan q{1, 128, tile_n, ring_split(steps, ks).ksplit, 0};
        if (gemm_plan_problem(M, K, N, q).empty()) {
          GemmPlan g = make_ring(M, K, N, tile_n, q.ksplit);
          if (g.ksplit == 1) g.order = MT_GEMM_ORDER_XCD_ROWS;
          return g;
        }
      }
    }
  }
  const int t128 = gemm_tiles(M, N, 2), t64 = gemm_tiles(M, N, 1);
  const int tile = t128 >= 200 ? 2 : 1;
  const int tiles = tile == 2 ? t128 : t64;
  int ksplit = (768 + tiles / 2) / tiles;
  const int max_split = steps / 24 > 0 ? steps / 24 : 1;
  if (ksplit > max_split) ksplit = max_split;
  if (ksplit < 1) ksplit = 1;
  return make_staged(M, K, N, tile, ksplit);
}

PlanKey gemm_key(int M, int K, int N, int group_size, int dtype) {
  return PlanKey{kOpGemm, row_bucket(M), K, N, 1, group_size, 4, dtype};
}

bool find_gemm_plan(const PlanKey& key, mt_gemm_plan* out) {
  if (g_plans_installed.load(std::memory_order_acquire) == 0) return false;
  std::shared_lock<std::shared_mutex> lock(g_plans_mu);
  const auto it = g_gemm_plans.find(key);
  if (it == g_gemm_plans.end()) return false;
  *out = it->second;
  return true;
}

GemmPlan plan_gemm(int M, int K, int N, int group_size, int dtype) {
  mt_gemm_plan q;
  if (find_gemm_plan(gemm_key(M, K, N, group_size, dtype), &q)) {
    if (q.kernel == 1) {
      GemmPlan g = make_ring(M, K, N, q.tile_n, q.ksplit);
      g.order = q.order;
      return g;
    }
    return make_staged(M, K, N, q.tile_m == 128 ? 2 : 1, q.ksplit);
  }
  return planner_gemm(M, K, N);
}

mt_gemm_plan gemm_to_public(const GemmPlan& g) {
  if (g.kernel == 1) return mt_gemm_plan{1, 128, g.tile_n, g.ksplit, g.order};
  const int t = g.tile == 2 ? 128 : 64;
  return mt_gemm_plan{0, t, t, g.ksplit, 0};
}

std::vector<mt_gemm_plan> gemm_candidates(int M, int K, int N) {
  std::vector<mt_gemm_plan> out;
  const int steps = K / 64;
  for (int tile : {64, 128}) {
    int last = 0;
    for (int ks = 1; ks <= steps && ks <= kMaxCandidateSplits / 2; ++ks) {
      const Plan p = split_plan(steps, ks);
      if (p.ksplit == last) continue;
      last = p.ksplit;
      const mt_gemm_plan q{0, tile, tile, p.ksplit, 0};
      if (gemm_plan_problem(M, K, N, q).empty()) out.push_back(q);
    }
  }
  for (int tile_n : {64, 96, 128, 160, 192, 256}) {
    int last = 0;
    for (int ks = 1; ks <= steps && ks <= mt::kGemmMaxSplits; ++ks) {
      const Plan p = ring_split(steps, ks);
      if (p.ksplit == last) continue;
      last = p.ksplit;
      for (int order : {MT_GEMM_ORDER_GRID, MT_GEMM_ORDER_XCD_COLUMNS, MT_GEMM_ORDER_XCD_ROWS}) {
        const mt_gemm_plan q{1, 128, tile_n, p.ksplit, order};
        if (gemm_plan_problem(M, K, N, q).empty()) out.push_back(q);
      }
    }
  }
  return out;
}

size_t gemm_workspace(int M, int K, int N, int group_size) {
  size_t need = 0;
  for (int dtype : {MT_BF16, MT_F16}) {
    const GemmPlan g = plan_gemm(M, K, N, group_size, dtype);
    if (g.ksplit > 1) {
      // kernel 0: [ksplit][M][N] fp32 partial sums; kernel 1: [ksplit][tile][128 x tile_n] in
      // the accumulators' register layout
      const size_t part = g.kernel == 0 ? (size_t)M * N : (size_t)g.tiles * 128 * g.tile_n;
      const size_t b = kCounterBytes + (size_t)g.ksplit * part * 4;
      if (b > need) need = b;
    }
  }
  return need;
}

// ---- MLP workspace ------------------------------------------------------------------------
// [counters + split-K partials of either projection | hidden activation]: the gate/up and down
// launches share the counter region (each leaves it zeroed) and the partial space, which lies
// below the hidden activation.
struct MlpPlan {
  size_t hidden, bytes;  // workspace offset of the hidden activation, and the total
};

MlpPlan plan_mlp(int M, int H, int I, int group_size, int bits) {
  const size_t a = qmv_workspace(M, H, I, 2, group_size, bits);
  const size_t b = qmv_workspace(M, I, H, 1, group_size, bits);
  const size_t split = align_up(a > b ? a : b);
  MlpPlan mp{};
  mp.hidden = split > kCounterBytes ? split : kCounterBytes;
  mp.bytes = mp.hidden + align_up((size_t)M * I * 2);
  return mp;
}

}  // namespace

namespace {

int affine_qmv_impl(const char* op, const void* x, const uint32_t* w_q, const void* scales,
                    const void* biases, const void* residual, void* y, int M, int K, int N,
                    int group_size, int bits, int dtype, void* workspace, size_t workspace_bytes,
                    void* stream, int layout) {
  const uint32_t* w[2] = {w_q, nullptr};
  const void* s[2] = {scales, nullptr};
  const void* b[2] = {biases, nullptr};
  return run_qmv(op, 1, x, w, s, b, residual, y, M, K, N, group_size, bits, dtype, workspace,
                 workspace_bytes, stream, layout);
}

int affine_swiglu_impl(const char* op, const void* x, const uint32_t* gate_w,
                       const void* gate_scales, const void* gate_biases, const uint32_t* up_w,
                       const void* up_scales, const void* up_biases, void* h, int M, int K, int N,
                       int group_size, int bits, int dtype, void* workspace,
                       size_t workspace_bytes, void* stream, int layout) {
  const uint32_t* w[2] = {gate_w, up_w};
  const void* s[2] = {gate_scales, up_scales};
  const void* b[2] = {gate_biases, up_biases};
  return run_qmv(op, 2, x, w, s, b, nullptr, h, M, K, N, group_size, bits, dtype, workspace,
                 workspace_bytes, stream, layout);
}

int mlp_check_shape(const char* op, int M, int H, int I, int group_size, int bits, int dtype) {
  const int st = check_affine(op, M, H, I, group_size, bits, dtype);
  return st ? st : check_affine(op, M, I, H, group_size, bits, dtype);
}

int mlp_check_pointers(const char* op, const void* x, const void* y, const void* const p[9]) {
  bool ok = x && y;
  for (int i = 0; i < 9; ++i) ok = ok && p[i];
  return ok ? MT_OK : fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": null pointer");
}

int affine_mlp_impl(const char* op, const void* x, const uint32_t* gate_w,
                    const void* gate_scales, const void* gate_biases, const uint32_t* up_w,
                    const void* up_scales, const void* up_biases, const uint32_t* down_w,
                    const void* down_scales, const void* down_biases, const void* residual,
                    void* y, int M, int H, int I, int group_size, int bits, int dtype,
                    void* workspace, size_t workspace_bytes, void* stream, int up_layout,
                    int down_layout) {
  int st = mlp_check_shape(op, M, H, I, group_size, bits, dtype);
  if (st) return st;
  const size_t need = plan_mlp(M, H, I, group_size, bits).bytes;
  if (!workspace || workspace_bytes < need)
    return fail(MT_ERR_WORKSPACE, std::string(op) + ": workspace of " + std::to_string(need) +
                                      " bytes required, got " + std::to_string(workspace_bytes));
  const void* const ptrs[9] = {gate_w, gate_scales, gate_biases, up_w, up_scales,
                               up_biases, down_w, down_scales, down_biases};
  st = mlp_check_pointers(op, x, y, ptrs);
  if (st) return st;
  const MlpPlan mp = plan_mlp(M, H, I, group_size, bits);
  void* h = static_cast<char*>(workspace) + mp.hidden;
  st = affine_swiglu_impl(op, x, gate_w, gate_scales, gate_biases, up_w, up_scales, up_biases, h,
                          M, H, I, group_size, bits, dtype, workspace, mp.hidden, stream,
                          up_layout);
  if (st) return st;
  return affine_qmv_impl(op, h, down_w, down_scales, down_biases, residual, y, M, I, H,
                         group_size, bits, dtype, workspace, mp.hidden, stream, down_layout);
}

}  // namespace

// Entry points in other source files that bring their own workspace (noalloc.hip) reach the MLP
// path and the error slot through these.
namespace mt {

int set_last_error(int status, const std::string& msg) { return fail(status, msg); }

size_t affine_mlp_workspace(int M, int H, int I, int group_size, int bits) {
  if (check_affine("mt_affine_mlp", M, H, I, group_size, bits, MT_BF16) ||
      check_affine("mt_affine_mlp", M, I, H, group_size, bits, MT_BF16))
    return 0;
  return plan_mlp(M, H, I, group_size, bits).bytes;
}

int affine_mlp_check(const char* op, const void* x, const uint32_t* gate_w,
                     const void* gate_scales, const void* gate_biases, const uint32_t* up_w,
                     const void* up_scales, const void* up_biases, const uint32_t* down_w,
                     const void* down_scales, const void* down_biases, const void* y, int M,
                     int H, int I, int group_size, int bits, int dtype) {
  const int st = mlp_check_shape(op, M, H, I, group_size, bits, dtype);
  if (st) return st;
  const void* const ptrs[9] = {gate_w, gate_scales, gate_biases, up_w, up_scales,
                               up_biases, down_w, down_scales, down_biases};
  return mlp_check_pointers(op, x, y, ptrs);
}

int affine_mlp(const char* op, const void* x, const uint32_t* gate_w, const void* gate_scales,
               const void* gate_biases, const uint32_t* up_w, const void* up_scales,
               const void* up_biases, const uint32_t* down_w, const void* down_scales,
               const void* down_biases, const void* residual, void* y, int M, int H, int I,
               int group_size, int bits, int dtype, void* workspace, size_t workspace_bytes,
               void* stream) {
  return affine_mlp_impl(op, x, gate_w, gate_scales, gate_biases, up_w, up_scales, up_biases,
                         down_w, down_scales, down_biases, residual, y, M, H, I, group_size,
                         bits, dtype, workspace, workspace_bytes, stream, kLayoutMlx, kLayoutMlx);
}

}  // namespace mt

extern "C" {

const char* mt_version(void) { return "metile_amd 0.1.0 (gfx950)"; }

const char* mt_last_error(void) { return g_last_error.c_str(); }

size_t mt_affine_qmv_workspace_bytes(int M, int K, int N, int group_size, int bits, int nproj) {
  if (check_affine("mt_affine_qmv_workspace_bytes", M, K, N, group_size, bits, MT_BF16))
    return 0;
  return qmv_workspace(M, K, N, nproj == 2 ? 2 : 1, group_size, bits);
}

int mt_affine_qmv(const void* x, const uint32_t* w_q, const void* scales, const void* biases,
                  const void* residual, void* y, int M, int K, int N, int group_size, int bits,
                  int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return affine_qmv_impl("mt_affine_qmv", x, w_q, scales, biases, residual, y, M, K, N,
                         group_size, bits, dtype, workspace, workspace_bytes, stream, kLayoutMlx);
}

int mt_affine_swiglu(const void* x, const uint32_t* gate_w, const void* gate_scales,
                     const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                     const void* up_biases, void* h, int M, int K, int N, int group_size,
                     int bits, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return affine_swiglu_impl("mt_affine_swiglu", x, gate_w, gate_scales, gate_biases, up_w,
                            up_scales, up_biases, h, M, K, N, group_size, bits, dtype, workspace,
                            workspace_bytes, stream, kLayoutMlx);
}

size_t mt_affine_mlp_workspace_bytes(int M, int H, int I, int group_size, int bits) {
  if (check_affine("mt_affine_mlp_workspace_bytes", M, H, I, group_size, bits, MT_BF16) ||
      check_affine("mt_affine_mlp_workspace_bytes", M, I, H, group_size, bits, MT_BF16))
    return 0;
  return plan_mlp(M, H, I, group_size, bits).bytes;
}

int mt_affine_mlp(const void* x, const uint32_t* gate_w, const void* gate_scales,
                  const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                  const void* up_biases, const uint32_t* down_w, const void* down_scales,
                  const void* down_biases, const void* residual, void* y, int M, int H, int I,
                  int group_size, int bits, int dtype, void* workspace, size_t workspace_bytes,
                  void* stream) {
  return affine_mlp_impl("mt_affine_mlp", x, gate_w, gate_scales, gate_biases, up_w, up_scales,
                         up_biases, down_w, down_scales, down_biases, residual, y, M, H, I,
                         group_size, bits, dtype, workspace, workspace_bytes, stream,
                         kLayoutMlx, kLayoutMlx);
}

int mt_affine_quantize(const void* w, uint32_t* w_q, void* scales, void* biases, int N, int K,
                       int group_size, int bits, int dtype, void* stream) {
  if (bits != 4 && bits != 8)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_quantize: bits must be 4 or 8");
  if (dtype != MT_BF16 && dtype != MT_F16)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_quantize: dtype must be MT_BF16 or MT_F16");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_quantize: group_size must be 32, 64 or 128");
  if (N < 1 || K < group_size || K % group_size)
    return fail(MT_ERR_INVALID_ARGUMENT,
                "mt_affine_quantize: N must be positive and K a positive multiple of group_size");
  if (!w || !w_q || !scales || !biases)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_quantize: null pointer");
  if ((size_t)N * K * 2 >= (1ull << 31))
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_quantize: tensor larger than 2 GiB");
  const hipError_t e = mt::launch_affine_quantize(
      static_cast<const uint16_t*>(w), w_q, static_cast<uint16_t*>(scales),
      static_cast<uint16_t*>(biases), N, K, group_size, bits, dtype,
      static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "mt_affine_quantize");
  return MT_OK;
}

int mt_affine_repack(const uint32_t* w_q, uint32_t* out, int N, int K, int bits, void* stream) {
  if (bits != 4 && bits != 8)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_repack: bits must be 4 or 8");
  if (N < 1 || K < 64 || K % 64)
    return fail(MT_ERR_INVALID_ARGUMENT,
                "mt_affine_repack: N must be positive and K a positive multiple of 64");
  if (!w_q || !out)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_repack: null pointer");
  if ((reinterpret_cast<uintptr_t>(w_q) | reinterpret_cast<uintptr_t>(out)) & 15u)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_repack: buffers must be 16-byte aligned");
  if ((size_t)N * K * bits / 8 >= (1ull << 31))
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_repack: tensor larger than 2 GiB");
  const hipError_t e =
      mt::launch_affine_repack(w_q, out, N, K, bits, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "mt_affine_repack");
  return MT_OK;
}

int mt_affine_qmv_repacked(const void* x, const uint32_t* w_packed, const void* scales,
                           const void* biases, const void* residual, void* y, int M, int K, int N,
                           int group_size, int bits, int dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return affine_qmv_impl("mt_affine_qmv_repacked", x, w_packed, scales, biases, residual, y, M, K,
                         N, group_size, bits, dtype, workspace, workspace_bytes, stream,
                         kLayoutStepMajor);
}

int mt_affine_swiglu_repacked(const void* x, const uint32_t* gate_packed, const void* gate_scales,
                              const void* gate_biases, const uint32_t* up_packed,
                              const void* up_scales, const void* up_biases, void* h, int M, int K,
                              int N, int group_size, int bits, int dtype, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return affine_swiglu_impl("mt_affine_swiglu_repacked", x, gate_packed, gate_scales, gate_biases,
                            up_packed, up_scales, up_biases, h, M, K, N, group_size, bits, dtype,
                            workspace, workspace_bytes, stream, kLayoutStepMajor);
}

int mt_affine_mlp_repacked(const void* x, const uint32_t* gate_packed, const void* gate_scales,
                           const void* gate_biases, const uint32_t* up_packed,
                           const void* up_scales, const void* up_biases,
                           const uint32_t* down_packed, const void* down_scales,
                           const void* down_biases, const void* residual, void* y, int M, int H,
                           int I, int group_size, int bits, int dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return affine_mlp_impl("mt_affine_mlp_repacked", x, gate_packed, gate_scales, gate_biases,
                         up_packed, up_scales, up_biases, down_packed, down_scales, down_biases,
                         residual, y, M, H, I, group_size, bits, dtype, workspace,
                         workspace_bytes, stream, kLayoutStepMajor, kLayoutStepMajor);
}

int mt_affine_mlp_layouts(const void* x, const uint32_t* gate_w, const void* gate_scales,
                          const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                          const void* up_biases, const uint32_t* down_w, const void* down_scales,
                          const void* down_biases, const void* residual, void* y, int M, int H,
                          int I, int group_size, int bits, int dtype, int up_layout,
                          int down_layout, void* workspace, size_t workspace_bytes,
                          void* stream) {
  for (int l : {up_layout, down_layout})
    if (l != MT_LAYOUT_MLX && l != MT_LAYOUT_REPACKED)
      return fail(MT_ERR_INVALID_ARGUMENT,
                  "mt_affine_mlp_layouts: layouts must be MT_LAYOUT_MLX or MT_LAYOUT_REPACKED");
  return affine_mlp_impl("mt_affine_mlp_layouts", x, gate_w, gate_scales, gate_biases, up_w,
                         up_scales, up_biases, down_w, down_scales, down_biases, residual, y, M,
                         H, I, group_size, bits, dtype, workspace, workspace_bytes, stream,
                         up_layout == MT_LAYOUT_REPACKED ? kLayoutStepMajor : kLayoutMlx,
                         down_layout == MT_LAYOUT_REPACKED ? kLayoutStepMajor : kLayoutMlx);
}

int mt_affine_dequantize(const uint32_t* w_q, const void* scales, const void* biases,
                         float* out, int N, int K, int group_size, int bits, int dtype,
                         void* stream) {
  if (bits != 4 && bits != 8)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_dequantize: bits must be 4 or 8");
  if (dtype != MT_BF16 && dtype != MT_F16)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_dequantize: dtype must be MT_BF16 or MT_F16");
  if (N < 1 || K < 1 || group_size < 1 || K % group_size || K % (32 / bits) ||
      group_size % (32 / bits))
    return fail(MT_ERR_INVALID_ARGUMENT,
                "mt_affine_dequantize: group_size must divide K and hold whole packed words");
  if (!w_q || !scales || !biases || !out)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_dequantize: null pointer");
  const hipError_t e = mt::launch_affine_dequantize(
      w_q, static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases), out, N, K,
      group_size, bits, dtype, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "mt_affine_dequantize");
  return MT_OK;
}

size_t mt_dense_workspace_bytes(int M, int K, int N, int nproj) {
  if (check_dense("mt_dense_workspace_bytes", M, K, N, MT_BF16)) return 0;
  return dense_workspace(M, K, N, nproj == 2 ? 2 : 1);
}

int mt_dense_swiglu(const void* x, const void* gate_w, const void* up_w, void* h, int M, int K,
                    int N, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const void* w[2] = {gate_w, up_w};
  return run_dense("mt_dense_swiglu", 2, x, w, nullptr, h, M, K, N, dtype, workspace,
                   workspace_bytes, stream);
}

int mt_dense_residual_qmv(const void* x, const void* w, const void* residual, void* y, int M,
                          int K, int N, int dtype, void* workspace, size_t workspace_bytes,
                          void* stream) {
  const void* ws[2] = {w, nullptr};
  return run_dense("mt_dense_residual_qmv", 1, x, ws, residual, y, M, K, N, dtype, workspace,
                   workspace_bytes, stream);
}

size_t mt_affine_gemm_workspace_bytes(int M, int K, int N, int group_size, int bits) {
  if (check_affine("mt_affine_gemm_workspace_bytes", 1, K, N, group_size, bits, MT_BF16) ||
      M < 1 || group_size < 64)
    return 0;
  return gemm_workspace(M, K, N, group_size);
}

int mt_affine_gemm(const void* x, const uint32_t* w_q, const void* scales, const void* biases,
                   void* y, int M, int K, int N, int group_size, int bits, int dtype,
                   void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_affine("mt_affine_gemm", 1, K, N, group_size, bits, dtype);
  if (st) return st;
  if (bits != 4)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm: the prefill GEMM takes 4-bit codes");
  if (group_size < 64)
    return fail(MT_ERR_INVALID_ARGUMENT,
                "mt_affine_gemm: the prefill GEMM takes groups of 64 or more");
  if (M < 1) return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm: M must be positive");
  if ((size_t)M * K * 2 >= (1ull << 31) || (size_t)M * N >= (1ull << 31))
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm: tensor larger than 2 GiB");
  if (!x || !w_q || !scales || !biases || !y)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm: null pointer");
  const GemmPlan g = plan_gemm(M, K, N, group_size, dtype);
  const size_t need = gemm_workspace(M, K, N, group_size);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MT_ERR_WORKSPACE, "mt_affine_gemm: workspace of " + std::to_string(need) +
                                      " bytes required, got " + std::to_string(workspace_bytes));
  if (g.ksplit > 1 && g.tiles > kMaxStrips)
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm: too many output tiles to split K");
  mt::GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.w = w_q;
  p.s = static_cast<const uint16_t*>(scales);
  p.b = static_cast<const uint16_t*>(biases);
  p.y = static_cast<uint16_t*>(y);
  if (g.ksplit > 1) {
    p.counters = static_cast<uint32_t*>(workspace);
    p.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  p.M = M;
  p.K = K;
  p.N = N;
  p.G = group_size;
  p.tile = g.tile;
  p.tile_n = g.tile_n;
  p.ksplit = g.ksplit;
  p.steps_per_split = g.steps_per_split;
  p.sb_words = g.sb_words;
  p.order = g.kernel == 1 ? g.order : 0;
  const hipError_t e =
      g.kernel == 1 ? mt::launch_affine_gemm_ring(p, dtype, static_cast<hipStream_t>(stream))
                    : mt::launch_affine_gemm(p, dtype, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "mt_affine_gemm");
  return MT_OK;
}

// ---- plans ------------------------------------------------------------------------------------

#ifndef MT_SOURCE_DIGEST
#define MT_SOURCE_DIGEST "unknown"
#endif

const char* mt_source_digest(void) { return MT_SOURCE_DIGEST; }

static int check_qmv_plan_shape(const char* op, int M, int K, int N, int group_size, int bits,
                                int nproj, int dtype) {
  const int st = check_affine(op, M, K, N, group_size, bits, dtype);
  if (st) return st;
  if (nproj != 1 && nproj != 2)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": nproj must be 1 or 2");
  if (M > row_chunk(group_size))
    return fail(MT_ERR_INVALID_ARGUMENT,
                std::string(op) + ": M is the rows of one dispatch, at most " +
                    std::to_string(row_chunk(group_size)) + " at this group size");
  return MT_OK;
}

int mt_affine_qmv_plan(int M, int K, int N, int group_size, int bits, int nproj, int dtype,
                       mt_qmv_plan* out) {
  const int st =
      check_qmv_plan_shape("mt_affine_qmv_plan", M, K, N, group_size, bits, nproj, dtype);
  if (st) return st;
  if (!out) return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_qmv_plan: null output");
  *out = to_public(plan_qmv(M, K, N, nproj, group_size, bits, dtype));
  return MT_OK;
}

int mt_affine_qmv_plan_candidates(int M, int K, int N, int group_size, int bits, int nproj,
                                  mt_qmv_plan* out, int capacity) {
  const int st = check_qmv_plan_shape("mt_affine_qmv_plan_candidates", M, K, N, group_size, bits,
                                      nproj, MT_BF16);
  if (st) return st;
  if (capacity < 0 || (capacity > 0 && !out))
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_qmv_plan_candidates: bad output buffer");
  const std::vector<mt_qmv_plan> c =
      qmv_candidates(row_bucket(M), K, N, nproj, group_size, bits);
  for (int i = 0; i < (int)c.size() && i < capacity; ++i) out[i] = c[i];
  return (int)c.size();
}

int mt_affine_qmv_plan_set(int M, int K, int N, int group_size, int bits, int nproj, int dtype,
                           const mt_qmv_plan* plan) {
  const int st =
      check_qmv_plan_shape("mt_affine_qmv_plan_set", M, K, N, group_size, bits, nproj, dtype);
  if (st) return st;
  const PlanKey key = qmv_key(M, K, N, nproj, group_size, bits, dtype);
  if (plan) {
    const std::string why = qmv_plan_problem(key.rows, K, N, nproj, group_size, bits, *plan);
    if (!why.empty()) return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_qmv_plan_set: " + why);
  }
  std::unique_lock<std::shared_mutex> lock(g_plans_mu);
  if (plan) g_qmv_plans[key] = *plan;
  else g_qmv_plans.erase(key);
  g_plans_installed.store(installed_plans(), std::memory_order_release);
  return MT_OK;
}

static int check_gemm_plan_shape(const char* op, int M, int K, int N, int group_size,
                                 int dtype) {
  const int st = check_affine(op, 1, K, N, group_size, 4, dtype);
  if (st) return st;
  if (M < 1) return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": M must be positive");
  if (group_size < 64)
    return fail(MT_ERR_INVALID_ARGUMENT,
                std::string(op) + ": the prefill GEMM takes groups of 64 or more");
  return MT_OK;
}

int mt_affine_gemm_plan(int M, int K, int N, int group_size, int dtype, mt_gemm_plan* out) {
  const int st = check_gemm_plan_shape("mt_affine_gemm_plan", M, K, N, group_size, dtype);
  if (st) return st;
  if (!out) return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm_plan: null output");
  *out = gemm_to_public(plan_gemm(M, K, N, group_size, dtype));
  return MT_OK;
}

int mt_affine_gemm_plan_candidates(int M, int K, int N, int group_size, mt_gemm_plan* out,
                                   int capacity) {
  const int st =
      check_gemm_plan_shape("mt_affine_gemm_plan_candidates", M, K, N, group_size, MT_BF16);
  if (st) return st;
  if (capacity < 0 || (capacity > 0 && !out))
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm_plan_candidates: bad output buffer");
  const std::vector<mt_gemm_plan> c = gemm_candidates(row_bucket(M), K, N);
  for (int i = 0; i < (int)c.size() && i < capacity; ++i) out[i] = c[i];
  return (int)c.size();
}

int mt_affine_gemm_plan_set(int M, int K, int N, int group_size, int dtype,
                            const mt_gemm_plan* plan) {
  const int st = check_gemm_plan_shape("mt_affine_gemm_plan_set", M, K, N, group_size, dtype);
  if (st) return st;
  const PlanKey key = gemm_key(M, K, N, group_size, dtype);
  if (plan) {
    const std::string why = gemm_plan_problem(key.rows, K, N, *plan);
    if (!why.empty()) return fail(MT_ERR_INVALID_ARGUMENT, "mt_affine_gemm_plan_set: " + why);
  }
  std::unique_lock<std::shared_mutex> lock(g_plans_mu);
  if (plan) g_gemm_plans[key] = *plan;
  else g_gemm_plans.erase(key);
  g_plans_installed.store(installed_plans(), std::memory_order_release);
  return MT_OK;
}

int mt_plans_clear(void) {
  std::unique_lock<std::shared_mutex> lock(g_plans_mu);
  g_qmv_plans.clear();
  g_gemm_plans.clear();
  g_dense_plans.clear();
  g_plans_installed.store(0, std::memory_order_release);
  return MT_OK;
}

static int check_dense_plan_shape(const char* op, int K, int N, int nproj, int dtype) {
  if (nproj != 1 && nproj != 2)
    return fail(MT_ERR_INVALID_ARGUMENT, std::string(op) + ": nproj must be 1 or 2");
  return check_dense(op, 1, K, N, dtype);
}

int mt_dense_qmv_plan(int K, int N, int nproj, int dtype, mt_dense_plan* out) {
  const int st = check_dense_plan_shape("mt_dense_qmv_plan", K, N, nproj, dtype);
  if (st) return st;
  if (!out) return fail(MT_ERR_INVALID_ARGUMENT, "mt_dense_qmv_plan: null output");
  *out = mt_dense_plan{plan_dense(K, N, nproj, dtype).ksplit};
  return MT_OK;
}

int mt_dense_qmv_plan_candidates(int K, int N, int nproj, mt_dense_plan* out, int capacity) {
  const int st = check_dense_plan_shape("mt_dense_qmv_plan_candidates", K, N, nproj, MT_BF16);
  if (st) return st;
  if (capacity < 0 || (capacity > 0 && !out))
    return fail(MT_ERR_INVALID_ARGUMENT, "mt_dense_qmv_plan_candidates: bad output buffer");
  const std::vector<mt_dense_plan> c = dense_candidates(K);
  for (int i = 0; i < (int)c.size() && i < capacity; ++i) out[i] = c[i];
  return (int)c.size();
}

int mt_dense_qmv_plan_set(int K, int N, int nproj, int dtype, const mt_dense_plan* plan) {
  const int st = check_dense_plan_shape("mt_dense_qmv_plan_set", K, N, nproj, dtype);
  if (st) return st;
  if (plan) {
    const std::string why = dense_plan_problem(K, *plan);
    if (!why.empty()) return fail(MT_ERR_INVALID_ARGUMENT, "mt_dense_qmv_plan_set: " + why);
  }
  std::unique_lock<std::shared_mutex> lock(g_plans_mu);
  if (plan) g_dense_plans[dense_key(K, N, nproj, dtype)] = *plan;
  else g_dense_plans.erase(dense_key(K, N, nproj, dtype));
  g_plans_installed.store(installed_plans(), std::memory_order_release);
  return MT_OK;
}

static int stream_read(const char* op, const void* p, size_t bytes, uint32_t* sink, int blocks,
                       bool blocked, void* stream) {
  if (!p || !sink || bytes == 0 || bytes >= (1ull << 31) || blocks < 1 || blocks > 65536)
    return fail(MT_ERR_INVALID_ARGUMENT,
                std::string(op) + ": need a buffer below 2 GiB, a sink and 1..65536 blocks");
  const hipError_t e = mt::launch_stream_read(p, (uint32_t)bytes, sink, blocks, blocked,
                                              static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, op);
  return MT_OK;
}

int mt_stream_read(const void* p, size_t bytes, uint32_t* sink, int blocks, void* stream) {
  return stream_read("mt_stream_read", p, bytes, sink, blocks, false, stream);
}

int mt_stream_read_blocked(const void* p, size_t bytes, uint32_t* sink, int blocks,
                           void* stream) {
  return stream_read("mt_stream_read_blocked", p, bytes, sink, blocks, true, stream);
}

}  // extern "C"

/* metile_amd — C ABI of the MI355X (gfx950) quantized-projection kernels.
 *
 * Every entry point takes caller-owned DEVICE pointers, plain integer sizes and a HIP stream
 * (hipStream_t passed as void*; NULL is the default stream), enqueues its kernels on that
 * stream and returns without synchronising. The library allocates nothing: split-K partial
 * sums and the MLP hidden activation live in a caller-provided workspace whose size the
 * matching *_workspace_bytes function reports. The first 64 KiB of every workspace hold
 * split-K arrival counters at fixed places; a workspace must be zero-filled once before
 * its first use; every call leaves its counter region zeroed again. Calls that share one
 * workspace must be ordered (same stream); calls on different streams need different
 * workspaces.
 *
 * Return value: MT_OK (0) or a negative mt_status. The message of the last failure on the
 * calling thread is available from mt_last_error(). Nothing throws across this boundary.
 *
 * Tensor formats (row-major, contiguous):
 *   x, residual, y, h     16-bit floats [M, K] / [M, N] (dtype MT_BF16 or MT_F16, as uint16)
 *   w_q                   uint32 [N, K*bits/32], MLX affine packing: code k of a row sits in
 *                         word k/(32/bits) at bit (k % (32/bits))*bits (low bits first)
 *   scales, biases        16-bit floats [N, K/group_size], same dtype as x
 *   dense weights         16-bit floats [N, K]
 * Kernels read x, w_q, dense weights and workspaces with 16-byte loads: these pointers must be
 * 16-byte aligned (allocations are; a row slice of a conforming tensor stays aligned, since
 * K % 64 == 0 and N % 32 == 0). Scales and biases need 4-byte alignment. Nothing checks this.
 */
#ifndef METILE_AMD_H
#define METILE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mt_status {
  MT_OK = 0,
  MT_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad shape, unsupported bits/group/dtype */
  MT_ERR_WORKSPACE = -2,        /* workspace missing or smaller than required */
  MT_ERR_HIP = -3               /* a HIP runtime call failed (launch error) */
} mt_status;

typedef enum mt_dtype { MT_BF16 = 0, MT_F16 = 1 } mt_dtype;

/* Library version string. */
const char* mt_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* mt_last_error(void);

/* Workspace bytes mt_affine_qmv (nproj = 1) or mt_affine_swiglu (nproj = 2) needs. */
size_t mt_affine_qmv_workspace_bytes(int M, int K, int N, int group_size, int bits, int nproj);

/* y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/G] + b[n, k/G]) (+ residual[m, n]).
 * Replaces mlx_affine_qmv (metile/backends/mlx_quantized.py:691-714) and, with a residual,
 * mlx_affine_residual_qmv (metile/backends/mlx_quantized.py:1538-1624); the kernels they
 * bind are kernels/affine_qmv.py:57-132. bits in {4, 8}; group_size a power of two >= 32
 * that divides K; K % 64 == 0; N % 32 == 0; any M >= 1 (rows beyond 32 run in 32-row
 * chunks, 16-row chunks for groups of 32). */
int mt_affine_qmv(const void* x, const uint32_t* w_q, const void* scales, const void* biases,
                  const void* residual, void* y, int M, int K, int N, int group_size, int bits,
                  int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* h[m, n] = silu(x @ Wg^T)[m, n] * (x @ Wu^T)[m, n], gate and up accumulated in fp32 from one
 * activation load and combined before the single output rounding. Replaces mlx_affine_swiglu
 * / mlx_affine_swiglu_qmv (metile/backends/mlx_quantized.py:717-751,1645-1720) and the kernel
 * kernels/affine_qmv.py:135-214. Shape rules as mt_affine_qmv. */
int mt_affine_swiglu(const void* x, const uint32_t* gate_w, const void* gate_scales,
                     const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                     const void* up_biases, void* h, int M, int K, int N, int group_size,
                     int bits, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for mt_affine_mlp (hidden activation plus split-K partials). */
size_t mt_affine_mlp_workspace_bytes(int M, int H, int I, int group_size, int bits);

/* y = down(swiglu(x)) (+ residual), x [M, H], gate/up [I, H], down [H, I]. The hidden
 * activation is rounded to the activation dtype between the two kernels, as the reference
 * executor's two dispatches do. Replaces the execute() closure of mlx_affine_mlp_executor
 * (metile/backends/mlx_quantized.py:1770-1832). */
int mt_affine_mlp(const void* x, const uint32_t* gate_w, const void* gate_scales,
                  const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                  const void* up_biases, const uint32_t* down_w, const void* down_scales,
                  const void* down_biases, const void* residual, void* y, int M, int H, int I,
                  int group_size, int bits, int dtype, void* workspace, size_t workspace_bytes,
                  void* stream);

/* mt_affine_mlp without a caller workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The workspace lives in a 16 MiB device array inside the library
 * (one per GPU, held until the process ends); a call whose mt_affine_mlp_workspace_bytes exceeds
 * 16 MiB fails with MT_ERR_WORKSPACE. It allocates nothing (no hipMalloc, no allocating library
 * call); the first call on a device clears the array's counter region with a small kernel on
 * `stream`. Every call on a GPU shares that array: calls that overlap on one GPU (other
 * streams, or a graph captured over this call replayed while another runs) race. Same arguments
 * (minus the workspace) and results as mt_affine_mlp, bit for bit. */
int mt_affine_mlp_noalloc(const void* x, const uint32_t* gate_w, const void* gate_scales,
                          const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                          const void* up_biases, const uint32_t* down_w, const void* down_scales,
                          const void* down_biases, const void* residual, void* y, int M, int H,
                          int I, int group_size, int bits, int dtype, void* stream);

/* out[n, k] = q[n, k] * s[n, k/G] + b[n, k/G] in fp32 (bit-exact dequantization, the decode
 * step of kernels/affine_qmv.py:41-51). Any group_size dividing K with K % (32/bits) == 0. */
int mt_affine_dequantize(const uint32_t* w_q, const void* scales, const void* biases,
                         float* out, int N, int K, int group_size, int bits, int dtype,
                         void* stream);

/* ---- affine group quantization (dense -> MLX affine format) ------------------------------- */

/* w [N, K] 16-bit (dtype) -> w_q [N, K*bits/32], scales and biases [N, K/group_size] in the
 * same dtype. Per group: scale = max((max - min) / (2^bits - 1), 1e-7) with the sign and
 * edge rule that makes the extreme of larger magnitude exactly representable, bias = that
 * extreme (or 0), codes = rint((w - bias) / scale) clamped to [0, 2^bits - 1], computed in fp32
 * with the stored (rounded) scale and bias. Restates MLX's affine quantize (mx.quantize,
 * mode="affine"), which the reference calls in metile/backends/mlx_compressed_down.py:41-48;
 * bit parity with MLX itself is not verified (MLX is not available here). bits in {4, 8};
 * group_size in {32, 64, 128} dividing K. */
int mt_affine_quantize(const void* w, uint32_t* w_q, void* scales, void* biases, int N, int K,
                       int group_size, int bits, int dtype, void* stream);

/* ---- ahead-of-time repack for the small-row kernels --------------------------------------- */

/* Step-major repack of MLX affine codes: the 8*bits bytes holding codes [64t, 64t + 64) of row
 * n move to byte (t*N + n)*8*bits of `out` (same size as w_q, 16-byte aligned buffers), so the
 * codes all columns of a strip need for one K step are contiguous. Scales and biases keep their
 * [N, K/group_size] layout. Replaces repack_mlx_affine_weight
 * (metile/backends/mlx_quantized.py:754-774), whose K-major nibble layout feeds the reference's
 * NAX kernels; this one is laid out for these kernels' loads. bits in {4, 8}; K % 64 == 0. */
int mt_affine_repack(const uint32_t* w_q, uint32_t* out, int N, int K, int bits, void* stream);

/* mt_affine_qmv, mt_affine_swiglu and mt_affine_mlp over repacked codes (mt_affine_repack);
 * same arguments, shape rules, workspace sizes and results, bit for bit. Replace the
 * reference's entries over pre-repacked weights, mlx_affine_qmv_nax and
 * mlx_affine_swiglu_qmv_nax (metile/backends/mlx_quantized.py:777-831), and the repacked
 * path its executors take (metile/backends/mlx_quantized.py:949-967,1082-1100). */
int mt_affine_qmv_repacked(const void* x, const uint32_t* w_packed, const void* scales,
                           const void* biases, const void* residual, void* y, int M, int K, int N,
                           int group_size, int bits, int dtype, void* workspace,
                           size_t workspace_bytes, void* stream);
int mt_affine_swiglu_repacked(const void* x, const uint32_t* gate_packed, const void* gate_scales,
                              const void* gate_biases, const uint32_t* up_packed,
                              const void* up_scales, const void* up_biases, void* h, int M, int K,
                              int N, int group_size, int bits, int dtype, void* workspace,
                              size_t workspace_bytes, void* stream);
int mt_affine_mlp_repacked(const void* x, const uint32_t* gate_packed, const void* gate_scales,
                           const void* gate_biases, const uint32_t* up_packed,
                           const void* up_scales, const void* up_biases,
                           const uint32_t* down_packed, const void* down_scales,
                           const void* down_biases, const void* residual, void* y, int M, int H,
                           int I, int group_size, int bits, int dtype, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Code layouts of one weight: MLX's rows or the step-major repack of mt_affine_repack. */
typedef enum mt_code_layout { MT_LAYOUT_MLX = 0, MT_LAYOUT_REPACKED = 1 } mt_code_layout;

/* mt_affine_mlp with the gate and up codes in `up_layout` and the down codes in `down_layout`,
 * so that each weight can be kept in the layout its plan reads fastest (at one row of
 * Qwen2.5-1.5B's MLP: gate/up repacked for the staged kernel, down in MLX rows for the GEMV
 * kernel). Same arguments, workspace and results as mt_affine_mlp, bit for bit. The reference's
 * executors likewise pick per stage between their repacked and plain schedules
 * (metile/backends/mlx_quantized.py:949-967,1082-1100). */
int mt_affine_mlp_layouts(const void* x, const uint32_t* gate_w, const void* gate_scales,
                          const void* gate_biases, const uint32_t* up_w, const void* up_scales,
                          const void* up_biases, const uint32_t* down_w, const void* down_scales,
                          const void* down_biases, const void* residual, void* y, int M, int H,
                          int I, int group_size, int bits, int dtype, int up_layout,
                          int down_layout, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ---- prefill (many rows) ---------------------------------------------------------------- */

/* Workspace bytes mt_affine_gemm needs (0 when K is not split). */
size_t mt_affine_gemm_workspace_bytes(int M, int K, int N, int group_size, int bits);

/* y = x @ dequantize(w_q)^T for many rows (prefill) on the matrix cores with fp32 accumulation.
 * Dequantization stays exact: the codes enter the MFMAs as exact 16-bit floats (offset + q) and
 * each 64-wide step's partial gets its group's scale and bias terms in fp32. Replaces mlx_affine_matmul / lower_affine_matmul
 * (metile/backends/mlx_affine.py:359-406, metile/compiler/affine_quantized.py:7-99).
 * bits = 4; group_size a power of two >= 64 dividing K; K % 64 == 0; N % 32 == 0. */
int mt_affine_gemm(const void* x, const uint32_t* w_q, const void* scales, const void* biases,
                   void* y, int M, int K, int N, int group_size, int bits, int dtype,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ---- dense 16-bit small-batch projections ------------------------------------------------ */

/* Workspace bytes mt_dense_swiglu (nproj = 2) or mt_dense_residual_qmv (nproj = 1) needs. */
size_t mt_dense_workspace_bytes(int M, int K, int N, int nproj);

/* h = typed SwiGLU of x @ gate^T and x @ up^T, gate/up [N, K] 16-bit weights: the fp32 dots
 * are rounded to the activation type, then silu and the product are evaluated with every
 * operation rounded to that type (metile/compiler/dense.py:193-299 with
 * metile/codegen/msl_emitter.py:1218-1252; entry mlx_dense_swiglu,
 * metile/backends/mlx_dense_swiglu.py:424-491). Each output row is bit-identical whatever
 * M is. K % 64 == 0, N % 32 == 0, N <= 262144. */
int mt_dense_swiglu(const void* x, const void* gate_w, const void* up_w, void* h, int M, int K,
                    int N, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* y = T(T(x @ w^T) + residual) (or T(x @ w^T) with a null residual), w [N, K]: the projected
 * value is rounded to the activation type T before the residual add
 * (metile/compiler/dense.py:302-381, metile/codegen/msl_emitter.py:1098-1120; entry
 * mlx_dense_residual_qmv, metile/backends/mlx_dense_residual.py:276-319). Each output row is
 * bit-identical whatever M is. K % 64 == 0, N % 32 == 0, N <= 262144. */
int mt_dense_residual_qmv(const void* x, const void* w, const void* residual, void* y, int M,
                          int K, int N, int dtype, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ---- plans: the tuner's knobs ------------------------------------------------------------ */

/* How one small-row dispatch runs: the kernel, the number of K splits, the number of column
 * strips (workgroup columns; N/32 for the register kernel, N/32 to 2N/32 for the staged kernel)
 * and the strips per workgroup (1 or 2, staged kernel only). The GEMV kernel (up to 4 rows)
 * never splits K: its strips are its workgroups, N / (columns x column groups) with 2, 4 or
 * 8 columns per group (8: one projection of up to 2 rows) and, when one pass of its lanes covers
 * K in whole rows of 16 lanes, several column groups per workgroup; `tiles` holds its waves per
 * workgroup (1 to 8) and `order` how workgroups take column groups (0: in index order; 1:
 * dealt out to the 8 XCDs in runs of adjacent groups). The column-block kernel (up to 32 rows,
 * groups of 64 or more) runs `strips` workgroups per K split, each a block of N / strips
 * columns (at most 64, also when N is counted in the 4-column (4-bit) or 2-column (8-bit)
 * units of the repacked layout) whose `tiles` waves (1 to 8) take consecutive runs of the
 * split's K steps over every column of the block. The 4x4x4-MFMA GEMV kernel (MT_QMV_GEMV4: up
 * to 4 rows, 4-bit codes, groups of 32 or more, no K split) runs `strips` = N / 4, N / 8 or
 * N / 16 workgroups of 1, 2 or 4 groups of 4 columns whose `tiles` waves (1 to 8) split K in
 * rounds of 512, at most four rounds each. `order` is 0 for every kernel but the GEMV. */
typedef enum mt_qmv_kernel {
  MT_QMV_STAGED = 1,
  MT_QMV_REGISTER = 2,
  MT_QMV_GEMV = 3,
  MT_QMV_BLOCK = 4,
  MT_QMV_GEMV4 = 5
} mt_qmv_kernel;
typedef struct mt_qmv_plan {
  int kernel;
  int ksplit;
  int strips;
  int tiles;
  int order;
} mt_qmv_plan;

/* How the prefill GEMM runs: the kernel, its output tile (tile_m x tile_n), the number of K
 * splits and the tile order. MT_GEMM_STAGED (v_mfma_f32_32x32x16, operands staged through
 * registers into LDS): square tiles of 64 or 128, K split into equal lengths, order 0.
 * MT_GEMM_RING (v_mfma_f32_16x16x32, activations and codes through three-stage LDS rings filled
 * by buffer_load...lds): tiles of 128 x 64, 96, 128, 160, 192 or 256, N a multiple of 8, at most
 * 8 splits of whole three-step lengths (steps of 64 along K), and the order in which workgroups
 * take (column tile, row block, split): MT_GEMM_ORDER_GRID (row-major, as launched), or each of
 * the 8 XCDs (which take workgroups in turn) a contiguous run of that sequence with column tiles
 * (MT_GEMM_ORDER_XCD_COLUMNS) or row blocks (MT_GEMM_ORDER_XCD_ROWS) varying fastest, so that
 * the tiles sharing activations or codes share an L2. The reference's matmul plans race tile
 * shapes and tile orders the same way (MLXAffineMatmulConfig, metile/backends/mlx_affine.py:36-63,
 * _candidate_configs :155-166). */
typedef enum mt_gemm_kernel { MT_GEMM_STAGED = 0, MT_GEMM_RING = 1 } mt_gemm_kernel;
typedef enum mt_gemm_order {
  MT_GEMM_ORDER_GRID = 0,
  MT_GEMM_ORDER_XCD_COLUMNS = 1,
  MT_GEMM_ORDER_XCD_ROWS = 2
} mt_gemm_order;
typedef struct mt_gemm_plan {
  int kernel;
  int tile_m;
  int tile_n;
  int ksplit;
  int order;
} mt_gemm_plan;

/* By default every call plans itself from its shape. A tuner lists the plans a shape can take,
 * measures them and installs the fastest; calls of that shape then take the installed plan
 * (results stay within the kernels' tolerance; summation order may change). Installed plans are
 * per process and keyed by (rows of one dispatch rounded up to a power of two, K, N, group_size,
 * bits, nproj, dtype); both code layouts take the installed plan, so that their results stay
 * bit-identical. The workspace queries cover every installed plan. These
 * functions are the analogue of the reference's tuned-config selection and its persistent
 * decisions (metile/backends/mlx_quantized.py:1225-1253,1275-1336,1393-1483; config lattice
 * MLXAffineSwiGLUConfig :61-67, MLXAffineResidualConfig :70-75, MLXAffineMatmulConfig
 * metile/backends/mlx_affine.py:36-41 with _candidate_configs :157-166). Host-only: they touch
 * no device.
 *
 * M is the rows of one dispatch (1..32, 1..16 for groups of 32; calls with more rows run
 * dispatches of that many); nproj 1 (QMV) or 2 (SwiGLU).
 * Within an MLP call, the gate/up dispatch is the nproj = 2 shape (K = H, N = I) and the down
 * dispatch the nproj = 1 shape (K = I, N = H). */

/* The plan a dispatch of this shape takes now (installed, else the planner's). */
int mt_affine_qmv_plan(int M, int K, int N, int group_size, int bits, int nproj, int dtype,
                       mt_qmv_plan* out);
/* Every plan valid for dispatches of up to row_bucket(M) rows: writes up to `capacity` and
 * returns how many there are (or a negative mt_status). */
int mt_affine_qmv_plan_candidates(int M, int K, int N, int group_size, int bits, int nproj,
                                  mt_qmv_plan* out, int capacity);
/* Install `plan` for the shape (rejects a plan the kernels cannot run); NULL removes it. */
int mt_affine_qmv_plan_set(int M, int K, int N, int group_size, int bits, int nproj, int dtype,
                           const mt_qmv_plan* plan);
/* The same three for the prefill GEMM (4-bit; M = rows of the call, bucketed likewise). */
int mt_affine_gemm_plan(int M, int K, int N, int group_size, int dtype, mt_gemm_plan* out);
int mt_affine_gemm_plan_candidates(int M, int K, int N, int group_size, mt_gemm_plan* out,
                                   int capacity);
int mt_affine_gemm_plan_set(int M, int K, int N, int group_size, int dtype,
                            const mt_gemm_plan* plan);
/* How a dense projection runs: its K splits. Keyed by (K, N, nproj, dtype) only, so that one
 * plan serves every row count and each output row stays bit-identical to that row run alone;
 * the analogue of the reference's tuned dense schedules under its per-row exactness gate
 * (metile/backends/mlx_dense_swiglu.py:343-421, metile/backends/mlx_dense_residual.py:202-273).
 * Splits are equal-length runs of at least 4 64-wide K steps, at most 32 of them. */
typedef struct mt_dense_plan {
  int ksplit;
} mt_dense_plan;
int mt_dense_qmv_plan(int K, int N, int nproj, int dtype, mt_dense_plan* out);
int mt_dense_qmv_plan_candidates(int K, int N, int nproj, mt_dense_plan* out, int capacity);
/* Install `plan` for the shape (rejects a plan the kernel cannot run); NULL removes it. The
 * workspace query (mt_dense_workspace_bytes) covers every installed plan. */
int mt_dense_qmv_plan_set(int K, int N, int nproj, int dtype, const mt_dense_plan* plan);

/* Remove every installed plan. */
int mt_plans_clear(void);
/* SHA-256 of the kernel and boundary sources this library was built from (hex): the part of a
 * persistent tuning key that retires decisions when the kernels change, as the reference's
 * source-hash keys do (metile/backends/mlx_quantized.py:1393-1427). */
const char* mt_source_digest(void);

/* ---- measurement -------------------------------------------------------------------------- */

/* Reads `bytes` from `p` with `blocks` workgroups of 256 threads issuing 16-byte loads (grid
 * stride; per thread the fewest loads in flight, 1, 2, 4 or 8, that cover the buffer in one
 * batch, else batches of 8) and no reduction: the streaming-read ceiling of one launch.
 * `sink` (at least `blocks` words) is written only when a thread's XOR of its data equals a
 * fixed sentinel, which keeps the loads alive. No counterpart entry point in the reference; it
 * is the analogue of its measured streaming-read constant (metile/target/agx.py:38). */
int mt_stream_read(const void* p, size_t bytes, uint32_t* sink, int blocks, void* stream);

/* The same probe with each block reading its own contiguous run (U x 4 KiB per batch, U as
 * above), the access pattern of kernels whose workgroups own whole columns of codes. No
 * counterpart entry point in the reference (metile/target/agx.py:38). */
int mt_stream_read_blocked(const void* p, size_t bytes, uint32_t* sink, int blocks,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* METILE_AMD_H */

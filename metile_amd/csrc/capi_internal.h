// Internal (not exported in include/metile_amd.h): what source files other than capi.cpp use
// of the boundary's MLP path and error reporting.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>

namespace mt {

// Every workspace starts with this many bytes of split-K arrival counters, zero between calls.
constexpr size_t kWorkspaceCounterBytes = 64 * 1024;

// Records `msg` as the calling thread's last error (mt_last_error) and returns `status`.
int set_last_error(int status, const std::string& msg);

// Workspace bytes mt_affine_mlp needs at this shape (0 for a shape it rejects).
size_t affine_mlp_workspace(int M, int H, int I, int group_size, int bits);

// The argument checks of mt_affine_mlp other than the workspace's (shapes, dtype, bits, group
// size, null pointers): MT_OK, or the status it would return, with the error recorded.
int affine_mlp_check(const char* op, const void* x, const uint32_t* gate_w,
                     const void* gate_scales, const void* gate_biases, const uint32_t* up_w,
                     const void* up_scales, const void* up_biases, const uint32_t* down_w,
                     const void* down_scales, const void* down_biases, const void* y, int M,
                     int H, int I, int group_size, int bits, int dtype);

// mt_affine_mlp with `op` naming the caller in error messages (MLX code layout for all three
// projections).
int affine_mlp(const char* op, const void* x, const uint32_t* gate_w, const void* gate_scales,
               const void* gate_biases, const uint32_t* up_w, const void* up_scales,
               const void* up_biases, const uint32_t* down_w, const void* down_scales,
               const void* down_biases, const void* residual, void* y, int M, int H, int I,
               int group_size, int bits, int dtype, void* workspace, size_t workspace_bytes,
               void* stream);

}  // namespace mt

// Streaming-read probe: the achievable HBM read rate of one launch over a buffer of a given
// size (the measured ceiling that the projection kernels are compared with; the reference
// keeps the same kind of constant for its GPU, metile/target/agx.py:38).
#include "common.h"
#include "stream_read.h"

namespace mt {

namespace {

constexpr int kUnroll = 8;
constexpr uint32_t kSentinel = 0x9E3779B9u;

// Grid-stride 16-byte loads: at each step the grid reads one contiguous span of
// gridDim.x * 4 KiB (block b its 4 KiB at b * 4 KiB), up to kUnroll steps in flight per thread.
// Each thread XOR-folds what it read and stores it only if it equals a sentinel, which keeps the
// loads alive without a reduction at the end: the probe is the stream alone, with no tail a
// reduction or store would add.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* p, uint32_t bytes,
                                                          uint32_t* sink) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p, bytes);
  const uint32_t stride = gridDim.x * 256u * 16u;
  uint32_t off = (blockIdx.x * 256u + threadIdx.x) * 16u;
  uint32_t acc = 0;
  for (; off + (kUnroll - 1) * stride < bytes; off += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = load16(r, off + (uint32_t)u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; off < bytes; off += stride) {
    const u32x4 v = load16(r, off);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == kSentinel) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_stream_read(const void* p, uint32_t bytes, uint32_t* sink, int blocks,
                              hipStream_t stream) {
  stream_read_kernel<<<blocks, 256, 0, stream>>>(static_cast<const uint8_t*>(p), bytes, sink);
  return hipGetLastError();
}

}  // namespace mt

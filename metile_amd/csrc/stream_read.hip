// Streaming-read probe: the achievable HBM read rate of one launch over a buffer of a given
// size (the measured ceiling that the projection kernels are compared with; the reference
// keeps the same kind of constant for its GPU, metile/target/agx.py:38).
#include "common.h"
#include "stream_read.h"

namespace mt {

namespace {

constexpr int kUnroll = 8;

__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* p, uint32_t bytes,
                                                          uint32_t* sink) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p, bytes);
  const uint32_t per_block = ((bytes + gridDim.x - 1) / gridDim.x + 4095u) & ~4095u;
  const uint32_t base = blockIdx.x * per_block;
  const uint32_t end = min(bytes, base + per_block);
  uint32_t acc = 0;
  for (uint32_t off = base + threadIdx.x * 16u; off < end; off += 256u * 16u * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t o = off + (uint32_t)u * 256u * 16u;
      v[u] = load16(r, o < end ? o : kOOB);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // One word per block keeps the loads alive; the value itself is meaningless.
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = 0;
    for (int i = 0; i < 256; ++i) a ^= red[i];
    sink[blockIdx.x] = a;
  }
}

}  // namespace

hipError_t launch_stream_read(const void* p, uint32_t bytes, uint32_t* sink, int blocks,
                              hipStream_t stream) {
  stream_read_kernel<<<blocks, 256, 0, stream>>>(static_cast<const uint8_t*>(p), bytes, sink);
  return hipGetLastError();
}

}  // namespace mt

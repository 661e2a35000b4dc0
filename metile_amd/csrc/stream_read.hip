// Streaming-read probe: the achievable HBM read rate of one launch over a buffer of a given
// size (the measured ceiling that the projection kernels are compared with; the reference
// keeps the same kind of constant for its GPU, metile/target/agx.py:38).
#include "common.h"
#include "stream_read.h"

namespace mt {

namespace {

constexpr uint32_t kSentinel = 0x9E3779B9u;

// 16-byte loads, U per thread in flight. Grid-stride: at each step the grid reads one
// contiguous span of gridDim.x * 4 KiB (block b its 4 KiB at b * 4 KiB), U steps per batch.
// Blocked: each block reads its own contiguous run of U * 4 KiB per batch, as a kernel whose
// workgroups own whole columns of codes does. Only the last
// batch can run past the end; its loads there take an out-of-range offset (bit 31 set; buffers
// are below 2 GiB) and read zero. (A second batch requested before the first is folded measured
// slower at every size.) The host picks U from the grid (the fewest loads per thread
// that cover the buffer, at most 8), so a grid of bytes / (4 KiB * U) blocks issues all of its
// loads in one batch, as a one-pass kernel does, with almost none out of range (those still
// cost issue slots). Each thread XOR-folds what it read and stores it only if it equals a
// sentinel, which keeps the loads alive without a reduction at the end: the probe is the stream
// alone, with no tail a reduction or store would add.
template <int U, bool BLOCKED>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* p, uint32_t bytes,
                                                          uint32_t* sink) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p, bytes);
  // Grid-stride: one step of the grid is gridDim.x * 4 KiB, block b's 4 KiB at b * 4 KiB.
  // Blocked: block b reads the contiguous run [b U 4 KiB, (b + 1) U 4 KiB), 4 KiB per step,
  // the next run one grid span (gridDim.x U 4 KiB) further on.
  const uint32_t stride = BLOCKED ? 256u * 16u : gridDim.x * 256u * 16u;
  const uint32_t first = BLOCKED ? blockIdx.x * (uint32_t)U * 4096u + threadIdx.x * 16u
                                 : (blockIdx.x * 256u + threadIdx.x) * 16u;
  const uint32_t next = BLOCKED ? gridDim.x * (uint32_t)U * 4096u : (uint32_t)U * stride;
  uint32_t acc = 0;
  for (uint32_t off = first; off < bytes; off += next) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t o = off + (uint32_t)u * stride;
      v[u] = load16(r, oob_unless(o < bytes, o));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == kSentinel) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_stream_read(const void* p, uint32_t bytes, uint32_t* sink, int blocks,
                              bool blocked, hipStream_t stream) {
  const uint64_t span = (uint64_t)blocks * 256u * 16u;
  const uint64_t steps = ((uint64_t)bytes + span - 1) / span;  // loads per thread
  const uint8_t* b = static_cast<const uint8_t*>(p);
  if (blocked) {
    if (steps <= 1) stream_read_kernel<1, true><<<blocks, 256, 0, stream>>>(b, bytes, sink);
    else if (steps <= 2) stream_read_kernel<2, true><<<blocks, 256, 0, stream>>>(b, bytes, sink);
    else if (steps <= 4) stream_read_kernel<4, true><<<blocks, 256, 0, stream>>>(b, bytes, sink);
    else stream_read_kernel<8, true><<<blocks, 256, 0, stream>>>(b, bytes, sink);
  } else {
    if (steps <= 1) stream_read_kernel<1, false><<<blocks, 256, 0, stream>>>(b, bytes, sink);
    else if (steps <= 2) stream_read_kernel<2, false><<<blocks, 256, 0, stream>>>(b, bytes, sink);
    else if (steps <= 4) stream_read_kernel<4, false><<<blocks, 256, 0, stream>>>(b, bytes, sink);
    else stream_read_kernel<8, false><<<blocks, 256, 0, stream>>>(b, bytes, sink);
  }
  return hipGetLastError();
}

}  // namespace mt

// Host-visible launch interface of the streaming-read probe.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

hipError_t launch_stream_read(const void* p, uint32_t bytes, uint32_t* sink, int blocks,
                              bool blocked, hipStream_t stream);

}  // namespace mt

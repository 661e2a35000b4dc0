// mt_affine_mlp_noalloc: mt_affine_mlp for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The workspace
// (split-K arrival counters, fp32 partial sums, the hidden activation) lives in `scratch`, a
// file-scope device array of kScratchBytes that each GPU the library runs on holds until the
// process ends. The caller still passes inputs and outputs.
//
// `scratch` names a host-side stand-in in host code, not a device address: the array's address
// on a device comes from hipGetSymbolAddress, taken once per device (with that device current)
// on the first call there, and kept in g_scratch[]; kernels receive that pointer.
//
// Every call on a GPU shares that GPU's array, which keeps the last call's contents. The split-K
// counters must start at zero: they are cleared once, by a fill kernel on the caller's stream at
// set-up, and every call leaves them at zero again. Calls that overlap on one GPU (concurrent
// streams, or a captured graph replayed while another call runs) race on the array.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/metile_amd.h"
#include "capi_internal.h"

namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;  // the stated maximum workspace
constexpr size_t kCounterBytes = 64 * 1024;         // the workspace's leading counter region

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void clear_words(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_setup_mu;
void* g_scratch[kMaxDevices];
std::atomic<bool> g_ready[kMaxDevices];

// The current device's scratch address, set up on its first use: the symbol's device address,
// and the counter region cleared on `stream`.
int device_scratch(void** out, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return mt::set_last_error(MT_ERR_HIP, std::string("mt_affine_mlp_noalloc: hipGetDevice: ") +
                                              hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return mt::set_last_error(MT_ERR_INVALID_ARGUMENT,
                              "mt_affine_mlp_noalloc: device index beyond 63");
  if (!g_ready[dev].load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> lock(g_setup_mu);
    if (!g_ready[dev].load(std::memory_order_relaxed)) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return mt::set_last_error(
            MT_ERR_HIP, std::string("mt_affine_mlp_noalloc: hipGetSymbolAddress(scratch): ") +
                            hipGetErrorString(e));
      const int words = (int)(kCounterBytes / 4);
      clear_words<<<(words + 255) / 256, 256, 0, stream>>>(static_cast<uint32_t*>(p), words);
      e = hipGetLastError();
      if (e != hipSuccess)
        return mt::set_last_error(
            MT_ERR_HIP, std::string("mt_affine_mlp_noalloc: clearing the scratch counters: ") +
                            hipGetErrorString(e));
      g_scratch[dev] = p;
      g_ready[dev].store(true, std::memory_order_release);
    }
  }
  *out = g_scratch[dev];
  return MT_OK;
}

}  // namespace

extern "C" int mt_affine_mlp_noalloc(const void* x, const uint32_t* gate_w, const void* gate_scales,
                                     const void* gate_biases, const uint32_t* up_w,
                                     const void* up_scales, const void* up_biases,
                                     const uint32_t* down_w, const void* down_scales,
                                     const void* down_biases, const void* residual, void* y, int M,
                                     int H, int I, int group_size, int bits, int dtype,
                                     void* stream) {
  const char* op = "mt_affine_mlp_noalloc";
  const size_t need = mt::affine_mlp_workspace(M, H, I, group_size, bits);
  if (need == 0)  // a shape the MLP rejects: let it report why (nothing is launched)
    return mt::affine_mlp(op, x, gate_w, gate_scales, gate_biases, up_w, up_scales, up_biases,
                          down_w, down_scales, down_biases, residual, y, M, H, I, group_size,
                          bits, dtype, nullptr, 0, stream);
  if (need > kScratchBytes)
    return mt::set_last_error(
        MT_ERR_WORKSPACE, std::string(op) + ": this call needs " + std::to_string(need) +
                              " bytes of workspace; the no-allocation entry point holds at most " +
                              std::to_string(kScratchBytes) +
                              " (use mt_affine_mlp with a caller workspace)");
  void* ws = nullptr;
  const int st = device_scratch(&ws, static_cast<hipStream_t>(stream));
  if (st) return st;
  return mt::affine_mlp(op, x, gate_w, gate_scales, gate_biases, up_w, up_scales, up_biases,
                        down_w, down_scales, down_biases, residual, y, M, H, I, group_size, bits,
                        dtype, ws, kScratchBytes, stream);
}

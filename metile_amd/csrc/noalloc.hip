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
// counters must start at zero: the array has static storage, so it is zero when the library's
// code object is loaded, and every call leaves the counters at zero again (no set-up kernel:
// nothing is launched besides the MLP's own two kernels, under graph capture too). Calls that
// overlap on one GPU (concurrent streams, or a captured graph replayed while another call runs)
// race on the array.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/metile_amd.h"
#include "capi_internal.h"

namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;  // the stated maximum workspace
static_assert(kScratchBytes > mt::kWorkspaceCounterBytes, "room beyond the counter region");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_setup_mu;
void* g_scratch[kMaxDevices];
std::atomic<bool> g_ready[kMaxDevices];

// The current device's scratch address, taken from the symbol on the device's first use (no
// stream work: the array needs no clearing).
int device_scratch(void** out) {
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
  // Every argument check of the MLP first: nothing touches the device for a call it rejects.
  int st = mt::affine_mlp_check(op, x, gate_w, gate_scales, gate_biases, up_w, up_scales,
                                up_biases, down_w, down_scales, down_biases, y, M, H, I,
                                group_size, bits, dtype);
  if (st) return st;
  const size_t need = mt::affine_mlp_workspace(M, H, I, group_size, bits);
  if (need > kScratchBytes)
    return mt::set_last_error(
        MT_ERR_WORKSPACE, std::string(op) + ": this call needs " + std::to_string(need) +
                              " bytes of workspace; the no-allocation entry point holds at most " +
                              std::to_string(kScratchBytes) +
                              " (use mt_affine_mlp with a caller workspace)");
  void* ws = nullptr;
  st = device_scratch(&ws);
  if (st) return st;
  return mt::affine_mlp(op, x, gate_w, gate_scales, gate_biases, up_w, up_scales, up_biases,
                        down_w, down_scales, down_biases, residual, y, M, H, I, group_size, bits,
                        dtype, ws, kScratchBytes, stream);
}

// abi_adam.hip -- the dense Adam entry points of include/churten_optim.h
// (the segmented ones are in abi_adam_segments.hip) and the allocation-free
// form's device scratch.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "optim_dispatch.h"

namespace churten {
namespace {

// Replicas whose per-replica constants fit ts_adam_step_noalloc's scratch.
constexpr int64_t kScratchReplicas = 65536;
constexpr int kMaxDevices = 64;

}  // namespace
}  // namespace churten

// The per-replica constants of ts_adam_step_noalloc (kPreStride doubles for up
// to kScratchReplicas replicas: 1 MiB), one copy on every device the library
// runs on, held until the process ends. In host code this name is only a
// stand-in: its device address comes from hipGetSymbolAddress
// (scratch_on_current_device), once per device.
static __device__ __align__(256) double scratch[churten::kPreStride * churten::kScratchReplicas];

namespace churten {
namespace {

// The device address of `scratch` on the calling thread's current device,
// looked up the first time the entry point runs on that device (with it
// current) and kept per device.
int scratch_on_current_device(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return kInvalid;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  const std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t s = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (s != hipSuccess) return static_cast<int>(s);
    if (p == nullptr) return kInvalid;
    addr[dev] = p;
  }
  *out = addr[dev];
  return 0;
}

}  // namespace
}  // namespace churten

using churten::make_call;

extern "C" {

int ts_adam_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                 const void* lr, const void* beta1, const void* beta2,
                 const void* eps, const void* weight_decay,
                 const uint8_t* active_mask, int64_t R, int64_t T,
                 uint32_t flags, void* out_zero, void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return churten::adam_run<false>(dtype, c, nullptr, 0);
}

int ts_adam_step_ws(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps, const void* lr,
                    const void* beta1, const void* beta2, const void* eps,
                    const void* weight_decay, const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream, workspace,
                           workspace_bytes);
  return churten::adam_run<false>(dtype, c, nullptr, 0);
}

int ts_adam_step_noalloc(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                         const void* lr, const void* beta1, const void* beta2, const void* eps,
                         const void* weight_decay, const uint8_t* active_mask, int64_t R,
                         int64_t T, uint32_t flags, void* out_zero, void* stream) {
  if (R < 0 || R > churten::kScratchReplicas) return churten::kInvalid;
  void* ws = nullptr;
  const int err = churten::scratch_on_current_device(&ws);
  if (err != 0) return err;
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream, ws,
                           sizeof(double) * churten::kPreStride * churten::kScratchReplicas);
  return churten::adam_run<false>(dtype, c, nullptr, 0);
}

}  // extern "C"

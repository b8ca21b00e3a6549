// abi_adam_segments.hip -- the segmented Adam entry points of
// include/churten_optim.h: one call takes the gradient as a table of
// per-parameter segments (segment_kernel).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "optim_dispatch.h"

using churten::make_call;

extern "C" {

int ts_adam_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                          ts_dtype dtype, void* state_steps, const void* lr,
                          const void* beta1, const void* beta2, const void* eps,
                          const void* weight_decay, const uint8_t* active_mask,
                          int64_t R, int64_t T, uint32_t flags, void* out_zero,
                          void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return churten::adam_run<true>(dtype, c, grads, n_grads);
}

int ts_adam_step_segments_ws(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                             ts_dtype dtype, void* state_steps, const void* lr,
                             const void* beta1, const void* beta2, const void* eps,
                             const void* weight_decay, const uint8_t* active_mask, int64_t R,
                             int64_t T, uint32_t flags, void* out_zero, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream, workspace,
                           workspace_bytes);
  return churten::adam_run<true>(dtype, c, grads, n_grads);
}

}  // extern "C"

// abi_adagrad.hip -- the Adagrad entry points of include/churten_optim.h,
// dense and segmented, with and without a workspace (adagrad_run in
// optim_dispatch.h picks AdagradPolicy, ATen's double math, or under
// TS_ADAGRAD_F32 AdagradF32Policy).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "optim_dispatch.h"

using churten::make_call;

extern "C" {

int ts_adagrad_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                    const void* lr, const void* lr_decay,
                    const void* weight_decay, const void* eps,
                    const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps},
                           active_mask, R, T, flags, out_zero, stream);
  return churten::adagrad_run<false>(dtype, c, nullptr, 0);
}

int ts_adagrad_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                             ts_dtype dtype, void* state_steps, const void* lr,
                             const void* lr_decay, const void* weight_decay,
                             const void* eps, const uint8_t* active_mask, int64_t R,
                             int64_t T, uint32_t flags, void* out_zero, void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps},
                           active_mask, R, T, flags, out_zero, stream);
  return churten::adagrad_run<true>(dtype, c, grads, n_grads);
}

int ts_adagrad_step_ws(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                       const void* lr, const void* lr_decay, const void* weight_decay,
                       const void* eps, const uint8_t* active_mask, int64_t R, int64_t T,
                       uint32_t flags, void* out_zero, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps}, active_mask,
                           R, T, flags, out_zero, stream, workspace, workspace_bytes);
  return churten::adagrad_run<false>(dtype, c, nullptr, 0);
}

int ts_adagrad_step_segments_ws(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                                ts_dtype dtype, void* state_steps, const void* lr,
                                const void* lr_decay, const void* weight_decay,
                                const void* eps, const uint8_t* active_mask, int64_t R,
                                int64_t T, uint32_t flags, void* out_zero, void* workspace,
                                size_t workspace_bytes, void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps}, active_mask,
                           R, T, flags, out_zero, stream, workspace, workspace_bytes);
  return churten::adagrad_run<true>(dtype, c, grads, n_grads);
}

}  // extern "C"

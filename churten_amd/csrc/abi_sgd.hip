// abi_sgd.hip -- the SGD entry points of include/churten_optim.h, dense and
// segmented (sgd_run in optim_dispatch.h picks the SgdPolicy from the call's
// dtype, flags and momentum buffers).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "optim_dispatch.h"

using churten::make_call;

extern "C" {

int ts_sgd_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                const void* lr, const void* momentum, const void* dampening,
                const void* weight_decay, const uint8_t* active_mask,
                int64_t R, int64_t T, uint32_t flags, void* out_zero,
                void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, momentum, dampening, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return churten::sgd_run<false>(dtype, c, nullptr, 0);
}

int ts_sgd_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                         ts_dtype dtype, void* state_steps, const void* lr,
                         const void* momentum, const void* dampening,
                         const void* weight_decay, const uint8_t* active_mask,
                         int64_t R, int64_t T, uint32_t flags, void* out_zero,
                         void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, momentum, dampening, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return churten::sgd_run<true>(dtype, c, grads, n_grads);
}

}  // extern "C"

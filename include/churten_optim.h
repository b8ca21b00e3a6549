/*
 * churten_optim.h -- C ABI of the MI355X fused batched optimizer step.
 *
 * One call updates every parameter of every replica of an N-replica ensemble
 * whose state is consolidated into replica-major (R, T) buffers: row r holds
 * all parameters of replica r, T is the per-replica width (padded to a
 * multiple of 4 by the layout producer). Per-replica hyperparameters are (R,)
 * device vectors and a per-replica active mask freezes whole rows.
 *
 * These entry points replace the device half of the reference's three
 * torch.library operators:
 *   ts_adam_step    <- torchstrap::adam_step_     (src/torchstrap/kernels/csrc/stubs.cpp:25-41,
 *                                                  CUDA impl csrc/cuda/adam.cu:250-331)
 *   ts_sgd_step     <- torchstrap::sgd_step_      (stubs.cpp:45-57, csrc/cuda/sgd.cu:295-359)
 *   ts_adagrad_step <- torchstrap::adagrad_step_  (stubs.cpp:61-72, csrc/cuda/adagrad.cu:238-283)
 *   ts_bump_steps   <- the `state_steps.add_(active_mask.to(...))` every op
 *                      runs first (adam.cu:277, sgd.cu:317, adagrad.cu:256)
 *
 * Contract shared by every entry point:
 *   - All pointers are device pointers on the device that is current for the
 *     calling thread; `stream` is a hipStream_t (NULL = the null stream).
 *   - Nothing is allocated, nothing is synchronised: work is enqueued on
 *     `stream` and the call returns. The return value is a hipError_t
 *     (0 = hipSuccess); invalid arguments give hipErrorInvalidValue (1) and
 *     enqueue nothing.
 *   - Buffers are described by ts_rt_buf: element (r, t) lives at
 *     data + r*stride_r + t*stride_t (strides in elements). Any strides are
 *     accepted; the 16-byte vector path is taken when every buffer has
 *     stride_t == 1, T % 4 == 0 and 16-byte-aligned rows (the layout `State`
 *     produces), otherwise an element-wise path with identical per-element
 *     arithmetic runs.
 *   - (R,) vectors (state_steps and the hyperparameters) are contiguous and
 *     in the parameter dtype; active_mask is R contiguous bytes (0 = frozen).
 *   - A frozen replica's rows are neither read nor written.
 *   - If TS_BUMP_STEPS is set, state_steps[r] += active_mask[r] is applied
 *     first (in the parameter dtype), and the update then reads the bumped
 *     value, as the reference does. Without it state_steps is read as given.
 *   - out_zero, if not NULL, receives one element of the parameter dtype set
 *     to zero: the reference operators return a fresh zero scalar.
 */
#ifndef CHURTEN_OPTIM_H
#define CHURTEN_OPTIM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ts_rt_buf {
  void* data;       /* address of element (0, 0) */
  int64_t stride_r; /* elements between consecutive replicas */
  int64_t stride_t; /* elements between consecutive parameters of a replica */
} ts_rt_buf;

/* Parameter / state dtypes (the reference dispatches all four:
 * AT_DISPATCH_FLOATING_TYPES_AND2(kHalf, kBFloat16, ...), adam.cu:302). */
typedef enum ts_dtype {
  TS_FLOAT32 = 0,
  TS_FLOAT64 = 1,
  TS_FLOAT16 = 2,
  TS_BFLOAT16 = 3
} ts_dtype;

/* Flag bits. */
#define TS_AMSGRAD 0x1u     /* Adam: keep and use max_exp_avg_sqs (bufs[4]) */
#define TS_ADAMW 0x2u       /* Adam: decoupled weight decay */
#define TS_MAXIMIZE 0x4u    /* all: ascend instead of descend */
#define TS_NESTEROV 0x8u    /* SGD: Nesterov momentum (needs a buffer) */
#define TS_BUMP_STEPS 0x10u /* all: state_steps += active_mask first */

/* state_steps[r] += active_mask[r] for r < R (in `dtype`), and *out_zero = 0
 * if out_zero is not NULL. One tiny launch. */
int ts_bump_steps(ts_dtype dtype, void* state_steps, const uint8_t* active_mask,
                  int64_t R, void* out_zero, void* stream);

/* Fused Adam / AdamW (+amsgrad, maximize) over (R, T).
 * bufs: [0] params (rw), [1] grads (r), [2] exp_avgs (rw), [3] exp_avg_sqs (rw),
 *       [4] max_exp_avg_sqs (rw, read only when TS_AMSGRAD is set).
 * Element math is ROCm ATen's `adam_math` (ATen/native/hip/fused_adam_utils.cuh),
 * which the reference calls verbatim (csrc/cuda/adam.cu:146-157). */
int ts_adam_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                 const void* lr, const void* beta1, const void* beta2,
                 const void* eps, const void* weight_decay,
                 const uint8_t* active_mask, int64_t R, int64_t T,
                 uint32_t flags, void* out_zero, void* stream);

/* Fused SGD (momentum, dampening, nesterov, maximize) over (R, T).
 * bufs: [0] params (rw), [1] grads (r), [2] momentum_buffers (rw) or
 *       data == NULL for the buffer-less (depth-2) form.
 * is_first_step is per replica: state_steps[r] == 1 after the bump
 * (csrc/cuda/sgd.cu:171). A momentum-0 replica in a call with buffers still
 * writes its buffer row (sgd.cu:43-50). */
int ts_sgd_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                const void* lr, const void* momentum, const void* dampening,
                const void* weight_decay, const uint8_t* active_mask,
                int64_t R, int64_t T, uint32_t flags, void* out_zero,
                void* stream);

/* Fused Adagrad (lr_decay, weight decay, maximize) over (R, T), fp64 element
 * math as ROCm ATen's `adagrad_math` (ATen/native/hip/fused_adagrad_utils.cuh,
 * called by the reference at csrc/cuda/adagrad.cu:141-148).
 * bufs: [0] params (rw), [1] grads (r), [2] state_sums (rw). */
int ts_adagrad_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                    const void* lr, const void* lr_decay,
                    const void* weight_decay, const void* eps,
                    const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* stream);

/* Library version, for INTEGRATION checks: major*10000 + minor*100 + patch. */
int ts_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CHURTEN_OPTIM_H */

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
 *   ts_*_step_segments, ts_scatter_segments
 *                   <- the gradient scatter `state._consolidated_grads.update_(grads)`
 *                      (src/torchstrap/optimizer/grad_transform.py:29) that precedes
 *                      every update: one copy per parameter tensor there; fused
 *                      into the update (or one launch) here
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
 *   - Optimizer-state buffers are in the parameter dtype, or bfloat16 with
 *     TS_STATE_BF16.
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
/* all: the optimizer-state buffers (bufs[2..]: exp_avgs, exp_avg_sqs,
 * max_exp_avg_sqs, momentum_buffers, state_sums) hold bfloat16 while params
 * and grads hold `dtype`, which must be TS_FLOAT32. The element math is the
 * float32 math of the same op; state is widened on load and rounded to
 * nearest-even on store, so parameters come out as the float32 op computes
 * them from the widened state. Low-precision optimizer state has no
 * counterpart in the reference operators (its README roadmap lists it). */
#define TS_STATE_BF16 0x20u
/* Adagrad: float32 element math -- the reference CPU kernel's loop
 * (cpu/adagrad.cpp:94-156), bit-identical to the reference's CPU build on
 * float32 parameters -- instead of ATen's fp64 device update. Explicitly not
 * bit-exact to torch._fused_adagrad_ (the reference's README/CLAUDE.md name
 * such a variant as a separate feature). Not available for float64. */
#define TS_ADAGRAD_F32 0x40u

/* A per-parameter gradient: an (R, numel) tensor with element (r, j) at
 * data + r*stride_r + j, standing for columns [col, col + numel) of the
 * consolidated (R, T) layout. Tables of segments are in ascending `col` order
 * and do not overlap. */
typedef struct ts_segment {
  const void* data;
  int64_t stride_r;
  int64_t col;
  int64_t numel;
} ts_segment;

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
 * bufs: [0] params (rw), [1] grads (r), [2] state_sums (rw).
 * float16: a row whose length is a multiple of 4, with unit inner stride and
 * all three row pointers aligned to 4 elements (the vector path of torch's
 * fused kernels and of adagrad.cu:119-133) stores its state sum rounded once
 * from the exact g*g + s, as torch's ROCm build does there; other rows store
 * the float sum rounded to half. */
int ts_adagrad_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                    const void* lr, const void* lr_decay,
                    const void* weight_decay, const void* eps,
                    const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* stream);

/* Segmented-gradient forms of the three updates: the gradient of the columns
 * a segment covers is read from the per-parameter tensors `grads[0..n_grads)`.
 * bufs[1].data may be NULL; if it is not, those gradients are also written
 * into that consolidated (R, T) buffer on the way through (all rows, frozen
 * replicas included, as the separate scatter would), and the columns no
 * segment covers take their gradient from it; with NULL they take zero. Element
 * math and flags as the consolidated forms, so every column ends up identical
 * to ts_scatter_segments into bufs[1] (or into a zeroed buffer) followed by
 * ts_*_step. One launch per 64 table entries (segments and the gaps between
 * them), plus the bump. */
int ts_adam_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                          ts_dtype dtype, void* state_steps, const void* lr,
                          const void* beta1, const void* beta2, const void* eps,
                          const void* weight_decay, const uint8_t* active_mask,
                          int64_t R, int64_t T, uint32_t flags, void* out_zero,
                          void* stream);
int ts_sgd_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                         ts_dtype dtype, void* state_steps, const void* lr,
                         const void* momentum, const void* dampening,
                         const void* weight_decay, const uint8_t* active_mask,
                         int64_t R, int64_t T, uint32_t flags, void* out_zero,
                         void* stream);
int ts_adagrad_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                             ts_dtype dtype, void* state_steps, const void* lr,
                             const void* lr_decay, const void* weight_decay,
                             const void* eps, const uint8_t* active_mask, int64_t R,
                             int64_t T, uint32_t flags, void* out_zero, void* stream);

/* Forms with a caller-provided workspace: the same updates, bit for bit, with
 * each active replica's constants (Adam's step size and bias-correction
 * divisor, from two fp64 pow; Adagrad's corrected learning rate: fp64 work
 * every workgroup otherwise repeats) computed once per call by the launch that
 * bumps the steps, and read by the update kernel. The update then runs a
 * shorter tile per workgroup: the config-5 Adam step (128 x 25.2M float32)
 * 6.46-6.51 TB/s against 6.14-6.18 for ts_adam_step on the same buffers.
 *   workspace:       device memory of at least ts_workspace_bytes(R) bytes,
 *                    8-byte aligned, not NULL. It is scratch: nothing is read
 *                    from it before the call writes it, and its contents after
 *                    the call mean nothing. It must not be shared with another
 *                    call that may run at the same time (another stream).
 *   workspace_bytes: its size; smaller than ts_workspace_bytes(R) is an
 *                    invalid argument.
 * Still two launches per call (preparation, update), as without a workspace.
 * These replace the same reference interfaces as ts_adam_step, ts_adagrad_step
 * and their segmented forms (stubs.cpp:25-41, 61-72; cuda/adam.cu:99-122 and
 * cuda/adagrad.cu:141-148 are the per-block prologues whose constants the
 * workspace hoists). */
size_t ts_workspace_bytes(int64_t R);
int ts_adam_step_ws(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps, const void* lr,
                    const void* beta1, const void* beta2, const void* eps,
                    const void* weight_decay, const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* workspace, size_t workspace_bytes,
                    void* stream);
int ts_adagrad_step_ws(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                       const void* lr, const void* lr_decay, const void* weight_decay,
                       const void* eps, const uint8_t* active_mask, int64_t R, int64_t T,
                       uint32_t flags, void* out_zero, void* workspace, size_t workspace_bytes,
                       void* stream);
int ts_adam_step_segments_ws(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                             ts_dtype dtype, void* state_steps, const void* lr,
                             const void* beta1, const void* beta2, const void* eps,
                             const void* weight_decay, const uint8_t* active_mask, int64_t R,
                             int64_t T, uint32_t flags, void* out_zero, void* workspace,
                             size_t workspace_bytes, void* stream);
int ts_adagrad_step_segments_ws(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                                ts_dtype dtype, void* state_steps, const void* lr,
                                const void* lr_decay, const void* weight_decay,
                                const void* eps, const uint8_t* active_mask, int64_t R,
                                int64_t T, uint32_t flags, void* out_zero, void* workspace,
                                size_t workspace_bytes, void* stream);

/* ts_adam_step_ws without a workspace argument, allocating nothing: the
 * per-replica constants go to a scratch array inside the library (1 MiB per
 * device, held until the process ends; its device address is looked up on the
 * first call on each device). No counterpart in the reference: it is for
 * callers that cannot allocate device memory at call time -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation.
 * Limits: R <= 65536 (larger R is hipErrorInvalidValue, before anything is
 * enqueued). Every call on one device shares that device's scratch: calls that
 * can overlap on one GPU (several streams, several threads) race and must be
 * serialised by the caller. Nothing in the scratch needs to start at zero:
 * each call writes every active replica's constants before its update reads
 * them. Results are bit-identical to ts_adam_step_ws. */
int ts_adam_step_noalloc(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                         const void* lr, const void* beta1, const void* beta2, const void* eps,
                         const void* weight_decay, const uint8_t* active_mask, int64_t R,
                         int64_t T, uint32_t flags, void* out_zero, void* stream);

/* Gradient scatter in one launch per 64 segments: copies every segment, all R
 * rows, into its columns of the (R, cols) buffer dst (row stride dst_stride_r,
 * unit column stride); other columns are not written. Replaces the
 * per-parameter copies of grad_transform.py:29. */
int ts_scatter_segments(const ts_segment* src, int n_src, ts_dtype dtype, void* dst,
                        int64_t dst_stride_r, int64_t cols, int64_t R, void* stream);

/* Replica-row transfer for the snapshot / checkpoint path: copies rows r of
 * an (R, ...) buffer with rows[r] != 0 (rows is a HOST array of R bytes; NULL
 * = every row), row_bytes bytes each, from src (row stride src_stride bytes)
 * to dst (row stride dst_stride bytes), with one DMA copy per run of
 * consecutive selected rows, enqueued on `stream`. The host side must be
 * pinned memory for the copy to be asynchronous. Replaces the gather + pinned
 * staging + host scatter of the reference's Snapshot.update / restore_to_live
 * (src/torchstrap/callbacks/training.py:45-116). */
#define TS_ROWS_TO_HOST 0   /* device buffer -> host mirror */
#define TS_ROWS_TO_DEVICE 1 /* host mirror -> device buffer */
#define TS_ROWS_DEVICE 2    /* device -> device */
int ts_copy_rows(void* dst, int64_t dst_stride, const void* src, int64_t src_stride,
                 int64_t row_bytes, const uint8_t* rows, int64_t R, int direction,
                 void* stream);

/* Library version, for INTEGRATION checks: major*10000 + minor*100 + patch. */
int ts_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CHURTEN_OPTIM_H */

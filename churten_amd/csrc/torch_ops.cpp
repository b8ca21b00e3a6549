// torch_ops.cpp -- the operator libraries over the C ABI.
//
// `torchstrap`: the three operator schemas with the reference's exact text
// (src/torchstrap/kernels/csrc/stubs.cpp:25-72), so code that calls
// torch.ops.torchstrap.{adam,sgd,adagrad}_step_ is served unchanged. The GPU
// dispatch key validates the tensors on the host and calls the extern "C"
// launchers of include/churten_optim.h on the current HIP stream. The module
// init function makes this file a drop-in for `torchstrap.kernels._C`
// (stubs.cpp:75-85): importing it registers the ops.
//
// `churten`: additions with no counterpart in the reference operator set, for
// the gradient scatter that precedes every update
// (src/torchstrap/optimizer/grad_transform.py:29): a one-launch scatter
// (`scatter_grads_`) and the three updates reading per-parameter gradients
// directly (`*_step_segments_`), optionally materialising the consolidated
// gradient on the way. Their CPU keys compose the scatter with the CPU
// kernels.
//
// Host-side behaviour kept from the reference operators:
//   - params must be a 2-D (R, T) buffer; amsgrad needs max_exp_avg_sqs,
//     nesterov needs momentum_buffers (RuntimeError otherwise);
//   - state_steps += active_mask happens on every call before the update reads
//     it, also when R or T is 0 (adam.cu:277-281);
//   - the (R,) inputs are used in the parameter dtype (adam.cu:287-294);
//   - the return value is a fresh 0-d zero tensor aliasing nothing.
// Added here, because the kernel trusts its operands: every (R, T) operand must
// match params' shape, dtype and device, and every (R,) input must have R
// elements on params' device -- the reference would read out of bounds.
// Extension: the optimizer-state buffers may be bfloat16 next to float32
// params (all of them, TS_STATE_BF16); the reference rejects mixed dtypes.
//
// The common case (steps in the param dtype, a bool mask, contiguous (R,)
// vectors) costs two launches: the preparation (step bump, zero result and,
// for Adam and Adagrad, the per-replica constants into a workspace) and the
// update. Anything else is first normalised with ATen ops.

#include <Python.h>

#include <ATen/ATen.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <numeric>
#include <optional>
#include <string>
#include <vector>

#include "../../include/churten_optim.h"

namespace churten {
namespace {

// Same cap the reference imposes (csrc/cuda/consolidated.cuh:30, 72-81), kept
// so callers see the same error for the same input.
constexpr int64_t kMaxReplicas = 65535;

ts_dtype ts_dtype_of(at::ScalarType t, const char* op) {
  switch (t) {
    case at::kFloat: return TS_FLOAT32;
    case at::kDouble: return TS_FLOAT64;
    case at::kHalf: return TS_FLOAT16;
    case at::kBFloat16: return TS_BFLOAT16;
    default: break;
  }
  TORCH_CHECK(false, op, ": unsupported parameter dtype ", t,
              " (float32, float64, float16 and bfloat16 are supported)");
}

ts_rt_buf rt_buf(const at::Tensor& t) {
  return ts_rt_buf{t.data_ptr(), t.stride(0), t.stride(1)};
}

constexpr ts_rt_buf kNoBuf{nullptr, 0, 1};

void check_params(const at::Tensor& params, const char* op) {
  TORCH_CHECK(params.dim() == 2, op, ": params must be a 2-D (R, T) buffer");
  TORCH_CHECK(params.size(0) <= kMaxReplicas, op,
              " maps one replica per row and supports at most ", kMaxReplicas,
              " replicas; got R = ", params.size(0));
  TORCH_CHECK(params.is_cuda(), op, ": params must be on a GPU for this kernel");
}

void check_like(const at::Tensor& params, const at::Tensor& t, const char* op,
                const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.sizes() == params.sizes(), op, ": ", name,
              " must have params' shape ", params.sizes(), ", got ", t.sizes());
  TORCH_CHECK(t.scalar_type() == params.scalar_type(), op, ": ", name,
              " must have params' dtype ", params.scalar_type(), ", got ",
              t.scalar_type());
  TORCH_CHECK(t.device() == params.device(), op, ": ", name,
              " must be on ", params.device(), ", got ", t.device());
}

// Optimizer state may be bfloat16 next to float32 params (TS_STATE_BF16);
// the first state buffer decides, and every state buffer must agree.
uint32_t state_flag(const at::Tensor& params, const at::Tensor& first_state) {
  return params.scalar_type() == at::kFloat && first_state.scalar_type() == at::kBFloat16
             ? TS_STATE_BF16
             : 0u;
}

void check_state(const at::Tensor& params, const at::Tensor& t, uint32_t sflag,
                 const char* op, const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.sizes() == params.sizes(), op, ": ", name,
              " must have params' shape ", params.sizes(), ", got ", t.sizes());
  const auto want = sflag != 0 ? at::kBFloat16 : params.scalar_type();
  TORCH_CHECK(t.scalar_type() == want, op, ": ", name, " must have dtype ", want,
              " (params' dtype, or bfloat16 for every state buffer next to float32 params),"
              " got ", t.scalar_type());
  TORCH_CHECK(t.device() == params.device(), op, ": ", name,
              " must be on ", params.device(), ", got ", t.device());
}

void check_vec(const at::Tensor& params, const at::Tensor& t, const char* op,
               const char* name) {
  TORCH_CHECK(t.numel() == params.size(0), op, ": ", name, " must have R = ",
              params.size(0), " elements (one per replica), got ", t.numel());
  TORCH_CHECK(t.device() == params.device(), op, ": ", name,
              " must be on ", params.device(), ", got ", t.device());
}

// The (R,) hyperparameters, in the param dtype and contiguous. The normal case,
// already such a vector, returns it without a dispatcher call (reshape, to and
// contiguous would each return it unchanged; at microsecond steps the host's
// per-call cost sets the step time).
at::Tensor hyper(const at::Tensor& t, at::ScalarType dtype) {
  if (t.dim() == 1 && t.scalar_type() == dtype && t.is_contiguous()) return t;
  return t.reshape({t.numel()}).to(dtype).contiguous();
}

void check_status(int status, const char* op) {
  TORCH_CHECK(status == 0, op, ": HIP launch failed with error ", status);
}

hipStream_t current_stream(const at::Tensor& params) {
  return c10::hip::getCurrentHIPStream(params.device().index()).stream();
}

// Everything a launcher needs besides the (R, T) operand table: the step
// counter (bumped by the launcher when TS_BUMP_STEPS is set), the mask, the
// normalised hyperparameter vectors, the fresh zero result and, when there is
// work, the workspace for the per-replica constants (ts_workspace_bytes(R)
// bytes from torch's caching allocator on the current stream: no device
// allocation once the allocator is warm, and stream-ordered reuse).
struct Prepared {
  ts_dtype dtype;
  uint32_t flags;
  at::Tensor steps;
  at::Tensor mask;
  std::vector<at::Tensor> hyp;
  at::Tensor out;
  at::Tensor ws;
  int64_t R, T;
  hipStream_t stream;

  const void* h(size_t i) const { return hyp[i].data_ptr(); }
  const uint8_t* m() const { return static_cast<const uint8_t*>(mask.data_ptr()); }
  bool has_ws() const { return ws.defined(); }
  void* ws_ptr() const { return ws.data_ptr(); }
  size_t ws_bytes() const { return static_cast<size_t>(ws.numel()); }
};

Prepared prepare(const at::Tensor& params, at::Tensor& state_steps,
                 const at::Tensor& active_mask, std::initializer_list<const at::Tensor*> hyp,
                 std::initializer_list<const char*> names, uint32_t flags, const char* op,
                 bool want_ws = true) {
  check_vec(params, state_steps, op, "state_steps");
  check_vec(params, active_mask, op, "active_mask");
  auto name = names.begin();
  for (const at::Tensor* t : hyp) check_vec(params, *t, op, *name++);
  Prepared p;
  const auto dtype = params.scalar_type();
  p.dtype = ts_dtype_of(dtype, op);
  p.flags = flags;
  if (state_steps.scalar_type() == dtype && state_steps.is_contiguous() &&
      active_mask.scalar_type() == at::kBool) {
    p.mask = active_mask.dim() == 1 && active_mask.is_contiguous()
                 ? active_mask
                 : active_mask.reshape({active_mask.numel()}).contiguous();
    p.steps = state_steps;
    p.flags |= TS_BUMP_STEPS;
  } else {
    state_steps.add_(active_mask.to(state_steps.scalar_type()));
    p.mask = active_mask.reshape({active_mask.numel()}).to(at::kBool).contiguous();
    p.steps = hyper(state_steps, dtype);
  }
  for (const at::Tensor* t : hyp) p.hyp.push_back(hyper(*t, dtype));
  p.out = at::empty({}, params.options());
  p.R = params.size(0);
  p.T = params.size(1);
  if (want_ws && p.R > 0 && p.T > 0) {
    p.ws = at::empty({static_cast<int64_t>(ts_workspace_bytes(p.R))},
                     params.options().dtype(at::kByte));
  }
  p.stream = current_stream(params);
  return p;
}

// ---------------------------------------------------------------------------
// Segment tables (per-parameter gradients)
// ---------------------------------------------------------------------------
struct SegTable {
  std::vector<ts_segment> segs;
  std::vector<at::Tensor> keep;  // (R, numel) views kept alive for the launch
};

// Each gradient is (R, *shape) and stands for columns [col, col + numel) of
// params; the table is returned in ascending column order, checked in range
// and non-overlapping.
SegTable segments_of(const at::Tensor& params, at::TensorList grads, at::IntArrayRef cols,
                     const char* op) {
  TORCH_CHECK(grads.size() == cols.size(), op, ": got ", grads.size(), " gradients but ",
              cols.size(), " column offsets");
  const int64_t R = params.size(0), T = params.size(1);
  std::vector<size_t> order(grads.size());
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return cols[a] < cols[b]; });
  SegTable st;
  int64_t end = 0;
  for (size_t i : order) {
    const at::Tensor& g = grads[i];
    TORCH_CHECK(g.scalar_type() == params.scalar_type(), op, ": gradient ", i,
                " must have params' dtype ", params.scalar_type());
    TORCH_CHECK(g.device() == params.device(), op, ": gradient ", i, " must be on ",
                params.device());
    TORCH_CHECK(g.dim() >= 1 && g.size(0) == R, op, ": gradient ", i,
                " must have the replica count R = ", R, " as its leading dimension");
    const int64_t numel = R > 0 ? g.numel() / R : 0;
    TORCH_CHECK(cols[i] >= 0 && cols[i] <= T - numel, op, ": gradient ", i, " (columns ",
                cols[i], "..", cols[i] + numel, ") lies outside the ", T, " columns");
    if (R == 0 || numel == 0) continue;
    TORCH_CHECK(cols[i] >= end, op, ": gradient ", i, " (columns ", cols[i], "..",
                cols[i] + numel, ") overlaps another gradient");
    end = cols[i] + numel;
    at::Tensor g2 = g.reshape({R, numel});
    if (g2.stride(1) != 1) g2 = g2.contiguous();
    st.segs.push_back(ts_segment{g2.data_ptr(), g2.stride(0), cols[i], numel});
    st.keep.push_back(std::move(g2));
  }
  return st;
}

// ---------------------------------------------------------------------------
// torchstrap::* on the GPU key
// ---------------------------------------------------------------------------
at::Tensor adam_step_gpu(at::Tensor params, at::Tensor grads, at::Tensor exp_avgs,
                         at::Tensor exp_avg_sqs, std::optional<at::Tensor> max_exp_avg_sqs,
                         at::Tensor state_steps, at::Tensor lr, at::Tensor beta1,
                         at::Tensor beta2, at::Tensor eps, at::Tensor weight_decay,
                         at::Tensor active_mask, bool amsgrad, bool maximize,
                         bool decoupled_weight_decay) {
  constexpr const char* op = "torchstrap::adam_step_";
  check_params(params, op);
  TORCH_CHECK(!amsgrad || max_exp_avg_sqs.has_value(), "amsgrad=True requires max_exp_avg_sqs");
  check_like(params, grads, op, "grads");
  const uint32_t sflag = state_flag(params, exp_avgs);
  check_state(params, exp_avgs, sflag, op, "exp_avgs");
  check_state(params, exp_avg_sqs, sflag, op, "exp_avg_sqs");
  if (amsgrad) check_state(params, *max_exp_avg_sqs, sflag, op, "max_exp_avg_sqs");
  const c10::DeviceGuard guard(params.device());
  const Prepared p = prepare(
      params, state_steps, active_mask, {&lr, &beta1, &beta2, &eps, &weight_decay},
      {"lr", "beta1", "beta2", "eps", "weight_decay"},
      sflag | (amsgrad ? TS_AMSGRAD : 0u) | (decoupled_weight_decay ? TS_ADAMW : 0u) |
          (maximize ? TS_MAXIMIZE : 0u),
      op);
  const ts_rt_buf bufs[5] = {rt_buf(params), rt_buf(grads), rt_buf(exp_avgs),
                             rt_buf(exp_avg_sqs),
                             amsgrad ? rt_buf(*max_exp_avg_sqs) : kNoBuf};
  check_status(
      p.has_ws()
          ? ts_adam_step_ws(bufs, p.dtype, p.steps.data_ptr(), p.h(0), p.h(1), p.h(2), p.h(3),
                            p.h(4), p.m(), p.R, p.T, p.flags, p.out.data_ptr(), p.ws_ptr(),
                            p.ws_bytes(), p.stream)
          : ts_adam_step(bufs, p.dtype, p.steps.data_ptr(), p.h(0), p.h(1), p.h(2), p.h(3),
                         p.h(4), p.m(), p.R, p.T, p.flags, p.out.data_ptr(), p.stream),
      op);
  return p.out;
}

at::Tensor sgd_step_gpu(at::Tensor params, at::Tensor grads,
                        std::optional<at::Tensor> momentum_buffers, at::Tensor state_steps,
                        at::Tensor lr, at::Tensor momentum, at::Tensor dampening,
                        at::Tensor weight_decay, at::Tensor active_mask, bool nesterov,
                        bool maximize) {
  constexpr const char* op = "torchstrap::sgd_step_";
  check_params(params, op);
  TORCH_CHECK(!nesterov || momentum_buffers.has_value(), "nesterov=True requires momentum_buffers");
  check_like(params, grads, op, "grads");
  const uint32_t sflag =
      momentum_buffers.has_value() ? state_flag(params, *momentum_buffers) : 0u;
  if (momentum_buffers.has_value()) {
    check_state(params, *momentum_buffers, sflag, op, "momentum_buffers");
  }
  const c10::DeviceGuard guard(params.device());
  const Prepared p = prepare(params, state_steps, active_mask,
                             {&lr, &momentum, &dampening, &weight_decay},
                             {"lr", "momentum", "dampening", "weight_decay"},
                             sflag | (nesterov ? TS_NESTEROV : 0u) |
                                 (maximize ? TS_MAXIMIZE : 0u),
                             op, /*want_ws=*/false);
  const ts_rt_buf bufs[3] = {rt_buf(params), rt_buf(grads),
                             momentum_buffers.has_value() ? rt_buf(*momentum_buffers) : kNoBuf};
  check_status(ts_sgd_step(bufs, p.dtype, p.steps.data_ptr(), p.h(0), p.h(1), p.h(2), p.h(3),
                           p.m(), p.R, p.T, p.flags, p.out.data_ptr(), p.stream),
               op);
  return p.out;
}

at::Tensor adagrad_gpu(at::Tensor params, at::Tensor grads, at::Tensor state_sums,
                       at::Tensor state_steps, at::Tensor lr, at::Tensor lr_decay,
                       at::Tensor weight_decay, at::Tensor eps, at::Tensor active_mask,
                       bool maximize, bool fp32_math, const char* op) {
  check_params(params, op);
  TORCH_CHECK(!fp32_math || params.scalar_type() != at::kDouble, op,
              ": the float32 Adagrad variant does not take float64 parameters");
  check_like(params, grads, op, "grads");
  const uint32_t sflag = state_flag(params, state_sums);
  check_state(params, state_sums, sflag, op, "state_sums");
  const c10::DeviceGuard guard(params.device());
  const Prepared p = prepare(params, state_steps, active_mask,
                             {&lr, &lr_decay, &weight_decay, &eps},
                             {"lr", "lr_decay", "weight_decay", "eps"},
                             sflag | (maximize ? TS_MAXIMIZE : 0u) |
                                 (fp32_math ? TS_ADAGRAD_F32 : 0u),
                             op);
  const ts_rt_buf bufs[3] = {rt_buf(params), rt_buf(grads), rt_buf(state_sums)};
  check_status(
      p.has_ws()
          ? ts_adagrad_step_ws(bufs, p.dtype, p.steps.data_ptr(), p.h(0), p.h(1), p.h(2),
                               p.h(3), p.m(), p.R, p.T, p.flags, p.out.data_ptr(), p.ws_ptr(),
                               p.ws_bytes(), p.stream)
          : ts_adagrad_step(bufs, p.dtype, p.steps.data_ptr(), p.h(0), p.h(1), p.h(2), p.h(3),
                            p.m(), p.R, p.T, p.flags, p.out.data_ptr(), p.stream),
      op);
  return p.out;
}

at::Tensor adagrad_step_gpu(at::Tensor params, at::Tensor grads, at::Tensor state_sums,
                            at::Tensor state_steps, at::Tensor lr, at::Tensor lr_decay,
                            at::Tensor weight_decay, at::Tensor eps, at::Tensor active_mask,
                            bool maximize) {
  return adagrad_gpu(params, grads, state_sums, state_steps, lr, lr_decay, weight_decay, eps,
                     active_mask, maximize, false, "torchstrap::adagrad_step_");
}

at::Tensor adagrad_step_f32_gpu(at::Tensor params, at::Tensor grads, at::Tensor state_sums,
                                at::Tensor state_steps, at::Tensor lr, at::Tensor lr_decay,
                                at::Tensor weight_decay, at::Tensor eps,
                                at::Tensor active_mask, bool maximize) {
  return adagrad_gpu(params, grads, state_sums, state_steps, lr, lr_decay, weight_decay, eps,
                     active_mask, maximize, true, "churten::adagrad_step_f32_");
}

// ---------------------------------------------------------------------------
// churten::* on the GPU key
// ---------------------------------------------------------------------------
void scatter_grads_gpu(at::Tensor dst, at::TensorList grads, at::IntArrayRef cols) {
  constexpr const char* op = "churten::scatter_grads_";
  TORCH_CHECK(dst.dim() == 2 && dst.is_cuda(), op, ": dst must be a 2-D (R, T) GPU buffer");
  TORCH_CHECK(dst.stride(1) == 1, op, ": dst rows must be contiguous");
  const c10::DeviceGuard guard(dst.device());
  const SegTable st = segments_of(dst, grads, cols, op);
  check_status(ts_scatter_segments(st.segs.data(), static_cast<int>(st.segs.size()),
                                   ts_dtype_of(dst.scalar_type(), op), dst.data_ptr(),
                                   dst.stride(0), dst.size(1), dst.size(0),
                                   current_stream(dst)),
               op);
}

at::Tensor adam_step_segments_gpu(at::Tensor params, at::TensorList grads, at::IntArrayRef cols,
                                  std::optional<at::Tensor> grads_out, at::Tensor exp_avgs,
                                  at::Tensor exp_avg_sqs,
                                  std::optional<at::Tensor> max_exp_avg_sqs,
                                  at::Tensor state_steps, at::Tensor lr, at::Tensor beta1,
                                  at::Tensor beta2, at::Tensor eps, at::Tensor weight_decay,
                                  at::Tensor active_mask, bool amsgrad, bool maximize,
                                  bool decoupled_weight_decay) {
  constexpr const char* op = "churten::adam_step_segments_";
  check_params(params, op);
  TORCH_CHECK(!amsgrad || max_exp_avg_sqs.has_value(), "amsgrad=True requires max_exp_avg_sqs");
  if (grads_out.has_value()) check_like(params, *grads_out, op, "grads_out");
  const uint32_t sflag = state_flag(params, exp_avgs);
  check_state(params, exp_avgs, sflag, op, "exp_avgs");
  check_state(params, exp_avg_sqs, sflag, op, "exp_avg_sqs");
  if (amsgrad) check_state(params, *max_exp_avg_sqs, sflag, op, "max_exp_avg_sqs");
  const c10::DeviceGuard guard(params.device());
  const SegTable st = segments_of(params, grads, cols, op);
  const Prepared p = prepare(
      params, state_steps, active_mask, {&lr, &beta1, &beta2, &eps, &weight_decay},
      {"lr", "beta1", "beta2", "eps", "weight_decay"},
      sflag | (amsgrad ? TS_AMSGRAD : 0u) | (decoupled_weight_decay ? TS_ADAMW : 0u) |
          (maximize ? TS_MAXIMIZE : 0u),
      op);
  const ts_rt_buf bufs[5] = {rt_buf(params), grads_out.has_value() ? rt_buf(*grads_out) : kNoBuf,
                             rt_buf(exp_avgs), rt_buf(exp_avg_sqs),
                             amsgrad ? rt_buf(*max_exp_avg_sqs) : kNoBuf};
  const int n = static_cast<int>(st.segs.size());
  check_status(
      p.has_ws()
          ? ts_adam_step_segments_ws(bufs, st.segs.data(), n, p.dtype, p.steps.data_ptr(),
                                     p.h(0), p.h(1), p.h(2), p.h(3), p.h(4), p.m(), p.R, p.T,
                                     p.flags, p.out.data_ptr(), p.ws_ptr(), p.ws_bytes(),
                                     p.stream)
          : ts_adam_step_segments(bufs, st.segs.data(), n, p.dtype, p.steps.data_ptr(), p.h(0),
                                  p.h(1), p.h(2), p.h(3), p.h(4), p.m(), p.R, p.T, p.flags,
                                  p.out.data_ptr(), p.stream),
      op);
  return p.out;
}

at::Tensor sgd_step_segments_gpu(at::Tensor params, at::TensorList grads, at::IntArrayRef cols,
                                 std::optional<at::Tensor> grads_out,
                                 std::optional<at::Tensor> momentum_buffers,
                                 at::Tensor state_steps, at::Tensor lr, at::Tensor momentum,
                                 at::Tensor dampening, at::Tensor weight_decay,
                                 at::Tensor active_mask, bool nesterov, bool maximize) {
  constexpr const char* op = "churten::sgd_step_segments_";
  check_params(params, op);
  TORCH_CHECK(!nesterov || momentum_buffers.has_value(), "nesterov=True requires momentum_buffers");
  if (grads_out.has_value()) check_like(params, *grads_out, op, "grads_out");
  const uint32_t sflag =
      momentum_buffers.has_value() ? state_flag(params, *momentum_buffers) : 0u;
  if (momentum_buffers.has_value()) {
    check_state(params, *momentum_buffers, sflag, op, "momentum_buffers");
  }
  const c10::DeviceGuard guard(params.device());
  const SegTable st = segments_of(params, grads, cols, op);
  const Prepared p = prepare(params, state_steps, active_mask,
                             {&lr, &momentum, &dampening, &weight_decay},
                             {"lr", "momentum", "dampening", "weight_decay"},
                             sflag | (nesterov ? TS_NESTEROV : 0u) |
                                 (maximize ? TS_MAXIMIZE : 0u),
                             op, /*want_ws=*/false);
  const ts_rt_buf bufs[3] = {rt_buf(params), grads_out.has_value() ? rt_buf(*grads_out) : kNoBuf,
                             momentum_buffers.has_value() ? rt_buf(*momentum_buffers) : kNoBuf};
  check_status(ts_sgd_step_segments(bufs, st.segs.data(), static_cast<int>(st.segs.size()),
                                    p.dtype, p.steps.data_ptr(), p.h(0), p.h(1), p.h(2), p.h(3),
                                    p.m(), p.R, p.T, p.flags, p.out.data_ptr(), p.stream),
               op);
  return p.out;
}

at::Tensor adagrad_step_segments_gpu(at::Tensor params, at::TensorList grads,
                                     at::IntArrayRef cols, std::optional<at::Tensor> grads_out,
                                     at::Tensor state_sums, at::Tensor state_steps,
                                     at::Tensor lr, at::Tensor lr_decay,
                                     at::Tensor weight_decay, at::Tensor eps,
                                     at::Tensor active_mask, bool maximize, bool fp32_math) {
  constexpr const char* op = "churten::adagrad_step_segments_";
  check_params(params, op);
  TORCH_CHECK(!fp32_math || params.scalar_type() != at::kDouble, op,
              ": the float32 Adagrad variant does not take float64 parameters");
  if (grads_out.has_value()) check_like(params, *grads_out, op, "grads_out");
  const uint32_t sflag = state_flag(params, state_sums);
  check_state(params, state_sums, sflag, op, "state_sums");
  const c10::DeviceGuard guard(params.device());
  const SegTable st = segments_of(params, grads, cols, op);
  const Prepared p = prepare(params, state_steps, active_mask,
                             {&lr, &lr_decay, &weight_decay, &eps},
                             {"lr", "lr_decay", "weight_decay", "eps"},
                             sflag | (maximize ? TS_MAXIMIZE : 0u) |
                                 (fp32_math ? TS_ADAGRAD_F32 : 0u),
                             op);
  const ts_rt_buf bufs[3] = {rt_buf(params), grads_out.has_value() ? rt_buf(*grads_out) : kNoBuf,
                             rt_buf(state_sums)};
  const int n = static_cast<int>(st.segs.size());
  check_status(
      p.has_ws()
          ? ts_adagrad_step_segments_ws(bufs, st.segs.data(), n, p.dtype, p.steps.data_ptr(),
                                        p.h(0), p.h(1), p.h(2), p.h(3), p.m(), p.R, p.T,
                                        p.flags, p.out.data_ptr(), p.ws_ptr(), p.ws_bytes(),
                                        p.stream)
          : ts_adagrad_step_segments(bufs, st.segs.data(), n, p.dtype, p.steps.data_ptr(),
                                     p.h(0), p.h(1), p.h(2), p.h(3), p.m(), p.R, p.T, p.flags,
                                     p.out.data_ptr(), p.stream),
      op);
  return p.out;
}

// ---------------------------------------------------------------------------
// churten::* on the CPU key: the scatter into a consolidated gradient (the
// caller's grads_out, or a zero buffer), then the torchstrap CPU kernel.
// ---------------------------------------------------------------------------
void scatter_grads_cpu(at::Tensor dst, at::TensorList grads, at::IntArrayRef cols) {
  constexpr const char* op = "churten::scatter_grads_";
  TORCH_CHECK(dst.dim() == 2, op, ": dst must be a 2-D (R, T) buffer");
  const SegTable st = segments_of(dst, grads, cols, op);
  for (size_t i = 0; i < st.segs.size(); ++i) {
    dst.narrow(1, st.segs[i].col, st.segs[i].numel).copy_(st.keep[i]);
  }
}

at::Tensor consolidated(const at::Tensor& params, const std::optional<at::Tensor>& grads_out,
                        at::TensorList grads, at::IntArrayRef cols) {
  at::Tensor dst = grads_out.has_value() ? *grads_out : at::zeros_like(params);
  scatter_grads_cpu(dst, grads, cols);
  return dst;
}

at::Tensor adam_step_segments_cpu(at::Tensor params, at::TensorList grads, at::IntArrayRef cols,
                                  std::optional<at::Tensor> grads_out, at::Tensor exp_avgs,
                                  at::Tensor exp_avg_sqs,
                                  std::optional<at::Tensor> max_exp_avg_sqs,
                                  at::Tensor state_steps, at::Tensor lr, at::Tensor beta1,
                                  at::Tensor beta2, at::Tensor eps, at::Tensor weight_decay,
                                  at::Tensor active_mask, bool amsgrad, bool maximize,
                                  bool decoupled_weight_decay) {
  static auto step = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchstrap::adam_step_", "")
                         .typed<at::Tensor(at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           std::optional<at::Tensor>, at::Tensor, at::Tensor,
                                           at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           at::Tensor, bool, bool, bool)>();
  TORCH_CHECK(params.dim() == 2, "churten::adam_step_segments_: params must be 2-D");
  return step.call(params, consolidated(params, grads_out, grads, cols), exp_avgs, exp_avg_sqs,
                   max_exp_avg_sqs, state_steps, lr, beta1, beta2, eps, weight_decay,
                   active_mask, amsgrad, maximize, decoupled_weight_decay);
}

at::Tensor sgd_step_segments_cpu(at::Tensor params, at::TensorList grads, at::IntArrayRef cols,
                                 std::optional<at::Tensor> grads_out,
                                 std::optional<at::Tensor> momentum_buffers,
                                 at::Tensor state_steps, at::Tensor lr, at::Tensor momentum,
                                 at::Tensor dampening, at::Tensor weight_decay,
                                 at::Tensor active_mask, bool nesterov, bool maximize) {
  static auto step = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchstrap::sgd_step_", "")
                         .typed<at::Tensor(at::Tensor, at::Tensor, std::optional<at::Tensor>,
                                           at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           at::Tensor, at::Tensor, bool, bool)>();
  TORCH_CHECK(params.dim() == 2, "churten::sgd_step_segments_: params must be 2-D");
  return step.call(params, consolidated(params, grads_out, grads, cols), momentum_buffers,
                   state_steps, lr, momentum, dampening, weight_decay, active_mask, nesterov,
                   maximize);
}

at::Tensor adagrad_step_segments_cpu(at::Tensor params, at::TensorList grads,
                                     at::IntArrayRef cols, std::optional<at::Tensor> grads_out,
                                     at::Tensor state_sums, at::Tensor state_steps,
                                     at::Tensor lr, at::Tensor lr_decay,
                                     at::Tensor weight_decay, at::Tensor eps,
                                     at::Tensor active_mask, bool maximize, bool fp32_math) {
  TORCH_CHECK(!fp32_math || params.scalar_type() != at::kDouble,
              "churten::adagrad_step_segments_: the float32 Adagrad variant does not take "
              "float64 parameters");
  // The CPU kernel already runs the float32 element math.
  static auto step = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchstrap::adagrad_step_", "")
                         .typed<at::Tensor(at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           at::Tensor, bool)>();
  TORCH_CHECK(params.dim() == 2, "churten::adagrad_step_segments_: params must be 2-D");
  return step.call(params, consolidated(params, grads_out, grads, cols), state_sums,
                   state_steps, lr, lr_decay, weight_decay, eps, active_mask, maximize);
}

// The reference's CPU Adagrad kernel is itself the float32 element loop, so
// the float32 variant on the CPU key is that kernel.
at::Tensor adagrad_step_f32_cpu(at::Tensor params, at::Tensor grads, at::Tensor state_sums,
                                at::Tensor state_steps, at::Tensor lr, at::Tensor lr_decay,
                                at::Tensor weight_decay, at::Tensor eps,
                                at::Tensor active_mask, bool maximize) {
  TORCH_CHECK(params.scalar_type() != at::kDouble,
              "churten::adagrad_step_f32_: the float32 Adagrad variant does not take float64 "
              "parameters");
  static auto step = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchstrap::adagrad_step_", "")
                         .typed<at::Tensor(at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           at::Tensor, at::Tensor, at::Tensor, at::Tensor,
                                           at::Tensor, bool)>();
  return step.call(params, grads, state_sums, state_steps, lr, lr_decay, weight_decay, eps,
                   active_mask, maximize);
}

}  // namespace

// Schema text identical to the reference (stubs.cpp:25-72): the alias
// annotations declare exactly which arguments are mutated in place, and the
// returned tensor is fresh (vmap rejects an op that returns nothing).
TORCH_LIBRARY(torchstrap, m) {
  m.def("adam_step_("
        "Tensor(a!) params, "
        "Tensor grads, "
        "Tensor(b!) exp_avgs, "
        "Tensor(c!) exp_avg_sqs, "
        "Tensor(d!)? max_exp_avg_sqs, "
        "Tensor(e!) state_steps, "
        "Tensor lr, "
        "Tensor beta1, "
        "Tensor beta2, "
        "Tensor eps, "
        "Tensor weight_decay, "
        "Tensor active_mask, "
        "bool amsgrad, "
        "bool maximize, "
        "bool decoupled_weight_decay"
        ") -> Tensor");
  m.def("sgd_step_("
        "Tensor(a!) params, "
        "Tensor grads, "
        "Tensor(b!)? momentum_buffers, "
        "Tensor(c!) state_steps, "
        "Tensor lr, "
        "Tensor momentum, "
        "Tensor dampening, "
        "Tensor weight_decay, "
        "Tensor active_mask, "
        "bool nesterov, "
        "bool maximize"
        ") -> Tensor");
  m.def("adagrad_step_("
        "Tensor(a!) params, "
        "Tensor grads, "
        "Tensor(b!) state_sums, "
        "Tensor(c!) state_steps, "
        "Tensor lr, "
        "Tensor lr_decay, "
        "Tensor weight_decay, "
        "Tensor eps, "
        "Tensor active_mask, "
        "bool maximize"
        ") -> Tensor");
}

// On ROCm builds of torch the GPU dispatch key is still called CUDA.
TORCH_LIBRARY_IMPL(torchstrap, CUDA, m) {
  m.impl("adam_step_", &adam_step_gpu);
  m.impl("sgd_step_", &sgd_step_gpu);
  m.impl("adagrad_step_", &adagrad_step_gpu);
}

TORCH_LIBRARY(churten, m) {
  m.def("scatter_grads_(Tensor(a!) dst, Tensor[] grads, int[] cols) -> ()");
  m.def("adam_step_segments_(Tensor(a!) params, Tensor[] grads, int[] cols, "
        "Tensor(b!)? grads_out, Tensor(c!) exp_avgs, Tensor(d!) exp_avg_sqs, "
        "Tensor(e!)? max_exp_avg_sqs, Tensor(f!) state_steps, Tensor lr, Tensor beta1, "
        "Tensor beta2, Tensor eps, Tensor weight_decay, Tensor active_mask, bool amsgrad, "
        "bool maximize, bool decoupled_weight_decay) -> Tensor");
  m.def("sgd_step_segments_(Tensor(a!) params, Tensor[] grads, int[] cols, "
        "Tensor(b!)? grads_out, Tensor(c!)? momentum_buffers, Tensor(d!) state_steps, "
        "Tensor lr, Tensor momentum, Tensor dampening, Tensor weight_decay, "
        "Tensor active_mask, bool nesterov, bool maximize) -> Tensor");
  m.def("adagrad_step_segments_(Tensor(a!) params, Tensor[] grads, int[] cols, "
        "Tensor(b!)? grads_out, Tensor(c!) state_sums, Tensor(d!) state_steps, Tensor lr, "
        "Tensor lr_decay, Tensor weight_decay, Tensor eps, Tensor active_mask, "
        "bool maximize, bool fp32_math=False) -> Tensor");
  // torchstrap::adagrad_step_'s schema; float32 element math instead of fp64.
  m.def("adagrad_step_f32_(Tensor(a!) params, Tensor grads, Tensor(b!) state_sums, "
        "Tensor(c!) state_steps, Tensor lr, Tensor lr_decay, Tensor weight_decay, Tensor eps, "
        "Tensor active_mask, bool maximize) -> Tensor");
}

TORCH_LIBRARY_IMPL(churten, CUDA, m) {
  m.impl("scatter_grads_", &scatter_grads_gpu);
  m.impl("adam_step_segments_", &adam_step_segments_gpu);
  m.impl("sgd_step_segments_", &sgd_step_segments_gpu);
  m.impl("adagrad_step_segments_", &adagrad_step_segments_gpu);
  m.impl("adagrad_step_f32_", &adagrad_step_f32_gpu);
}

TORCH_LIBRARY_IMPL(churten, CPU, m) {
  m.impl("scatter_grads_", &scatter_grads_cpu);
  m.impl("adam_step_segments_", &adam_step_segments_cpu);
  m.impl("sgd_step_segments_", &sgd_step_segments_cpu);
  m.impl("adagrad_step_segments_", &adagrad_step_segments_cpu);
  m.impl("adagrad_step_f32_", &adagrad_step_f32_cpu);
}

}  // namespace churten

extern "C" PyObject* PyInit__C(void) {
  static struct PyModuleDef module_def = {
      PyModuleDef_HEAD_INIT, "_C", "torchstrap operators on MI355X (gfx950 HIP kernels)",
      -1, nullptr,
  };
  return PyModule_Create(&module_def);
}

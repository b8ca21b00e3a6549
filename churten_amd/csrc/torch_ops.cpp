// torch_ops.cpp -- the `torchstrap` operator library over the C ABI.
//
// Declares the three operator schemas with the reference's exact text
// (src/torchstrap/kernels/csrc/stubs.cpp:25-72), so code that calls
// torch.ops.torchstrap.{adam,sgd,adagrad}_step_ is served unchanged, and
// implements the GPU dispatch key by validating the tensors on the host and
// calling the extern "C" launchers of include/churten_optim.h on the current
// HIP stream. The module init function makes this file a drop-in for
// `torchstrap.kernels._C` (stubs.cpp:75-85): importing it registers the ops.
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
//
// The common case (steps in the param dtype, a bool mask, contiguous (R,)
// vectors) costs two launches: the step bump (which also writes the zero
// result) and the update. Anything else is first normalised with ATen ops.

#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <optional>
#include <string>

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

void check_vec(const at::Tensor& params, const at::Tensor& t, const char* op,
               const char* name) {
  TORCH_CHECK(t.numel() == params.size(0), op, ": ", name, " must have R = ",
              params.size(0), " elements (one per replica), got ", t.numel());
  TORCH_CHECK(t.device() == params.device(), op, ": ", name,
              " must be on ", params.device(), ", got ", t.device());
}

// The (R,) hyperparameters, in the param dtype and contiguous; a no-op in the
// normal case.
at::Tensor hyper(const at::Tensor& t, at::ScalarType dtype) {
  return t.reshape({t.numel()}).to(dtype).contiguous();
}

// Prepares state_steps and the mask. Returns the steps pointer the kernel
// reads and adds TS_BUMP_STEPS to `flags` when the bump is left to the
// launcher (same dtype, contiguous, bool mask).
struct Steps {
  at::Tensor steps;  // what the kernel reads (may alias state_steps)
  at::Tensor mask;
};

Steps prepare_steps(at::Tensor& state_steps, const at::Tensor& active_mask,
                    at::ScalarType dtype, uint32_t& flags) {
  Steps s;
  const bool fused = state_steps.scalar_type() == dtype &&
                     state_steps.is_contiguous() &&
                     active_mask.scalar_type() == at::kBool;
  if (fused) {
    s.mask = active_mask.reshape({active_mask.numel()}).contiguous();
    s.steps = state_steps;
    flags |= TS_BUMP_STEPS;
  } else {
    state_steps.add_(active_mask.to(state_steps.scalar_type()));
    s.mask = active_mask.reshape({active_mask.numel()}).to(at::kBool).contiguous();
    s.steps = hyper(state_steps, dtype);
  }
  return s;
}

void check_status(int status, const char* op) {
  TORCH_CHECK(status == 0, op, ": HIP launch failed with error ", status);
}

hipStream_t current_stream(const at::Tensor& params) {
  return c10::hip::getCurrentHIPStream(params.device().index()).stream();
}

at::Tensor adam_step_gpu(at::Tensor params, at::Tensor grads, at::Tensor exp_avgs,
                         at::Tensor exp_avg_sqs,
                         std::optional<at::Tensor> max_exp_avg_sqs,
                         at::Tensor state_steps, at::Tensor lr, at::Tensor beta1,
                         at::Tensor beta2, at::Tensor eps,
                         at::Tensor weight_decay, at::Tensor active_mask,
                         bool amsgrad, bool maximize,
                         bool decoupled_weight_decay) {
  constexpr const char* op = "torchstrap::adam_step_";
  check_params(params, op);
  TORCH_CHECK(!amsgrad || max_exp_avg_sqs.has_value(),
              "amsgrad=True requires max_exp_avg_sqs");
  check_like(params, grads, op, "grads");
  check_like(params, exp_avgs, op, "exp_avgs");
  check_like(params, exp_avg_sqs, op, "exp_avg_sqs");
  if (amsgrad) {
    check_like(params, *max_exp_avg_sqs, op, "max_exp_avg_sqs");
  }
  check_vec(params, state_steps, op, "state_steps");
  check_vec(params, lr, op, "lr");
  check_vec(params, beta1, op, "beta1");
  check_vec(params, beta2, op, "beta2");
  check_vec(params, eps, op, "eps");
  check_vec(params, weight_decay, op, "weight_decay");
  check_vec(params, active_mask, op, "active_mask");

  const c10::DeviceGuard guard(params.device());
  const auto dtype = params.scalar_type();
  const ts_dtype td = ts_dtype_of(dtype, op);
  uint32_t flags = (amsgrad ? TS_AMSGRAD : 0u) |
                   (decoupled_weight_decay ? TS_ADAMW : 0u) |
                   (maximize ? TS_MAXIMIZE : 0u);
  Steps s = prepare_steps(state_steps, active_mask, dtype, flags);
  const auto lr_c = hyper(lr, dtype);
  const auto b1_c = hyper(beta1, dtype);
  const auto b2_c = hyper(beta2, dtype);
  const auto eps_c = hyper(eps, dtype);
  const auto wd_c = hyper(weight_decay, dtype);

  ts_rt_buf bufs[5] = {rt_buf(params), rt_buf(grads), rt_buf(exp_avgs),
                       rt_buf(exp_avg_sqs), ts_rt_buf{nullptr, 0, 1}};
  if (amsgrad) {
    bufs[4] = rt_buf(*max_exp_avg_sqs);
  }
  at::Tensor out = at::empty({}, params.options());
  check_status(
      ts_adam_step(bufs, td, s.steps.data_ptr(), lr_c.data_ptr(), b1_c.data_ptr(),
                   b2_c.data_ptr(), eps_c.data_ptr(), wd_c.data_ptr(),
                   static_cast<const uint8_t*>(s.mask.data_ptr()), params.size(0),
                   params.size(1), flags, out.data_ptr(), current_stream(params)),
      op);
  return out;
}

at::Tensor sgd_step_gpu(at::Tensor params, at::Tensor grads,
                        std::optional<at::Tensor> momentum_buffers,
                        at::Tensor state_steps, at::Tensor lr,
                        at::Tensor momentum, at::Tensor dampening,
                        at::Tensor weight_decay, at::Tensor active_mask,
                        bool nesterov, bool maximize) {
  constexpr const char* op = "torchstrap::sgd_step_";
  check_params(params, op);
  TORCH_CHECK(!nesterov || momentum_buffers.has_value(),
              "nesterov=True requires momentum_buffers");
  check_like(params, grads, op, "grads");
  const bool has_buf = momentum_buffers.has_value();
  if (has_buf) {
    check_like(params, *momentum_buffers, op, "momentum_buffers");
  }
  check_vec(params, state_steps, op, "state_steps");
  check_vec(params, lr, op, "lr");
  check_vec(params, momentum, op, "momentum");
  check_vec(params, dampening, op, "dampening");
  check_vec(params, weight_decay, op, "weight_decay");
  check_vec(params, active_mask, op, "active_mask");

  const c10::DeviceGuard guard(params.device());
  const auto dtype = params.scalar_type();
  const ts_dtype td = ts_dtype_of(dtype, op);
  uint32_t flags = (nesterov ? TS_NESTEROV : 0u) | (maximize ? TS_MAXIMIZE : 0u);
  Steps s = prepare_steps(state_steps, active_mask, dtype, flags);
  const auto lr_c = hyper(lr, dtype);
  const auto mom_c = hyper(momentum, dtype);
  const auto damp_c = hyper(dampening, dtype);
  const auto wd_c = hyper(weight_decay, dtype);

  ts_rt_buf bufs[3] = {rt_buf(params), rt_buf(grads), ts_rt_buf{nullptr, 0, 1}};
  if (has_buf) {
    bufs[2] = rt_buf(*momentum_buffers);
  }
  at::Tensor out = at::empty({}, params.options());
  check_status(
      ts_sgd_step(bufs, td, s.steps.data_ptr(), lr_c.data_ptr(), mom_c.data_ptr(),
                  damp_c.data_ptr(), wd_c.data_ptr(),
                  static_cast<const uint8_t*>(s.mask.data_ptr()), params.size(0),
                  params.size(1), flags, out.data_ptr(), current_stream(params)),
      op);
  return out;
}

at::Tensor adagrad_step_gpu(at::Tensor params, at::Tensor grads,
                            at::Tensor state_sums, at::Tensor state_steps,
                            at::Tensor lr, at::Tensor lr_decay,
                            at::Tensor weight_decay, at::Tensor eps,
                            at::Tensor active_mask, bool maximize) {
  constexpr const char* op = "torchstrap::adagrad_step_";
  check_params(params, op);
  check_like(params, grads, op, "grads");
  check_like(params, state_sums, op, "state_sums");
  check_vec(params, state_steps, op, "state_steps");
  check_vec(params, lr, op, "lr");
  check_vec(params, lr_decay, op, "lr_decay");
  check_vec(params, weight_decay, op, "weight_decay");
  check_vec(params, eps, op, "eps");
  check_vec(params, active_mask, op, "active_mask");

  const c10::DeviceGuard guard(params.device());
  const auto dtype = params.scalar_type();
  const ts_dtype td = ts_dtype_of(dtype, op);
  uint32_t flags = maximize ? TS_MAXIMIZE : 0u;
  Steps s = prepare_steps(state_steps, active_mask, dtype, flags);
  const auto lr_c = hyper(lr, dtype);
  const auto lrd_c = hyper(lr_decay, dtype);
  const auto wd_c = hyper(weight_decay, dtype);
  const auto eps_c = hyper(eps, dtype);

  ts_rt_buf bufs[3] = {rt_buf(params), rt_buf(grads), rt_buf(state_sums)};
  at::Tensor out = at::empty({}, params.options());
  check_status(
      ts_adagrad_step(bufs, td, s.steps.data_ptr(), lr_c.data_ptr(),
                      lrd_c.data_ptr(), wd_c.data_ptr(), eps_c.data_ptr(),
                      static_cast<const uint8_t*>(s.mask.data_ptr()),
                      params.size(0), params.size(1), flags, out.data_ptr(),
                      current_stream(params)),
      op);
  return out;
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

}  // namespace churten

extern "C" PyObject* PyInit__C(void) {
  static struct PyModuleDef module_def = {
      PyModuleDef_HEAD_INIT, "_C", "torchstrap operators on MI355X (gfx950 HIP kernels)",
      -1, nullptr,
  };
  return PyModule_Create(&module_def);
}

"""The ``churten`` operators: the gradient scatter fused into the update.

The reference's training step scatters a per-parameter gradient dict into the
consolidated ``(N, T)`` gradient buffer, one copy per parameter, and then runs
the fused update (src/torchstrap/optimizer/grad_transform.py:29-30). These ops
(C++/HIP, churten_amd/csrc) take the per-parameter gradients directly:

* ``scatter_grads_(dst, grads, cols)`` -- the whole scatter in one launch per
  64 parameters;
* ``{adam,sgd,adagrad}_step_segments_(params, grads, cols, grads_out, ...)``
  -- the update reads each parameter's gradient where it lies; ``grads_out``
  (optional) receives the consolidated gradient on the way through. Every
  column ends up as ``scatter_grads_`` into ``grads_out`` (or into a zero
  buffer) followed by the matching ``torchstrap`` op would leave it.

``grads[i]`` is ``(N, *shape)`` and stands for columns ``cols[i] ..
cols[i] + prod(shape)`` of the layout. This module adds the fake kernels so the
ops trace under meta tensors and ``torch.compile``.
"""

from __future__ import annotations

import torch

from churten_amd.kernels import _C  # noqa: F401  (registers the ops)

scatter_grads_ = torch.ops.churten.scatter_grads_
adam_step_segments_ = torch.ops.churten.adam_step_segments_
sgd_step_segments_ = torch.ops.churten.sgd_step_segments_
adagrad_step_segments_ = torch.ops.churten.adagrad_step_segments_

__all__ = ["scatter_grads_", "adam_step_segments_", "sgd_step_segments_",
           "adagrad_step_segments_"]


@torch.library.register_fake("churten::scatter_grads_")
def _scatter_grads_fake(dst, grads, cols):
    return None


@torch.library.register_fake("churten::adam_step_segments_")
def _adam_step_segments_fake(params, grads, cols, grads_out, exp_avgs, exp_avg_sqs,
                             max_exp_avg_sqs, state_steps, lr, beta1, beta2, eps,
                             weight_decay, active_mask, amsgrad, maximize,
                             decoupled_weight_decay):
    return params.new_empty(())


@torch.library.register_fake("churten::sgd_step_segments_")
def _sgd_step_segments_fake(params, grads, cols, grads_out, momentum_buffers, state_steps,
                            lr, momentum, dampening, weight_decay, active_mask, nesterov,
                            maximize):
    return params.new_empty(())


@torch.library.register_fake("churten::adagrad_step_segments_")
def _adagrad_step_segments_fake(params, grads, cols, grads_out, state_sums, state_steps, lr,
                                lr_decay, weight_decay, eps, active_mask, maximize,
                                fp32_math=False):
    return params.new_empty(())

"""``torchstrap::adam_step_`` -- handle, fake rule and vmap rule.

The op and its GPU kernel are C++/HIP (churten_amd/csrc); this module adds the
two rules the dispatcher cannot derive, as the reference does
(src/torchstrap/kernels/adam.py:52-134): a fake kernel for meta tensors and
``torch.compile`` (a fresh 0-d tensor of the params' dtype/device), and a vmap
rule that maps an outer vmap dimension onto the replica dimension.
"""

from __future__ import annotations

import torch

from churten_amd.kernels import _C  # noqa: F401  (registers the op)
from churten_amd.kernels._consolidated import hyp, hyp_mask, lead_squeeze

adam_step_ = torch.ops.torchstrap.adam_step_

__all__ = ["adam_step_"]


@torch.library.register_fake("torchstrap::adam_step_")
def _adam_step_fake(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs,
                    state_steps, lr, beta1, beta2, eps, weight_decay,
                    active_mask, amsgrad, maximize, decoupled_weight_decay):
    return params.new_empty(())


def _adam_step_vmap(info, in_dims, params, grads, exp_avgs, exp_avg_sqs,
                    max_exp_avg_sqs, state_steps, lr, beta1, beta2, eps,
                    weight_decay, active_mask, amsgrad, maximize,
                    decoupled_weight_decay):
    p = lead_squeeze(params, in_dims[0])
    B = p.shape[0]
    mx = None if max_exp_avg_sqs is None else lead_squeeze(max_exp_avg_sqs, in_dims[4])
    out = adam_step_(
        p,
        lead_squeeze(grads, in_dims[1]),
        lead_squeeze(exp_avgs, in_dims[2]),
        lead_squeeze(exp_avg_sqs, in_dims[3]),
        mx,
        lead_squeeze(state_steps, in_dims[5]),
        hyp(lr, in_dims[6], B),
        hyp(beta1, in_dims[7], B),
        hyp(beta2, in_dims[8], B),
        hyp(eps, in_dims[9], B),
        hyp(weight_decay, in_dims[10], B),
        hyp_mask(active_mask, in_dims[11], B),
        amsgrad=amsgrad,
        maximize=maximize,
        decoupled_weight_decay=decoupled_weight_decay,
    )
    return out, None


torch.library.register_vmap("torchstrap::adam_step_", _adam_step_vmap)

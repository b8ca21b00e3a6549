"""``torchstrap::sgd_step_`` -- handle, fake rule and vmap rule.

Rules restated from the reference (src/torchstrap/kernels/sgd.py:35-103).
"""

from __future__ import annotations

import torch

from churten_amd.kernels import _C  # noqa: F401  (registers the op)
from churten_amd.kernels._consolidated import hyp, hyp_mask, lead_squeeze

sgd_step_ = torch.ops.torchstrap.sgd_step_

__all__ = ["sgd_step_"]


@torch.library.register_fake("torchstrap::sgd_step_")
def _sgd_step_fake(params, grads, momentum_buffers, state_steps, lr, momentum,
                   dampening, weight_decay, active_mask, nesterov, maximize):
    return params.new_empty(())


def _sgd_step_vmap(info, in_dims, params, grads, momentum_buffers, state_steps,
                   lr, momentum, dampening, weight_decay, active_mask, nesterov,
                   maximize):
    p = lead_squeeze(params, in_dims[0])
    B = p.shape[0]
    mb = None if momentum_buffers is None else lead_squeeze(momentum_buffers, in_dims[2])
    out = sgd_step_(
        p,
        lead_squeeze(grads, in_dims[1]),
        mb,
        lead_squeeze(state_steps, in_dims[3]),
        hyp(lr, in_dims[4], B),
        hyp(momentum, in_dims[5], B),
        hyp(dampening, in_dims[6], B),
        hyp(weight_decay, in_dims[7], B),
        hyp_mask(active_mask, in_dims[8], B),
        nesterov=nesterov,
        maximize=maximize,
    )
    return out, None


torch.library.register_vmap("torchstrap::sgd_step_", _sgd_step_vmap)

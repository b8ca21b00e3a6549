"""``torchstrap::adagrad_step_`` -- handle, fake rule and vmap rule.

Rules restated from the reference (src/torchstrap/kernels/adagrad.py:36-94).
"""

from __future__ import annotations

import torch

from churten_amd.kernels import _C  # noqa: F401  (registers the op)
from churten_amd.kernels._consolidated import hyp, hyp_mask, lead_squeeze

adagrad_step_ = torch.ops.torchstrap.adagrad_step_

__all__ = ["adagrad_step_"]


@torch.library.register_fake("torchstrap::adagrad_step_")
def _adagrad_step_fake(params, grads, state_sums, state_steps, lr, lr_decay,
                       weight_decay, eps, active_mask, maximize):
    return params.new_empty(())


def _adagrad_step_vmap(info, in_dims, params, grads, state_sums, state_steps, lr,
                       lr_decay, weight_decay, eps, active_mask, maximize):
    p = lead_squeeze(params, in_dims[0])
    B = p.shape[0]
    out = adagrad_step_(
        p,
        lead_squeeze(grads, in_dims[1]),
        lead_squeeze(state_sums, in_dims[2]),
        lead_squeeze(state_steps, in_dims[3]),
        hyp(lr, in_dims[4], B),
        hyp(lr_decay, in_dims[5], B),
        hyp(weight_decay, in_dims[6], B),
        hyp(eps, in_dims[7], B),
        hyp_mask(active_mask, in_dims[8], B),
        maximize=maximize,
    )
    return out, None


torch.library.register_vmap("torchstrap::adagrad_step_", _adagrad_step_vmap)

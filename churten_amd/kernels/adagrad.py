"""``torchstrap::adagrad_step_`` -- handle, fake rule and vmap rule.

Rules restated from the reference (src/torchstrap/kernels/adagrad.py:36-94).
``churten::adagrad_step_f32_`` (same schema) is this build's float32 variant:
the reference CPU kernel's float element math on every device instead of
ATen's fp64 device update -- bit-identical to the reference's CPU build on
float32 parameters, explicitly not to ``torch._fused_adagrad_``.
"""

from __future__ import annotations

import torch

from churten_amd.kernels import _C  # noqa: F401  (registers the op)
from churten_amd.kernels._consolidated import hyp, hyp_mask, lead_squeeze

adagrad_step_ = torch.ops.torchstrap.adagrad_step_
adagrad_step_f32_ = torch.ops.churten.adagrad_step_f32_

__all__ = ["adagrad_step_", "adagrad_step_f32_"]


@torch.library.register_fake("torchstrap::adagrad_step_")
def _adagrad_step_fake(params, grads, state_sums, state_steps, lr, lr_decay,
                       weight_decay, eps, active_mask, maximize):
    return params.new_empty(())


@torch.library.register_fake("churten::adagrad_step_f32_")
def _adagrad_step_f32_fake(params, grads, state_sums, state_steps, lr, lr_decay,
                           weight_decay, eps, active_mask, maximize):
    return params.new_empty(())


def _vmap_rule(op):
    def rule(info, in_dims, *args):
        return _adagrad_step_vmap(info, in_dims, *args, op=op)

    return rule


def _adagrad_step_vmap(info, in_dims, params, grads, state_sums, state_steps, lr,
                       lr_decay, weight_decay, eps, active_mask, maximize, op=None):
    p = lead_squeeze(params, in_dims[0])
    B = p.shape[0]
    out = (op or adagrad_step_)(
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
torch.library.register_vmap("churten::adagrad_step_f32_", _vmap_rule(adagrad_step_f32_))

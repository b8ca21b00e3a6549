"""``Adam`` -- a GradientTransformation over the consolidated state.

Restates src/torchstrap/optimizer/adam.py:18-112: ``init`` registers the
per-replica ``(N,)`` hyperparameters (floats or tensors, stored in the param
dtype), a zero ``state_steps`` counter, ``(N, T)`` moments (plus
``max_exp_avg_sqs`` under amsgrad) and the static variant flags; ``update``
issues one ``torchstrap::adam_step_`` call over the whole ensemble, and
``update_segments`` the same step with the gradient scatter fused in.
Defaults are the reference's: AdamW-style decoupled decay with
weight_decay = 1e-2.
"""

from __future__ import annotations

import torch

from churten_amd.kernels.adam import adam_step_
from churten_amd.kernels.segments import adam_step_segments_
from churten_amd.optimizer.grad_transform import GradientTransformation
from churten_amd.state import State

__all__ = ["Adam", "adam_step_"]


class Adam(metaclass=GradientTransformation):
    @classmethod
    def init(cls, state: State, *, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
             weight_decay=1e-2, amsgrad: bool = False, maximize: bool = False,
             decoupled_weight_decay: bool = True,
             state_dtype: torch.dtype | None = None) -> State:
        """``state_dtype=torch.bfloat16`` keeps the moments in bfloat16 next to
        float32 params (20 instead of 28 bytes per element and step)."""
        for key, value in (("lr", lr), ("beta1", beta1), ("beta2", beta2), ("eps", eps),
                           ("weight_decay", weight_decay), ("state_steps", 0)):
            state.add_optim_state(key, value)
        state.add_optim_state("exp_avgs", per_param=True, dtype=state_dtype)
        state.add_optim_state("exp_avg_sqs", per_param=True, dtype=state_dtype)
        if amsgrad:
            state.add_optim_state("max_exp_avg_sqs", per_param=True, dtype=state_dtype)
        state.add_optim_meta("amsgrad", amsgrad)
        state.add_optim_meta("maximize", maximize)
        state.add_optim_meta("decoupled_weight_decay", decoupled_weight_decay)
        return state

    @classmethod
    def _state_args(cls, state: State, decoupled_weight_decay=True, maximize=False,
                    amsgrad=False):
        opt = state.optimizer_state
        mx = opt.get("max_exp_avg_sqs")
        args = (
            torch.atleast_2d(opt["exp_avgs"]),
            torch.atleast_2d(opt["exp_avg_sqs"]),
            torch.atleast_2d(mx) if mx is not None else None,
            torch.atleast_1d(opt["state_steps"]),
            torch.atleast_1d(opt["lr"]),
            torch.atleast_1d(opt["beta1"]),
            torch.atleast_1d(opt["beta2"]),
            torch.atleast_1d(opt["eps"]),
            torch.atleast_1d(opt["weight_decay"]),
            torch.atleast_1d(state.active_mask),
        )
        flags = dict(
            amsgrad=bool(opt.get("amsgrad", amsgrad)),
            maximize=bool(opt.get("maximize", maximize)),
            decoupled_weight_decay=bool(opt.get("decoupled_weight_decay",
                                                decoupled_weight_decay)),
        )
        return args, flags

    @classmethod
    def update(cls, state: State, decoupled_weight_decay: bool = True, maximize: bool = False,
               amsgrad: bool = False) -> State:
        args, flags = cls._state_args(state, decoupled_weight_decay, maximize, amsgrad)
        adam_step_(torch.atleast_2d(state.flat_params), torch.atleast_2d(state.flat_grads),
                   *args, **flags)
        return state

    @classmethod
    def update_segments(cls, state: State, grads, cols, grads_out) -> State:
        """``update`` with the gradient read from the per-parameter tensors
        (``churten::adam_step_segments_``); ``grads_out`` receives the
        consolidated gradient unless it is None."""
        args, flags = cls._state_args(state)
        adam_step_segments_(torch.atleast_2d(state.flat_params), grads, cols, grads_out,
                            *args, **flags)
        return state

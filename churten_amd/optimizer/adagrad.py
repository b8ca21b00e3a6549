"""``Adagrad`` -- a GradientTransformation over the consolidated state.

Restates src/torchstrap/optimizer/adagrad.py:18-90: ``init`` registers the
``(N,)`` hyperparameters, the step counter and the ``(N, T)`` accumulator,
filled with ``initial_accumulator_value`` (pad lanes included: they never see
a gradient, so they never move the pad parameters); ``update`` issues one
``torchstrap::adagrad_step_`` call.
"""

from __future__ import annotations

import torch

from churten_amd.kernels.adagrad import adagrad_step_, adagrad_step_f32_
from churten_amd.kernels.segments import adagrad_step_segments_
from churten_amd.optimizer.grad_transform import GradientTransformation
from churten_amd.state import State

__all__ = ["Adagrad", "adagrad_step_"]


class Adagrad(metaclass=GradientTransformation):
    @classmethod
    def init(cls, state: State, *, lr=1e-2, lr_decay=0.0, weight_decay=0.0, eps=1e-10,
             initial_accumulator_value=0.0, maximize: bool = False,
             state_dtype: torch.dtype | None = None, fp32_math: bool = False) -> State:
        """``state_dtype=torch.bfloat16`` keeps the accumulators in bfloat16
        next to float32 params. ``fp32_math=True`` selects the float32 variant
        (``churten::adagrad_step_f32_``): the reference CPU kernel's float
        element math on the GPU too, not torch's fp64 device update."""
        for key, value in (("lr", lr), ("lr_decay", lr_decay), ("weight_decay", weight_decay),
                           ("eps", eps), ("state_steps", 0)):
            state.add_optim_state(key, value)
        state.add_optim_state("state_sums", per_param=True, dtype=state_dtype)
        sums = state.optimizer_state["state_sums"]
        if isinstance(initial_accumulator_value, torch.Tensor):
            sums.copy_(initial_accumulator_value.expand_as(sums))
        elif initial_accumulator_value != 0.0:
            sums.fill_(initial_accumulator_value)
        state.add_optim_meta("maximize", maximize)
        state.add_optim_meta("fp32_math", fp32_math)
        return state

    @classmethod
    def _state_args(cls, state: State, maximize=False):
        opt = state.optimizer_state
        args = (
            torch.atleast_2d(opt["state_sums"]),
            torch.atleast_1d(opt["state_steps"]),
            torch.atleast_1d(opt["lr"]),
            torch.atleast_1d(opt["lr_decay"]),
            torch.atleast_1d(opt["weight_decay"]),
            torch.atleast_1d(opt["eps"]),
            torch.atleast_1d(state.active_mask),
        )
        return args, dict(maximize=bool(opt.get("maximize", maximize)))

    @classmethod
    def update(cls, state: State, maximize: bool = False) -> State:
        args, flags = cls._state_args(state, maximize)
        op = adagrad_step_f32_ if state.optimizer_state.get("fp32_math") else adagrad_step_
        op(torch.atleast_2d(state.flat_params), torch.atleast_2d(state.flat_grads), *args,
           **flags)
        return state

    @classmethod
    def update_segments(cls, state: State, grads, cols, grads_out) -> State:
        """``update`` with the gradient read from the per-parameter tensors
        (``churten::adagrad_step_segments_``); ``grads_out`` receives the
        consolidated gradient unless it is None."""
        args, flags = cls._state_args(state)
        adagrad_step_segments_(torch.atleast_2d(state.flat_params), grads, cols, grads_out,
                               *args, fp32_math=bool(state.optimizer_state.get("fp32_math")),
                               **flags)
        return state

"""``SGD`` -- a GradientTransformation over the consolidated state.

Restates src/torchstrap/optimizer/sgd.py:17-113: ``init`` applies
torch.optim.SGD's Nesterov validation across the ensemble (non-zero momentum
somewhere and no dampening anywhere), registers the ``(N,)``
hyperparameters and the step counter, and allocates the ``(N, T)`` momentum
buffers iff any replica has non-zero momentum -- whether the buffer exists is
one call-level decision, as in ATen, while its value stays per replica. A
momentum-0 replica in a buffered call runs the momentum recursion with
momentum 0 (its buffer row is written), as the reference kernels do.
"""

from __future__ import annotations

import torch

from churten_amd.kernels.segments import sgd_step_segments_
from churten_amd.kernels.sgd import sgd_step_
from churten_amd.optimizer.grad_transform import GradientTransformation
from churten_amd.state import State

__all__ = ["SGD", "sgd_step_"]


def _any_nonzero(value) -> bool:
    return bool(torch.as_tensor(value).ne(0).any())


class SGD(metaclass=GradientTransformation):
    @classmethod
    def init(cls, state: State, *, lr=1e-3, momentum=0.0, dampening=0.0, weight_decay=0.0,
             nesterov: bool = False, maximize: bool = False,
             state_dtype: torch.dtype | None = None) -> State:
        """``state_dtype=torch.bfloat16`` keeps the momentum buffers in bfloat16
        next to float32 params."""
        if nesterov and (not _any_nonzero(momentum) or _any_nonzero(dampening)):
            raise ValueError("Nesterov momentum requires a non-zero momentum and zero dampening")
        for key, value in (("lr", lr), ("momentum", momentum), ("dampening", dampening),
                           ("weight_decay", weight_decay), ("state_steps", 0)):
            state.add_optim_state(key, value)
        has_momentum = _any_nonzero(momentum)
        if has_momentum:
            state.add_optim_state("momentum_buffers", per_param=True, dtype=state_dtype)
        state.add_optim_meta("nesterov", nesterov)
        state.add_optim_meta("maximize", maximize)
        state.add_optim_meta("has_momentum", has_momentum)
        return state

    @classmethod
    def _state_args(cls, state: State, nesterov=False, maximize=False):
        opt = state.optimizer_state
        mb = opt.get("momentum_buffers")
        args = (
            torch.atleast_1d(opt["state_steps"]),
            torch.atleast_1d(opt["lr"]),
            torch.atleast_1d(opt["momentum"]),
            torch.atleast_1d(opt["dampening"]),
            torch.atleast_1d(opt["weight_decay"]),
            torch.atleast_1d(state.active_mask),
        )
        flags = dict(nesterov=bool(opt.get("nesterov", nesterov)),
                     maximize=bool(opt.get("maximize", maximize)))
        return torch.atleast_2d(mb) if mb is not None else None, args, flags

    @classmethod
    def update(cls, state: State, nesterov: bool = False, maximize: bool = False) -> State:
        mb, args, flags = cls._state_args(state, nesterov, maximize)
        sgd_step_(torch.atleast_2d(state.flat_params), torch.atleast_2d(state.flat_grads), mb,
                  *args, **flags)
        return state

    @classmethod
    def update_segments(cls, state: State, grads, cols, grads_out) -> State:
        """``update`` with the gradient read from the per-parameter tensors
        (``churten::sgd_step_segments_``); ``grads_out`` receives the
        consolidated gradient unless it is None."""
        mb, args, flags = cls._state_args(state)
        sgd_step_segments_(torch.atleast_2d(state.flat_params), grads, cols, grads_out, mb,
                           *args, **flags)
        return state

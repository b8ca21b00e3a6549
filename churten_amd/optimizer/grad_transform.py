"""``GradientTransformation``: optimizers as classes, not instances.

Restates src/torchstrap/optimizer/grad_transform.py:10-31. A class built with
this metaclass must define ``init(state, **hyperparameters)`` (allocates the
per-replica hyperparameters and moments in the state) and ``update(state)``
(one fused operator call); ``apply_gradient(state, grads)`` scatters a per-name
gradient dict into the consolidated gradient buffer and runs ``update``.
"""

from __future__ import annotations

from typing import Any

from torch import Tensor

from churten_amd.state import State

__all__ = ["GradientTransformation"]


class GradientTransformation(type):
    def __new__(cls, name: str, bases: tuple, attrs: dict[str, Any]):
        for required in ("init", "update"):
            if required not in attrs:
                raise TypeError(
                    f"Need to define an '{required}' method to make an optimizer class!")
        return super().__new__(cls, name, bases, attrs)

    def apply_gradient(cls, state: State, grads: dict[str, Tensor]) -> State:
        state._consolidated_grads.update_(grads)
        cls.update(state)
        return state

"""``GradientTransformation``: optimizers as classes, not instances.

Restates src/torchstrap/optimizer/grad_transform.py:10-31. A class built with
this metaclass must define ``init(state, **hyperparameters)`` (allocates the
per-replica hyperparameters and moments in the state) and ``update(state)``
(one fused operator call); ``apply_gradient(state, grads)`` scatters a per-name
gradient dict into the consolidated gradient buffer and runs ``update``.

A class may also define ``update_segments(state, grads, cols, grads_out)``,
the same update reading the per-parameter gradients in place (the
``churten::*_step_segments_`` ops). ``apply_gradient`` then takes that single
fused call whenever the dict holds every parameter's gradient as an exact
``(N, *shape)`` tensor; the result, ``state.grads`` included, is the same as
the scatter followed by ``update``. ``keep_grads=False`` skips writing
``state.grads`` (it then keeps its previous contents), saving that traffic.
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

    def apply_gradient(cls, state: State, grads: dict[str, Tensor], *,
                       keep_grads: bool = True) -> State:
        # Only a class's own update_segments is trusted to match its update: a
        # subclass that overrides update takes the scatter path.
        segs = None
        if "update_segments" in cls.__dict__ and len(grads) == len(state.param_meta):
            segs = state._consolidated_grads.segments(grads)
        if segs is None:
            state._consolidated_grads.update_(grads)
            cls.update(state)
        else:
            cls.update_segments(state, *segs, state.flat_grads if keep_grads else None)
        return state

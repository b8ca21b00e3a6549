"""Consolidated ensemble state: the (N, T) layout the fused operators consume.

Restates the layout contract of the reference's ``State``
(src/torchstrap/state.py:35-66, 128-132, 135-292) without tensordict, which is
not part of this build's dependencies:

* every parameter of every replica lives in one replica-major ``(N, T)``
  buffer (row i = replica i), parameters concatenated in registration order;
* ``T`` is padded up to a multiple of ``_CONSOLIDATION_ALIGNMENT`` (4) with
  zero lanes, so each row starts 16-byte aligned and the operators take their
  vector path; the offset table never covers the pad, so no gradient ever
  reaches it and the pad stays exactly zero under every optimizer;
* an empty consolidation stays ``(N, 0)``;
* per-name ``(N, *shape)`` views alias the buffer (``params_dict``), and the
  gradient buffer is written through the same views (``_consolidated_grads``);
* optimizer hyperparameters are ``(N,)`` tensors in the parameter dtype,
  moments are ``(N, T)`` buffers, ``active_mask`` is ``(N,)`` bool.

Only what the optimizers and a training loop touch is provided: construction
from models, the flat buffers, the aliased views, the gradient scatter and the
optimizer-state registry. Tensordict features of the reference's class
(memmap, masked indexing, device moves) are outside this build's scope.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any

import torch
from torch.func import stack_module_state
from torch.nn import Module

__all__ = [
    "_CONSOLIDATION_ALIGNMENT",
    "State",
    "consolidate_params_and_buffers_dict",
    "consolidate_params_and_bufffers_dict",
    "consolidated_dict_view",
]

_CONSOLIDATION_ALIGNMENT = 4


def _cat_consolidated(flat: list[torch.Tensor], batch_size: tuple, device, dtype) -> torch.Tensor:
    """Concatenate flattened leaves into one ``(*batch_size, T)`` buffer, T
    rounded up to the alignment with zero lanes; no leaves -> ``(*batch, 0)``."""
    if not flat:
        return torch.empty((*batch_size, 0), device=device, dtype=dtype)
    raw = sum(t.shape[-1] for t in flat)
    width = raw + (-raw % _CONSOLIDATION_ALIGNMENT)
    out = torch.zeros((*batch_size, width), device=device, dtype=dtype)
    off = 0
    for t in flat:
        n = t.shape[-1]
        out[..., off : off + n].copy_(t)
        off += n
    return out


def consolidate_params_and_buffers_dict(params_and_buffers, batch_size=None, device=None,
                                        dtype=None) -> dict:
    """``{"params"|"buffers": {"storage": (N, T), "metadata": [(name, shape,
    offset, numel), ...]}}`` from stacked ``(N, *shape)`` dicts."""
    params_dict, buffers_dict = params_and_buffers
    first = next(iter(params_dict.values()))
    device = device or first.device
    dtype = dtype or first.dtype
    batch_size = tuple(batch_size or ())
    nb = len(batch_size)
    out: dict[str, dict[str, Any]] = {}
    for group, d in (("params", params_dict), ("buffers", buffers_dict)):
        meta, flat, off = [], [], 0
        for name, t in d.items():
            if tuple(t.shape[:nb]) != batch_size:
                raise ValueError(
                    f"Tensor at key={name} has incompatible shape {t.shape} for batch size "
                    f"{batch_size}")
            # The consolidated buffers are plain data: the fused operators update
            # them in place, and torch.func transforms need no autograd leaves.
            f = t.detach().reshape(*batch_size, -1)
            meta.append((name, t.shape, off, f.shape[-1]))
            flat.append(f)
            off += f.shape[-1]
        out[group] = {"metadata": meta,
                      "storage": _cat_consolidated(flat, batch_size, device, dtype)}
    return out


# The reference's spelling (state.py:69), kept so imports of it keep working.
consolidate_params_and_bufffers_dict = consolidate_params_and_buffers_dict


def consolidated_dict_view(tcons: torch.Tensor, metadata) -> dict[str, torch.Tensor]:
    """Aliased ``(N, *shape)`` views into a consolidated buffer."""
    return {name: tcons[..., off : off + n].view(*shape) for name, shape, off, n in metadata}


class _GradScatter:
    """The gradient buffer seen through per-name views; ``update_`` writes a
    per-name gradient dict into the consolidated ``(N, T)`` buffer -- in one
    ``churten::scatter_grads_`` launch when every gradient is exactly
    ``(N, *shape)`` in the buffer's dtype and device, else one ``copy_`` per
    name (which also broadcasts and converts, as the views' ``copy_`` would)."""

    def __init__(self, buffer: torch.Tensor, metadata):
        self._buffer = buffer
        self._meta = {name: (shape, off, n) for name, shape, off, n in metadata}
        self._views = consolidated_dict_view(buffer, metadata)

    def keys(self):
        return self._views.keys()

    def __getitem__(self, k):
        return self._views[k]

    def segments(self, grads: dict[str, torch.Tensor]):
        """``(tensors, cols)`` for the fused scatter, or None when some
        gradient needs the per-name path (unknown name, other shape, dtype or
        device)."""
        buf = self._buffer
        tensors, cols = [], []
        for name, g in grads.items():
            meta = self._meta.get(name)
            # meta[0] is the stacked (N, *shape)
            if (meta is None or not isinstance(g, torch.Tensor) or g.dtype != buf.dtype
                    or g.device != buf.device or tuple(g.shape) != tuple(meta[0])):
                return None
            tensors.append(g.detach())
            cols.append(meta[1])
        return tensors, cols

    def update_(self, grads: dict[str, torch.Tensor]) -> "_GradScatter":
        with torch.no_grad():
            segs = self.segments(grads) if self._buffer.dim() == 2 else None
            if segs is not None:
                from churten_amd.kernels.segments import scatter_grads_

                scatter_grads_(self._buffer, *segs)
            else:
                for name, g in grads.items():
                    self._views[name].copy_(g)
        return self


class State:
    """Replica-major consolidated state of an N-replica ensemble."""

    def __init__(self, params: torch.Tensor, buffers: torch.Tensor, param_meta, buffer_meta,
                 param_buffer_dtype: torch.dtype | None = None,
                 optimizer_state: dict | None = None,
                 active_mask: torch.Tensor | None = None, grads: torch.Tensor | None = None):
        self.params = params
        self.buffers = buffers
        self.param_meta = list(param_meta)
        self.buffer_meta = list(buffer_meta)
        self.param_buffer_dtype = param_buffer_dtype or params.dtype
        self.optimizer_state: dict[str, Any] = dict(optimizer_state or {})
        self.batch_size = torch.Size(params.shape[:1])
        self.device = params.device
        self.active_mask = (active_mask if active_mask is not None
                            else torch.ones(self.batch_size, dtype=torch.bool, device=self.device))
        self.grads = grads if grads is not None else torch.zeros_like(params)

    @classmethod
    def from_models(cls, modules: Sequence[Module]) -> "State":
        batch = (len(modules),)
        cons = consolidate_params_and_buffers_dict(stack_module_state(list(modules)),
                                                   batch_size=batch)
        params = cons["params"]["storage"]
        return cls(params=params, buffers=cons["buffers"]["storage"],
                   param_meta=cons["params"]["metadata"],
                   buffer_meta=cons["buffers"]["metadata"], param_buffer_dtype=params.dtype)

    # -- views -------------------------------------------------------------
    @property
    def flat_params(self) -> torch.Tensor:
        return self.params

    @property
    def flat_grads(self) -> torch.Tensor:
        return self.grads

    @property
    def params_dict(self) -> dict[str, torch.Tensor]:
        return consolidated_dict_view(self.params, self.param_meta)

    @property
    def buffers_dict(self) -> dict[str, torch.Tensor]:
        return consolidated_dict_view(self.buffers, self.buffer_meta)

    @property
    def _consolidated_grads(self) -> _GradScatter:
        return _GradScatter(self.grads, self.param_meta)

    # -- optimizer state ---------------------------------------------------
    def add_optim_state(self, key: str, value: Any = None, per_param: bool = False,
                        dtype: torch.dtype | None = None) -> None:
        self.optimizer_state[key] = self.like_tensor(value, per_param=per_param, dtype=dtype)

    def add_optim_meta(self, key: str, value: Any) -> None:
        """A static, non-tensor optimizer flag (amsgrad, maximize, ...)."""
        self.optimizer_state[key] = value

    def like_tensor(self, value: Any = None, per_param: bool = False,
                    dtype: torch.dtype | None = None) -> torch.Tensor:
        """``(N,)`` (or ``(N, T)`` if ``per_param``) tensor in the param dtype:
        zeros for None, filled for a number, broadcast copy of a tensor. A
        ``per_param`` buffer may take another ``dtype`` (bfloat16 optimizer
        state next to float32 params)."""
        like = dict(dtype=self.param_buffer_dtype, device=self.device)
        if per_param:
            out = torch.zeros_like(self.flat_params, dtype=dtype or self.param_buffer_dtype,
                                   memory_format=torch.preserve_format)
            if isinstance(value, torch.Tensor):
                out.copy_(torch.as_tensor(value, **like).expand_as(out))
            elif value is not None:
                out.fill_(value)
            return out
        if value is None:
            return torch.zeros(self.batch_size, **like)
        if isinstance(value, torch.Tensor):
            return torch.as_tensor(value, **like).expand(self.batch_size).clone()
        return torch.full(self.batch_size, fill_value=value, **like)

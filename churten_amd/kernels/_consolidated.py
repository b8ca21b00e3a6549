"""Reshaping helpers shared by the operators' ``register_vmap`` rules.

Rule restated from the reference (src/torchstrap/kernels/_consolidated.py:25-44):
an outer ``torch.func.vmap`` dimension is treated as the replica dimension.
Callers step single-replica state inside the vmapped function, so the
consolidated buffers arrive as ``(B, 1, T)`` (or ``(B, T)``) and the (R,)
inputs as ``(B, 1)`` / ``(B,)``; the batch dim is moved to the front and a
singleton replica dim squeezed, giving the kernels a plain ``(R=B, T)`` call.
Moving a batch dim other than 0 to the front yields a strided view, which the
element path of the kernels handles.
"""

from __future__ import annotations

import torch

__all__ = ["lead_squeeze", "hyp", "hyp_mask"]


def lead_squeeze(t: torch.Tensor, d: int | None) -> torch.Tensor:
    """Batch dim to the front, then drop a singleton replica dim behind it."""
    if d is None:
        return t
    out = torch.movedim(t, d, 0)
    if out.dim() >= 2 and out.size(1) == 1:
        out = out.squeeze(1)
    return out


def hyp(t: torch.Tensor, d: int | None, batch_size: int) -> torch.Tensor:
    """An (R,) input under vmap: batched -> ``lead_squeeze``; an unbatched
    scalar is broadcast to ``batch_size``; an unbatched vector is kept."""
    if d is not None:
        return lead_squeeze(t, d)
    if t.dim() == 0:
        return t.expand(batch_size)
    return t


def hyp_mask(t: torch.Tensor, d: int | None, batch_size: int) -> torch.Tensor:
    """``hyp`` for the active mask, which the kernels read as bool."""
    return hyp(t, d, batch_size).to(dtype=torch.bool)

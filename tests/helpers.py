"""Runs the parity cases of tests/golden/cases.py through the product.

``run_hip(case)`` moves a case's numpy inputs to the GPU, calls the
``torch.ops.torchstrap.*_step_`` operators (HIP kernels) once per gradient and
returns the outputs as numpy arrays, so they can be compared with the C oracle
and with the golden vectors.
"""

from __future__ import annotations

import numpy as np
import torch

import cases as C


def to_layout(a: np.ndarray, dev, strided: bool) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    if not strided:
        return t
    R, T = a.shape
    backing = torch.empty(T, R, dtype=t.dtype, device=dev).t()
    backing.copy_(t)
    return backing


STATE_NAMES = ("m", "v", "mx", "mb", "s")


def to_layout_tensor(t: torch.Tensor, strided: bool) -> torch.Tensor:
    """The same values in a transposed-backing (R, T) view when ``strided``."""
    if not strided:
        return t
    R, T = t.shape
    backing = torch.empty(T, R, dtype=t.dtype, device=t.device).t()
    backing.copy_(t)
    return backing


def run_hip(c, strided: bool = False, dev: str = "cuda", state_bf16: bool = False,
            state_dtype=None, adagrad_f32: bool = False):
    """``state_bf16``: the case's optimizer state starts bfloat16-valued and is
    held in bfloat16 tensors (params and grads stay float32), unless
    ``state_dtype`` names another dtype for those tensors. Outputs are returned
    widened to float32. ``adagrad_f32`` runs Adagrad cases through the float32
    variant ``churten::adagrad_step_f32_``."""
    import churten_amd.kernels  # noqa: F401

    x = C.make_inputs(c, state_bf16)
    names = C.state_names(c, x)
    st = {k: to_layout(x[k], dev, strided) for k in names}
    if state_bf16 and state_dtype in (None, torch.bfloat16):
        for k in names:
            if k in STATE_NAMES:
                t = st[k].to(torch.bfloat16)
                st[k] = t if not strided else to_layout_tensor(t, strided)

    def vec(k):
        return torch.from_numpy(x[k].copy()).to(dev)

    mask = torch.from_numpy(x["mask"].copy()).to(dev)
    steps = vec("steps")
    ops = torch.ops.torchstrap
    for g in x["grads"]:
        gt = to_layout(g, dev, strided)
        if c["op"] == "adam":
            ops.adam_step_(st["p"], gt, st["m"], st["v"], st.get("mx"), steps, vec("lr"),
                           vec("beta1"), vec("beta2"), vec("eps"), vec("wd"), mask,
                           amsgrad=c["amsgrad"], maximize=c["maximize"],
                           decoupled_weight_decay=c["decoupled"])
        elif c["op"] == "sgd":
            ops.sgd_step_(st["p"], gt, st.get("mb"), steps, vec("lr"), vec("momentum"),
                          vec("dampening"), vec("wd"), mask, nesterov=c["nesterov"],
                          maximize=c["maximize"])
        else:
            fn = torch.ops.churten.adagrad_step_f32_ if adagrad_f32 else ops.adagrad_step_
            fn(st["p"], gt, st["s"], steps, vec("lr"), vec("lr_decay"), vec("wd"), vec("eps"),
               mask, maximize=c["maximize"])
    if torch.device(dev).type == "cuda":
        torch.cuda.synchronize()
    out = {k: st[k].float().contiguous().cpu().numpy() for k in names}
    out["steps"] = steps.cpu().numpy()
    return out


def mismatch(a: np.ndarray, b: np.ndarray) -> str:
    """Human-readable summary of where two float32 arrays differ."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    ne = a.view(np.uint32) != b.view(np.uint32)
    if not ne.any():
        return "identical"
    idx = np.argwhere(ne)
    diff = np.abs(a.astype(np.float64) - b.astype(np.float64))
    return (f"{int(ne.sum())}/{a.size} differ; first at {tuple(idx[0])}: "
            f"{a[tuple(idx[0])]!r} vs {b[tuple(idx[0])]!r}; max abs diff {diff.max():.3e}")

"""Deterministic parity cases shared by the golden-vector scripts and the tests.

A case is a small dict: the operator, (R, T), its flags, a seed, the
hyperparameter pattern, the freeze pattern, the starting step and the number of
steps. ``make_inputs`` expands it with numpy's PCG64 (bit-reproducible on every
platform) into float32 state, per-replica vectors and one gradient per step;
the golden files store only the case, a SHA-256 digest of every output array
and, for small cases, the arrays themselves.
"""

from __future__ import annotations

import hashlib
import itertools

import numpy as np

F32 = np.float32


def f32(x: float) -> float:
    return float(np.float32(x))


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f4").tobytes()).hexdigest()


# ---------------------------------------------------------------------------
# case lists
# ---------------------------------------------------------------------------
# T values: 45 (ragged: T % 4 and T % 8 != 0), 52 (T % 4 == 0, AVX2 tail of 4),
# 64 (no tail anywhere), 1000 (tail of 0 on 8 lanes, > one GPU tile row? no),
# 16397 (crosses the CPU 16384-element chunk and several GPU tiles, ragged).
_TS = (45, 52, 64, 1000)


def adam_cases():
    out = []
    for T, ams, mx, dec, wd in itertools.product(_TS, (False, True), (False, True),
                                                  (False, True), (0.0, 1e-2)):
        out.append(dict(op="adam", R=3, T=T, amsgrad=ams, maximize=mx,
                        decoupled=dec, wd=wd, hypers="distinct", mask="one_frozen",
                        steps0=0, nsteps=3, seed=len(out)))
    # step-0 freeze, late steps, big ragged row
    out.append(dict(op="adam", R=4, T=16397, amsgrad=True, maximize=False, decoupled=True,
                    wd=1e-2, hypers="distinct", mask="one_frozen", steps0=0, nsteps=2,
                    seed=1001))
    out.append(dict(op="adam", R=4, T=45, amsgrad=False, maximize=False, decoupled=False,
                    wd=1e-2, hypers="distinct", mask="one_frozen", steps0=250, nsteps=2,
                    seed=1002))
    return out


def sgd_cases():
    out = []
    for T, mom, damp, wd, nest, mx in itertools.product(_TS, (0.0, 0.9), (0.0, 0.3),
                                                        (0.0, 1e-2), (False, True),
                                                        (False, True)):
        if nest and mom == 0.0:  # nesterov needs momentum buffers
            continue
        out.append(dict(op="sgd", R=3, T=T, momentum=mom, dampening=damp, wd=wd,
                        nesterov=nest, maximize=mx, hypers="uniform", mask="one_frozen",
                        steps0=0, nsteps=3, seed=2000 + len(out)))
    # per-replica momentum incl. a momentum-0 replica inside a buffered call
    out.append(dict(op="sgd", R=4, T=1000, momentum="mixed", dampening=0.1, wd=1e-2,
                    nesterov=False, maximize=False, hypers="distinct", mask="one_frozen",
                    steps0=0, nsteps=3, seed=2901))
    out.append(dict(op="sgd", R=4, T=16397, momentum="mixed", dampening=0.0, wd=0.0,
                    nesterov=True, maximize=False, hypers="distinct", mask="one_frozen",
                    steps0=0, nsteps=2, seed=2902))
    # BASELINE config 3's flags: per-replica momentum {0, .5, .9, .99}, dampening
    # 0.1 with nesterov, some replicas on their first step and some not
    out.append(dict(op="sgd", R=6, T=1001, momentum="mixed", dampening=0.1, wd=0.0,
                    nesterov=True, maximize=False, hypers="distinct", mask="one_frozen",
                    steps0=[0, 3, 0, 7, 1, 0], nsteps=3, seed=2903))
    out.append(dict(op="sgd", R=6, T=52, momentum="mixed", dampening=0.1, wd=1e-2,
                    nesterov=True, maximize=True, hypers="distinct", mask="one_frozen",
                    steps0=[2, 0, 0, 5, 0, 1], nsteps=2, seed=2904))
    return out


def adagrad_cases():
    out = []
    for T, lrd, wd, eps, mx in itertools.product(_TS, (0.0, 1e-2), (0.0, 1e-2),
                                                 (1e-10, 1e-6), (False, True)):
        out.append(dict(op="adagrad", R=3, T=T, lr_decay=lrd, wd=wd, eps=eps,
                        maximize=mx, hypers="distinct", mask="one_frozen", steps0=0,
                        nsteps=3, seed=3000 + len(out)))
    out.append(dict(op="adagrad", R=4, T=16397, lr_decay=1e-4, wd=1e-4, eps=1e-10,
                    maximize=False, hypers="distinct", mask="one_frozen", steps0=120,
                    nsteps=2, seed=3901))
    return out


def all_cases():
    return adam_cases() + sgd_cases() + adagrad_cases()


def dtype_cases():
    """Cases replayed in float64, float16 and bfloat16: each optimizer's whole
    flag matrix at T = 45 (ragged) and T = 1000, plus every special case (the
    16397-element rows that cross the CPU chunk, late steps, per-replica
    momentum with a momentum-0 replica inside a buffered call, first steps)."""
    return [c for c in all_cases() if c["T"] not in (52, 64)]


def digest_bytes(a) -> str:
    """SHA-256 of an array's raw bytes in its own dtype (numpy array, or a torch
    tensor of any dtype, bfloat16 included), tagged with the dtype name."""
    if hasattr(a, "numpy"):
        import torch

        tag = str(a.dtype).replace("torch.", "")
        raw = a.detach().contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()
    else:
        tag, raw = str(a.dtype), np.ascontiguousarray(a).tobytes()
    return tag + ":" + hashlib.sha256(raw).hexdigest()


def case_id(c) -> str:
    keys = [k for k in c if k not in ("op",)]
    return c["op"] + "-" + "-".join(f"{k}={c[k]}" for k in keys)


# ---------------------------------------------------------------------------
# inputs
# ---------------------------------------------------------------------------
def _mask(c, R):
    m = np.ones(R, dtype=bool)
    if c["mask"] == "one_frozen" and R > 1:
        m[1] = False
    return m


def to_bf16_values(a: np.ndarray) -> np.ndarray:
    """float32 array of the nearest-even bfloat16 values of ``a`` (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=F32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(F32)


def make_inputs(c, state_bf16=False):
    """All inputs of a case as float32 numpy arrays (state is (R, T)). With
    ``state_bf16`` the optimizer-state arrays start bfloat16-representable."""
    x = _make_inputs(c)
    if state_bf16:
        for k in ("m", "v", "mx", "mb", "s"):
            if x.get(k) is not None:
                x[k] = to_bf16_values(x[k])
    return x


def _make_inputs(c):
    rng = np.random.Generator(np.random.PCG64(c["seed"]))
    R, T = c["R"], c["T"]

    def n(*shape, scale=1.0):
        return (rng.standard_normal(shape) * scale).astype(F32)

    s0 = c["steps0"]  # one starting step for every replica, or one per replica
    steps = (np.array(s0, dtype=F32) if isinstance(s0, (list, tuple))
             else np.full(R, s0, dtype=F32))
    x = {"mask": _mask(c, R), "steps": steps}
    x["p"] = n(R, T)
    if c["op"] == "adam":
        x["m"] = np.abs(n(R, T))
        x["v"] = np.abs(n(R, T))
        x["mx"] = np.abs(n(R, T)) if c["amsgrad"] else None
        if c["hypers"] == "distinct":
            x["lr"] = np.linspace(1e-3, 5e-2, R, dtype=F32)
            x["beta1"] = np.linspace(0.80, 0.95, R, dtype=F32)
            x["beta2"] = np.linspace(0.990, 0.9999, R, dtype=F32)
            x["eps"] = np.linspace(1e-9, 1e-7, R, dtype=F32)
        else:
            x["lr"] = np.full(R, 1e-2, F32)
            x["beta1"] = np.full(R, 0.9, F32)
            x["beta2"] = np.full(R, 0.999, F32)
            x["eps"] = np.full(R, 1e-8, F32)
        x["wd"] = np.full(R, c["wd"], F32)
    elif c["op"] == "sgd":
        mom = c["momentum"]
        if mom == "mixed":
            x["momentum"] = np.array(([0.0, 0.5, 0.9, 0.99] * 2)[:R] + [0.9] * max(0, R - 8),
                                     F32)
        else:
            x["momentum"] = np.full(R, mom, F32)
        has_buf = bool(np.any(x["momentum"] != 0))
        x["mb"] = n(R, T) if has_buf else None
        x["lr"] = (np.linspace(1e-3, 5e-2, R, dtype=F32) if c["hypers"] == "distinct"
                   else np.full(R, 1e-2, F32))
        x["dampening"] = np.full(R, c["dampening"], F32)
        x["wd"] = np.full(R, c["wd"], F32)
    else:
        x["s"] = np.abs(n(R, T))
        x["lr"] = (np.linspace(1e-3, 5e-2, R, dtype=F32) if c["hypers"] == "distinct"
                   else np.full(R, 1e-2, F32))
        x["lr_decay"] = np.full(R, c["lr_decay"], F32)
        x["wd"] = np.full(R, c["wd"], F32)
        x["eps"] = np.full(R, c["eps"], F32)
    x["grads"] = [n(R, T) for _ in range(c["nsteps"])]
    return x


def state_names(c, x):
    if c["op"] == "adam":
        return ["p", "m", "v"] + (["mx"] if c["amsgrad"] else [])
    if c["op"] == "sgd":
        return ["p"] + (["mb"] if x["mb"] is not None else [])
    return ["p", "s"]


def run_oracle(c, form, unit_stride=True, state_bf16=False):
    """Runs the case through the C oracle; returns {name: array} incl. steps.
    ``state_bf16``: bfloat16 optimizer state next to float32 params."""
    from oracle import oracle as O

    x = make_inputs(c, state_bf16)
    kw = dict(unit_stride=unit_stride, state_bf16=state_bf16)
    for g in x["grads"]:
        if c["op"] == "adam":
            O.adam_step(form, x["p"], g, x["m"], x["v"], x["mx"], x["steps"], x["lr"],
                        x["beta1"], x["beta2"], x["eps"], x["wd"], x["mask"],
                        amsgrad=c["amsgrad"], maximize=c["maximize"],
                        decoupled_weight_decay=c["decoupled"], **kw)
        elif c["op"] == "sgd":
            O.sgd_step(form, x["p"], g, x["mb"], x["steps"], x["lr"], x["momentum"],
                       x["dampening"], x["wd"], x["mask"], nesterov=c["nesterov"],
                       maximize=c["maximize"], **kw)
        else:
            O.adagrad_step(form, x["p"], g, x["s"], x["steps"], x["lr"], x["lr_decay"],
                           x["wd"], x["eps"], x["mask"], maximize=c["maximize"], **kw)
    out = {k: x[k] for k in state_names(c, x)}
    out["steps"] = x["steps"]
    return out

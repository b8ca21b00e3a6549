"""TEST INFRASTRUCTURE ONLY -- ctypes front end of oracle/liboracle.so.

The C file (optim_oracle.c) restates the reference's fused optimizer step in
two formulations: ``DEVICE`` (the element math of the reference's GPU kernels,
in torch's ROCm form -- the HIP kernels must match it bit for bit) and ``CPU``
(the reference's own CPU kernels, src/torchstrap/kernels/csrc/cpu/*.cpp -- the
HIP kernels must agree within atol = rtol = 1e-5). All arrays are numpy
float32, C-contiguous, (R, T) for state and (R,) for the per-replica inputs;
``mask`` is (R,) bool. Everything is updated in place, ``steps`` included
(steps += mask first, as the reference operators do).

``state_bf16=True`` models bfloat16 optimizer state next to float32 params:
the state arrays hold bfloat16-representable float32 values, the float32 step
runs, then the active rows' state is rounded to nearest-even bfloat16.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "torchstrap_ref_C.so"

DEVICE = 0
CPU = 1

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        f = ctypes.c_void_p
        i64 = ctypes.c_int64
        ci = ctypes.c_int
        lib.oracle_adam_step.argtypes = [ci] + [f] * 12 + [i64, i64, ci, ci, ci, ci]
        lib.oracle_sgd_step.argtypes = [ci] + [f] * 9 + [i64, i64, ci, ci, ci]
        lib.oracle_adagrad_step.argtypes = [ci] + [f] * 9 + [i64, i64, ci, ci]
        lib.oracle_round_bf16_rows.argtypes = [f, f, i64, i64]
        for fn in (lib.oracle_adam_step, lib.oracle_sgd_step, lib.oracle_adagrad_step,
                   lib.oracle_round_bf16_rows):
            fn.restype = ci
        _lib = lib
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.dtype in (np.float32, np.uint8) and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data


def _mask(mask):
    return np.ascontiguousarray(mask, dtype=np.uint8)


def round_bf16_rows(x, mask):
    """Round the rows of (R, T) float32 ``x`` selected by ``mask`` to bfloat16."""
    R, T = x.shape
    assert _load().oracle_round_bf16_rows(_ptr(x), _ptr(_mask(mask)), R, T) == 0


def _round_state(state, mask):
    for s in state:
        if s is not None:
            round_bf16_rows(s, mask)


def adam_step(form, p, g, m, v, mx, steps, lr, beta1, beta2, eps, weight_decay,
              mask, amsgrad=False, maximize=False, decoupled_weight_decay=True,
              unit_stride=True, state_bf16=False):
    R, T = p.shape
    mk = _mask(mask)
    rc = _load().oracle_adam_step(
        form, _ptr(p), _ptr(g), _ptr(m), _ptr(v), _ptr(mx if amsgrad else None),
        _ptr(steps), _ptr(lr), _ptr(beta1), _ptr(beta2), _ptr(eps),
        _ptr(weight_decay), _ptr(mk), R, T, int(amsgrad),
        int(decoupled_weight_decay), int(maximize), int(unit_stride))
    assert rc == 0
    if state_bf16:
        _round_state((m, v, mx if amsgrad else None), mk)


def sgd_step(form, p, g, mb, steps, lr, momentum, dampening, weight_decay,
             mask, nesterov=False, maximize=False, unit_stride=True, state_bf16=False):
    R, T = p.shape
    mk = _mask(mask)
    rc = _load().oracle_sgd_step(
        form, _ptr(p), _ptr(g), _ptr(mb), _ptr(steps), _ptr(lr), _ptr(momentum),
        _ptr(dampening), _ptr(weight_decay), _ptr(mk), R, T, int(nesterov),
        int(maximize), int(unit_stride))
    if rc != 0:
        raise RuntimeError("nesterov=True requires momentum_buffers")
    if state_bf16:
        _round_state((mb,), mk)


def adagrad_step(form, p, g, s, steps, lr, lr_decay, weight_decay, eps, mask,
                 maximize=False, unit_stride=True, state_bf16=False):
    R, T = p.shape
    mk = _mask(mask)
    rc = _load().oracle_adagrad_step(
        form, _ptr(p), _ptr(g), _ptr(s), _ptr(steps), _ptr(lr), _ptr(lr_decay),
        _ptr(weight_decay), _ptr(eps), _ptr(mk), R, T, int(maximize),
        int(unit_stride))
    assert rc == 0
    if state_bf16:
        _round_state((s,), mk)

"""bfloat16 optimizer state next to float32 parameters.

An extension of the operators (the reference rejects mixed dtypes; its README
roadmap lists low-precision optimizer state): exp_avgs / exp_avg_sqs /
max_exp_avg_sqs, momentum_buffers or state_sums may be bfloat16 while params
and grads are float32. The step is the float32 step on the widened state, and
the state is rounded to nearest-even bfloat16 when stored.

Pinning: the oracle's rounding is checked against torch's own float ->
bfloat16 conversion; on the GPU the HIP kernels must equal the oracle bit for
bit, and a single step must equal the float32 path (itself bit-exact to
torch's fused kernels) followed by that rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import cases as C
import churten_amd.kernels as K
from helpers import mismatch, run_hip
from oracle import oracle as O

CASES = C.all_cases()
SUBSET = CASES[::5]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bit_equal(got, want):
    for k in want:
        assert np.array_equal(bits(got[k]), bits(want[k])), f"{k}: {mismatch(got[k], want[k])}"


# ---------------------------------------------------------------------------
# oracle pinning (CPU)
# ---------------------------------------------------------------------------
def _torch_bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()


def test_oracle_rounding_matches_torch_conversion():
    rng = np.random.Generator(np.random.PCG64(0))
    pats = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    hi = rng.integers(0, 2**16, size=4096, dtype=np.uint64).astype(np.uint32) << 16
    special = np.concatenate([
        hi | 0x8000,                      # exact ties, even and odd upper halves
        hi | 0x7FFF, hi | 0x8001,         # either side of a tie
        np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00001, 0xFFFFFFFF,
                  0x00000001, 0x80008000, 0x00008000, 0x00018000, 0x0], dtype=np.uint32),
    ])
    x = np.concatenate([pats, special]).view(np.float32).reshape(1, -1)
    got = x.copy()
    O.round_bf16_rows(got, np.ones(1, bool))
    want = _torch_bf16(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.all(bits(got)[nan] == 0x7FC00000)


def test_oracle_rounds_active_rows_only():
    x = np.full((3, 5), 1.00390625, np.float32)  # exactly between two bfloat16 values
    O.round_bf16_rows(x, np.array([True, False, True]))
    assert np.all(x[[0, 2]] == 1.0) and np.all(x[1] == 1.00390625)


def test_case_state_values_are_bf16():
    x = C.make_inputs(CASES[0], state_bf16=True)
    for k in ("m", "v"):
        assert np.array_equal(bits(x[k]), bits(_torch_bf16(x[k])))


# ---------------------------------------------------------------------------
# CPU key
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("c", SUBSET, ids=C.case_id)
def test_cpu_bf16_state_bit_exact_to_cpu_oracle(c):
    got = run_hip(c, dev="cpu", state_bf16=True)
    want = C.run_oracle(c, O.CPU, state_bf16=True)
    assert_bit_equal(got, want)


def test_mixed_state_dtypes_rejected():
    R, T = 2, 8
    p, g = torch.zeros(R, T), torch.zeros(R, T)
    vec = [torch.zeros(R)] + [torch.full((R,), x) for x in (1e-3, 0.9, 0.999, 1e-8, 0.0)]
    mask = torch.ones(R, dtype=torch.bool)
    bf = torch.zeros(R, T, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="bfloat16"):
        K.adam_step_(p, g, bf, torch.zeros(R, T), None, *vec, mask, amsgrad=False,
                     maximize=False, decoupled_weight_decay=True)
    with pytest.raises(RuntimeError):
        K.adam_step_(p.double(), g.double(), bf, bf.clone(), None, *vec, mask, amsgrad=False,
                     maximize=False, decoupled_weight_decay=True)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=C.case_id)
def test_hip_bf16_state_bit_exact_to_device_oracle(c):
    got = run_hip(c, state_bf16=True)
    want = C.run_oracle(c, O.DEVICE, state_bf16=True)
    assert_bit_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("c", SUBSET, ids=C.case_id)
def test_hip_bf16_state_strided_bit_exact(c):
    got = run_hip(c, strided=True, state_bf16=True)
    want = C.run_oracle(c, O.DEVICE, state_bf16=True)
    assert_bit_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=C.case_id)
def test_hip_bf16_state_is_float32_step_then_rounding(c):
    """One step: params equal the float32 path's (bit-exact to torch's fused
    kernels elsewhere) from the same bfloat16-valued state, and the stored state
    is the float32 path's state rounded to bfloat16."""
    c1 = dict(c, nsteps=1)
    mixed = run_hip(c1, state_bf16=True)
    full = run_hip(c1, state_bf16=True, state_dtype=torch.float32)
    for k, want in full.items():
        if k in ("m", "v", "mx", "mb", "s"):
            want = _torch_bf16(want)  # frozen rows are bfloat16-valued already
        assert np.array_equal(bits(mixed[k]), bits(want)), f"{k}: {mismatch(mixed[k], want)}"

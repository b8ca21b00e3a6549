"""The float32 Adagrad variant (``churten::adagrad_step_f32_``).

ATen's device Adagrad runs its update in fp64 (fused_adagrad_utils.cuh:16-50);
the reference keeps that for bit-exactness and names a float32 variant, "sold as
such and not bit-exact", as a separate feature (test/optimizer/bench_adagrad.py
docstring). This build's variant runs the element loop of the reference's CPU
kernel (cpu/adagrad.cpp:94-156) on every device, so it is pinned bit for bit to
the oracle's CPU formulation -- itself bit-exact to the compiled reference CPU
build -- and stays within float32 rounding of the fp64 device update.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import cases as C
import churten_amd.kernels as K
from churten_amd.optimizer import Adagrad
from helpers import mismatch, run_hip
from oracle import oracle as O

CASES = C.adagrad_cases()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bit_equal(got, want):
    for k in want:
        assert np.array_equal(bits(got[k]), bits(want[k])), f"{k}: {mismatch(got[k], want[k])}"


def test_schema_is_the_reference_adagrad_schema():
    ref = str(torch.ops.torchstrap.adagrad_step_.default._schema)
    got = str(torch.ops.churten.adagrad_step_f32_.default._schema)
    assert got == ref.replace("torchstrap::adagrad_step_", "churten::adagrad_step_f32_")


@pytest.mark.parametrize("c", CASES[::3], ids=C.case_id)
def test_cpu_variant_bit_exact_to_cpu_oracle(c):
    assert_bit_equal(run_hip(c, dev="cpu", adagrad_f32=True), C.run_oracle(c, O.CPU))


def test_float64_params_rejected():
    R, T = 2, 8
    d = dict(dtype=torch.float64)
    args = [torch.zeros(R, T, **d) for _ in range(3)] + [torch.zeros(R, **d)] + [
        torch.full((R,), x, **d) for x in (1e-2, 0.0, 0.0, 1e-10)]
    with pytest.raises(RuntimeError, match="float64"):
        K.adagrad_step_f32_(*args, torch.ones(R, dtype=torch.bool), maximize=False)


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=C.case_id)
def test_hip_variant_bit_exact_to_cpu_oracle(c):
    assert_bit_equal(run_hip(c, adagrad_f32=True), C.run_oracle(c, O.CPU))


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES[::2], ids=C.case_id)
def test_hip_variant_strided_and_bf16_state(c):
    assert_bit_equal(run_hip(c, strided=True, adagrad_f32=True), C.run_oracle(c, O.CPU))
    assert_bit_equal(run_hip(c, adagrad_f32=True, state_bf16=True),
                     C.run_oracle(c, O.CPU, state_bf16=True))


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=C.case_id)
def test_hip_variant_close_to_fp64_device_update(c):
    got = run_hip(c, adagrad_f32=True)
    want = run_hip(c)
    for k in want:
        np.testing.assert_allclose(got[k], want[k], rtol=2e-6, atol=1e-7, err_msg=k)


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
def test_adagrad_fp32_math_through_apply_gradient(device):
    """fp32_math=True end to end, fused gradient path included; GPU and CPU
    states agree bit for bit (both run the CPU kernel's float math)."""
    torch.manual_seed(0)
    net = torch.nn.Sequential(torch.nn.Linear(5, 7), torch.nn.Tanh(), torch.nn.Linear(7, 1))
    from churten_amd.state import State

    out = {}
    for dev in ("cpu", device):
        state = State.from_models([net, net, net])
        state.params = state.params.to(dev)
        state.grads = state.grads.to(dev)
        state.device = torch.device(dev)
        state.active_mask = state.active_mask.to(dev)
        Adagrad.init(state, lr=5e-2, lr_decay=1e-3, weight_decay=1e-3,
                     initial_accumulator_value=0.1, fp32_math=True)
        g = torch.Generator().manual_seed(3)
        for _ in range(4):
            grads = {name: torch.randn(*shape, generator=g).to(dev)
                     for name, shape, _, _ in state.param_meta}
            Adagrad.apply_gradient(state, grads)
        out[dev] = state
    assert out["cpu"].optimizer_state["fp32_math"] is True
    if device != "cpu":
        a, b = out["cpu"], out[device]
        assert torch.equal(a.params, b.params.cpu())
        assert torch.equal(a.optimizer_state["state_sums"], b.optimizer_state["state_sums"].cpu())

"""HIP kernels against the C oracle, on every parity case.

Bar (from the operator's contract): every element of every active replica is
bit-identical to the device formulation -- torch's ROCm fused math, which the
reference's GPU kernels run -- and within atol = rtol = 1e-5 of the reference's
CPU kernels (the CPU formulation). Frozen rows and the step counters are
covered by the same comparisons (the oracle leaves frozen rows as they were).
"""

from __future__ import annotations

import numpy as np
import pytest

import cases as C
from helpers import mismatch, run_hip
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CASES = C.all_cases()
CPU_TOL = 1e-5


@pytest.mark.parametrize("c", CASES, ids=C.case_id)
def test_hip_bit_exact_to_device_oracle(c):
    got = run_hip(c)
    want = C.run_oracle(c, O.DEVICE)
    for k in want:
        assert np.array_equal(got[k].view(np.uint32), want[k].view(np.uint32)), (
            f"{k}: {mismatch(got[k], want[k])}")


@pytest.mark.parametrize("c", CASES[::4], ids=C.case_id)
def test_strided_layout_bit_exact(c):
    """A transposed (R, T) view takes the element path; same bits per element."""
    got = run_hip(c, strided=True)
    want = C.run_oracle(c, O.DEVICE)
    for k in want:
        assert np.array_equal(got[k].view(np.uint32), want[k].view(np.uint32)), (
            f"{k}: {mismatch(got[k], want[k])}")


@pytest.mark.parametrize("c", CASES, ids=C.case_id)
def test_hip_close_to_reference_cpu_kernel(c):
    got = run_hip(c)
    want = C.run_oracle(c, O.CPU)
    for k in want:
        np.testing.assert_allclose(got[k], want[k], atol=CPU_TOL, rtol=CPU_TOL, err_msg=k)

"""Adam's float update adds eps in float: ATen adds the double eps to the float
quotient in double and narrows, and since eps holds a float value (the
hyperparameters are float tensors, or half / bfloat16 ones, widened) the twice
rounded sum equals the once rounded float sum. Checked on the GPU on every one
of the 2^32 float bit patterns x, bit for bit (NaN payloads included), for eps
values Adam uses and a few others, through torch's float and double adds. A
plausible wrong form (eps rounded to bfloat16 first) fails the comparison."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

CHUNK = 1 << 30
EPS = [1e-8, 1e-6, 1e-4, 0.1, 3.0, 2.0 ** -149, -1e-8]


@pytest.mark.parametrize("eps", EPS, ids=[f"{e:.3g}" for e in EPS])
def test_float_add_of_eps_matches_double_then_narrow(eps):
    e32 = torch.tensor(eps, dtype=torch.float32, device="cuda")  # the hyperparameter's value
    e64 = e32.double()
    for part in range(4):
        start = part * CHUNK - (1 << 31)
        x = torch.arange(start, start + CHUNK, dtype=torch.int64, device="cuda").to(
            torch.int32).view(torch.float32)
        want = (x.double() + e64).float()
        got = x + e32
        bad = (got.view(torch.int32) != want.view(torch.int32)).nonzero()
        if bad.numel():
            i = int(bad[0])
            pytest.fail(f"eps={eps!r}: {bad.numel()} x differ; first x bits "
                        f"0x{int(x[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}")
        if part == 2:  # positive floats: the same check catches eps rounded to bfloat16
            wrong = x + e32.bfloat16().float()
            if e32.bfloat16().float() != e32:
                assert (wrong.view(torch.int32) != want.view(torch.int32)).any()
        del x, want, got

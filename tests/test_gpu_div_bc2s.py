"""Adam's float update divides sqrt(v) by the replica's bias_correction2_sqrt
as a multiply by that divisor's correctly rounded double reciprocal. That is
exact whenever the quotient is not a subnormal float: the rounded product then
equals the correctly rounded quotient, NaN bit patterns included, except where
both operands are NaN (both results are NaN; the divide keeps x's payload, the
product b's). A subnormal quotient can be an exact midpoint, which the product
may round the other way; Adam's divisor reaches that range (b > 2^51) only
with |beta2| > 1, so its tests treat it as a documented exception: every
mismatch over all 2^32 x must be such a tie.
Checked here against torch's true division on the GPU, bit for bit, on every
one of the 2^32 float bit patterns for a set of divisors (divisors Adam
produces, odd significands, a subnormal and a huge one) and on random
bit-pattern pairs. A plausible wrong form (the reciprocal rounded to float)
fails the same comparison."""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / "churten_amd" / "lib" / "libchurten_bench.so"
CHUNK = 1 << 30


def _bc2s(beta2: float, step: float) -> float:
    return float(np.float32(math.sqrt(1.0 - beta2 ** step)))


DIVISORS = [
    _bc2s(0.999, 1),
    _bc2s(0.999, 7),
    _bc2s(0.9999, 1),
    _bc2s(0.999, 10000),
    1.0,
    3.0,
    float(np.float32(0.1)),
    float(np.float32(1.5 * 2.0 ** -130)),  # subnormal
    float(np.float32(1.37 * 2.0 ** 100)),
]


def _div(lib, x, b, b_stride):
    out = torch.empty_like(x)
    rc = lib.cb_div_bc2s(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                         ctypes.c_int64(b_stride), ctypes.c_void_p(out.data_ptr()),
                         ctypes.c_int64(x.numel()),
                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    return out


def _mismatches(got, want, both_nan=None):
    # bit for bit, NaN payloads included; `both_nan` marks pairs whose operands
    # are both NaN, where only NaN-ness has to agree
    bad = got.view(torch.int32) != want.view(torch.int32)
    if both_nan is not None:
        bad &= ~(both_nan & torch.isnan(got) & torch.isnan(want))
    return bad.nonzero()


@pytest.mark.parametrize("b", DIVISORS, ids=[f"{d:.6g}" for d in DIVISORS])
def test_div_bc2s_on_every_float(b):
    lib = ctypes.CDLL(str(LIB))
    bt = torch.tensor([b], dtype=torch.float32, device="cuda")
    for part in range(4):
        start = part * CHUNK - (1 << 31)
        x = torch.arange(start, start + CHUNK, dtype=torch.int64, device="cuda").to(
            torch.int32).view(torch.float32)
        got = _div(lib, x, bt, 0)
        # A one-element device tensor, not a Python scalar: torch then divides
        # elementwise (a CPU scalar divisor would be turned into a multiply).
        want = x / bt
        bad = _mismatches(got, want)
        if bad.numel():
            i = int(bad[0])
            pytest.fail(f"b={b!r}: {bad.numel()} x differ; first x bits "
                        f"0x{int(x[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}: "
                        f"{float(got[i])!r} vs {float(want[i])!r}")
        del x, got, want


def test_div_bc2s_random_pairs_and_sensitivity():
    lib = ctypes.CDLL(str(LIB))
    gen = torch.Generator(device="cuda").manual_seed(2024)
    n = 1 << 28
    x = torch.randint(-(1 << 31), 1 << 31, (n,), generator=gen, device="cuda",
                      dtype=torch.int64).to(torch.int32).view(torch.float32)
    # divisors over the whole exponent range, and divisors like Adam's
    b = torch.randint(-(1 << 31), 1 << 31, (n,), generator=gen, device="cuda",
                      dtype=torch.int64).to(torch.int32).view(torch.float32)
    b[: n // 2] = torch.rand(n // 2, generator=gen, device="cuda") + 2.0 ** -12
    got = _div(lib, x, b, 1)
    want = x / b
    assert _mismatches(got, want, torch.isnan(x) & torch.isnan(b)).numel() == 0
    # The same comparison catches the reciprocal rounded to float first.
    wrong = x * (1.0 / b)
    finite = torch.isfinite(want)
    assert _mismatches(wrong[finite], want[finite]).numel() > 1000


# Divisors whose odd part is small, so that subnormal quotients can be exact
# midpoints (b = 49 * 2^10 = 50176 gives one at x = 0x00012600).
TIE_DIVISORS = [49.0 * 2.0 ** 10, 49.0 * 2.0 ** 52, 3.0 * 2.0 ** 60]


@pytest.mark.parametrize("b", TIE_DIVISORS, ids=[f"{d:.6g}" for d in TIE_DIVISORS])
def test_div_bc2s_only_exceptions_are_subnormal_ties(b):
    """Over every float x: wherever the product and the divide differ, the
    correctly rounded quotient is subnormal, x / b is exactly the midpoint of
    the two results (checked in double, where b times a subnormal midpoint is
    exact), and the two results are neighbours. For b = 50176 the exceptions
    exist (x = 0x00012600 is one)."""
    lib = ctypes.CDLL(str(LIB))
    bt = torch.tensor([b], dtype=torch.float32, device="cuda")
    n_bad = 0
    for part in range(4):
        start = part * CHUNK - (1 << 31)
        x = torch.arange(start, start + CHUNK, dtype=torch.int64, device="cuda").to(
            torch.int32).view(torch.float32)
        got = _div(lib, x, bt, 0)
        want = x / bt
        bad = _mismatches(got, want).flatten()
        n_bad += bad.numel()
        if bad.numel():
            xb, gb, wb = x[bad], got[bad], want[bad]
            assert (wb.abs() < 2.0 ** -126).all() and (gb.abs() < 2.0 ** -126).all()
            gi, wi = gb.view(torch.int32).long(), wb.view(torch.int32).long()
            assert ((gi - wi).abs() == 1).all()
            mid = (gb.double() + wb.double()) / 2
            assert torch.equal(mid * b, xb.double())
        del x, got, want
    if b == TIE_DIVISORS[0]:
        assert n_bad > 0
        x = torch.tensor([0x00012600], dtype=torch.int32, device="cuda").view(torch.float32)
        got, want = _div(lib, x, bt, 0), x / bt
        assert got.view(torch.int32).item() == 1 and want.view(torch.int32).item() == 2

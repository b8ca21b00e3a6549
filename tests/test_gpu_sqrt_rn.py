"""The update kernels' float square root (a short path when no lane of the
wavefront holds a value below 2^-96, zero or negative; hipcc's full expansion
otherwise) against torch's sqrt on the GPU, bit for bit (NaN bits included),
in both of its forms (the float16-state policies' form also sends wavefronts
whose only small values are zeros down the short path): every one of the
2^32 float bit patterns in order (wavefronts of neighbouring patterns: the
short path for every value it serves), then shuffled values so that
wavefronts mix tiny and ordinary ones, and wavefronts whose small values are
zeros of either sign."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / "churten_amd" / "lib" / "libchurten_bench.so"
CHUNK = 1 << 30


def _sqrt_rn(lib, x, zeros):
    out = torch.empty_like(x)
    rc = lib.cb_sqrt_rn(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                        ctypes.c_int64(x.numel()), ctypes.c_int(int(zeros)),
                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    return out


def _check(x, got):
    want = torch.sqrt(x)
    bad = (got.view(torch.int32) != want.view(torch.int32)).nonzero()
    if bad.numel():
        i = int(bad[0])
        pytest.fail(f"{bad.numel()} values differ; first x bits "
                    f"0x{int(x[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}: kernel "
                    f"0x{int(got[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}, torch "
                    f"0x{int(want[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}")


@pytest.mark.parametrize("zeros", [False, True], ids=["plain", "zeros"])
@pytest.mark.parametrize("part", range(4))
def test_sqrt_rn_matches_torch_on_every_float(part, zeros):
    lib = ctypes.CDLL(str(LIB))
    start = part * CHUNK - (1 << 31)
    x = torch.arange(start, start + CHUNK, dtype=torch.int64, device="cuda").to(
        torch.int32).view(torch.float32)
    _check(x, _sqrt_rn(lib, x, zeros))


@pytest.mark.parametrize("zeros", [False, True], ids=["plain", "zeros"])
def test_sqrt_rn_mixed_wavefronts(zeros):
    lib = ctypes.CDLL(str(LIB))
    gen = torch.Generator(device="cuda").manual_seed(7)
    n = 1 << 26
    # half ordinary magnitudes, half from every bit pattern (tiny, zero, negative, NaN, inf)
    x = torch.rand(n, generator=gen, device="cuda") * 10
    x[: n // 2] = torch.randint(-(1 << 31), 1 << 31, (n // 2,), generator=gen, device="cuda",
                                dtype=torch.int64).to(torch.int32).view(torch.float32)
    x = x[torch.randperm(n, generator=gen, device="cuda")]
    _check(x, _sqrt_rn(lib, x, zeros))
    # a wavefront's one tiny value sends all its lanes down the full expansion
    y = torch.rand(n, generator=gen, device="cuda") + 0.5
    y[::64] = 2.0 ** -100
    _check(y, _sqrt_rn(lib, y, zeros))
    # zeros: one or many per wavefront, either sign, and beside a tiny value
    # (the full expansion); with `zeros` the first ones take the short path
    z = torch.rand(n, generator=gen, device="cuda") + 0.5
    z[::64] = 0.0
    z[1::128] = -0.0
    z[5::256] = 0.0
    _check(z, _sqrt_rn(lib, z, zeros))
    z[3::512] = 2.0 ** -120
    _check(z, _sqrt_rn(lib, z, zeros))
    pos0 = torch.zeros(4096, device="cuda")
    _check(pos0, _sqrt_rn(lib, pos0, zeros))
    neg0 = torch.full((4096,), -0.0, device="cuda")
    _check(neg0, _sqrt_rn(lib, neg0, zeros))

"""The kernels' float -> bfloat16 and float -> half narrowing (the store of
16-bit parameters and of bfloat16 optimizer state) against torch's own
conversions on the GPU, on every one of the 2^32 float bit patterns: normals,
subnormals, ties, the largest values that round to infinity, infinities and
NaNs."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / "churten_amd" / "lib" / "libchurten_bench.so"
CHUNK = 1 << 30


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("part", range(4))
def test_narrow_matches_torch_on_every_float(part, dtype):
    lib = ctypes.CDLL(str(LIB))
    start = part * CHUNK - (1 << 31)  # int32 range, as the float bit patterns
    bits = torch.arange(start, start + CHUNK, dtype=torch.int64, device="cuda").to(torch.int32)
    x = bits.view(torch.float32)
    del bits
    out = torch.empty(CHUNK, dtype=torch.int16, device="cuda")
    fn = lib.cb_narrow_bf16 if dtype == torch.bfloat16 else lib.cb_narrow_f16
    rc = fn(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()), ctypes.c_int64(CHUNK),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    want = x.to(dtype).view(torch.int16)
    bad = (out != want).nonzero()
    if bad.numel():
        i = int(bad[0])
        pytest.fail(f"{bad.numel()} patterns differ; first 0x{int(x[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}: "
                    f"kernel 0x{int(out[i]) & 0xFFFF:04x}, torch 0x{int(want[i]) & 0xFFFF:04x}")


@pytest.mark.parametrize("shift", [0, 1], ids=["first", "second"])
@pytest.mark.parametrize("part", range(4))
def test_paired_bf16_narrow_matches_torch_on_every_float(part, shift):
    """The drivers narrow bfloat16 packs two values per conversion; every float
    bit pattern, once in the first and once in the second position of a pair."""
    lib = ctypes.CDLL(str(LIB))
    start = part * CHUNK - (1 << 31) + shift
    bits = torch.arange(start, start + CHUNK, dtype=torch.int64, device="cuda").to(torch.int32)
    x = bits.view(torch.float32)
    del bits
    out = torch.empty(CHUNK // 2, dtype=torch.int32, device="cuda")
    rc = lib.cb_narrow2_bf16(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                             ctypes.c_int64(CHUNK // 2),
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    got = out.view(torch.int16)  # low half first: element order
    want = x.to(torch.bfloat16).view(torch.int16)
    bad = (got != want).nonzero()
    if bad.numel():
        i = int(bad[0])
        pytest.fail(f"{bad.numel()} patterns differ; first 0x{int(x[i:i + 1].view(torch.int32)) & 0xFFFFFFFF:08x}: "
                    f"kernel 0x{int(got[i]) & 0xFFFF:04x}, torch 0x{int(want[i]) & 0xFFFF:04x}")

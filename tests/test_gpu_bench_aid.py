"""The traffic-ceiling kernels bench.py times (churten_amd/lib/libchurten_bench.so):
they touch exactly the active rows they claim to, with the values they claim
to write, and reject arguments they cannot serve."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / "churten_amd" / "lib" / "libchurten_bench.so"


def call(lib, mode, ts, mask, c, sink, R=None, T=None, packs=2):
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    R = ts[0].shape[0] if R is None else R
    T = ts[0].shape[1] if T is None else T
    return lib.cb_traffic(ctypes.c_int(mode), *[vp(t) for t in ts], vp(mask), ctypes.c_int64(R),
                          ctypes.c_int64(T), ctypes.c_float(c), ctypes.c_uint32(0),
                          ctypes.c_int(packs), vp(sink),
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("packs", [1, 2])
@pytest.mark.parametrize("T", [4, 1000, 1028, 4096])
def test_traffic_modes(T, packs):
    lib = ctypes.CDLL(str(LIB))
    R = 3
    g = torch.Generator(device="cuda").manual_seed(T)
    ts = [torch.randn(R, T, device="cuda", generator=g) for _ in range(4)]
    before = [t.clone() for t in ts]
    mask = torch.tensor([True, False, True], device="cuda")
    sink = torch.full((1,), 7.0, device="cuda")
    assert call(lib, 0, ts, mask, 0.0, sink, packs=packs) == 0      # x + g * 0: unchanged
    assert call(lib, 1, ts, mask, -3.0e38, sink, packs=packs) == 0  # reads only
    torch.cuda.synchronize()
    for a, b in zip(ts, before):
        assert torch.equal(a, b)
    assert sink.item() == 7.0
    assert call(lib, 2, ts, mask, 1.5, sink, packs=packs) == 0      # writes c to p, m, v of active rows
    torch.cuda.synchronize()
    for i in (0, 2, 3):
        assert torch.equal(ts[i][mask], torch.full_like(ts[i][mask], 1.5))
        assert torch.equal(ts[i][~mask], before[i][~mask])
    assert torch.equal(ts[1], before[1])                # the gradient is only read


@pytest.mark.parametrize("packs", [1, 2])
@pytest.mark.parametrize("T", [4, 1000, 1028, 4096])
def test_traffic_bf16_moments_mode(T, packs):
    """Mode 3: float32 params and grads, bfloat16 moments. With c = 0 nothing
    changes; with c != 0 the active rows' params become p + g * c and their
    moments' bits flip in the lowest bit, frozen rows and the gradient stay."""
    lib = ctypes.CDLL(str(LIB))
    R = 3
    g = torch.Generator(device="cuda").manual_seed(T + 1)
    p, gr = (torch.randn(R, T, device="cuda", generator=g) for _ in range(2))
    m, v = (torch.randn(R, T, device="cuda", generator=g).to(torch.bfloat16) for _ in range(2))
    ts = [p, gr, m, v]
    before = [t.clone() for t in ts]
    mask = torch.tensor([True, False, True], device="cuda")
    sink = torch.zeros(1, device="cuda")
    assert call(lib, 3, ts, mask, 0.0, sink, packs=packs) == 0
    torch.cuda.synchronize()
    for a, b in zip(ts, before):
        assert torch.equal(a.view(torch.int32 if a.dtype == torch.float32 else torch.int16),
                           b.view(torch.int32 if b.dtype == torch.float32 else torch.int16))
    assert call(lib, 3, ts, mask, 0.5, sink, packs=packs) == 0
    torch.cuda.synchronize()
    assert torch.equal(p[mask], before[0][mask] + before[1][mask] * 0.5)
    assert torch.equal(p[~mask], before[0][~mask]) and torch.equal(gr, before[1])
    for t, b in ((m, before[2]), (v, before[3])):
        ti, bi = t.view(torch.int16), b.view(torch.int16)
        assert torch.equal(ti[mask], bi[mask] ^ 1) and torch.equal(ti[~mask], bi[~mask])


def test_traffic_rejects_bad_arguments():
    lib = ctypes.CDLL(str(LIB))
    ts = [torch.zeros(2, 8, device="cuda") for _ in range(4)]
    mask = torch.ones(2, dtype=torch.bool, device="cuda")
    sink = torch.zeros(1, device="cuda")
    assert call(lib, 4, ts, mask, 0.0, sink) == 1                 # no such mode
    assert call(lib, 0, ts, mask, 0.0, sink, packs=3) == 1        # 1 or 2 packs only
    assert call(lib, 0, ts, mask, 0.0, sink, T=6) == 1            # T not a multiple of 4
    odd = [t.view(-1)[1:9].view(1, 8) for t in ts]               # 4-byte aligned only
    assert call(lib, 0, odd, mask, 0.0, sink, R=1) == 1


DIVISORS = [1, 2, 3, 5, 7, 64, 255, 256, 257, 430, 1037, 4099, 98_328, 8_388_625,
            2**20 - 1, 2**24 + 1, 2**31 - 1, 2**31, 2**31 + 1, 2**32 - 1]


@pytest.mark.parametrize("d", DIVISORS)
def test_div_tiles_is_integer_division(d):
    """The streaming driver finds a workgroup's row as index / tiles-per-row
    with a multiply and shifts (Granlund-Montgomery constants set on the host).
    Against integer division: 2^20 random 32-bit indices plus the edges (0,
    d - 1, d, d + 1, multiples of d and their neighbours, 2^32 - 1)."""
    lib = ctypes.CDLL(str(LIB))
    g = torch.Generator().manual_seed(d % 1_000_003)
    rnd = torch.randint(0, 2**32, (1 << 20,), generator=g, dtype=torch.int64)
    edges = [0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, 2**32 - 1, 2**32 - 2, 2**31, 2**31 - 1]
    k = (2**32 - 1) // d
    edges += [k * d, k * d - 1, (k // 2) * d, (k // 2) * d - 1, (k // 2) * d + 1]
    m = torch.cat([rnd, torch.tensor([e % 2**32 for e in edges], dtype=torch.int64)])
    dev_m = m.to(torch.uint32).cuda()
    q = torch.empty_like(dev_m)
    assert lib.cb_div_tiles(ctypes.c_uint32(d), ctypes.c_void_p(dev_m.data_ptr()),
                            ctypes.c_void_p(q.data_ptr()), ctypes.c_int64(m.numel()),
                            None) == 0
    torch.cuda.synchronize()
    got = q.cpu().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    assert torch.equal(got, m // d)


def test_div_tiles_rejects_a_zero_divisor():
    lib = ctypes.CDLL(str(LIB))
    assert lib.cb_div_tiles(ctypes.c_uint32(0), None, None, ctypes.c_int64(4), None) == 1

"""The allocation-free Adam entry point against the workspace entry point.

ts_adam_step_noalloc keeps the per-replica constants in the library's own
device scratch array instead of a caller's workspace. On every call it must
give what ts_adam_step_ws gives, bit for bit; calls run back to back, the
later ones with smaller inputs (the scratch keeps the previous call's
contents, which no call may depend on). The first call in the process is made
under HIP graph capture (the first call on a device looks up the scratch's
address), and eager calls change neither torch's allocated bytes nor the
device's free memory.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LIB = ctypes.CDLL(str(ROOT / "churten_amd" / "lib" / "libchurten_optim.so"))
DEV = torch.device("cuda")
TS_AMSGRAD, TS_ADAMW, TS_MAXIMIZE, TS_BUMP_STEPS = 0x1, 0x2, 0x4, 0x10
DTYPE_CODE = {torch.float32: 0, torch.float64: 1, torch.float16: 2, torch.bfloat16: 3}


class RtBuf(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride_r", ctypes.c_int64),
                ("stride_t", ctypes.c_int64)]


_P, _I64, _U32, _SZ, _I = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_size_t,
                           ctypes.c_int)
_HEAD = [ctypes.POINTER(RtBuf), _I, _P, _P, _P, _P, _P, _P, ctypes.POINTER(ctypes.c_uint8),
         _I64, _I64, _U32, _P]
LIB.ts_adam_step_noalloc.argtypes = _HEAD + [_P]
LIB.ts_adam_step_ws.argtypes = _HEAD + [_P, _SZ, _P]
LIB.ts_workspace_bytes.argtypes = [_I64]
LIB.ts_workspace_bytes.restype = _SZ


def _inputs(R, T, dtype, seed, amsgrad):
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)  # noqa: E731
    bufs = [rnd(), rnd(), rnd().abs(), rnd().abs()] + ([rnd().abs()] if amsgrad else [])
    steps = torch.randint(0, 50, (R,), generator=g, device=DEV).to(dtype)
    mask = (torch.rand(R, generator=g, device=DEV) < 0.7).to(torch.uint8)
    mask[0] = 1
    lr = torch.rand(R, generator=g, device=DEV) * 1e-2
    hyp = [lr, torch.full((R,), 0.9, device=DEV), torch.full((R,), 0.999, device=DEV),
           torch.full((R,), 1e-4 if dtype == torch.float16 else 1e-8, device=DEV),
           torch.full((R,), 1e-2, device=DEV)]
    hyp = [h.to(dtype) for h in hyp]
    return bufs, steps, hyp, mask


def _call(noalloc, bufs, steps, hyp, mask, flags, dtype, out_zero, sync=True):
    R, T = bufs[0].shape
    table = (RtBuf * 5)(*[RtBuf(t.data_ptr(), t.stride(0), t.stride(1)) for t in bufs]
                        + [RtBuf(0, 0, 1)] * (5 - len(bufs)))
    args = [table, DTYPE_CODE[dtype], steps.data_ptr(), *[h.data_ptr() for h in hyp],
            ctypes.cast(mask.data_ptr(), ctypes.POINTER(ctypes.c_uint8)), R, T, flags,
            out_zero.data_ptr()]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = LIB.ts_adam_step_noalloc(*args, stream)
    else:
        ws = torch.empty(LIB.ts_workspace_bytes(R), dtype=torch.uint8, device=DEV)
        rc = LIB.ts_adam_step_ws(*args, ws.data_ptr(), ws.numel(), stream)
    if sync:
        torch.cuda.synchronize()
    return rc


INTS = {torch.float32: torch.int32, torch.float64: torch.int64, torch.float16: torch.int16}


def test_a_first_call_under_graph_capture_replays_match_workspace_entry_point():
    """The process's first noalloc call is captured in a torch.cuda graph (the
    scratch address lookup runs during capture). Three replays, each after a
    new gradient is copied into the captured one and with eager calls of
    ts_adam_step_ws on a twin state between them, equal the eager results bit
    for bit; the captured steps bump and zero result replay too."""
    R, T, dtype, flags = 12, 4 * 1000 + 12, torch.float32, TS_ADAMW | TS_BUMP_STEPS
    bufs, steps, hyp, mask = _inputs(R, T, dtype, 7, False)
    twin, twin_steps = [t.clone() for t in bufs], steps.clone()
    z, tz = torch.full((1,), 5.0, device=DEV), torch.full((1,), 5.0, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(8)
    grads = [torch.randn(R, T, device=DEV, generator=g) for _ in range(3)]
    # warm up the library (its kernels load) on the workspace entry point only
    warm = [t.clone() for t in bufs]
    assert _call(False, warm, steps.clone(), hyp, mask, flags, dtype, z.clone()) == 0
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call(True, bufs, steps, hyp, mask, flags, dtype, z, sync=False)
    assert rc == 0
    for gr in grads:
        bufs[1].copy_(gr)
        twin[1].copy_(gr)
        z.fill_(5.0)
        graph.replay()
        torch.cuda.synchronize()
        assert _call(False, twin, twin_steps, hyp, mask, flags, dtype, tz) == 0
        for k, (a, b) in enumerate(zip(bufs, twin)):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), k
        assert torch.equal(steps, twin_steps)
        assert z.item() == 0.0 and tz.item() == 0.0


def test_eager_calls_allocate_nothing():
    """After the first call on the device, noalloc calls (including a new
    shape and dtype) leave torch's allocated bytes and hipMemGetInfo's free
    bytes exactly as they were."""
    inputs = [_inputs(R, T, dt, 50 + i, bool(f & TS_AMSGRAD)) + (dt, f)
              for i, (R, T, dt, f) in enumerate(SEQUENCE[1:])]
    z = [torch.zeros(1, device=DEV, dtype=x[4]) for x in inputs]
    bufs, steps, hyp, mask, dt, f = inputs[0]
    assert _call(True, bufs, steps, hyp, mask, f | TS_BUMP_STEPS, dt, z[0]) == 0
    torch.cuda.synchronize()
    before = (torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0])
    for (bufs, steps, hyp, mask, dt, f), zi in zip(inputs, z):
        assert _call(True, bufs, steps, hyp, mask, f | TS_BUMP_STEPS, dt, zi) == 0
        assert (torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]) == before


# Calls in this order, one after the other: each later input is smaller.
SEQUENCE = [
    (70, 5_592_410, torch.float32, TS_ADAMW),         # the large (non-temporal) shape
    (64, 70_001, torch.float32, TS_AMSGRAD | TS_MAXIMIZE),
    (9, 1_001, torch.float16, TS_ADAMW),
    (3, 45, torch.float32, 0),
    (1, 7, torch.float64, TS_AMSGRAD),
]


def test_noalloc_equals_workspace_entry_point_on_successive_calls():
    for i, (R, T, dtype, flags) in enumerate(SEQUENCE):
        amsgrad = bool(flags & TS_AMSGRAD)
        a_bufs, a_steps, hyp, mask = _inputs(R, T, dtype, 100 + i, amsgrad)
        b_bufs, b_steps = [t.clone() for t in a_bufs], a_steps.clone()
        za = torch.full((1,), float("nan"), device=DEV, dtype=dtype)
        zb = za.clone()
        for _ in range(2):  # two steps of each input
            assert _call(False, a_bufs, a_steps, hyp, mask, flags | TS_BUMP_STEPS, dtype, za) == 0
            assert _call(True, b_bufs, b_steps, hyp, mask, flags | TS_BUMP_STEPS, dtype, zb) == 0
        for k, (a, b) in enumerate(zip(a_bufs, b_bufs)):
            assert torch.equal(a.view(INTS[dtype]), b.view(INTS[dtype])), (i, R, T, k)
        assert torch.equal(a_steps, b_steps), (i, "steps")
        assert za.item() == 0 and zb.item() == 0


def test_noalloc_at_its_largest_replica_count():
    """R = 65536, the scratch's capacity, every replica's constants in use
    (the last entry at the array's end): equal to the workspace form."""
    R, T = 65536, 8
    bufs, steps, hyp, mask = _inputs(R, T, torch.float32, 11, False)
    mask.fill_(1)
    b_bufs, b_steps = [t.clone() for t in bufs], steps.clone()
    za, zb = torch.ones(1, device=DEV), torch.ones(1, device=DEV)
    assert _call(False, bufs, steps, hyp, mask, TS_ADAMW | TS_BUMP_STEPS, torch.float32, za) == 0
    assert _call(True, b_bufs, b_steps, hyp, mask, TS_ADAMW | TS_BUMP_STEPS, torch.float32, zb) == 0
    for k, (a, b) in enumerate(zip(bufs, b_bufs)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), k
    assert torch.equal(steps, b_steps) and za.item() == 0 and zb.item() == 0


def test_noalloc_rejects_more_replicas_than_its_scratch_holds():
    R, T = 65537, 4
    bufs = [torch.zeros(R, T, device=DEV) for _ in range(4)]
    steps = torch.zeros(R, device=DEV)
    hyp = [torch.zeros(R, device=DEV) for _ in range(5)]
    mask = torch.ones(R, dtype=torch.uint8, device=DEV)
    z = torch.full((1,), 7.0, device=DEV)
    assert _call(True, bufs, steps, hyp, mask, TS_BUMP_STEPS, torch.float32, z) == 1
    assert torch.equal(steps, torch.zeros(R, device=DEV)) and z.item() == 7.0

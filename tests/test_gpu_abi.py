"""The C ABI on the GPU, called as a foreign-function caller would call it.

include/churten_optim.h is the drop-in boundary (the device half of the
reference's torch.library operators, src/torchstrap/kernels/csrc/stubs.cpp:
25-72). These tests call its entry points through ctypes on device buffers
that torch allocates, on torch's current stream, and compare every output bit
for bit with the oracle's device formulation:

* every update entry point -- dense, segmented, with and without a workspace;
* TS_BUMP_STEPS on (the library bumps) and off (the caller bumps first);
* out_zero set (it must read 0 afterwards) and NULL;
* R or T of 0 and 1;
* the segmented forms against the oracle directly, with and without the
  consolidated gradient written on the way, and with a gap column range;
* the large-launch shapes (non-temporal, residency-capped) of every policy and
  dtype just above the size where the small, MALL-resident shape stops, against
  torch's own fused kernels row by row (and the oracle for float32);
* Adam's per-replica constants derived without a workspace (once per
  wavefront) against those of the workspace form, replica by replica.
"""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import cases as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LIB = ctypes.CDLL(str(ROOT / "churten_amd" / "lib" / "libchurten_optim.so"))
DEV = torch.device("cuda")

TS_AMSGRAD, TS_ADAMW, TS_MAXIMIZE, TS_NESTEROV = 0x1, 0x2, 0x4, 0x8
TS_BUMP_STEPS, TS_STATE_BF16, TS_ADAGRAD_F32 = 0x10, 0x20, 0x40
DTYPE_CODE = {torch.float32: 0, torch.float64: 1, torch.float16: 2, torch.bfloat16: 3}
# the small/large switch: (R, T) operand bytes of a launch (256 MiB)
MALL_BYTES = 256 << 20


class RtBuf(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride_r", ctypes.c_int64),
                ("stride_t", ctypes.c_int64)]


class Segment(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride_r", ctypes.c_int64),
                ("col", ctypes.c_int64), ("numel", ctypes.c_int64)]


_P, _I64, _U32, _SZ, _I = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_size_t,
                           ctypes.c_int)
_BUFS, _SEGS = ctypes.POINTER(RtBuf), ctypes.POINTER(Segment)
_HEAD = [_BUFS, _I, _P, _P, _P, _P, _P]  # bufs, dtype, steps, 4 hyperparameters
for name, nh in (("ts_adam_step", 5), ("ts_sgd_step", 4), ("ts_adagrad_step", 4)):
    common = [_P] * (nh - 4) + [ctypes.POINTER(ctypes.c_uint8), _I64, _I64, _U32, _P]
    getattr(LIB, name).argtypes = _HEAD + common + [_P]
    getattr(LIB, name + "_segments").argtypes = (
        [_BUFS, _SEGS, _I] + _HEAD[1:] + common + [_P])
    if name != "ts_sgd_step":
        getattr(LIB, name + "_ws").argtypes = _HEAD + common + [_P, _SZ, _P]
        getattr(LIB, name + "_segments_ws").argtypes = (
            [_BUFS, _SEGS, _I] + _HEAD[1:] + common + [_P, _SZ, _P])
LIB.ts_workspace_bytes.argtypes = [_I64]
LIB.ts_workspace_bytes.restype = _SZ


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_INT_OF = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32,
           torch.float64: torch.int64}


def _same(name, got, want):
    """Bit equality of two tensors (NaNs included: float16 rounds beta2 =
    0.9999 to 1, so a zero exp_avg_sq gives 0/0 in torch and here alike),
    with the first differences on failure."""
    it = _INT_OF[got.dtype]
    if torch.equal(got.view(it), want.view(it)):
        return
    g, w = got.float().cpu(), want.float().cpu()
    ne = got.view(it).cpu() != want.view(it).cpu()
    idx = ne.nonzero().flatten()[:4].tolist()
    raise AssertionError(f"{name}: {int(ne.sum())} of {g.numel()} differ; at {idx}: "
                         f"{[g[i].item() for i in idx]} vs {[w[i].item() for i in idx]}")


def abi_step(op, bufs, steps, hyp, mask, flags, *, dtype=torch.float32, workspace=False,
             out_zero=None, segments=None, shape=None):
    """One call of the entry point for `op` ("adam" | "sgd" | "adagrad") on
    device tensors. `bufs`: the (R, T) operands in the header's order (None =
    a NULL buffer); `segments`: a list of (tensor, col) per-parameter
    gradients for the segmented forms. Returns the library's status."""
    R, T = shape if shape is not None else bufs[0].shape
    table = (RtBuf * 5)(*[RtBuf(t.data_ptr(), t.stride(0), t.stride(1)) if t is not None
                          else RtBuf(0, 0, 1) for t in bufs]
                        + [RtBuf(0, 0, 1)] * (5 - len(bufs)))
    mask_p = ctypes.cast(mask.data_ptr(), ctypes.POINTER(ctypes.c_uint8)) if mask.numel() else None
    args = [table, DTYPE_CODE[dtype], _ptr(steps), *[_ptr(h) for h in hyp], mask_p, R, T, flags,
            _ptr(out_zero)]
    name = f"ts_{op}_step"
    if segments is not None:
        segs = (Segment * max(1, len(segments)))(
            *[Segment(t.data_ptr(), t.stride(0), col, t.shape[1]) for t, col in segments])
        args = [table, segs, len(segments)] + args[1:]
        name += "_segments"
    ws = None
    if workspace:
        ws = torch.empty(max(1, LIB.ts_workspace_bytes(R)), dtype=torch.uint8, device=DEV)
        args += [_ptr(ws), ws.numel()]
        name += "_ws"
    rc = getattr(LIB, name)(*args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return rc


# ---------------------------------------------------------------------------
# golden cases through every entry point, against the oracle
# ---------------------------------------------------------------------------
def _picked_cases():
    out = []
    for c in C.all_cases():
        if c["T"] in (45, 1001, 16397) or (c["op"] == "adam" and c["T"] == 64 and c["wd"] > 0):
            out.append(c)
    return out


CASES = _picked_cases()


def _flags(c):
    if c["op"] == "adam":
        return ((TS_AMSGRAD if c["amsgrad"] else 0) | (TS_ADAMW if c["decoupled"] else 0)
                | (TS_MAXIMIZE if c["maximize"] else 0))
    if c["op"] == "sgd":
        return (TS_NESTEROV if c["nesterov"] else 0) | (TS_MAXIMIZE if c["maximize"] else 0)
    return TS_MAXIMIZE if c["maximize"] else 0


def _hyper_names(c):
    return {"adam": ("lr", "beta1", "beta2", "eps", "wd"),
            "sgd": ("lr", "momentum", "dampening", "wd"),
            "adagrad": ("lr", "lr_decay", "wd", "eps")}[c["op"]]


def _operand_names(c, x):
    if c["op"] == "adam":
        return ["p", "g", "m", "v"] + (["mx"] if c["amsgrad"] else [])
    if c["op"] == "sgd":
        return ["p", "g"] + (["mb"] if x["mb"] is not None else [])
    return ["p", "g", "s"]


def _split_segments(g, T):
    """Three per-parameter gradients covering columns [0, T) irregularly."""
    cuts = sorted({0, T // 3 + 1, (2 * T) // 3 - 2, T}) if T > 8 else [0, T]
    return [(g[:, a:b].contiguous(), a) for a, b in zip(cuts[:-1], cuts[1:]) if b > a]


# SGD has no workspace entry points (nothing to precompute)
_CASE_WS = [pytest.param(c, ws, id=C.case_id(c) + ("-ws" if ws else "-no_ws"))
            for c in CASES for ws in (False, True) if not (ws and c["op"] == "sgd")]


@pytest.mark.parametrize("form", ["dense", "segments", "segments_no_grad_out"])
@pytest.mark.parametrize("bump", [True, False], ids=["bump", "caller_bumps"])
@pytest.mark.parametrize("c,workspace", _CASE_WS)
def test_entry_points_bit_exact_to_oracle(c, form, workspace, bump):
    x = C.make_inputs(c)
    names = _operand_names(c, x)
    dev = {k: torch.from_numpy(x[k].copy()).to(DEV) for k in names if k != "g"}
    steps = torch.from_numpy(x["steps"].copy()).to(DEV)
    mask = torch.from_numpy(x["mask"].astype(np.uint8)).to(DEV)
    hyp = [torch.from_numpy(x[k].copy()).to(DEV) for k in _hyper_names(c)]
    R, T = c["R"], c["T"]
    out_zero = torch.full((1,), float("nan"), device=DEV)
    want = C.run_oracle(c, O.DEVICE)
    for g_np in x["grads"]:
        g = torch.from_numpy(g_np.copy()).to(DEV)
        if not bump:
            steps += mask.to(steps.dtype)
        segments, grad_buf = None, g
        if form != "dense":
            segments = _split_segments(g, T)
            grad_buf = torch.zeros_like(g) if form == "segments" else None
        bufs = [dev["p"], grad_buf] + [dev[k] for k in names[2:]]
        out_zero.fill_(float("nan"))
        rc = abi_step(c["op"], bufs, steps, hyp, mask, _flags(c) | (TS_BUMP_STEPS if bump else 0),
                      workspace=workspace, out_zero=out_zero, segments=segments, shape=(R, T))
        assert rc == 0
        assert out_zero.item() == 0.0
        if form == "segments":  # the consolidated gradient, all rows
            assert torch.equal(grad_buf, g)
    for k in names:
        if k == "g":
            continue
        got = dev[k].cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want[k].view(np.uint32)), k
    assert np.array_equal(steps.cpu().numpy(), want["steps"])


@pytest.mark.parametrize("workspace", [False, True], ids=["no_ws", "ws"])
@pytest.mark.parametrize("op", ["adam", "adagrad"])
def test_segments_with_gap_take_zero_gradient(op, workspace):
    """Columns no segment covers take zero gradient when no consolidated
    buffer is given (and the update still runs there): the oracle with those
    gradient columns zeroed."""
    c = dict(op=op, R=3, T=1000, amsgrad=False, maximize=False, decoupled=True, wd=1e-2,
             lr_decay=1e-2, eps=1e-10, hypers="distinct", mask="one_frozen", steps0=0,
             nsteps=1, seed=77)
    x = C.make_inputs(c)
    names = _operand_names(c, x)
    g_np = x["grads"][0]
    g_np[:, 300:420] = 0.0
    want = {k: (x[k].copy() if x[k] is not None else None) for k in x if k != "grads"}
    if op == "adam":
        O.adam_step(O.DEVICE, want["p"], g_np, want["m"], want["v"], None, want["steps"],
                    want["lr"], want["beta1"], want["beta2"], want["eps"], want["wd"],
                    want["mask"], amsgrad=False, maximize=False, decoupled_weight_decay=True)
    else:
        O.adagrad_step(O.DEVICE, want["p"], g_np, want["s"], want["steps"], want["lr"],
                       want["lr_decay"], want["wd"], want["eps"], want["mask"])
    dev = {k: torch.from_numpy(x[k].copy()).to(DEV) for k in names if k != "g"}
    g = torch.from_numpy(g_np.copy()).to(DEV)
    segments = [(g[:, :300].contiguous(), 0), (g[:, 420:].contiguous(), 420)]
    steps = torch.from_numpy(x["steps"].copy()).to(DEV)
    mask = torch.from_numpy(x["mask"].astype(np.uint8)).to(DEV)
    hyp = [torch.from_numpy(x[k].copy()).to(DEV) for k in _hyper_names(c)]
    bufs = [dev["p"], None] + [dev[k] for k in names[2:]]
    assert abi_step(op, bufs, steps, hyp, mask, TS_BUMP_STEPS | (TS_ADAMW if op == "adam" else 0),
                    workspace=workspace, segments=segments, shape=(3, 1000)) == 0
    for k in names:
        if k != "g":
            assert np.array_equal(dev[k].cpu().numpy().view(np.uint32),
                                  want[k].view(np.uint32)), k


def _op_ws(ops):
    """(op, workspace) pairs; SGD has no workspace entry points."""
    return [pytest.param(op, ws, id=op + ("-ws" if ws else "-no_ws"))
            for op in ops for ws in (False, True) if not (ws and op == "sgd")]


@pytest.mark.parametrize("op,workspace", _op_ws(["adam", "sgd", "adagrad"]))
@pytest.mark.parametrize("R,T", [(0, 5), (3, 0), (0, 0), (1, 1), (1, 3), (2, 1)])
def test_empty_and_unit_shapes(op, R, T, workspace):
    """R or T of 0: the steps of active replicas still tick (when the library
    bumps), out_zero is written, nothing else is touched. R or T of 1: the
    update itself, against the oracle."""
    g = torch.Generator(device=DEV).manual_seed(R * 10 + T)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g)  # noqa: E731
    p, gr = rnd(), rnd()
    state = [rnd().abs() for _ in range(2 if op == "adam" else 1)]
    steps = torch.arange(R, device=DEV, dtype=torch.float32) + 3
    mask = torch.ones(R, dtype=torch.uint8, device=DEV)
    if R > 1:
        mask[1] = 0
    nh = 5 if op == "adam" else 4
    hyp = [torch.full((R,), v, device=DEV) for v in
           {"adam": (1e-2, 0.9, 0.999, 1e-8, 1e-2), "sgd": (1e-2, 0.9, 0.1, 1e-2),
            "adagrad": (1e-2, 1e-2, 1e-2, 1e-10)}[op][:nh]]
    host = [t.cpu().numpy().copy() for t in [p, gr, *state, steps, *hyp]]
    out_zero = torch.full((1,), float("nan"), device=DEV)
    flags = TS_BUMP_STEPS | (TS_NESTEROV if op == "sgd" else 0)
    assert abi_step(op, [p, gr, *state], steps, hyp, mask, flags, workspace=workspace,
                    out_zero=out_zero, shape=(R, T)) == 0
    assert out_zero.item() == 0.0
    hp, hg, *rest = host
    hstate, hsteps, hhyp = rest[:len(state)], rest[len(state)], rest[len(state) + 1:]
    hmask = mask.cpu().numpy().astype(bool)
    if R * T == 0:
        assert np.array_equal(steps.cpu().numpy(), hsteps + hmask.astype(np.float32))
        return
    if op == "adam":
        O.adam_step(O.DEVICE, hp, hg, hstate[0], hstate[1], None, hsteps, *hhyp, hmask,
                    amsgrad=False, maximize=False, decoupled_weight_decay=False)
    elif op == "sgd":
        O.sgd_step(O.DEVICE, hp, hg, hstate[0], hsteps, *hhyp, hmask, nesterov=True)
    else:
        O.adagrad_step(O.DEVICE, hp, hg, hstate[0], hsteps, *hhyp, hmask)
    for got, want in zip([p, *state, steps], [hp, *hstate, hsteps]):
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_null_out_zero_and_no_bump_leave_steps_alone():
    """Without TS_BUMP_STEPS the steps are read as given and not written; a
    NULL out_zero writes nothing."""
    R, T = 3, 64
    g = torch.Generator(device=DEV).manual_seed(5)
    p, gr, m, v = (torch.randn(R, T, device=DEV, generator=g) for _ in range(4))
    m, v = m.abs(), v.abs()
    steps = torch.tensor([4.0, 2.0, 9.0], device=DEV)
    mask = torch.tensor([1, 0, 1], dtype=torch.uint8, device=DEV)
    hyp = [torch.full((R,), x, device=DEV) for x in (1e-2, 0.9, 0.999, 1e-8, 0.0)]
    for ws in (False, True):
        s = steps.clone()
        assert abi_step("adam", [p, gr, m, v], s, hyp, mask, 0, workspace=ws) == 0
        assert torch.equal(s, steps)


LIB.ts_bump_steps.argtypes = [_I, _P, ctypes.POINTER(ctypes.c_uint8), _I64, _P, _P]


@pytest.mark.parametrize("with_zero", [True, False], ids=["out_zero", "null_out_zero"])
@pytest.mark.parametrize("R", [0, 1, 1000])
@pytest.mark.parametrize("dtype", list(DTYPE_CODE), ids=str)
def test_bump_steps_on_device(dtype, R, with_zero):
    """ts_bump_steps, the reference's `state_steps.add_(active_mask.to(dtype))`
    (cuda/adam.cu:277), on device buffers: two calls with complementary masks;
    after each, the steps equal torch's own add of the mask in the steps' dtype
    bit for bit (including its rounding: 256 + 1 rounds back to 256 in
    bfloat16), the frozen replicas keep their bits, and out_zero reads +0 (a
    NULL out_zero is accepted and writes nothing)."""
    g = torch.Generator().manual_seed(R)
    steps = torch.randint(0, 3000, (R,), generator=g).to(dtype)
    if R:
        steps[0] = 256.0
    mask = torch.rand(R, generator=g) < 0.7
    if R > 1:
        mask[:2] = torch.tensor([True, False])
    d_steps = steps.to(DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for m in (mask, ~mask):
        before = d_steps.clone()
        want = before.clone().add_(m.to(DEV).to(dtype))
        d_mask = m.to(torch.uint8).to(DEV)
        mask_p = (ctypes.cast(d_mask.data_ptr(), ctypes.POINTER(ctypes.c_uint8)) if R
                  else None)
        zero = torch.full((), 7.0, dtype=dtype, device=DEV) if with_zero else None
        rc = LIB.ts_bump_steps(DTYPE_CODE[dtype], _ptr(d_steps) if R else None, mask_p, R,
                               _ptr(zero), stream)
        torch.cuda.synchronize()
        assert rc == 0
        _same("steps", d_steps, want)
        frozen = ~m.to(DEV)
        _same("frozen steps", d_steps[frozen], before[frozen])
        if with_zero:
            _same("out_zero", zero, torch.zeros((), dtype=dtype, device=DEV))


@pytest.mark.parametrize("layout", ["rows", "replica_minor"])
@pytest.mark.parametrize("amsgrad", [False, True])
def test_workspace_entries_of_frozen_replicas_are_never_written(amsgrad, layout):
    """ts_adam_step_ws writes workspace constants for active replicas only:
    with the workspace filled with NaN bit patterns before the call and the
    frozen replicas at step 0 (whose bias corrections would divide by
    1 - beta^0 = 0) holding NaN state, the frozen replicas' 16-byte entries
    keep the NaN bytes, their rows or columns stay bit-identical, and every
    operand equals the oracle's device form."""
    R, T = 70, 45
    rng = np.random.default_rng(21)
    flags = TS_BUMP_STEPS | TS_ADAMW | (TS_AMSGRAD if amsgrad else 0)
    host = [rng.standard_normal((R, T)).astype(np.float32) for _ in range(5)]
    for a in host[2:]:
        np.abs(a, out=a)
    mask = np.ones(R, dtype=bool)
    frozen = [0, 33, 69]
    mask[frozen] = False
    for a in host[2:]:
        a[frozen] = np.nan
    steps = np.where(mask, 3.0, 0.0).astype(np.float32)
    hyp = [np.linspace(lo, hi, R, dtype=np.float32) for lo, hi in
           ((1e-3, 5e-2), (0.8, 0.95), (0.99, 0.9999), (1e-9, 1e-7), (1e-2, 1e-2))]

    def dev(a):
        if layout == "rows":
            return torch.from_numpy(a).to(DEV)
        return torch.from_numpy(np.ascontiguousarray(a.T)).to(DEV).t()

    ops = [dev(a) for a in host[:5 if amsgrad else 4]]
    d_steps = torch.from_numpy(steps).to(DEV)
    d_hyp = [torch.from_numpy(h).to(DEV) for h in hyp]
    d_mask = torch.from_numpy(mask.astype(np.uint8)).to(DEV)
    table = (RtBuf * 5)(*[RtBuf(t.data_ptr(), t.stride(0), t.stride(1)) for t in ops]
                        + [RtBuf(0, 0, 1)] * (5 - len(ops)))
    ws = torch.full((LIB.ts_workspace_bytes(R),), 0xFF, dtype=torch.uint8, device=DEV)
    rc = LIB.ts_adam_step_ws(table, 0, _ptr(d_steps), *[_ptr(h) for h in d_hyp],
                             ctypes.cast(d_mask.data_ptr(), ctypes.POINTER(ctypes.c_uint8)),
                             R, T, flags, None, _ptr(ws), ws.numel(),
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0
    entries = ws.view(R, 16).cpu()
    assert (entries[frozen] == 0xFF).all()
    assert not (entries[torch.from_numpy(mask)] == 0xFF).all(dim=1).any()
    want = [a.copy() for a in host]
    O.adam_step(O.DEVICE, want[0], want[1], want[2], want[3], want[4] if amsgrad else None,
                steps, *hyp, mask, amsgrad=amsgrad, maximize=False, decoupled_weight_decay=True)
    for i, t in enumerate(ops):
        got = t.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), i
        assert np.array_equal(got[frozen].view(np.uint32), host[i][frozen].view(np.uint32)), i
    assert np.array_equal(d_steps.cpu().numpy(), steps)


# ---------------------------------------------------------------------------
# the large-launch shapes, just above the small/large switch
# ---------------------------------------------------------------------------
def _large_T(R, bytes_per_elem, extra=3):
    """A ragged width whose (R, T) operands pass MALL_BYTES."""
    return MALL_BYTES // bytes_per_elem // R + extra


def _fused_rows_adam(p, g, m, v, mx, steps, hyp, mask, amsgrad, adamw, maximize):
    """torch's own fused Adam/AdamW on each active row, with that row's
    bumped step; returns the expected (p, m, v, mx)."""
    want = [t.clone() if t is not None else None for t in (p, m, v, mx)]
    fused = torch._fused_adamw_ if adamw else torch._fused_adam_
    lr, b1, b2, eps, wd = hyp
    for r in range(p.shape[0]):
        if not mask[r]:
            continue
        step = (steps[r].float() + 1).reshape(())
        fused([want[0][r]], [g[r].clone()], [want[1][r]], [want[2][r]],
              [want[3][r]] if amsgrad else [], [step], lr=lr[r].item(), beta1=b1[r].item(),
              beta2=b2[r].item(), weight_decay=wd[r].item(), eps=eps[r].item(), amsgrad=amsgrad,
              maximize=maximize, grad_scale=None, found_inf=None)
    return want


@pytest.mark.parametrize("workspace", [False, True], ids=["no_ws", "ws"])
@pytest.mark.parametrize("dtype,amsgrad,adamw,maximize", [
    (torch.float32, False, False, False), (torch.float32, True, True, True),
    (torch.float16, False, True, False), (torch.bfloat16, True, False, False),
    (torch.bfloat16, False, False, False), (torch.float64, False, True, True),
    (torch.float64, True, False, False)], ids=str)
def test_large_adam_rows_bit_identical_to_aten(dtype, amsgrad, adamw, maximize, workspace):
    R = 3
    bpe = torch.finfo(dtype).bits // 8 * (5 if amsgrad else 4)
    T = _large_T(R, bpe)
    g = torch.Generator(device=DEV).manual_seed(T)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)  # noqa: E731
    p, gr, m, v = rnd(), rnd(), rnd().abs(), rnd().abs()
    mx = rnd().abs() if amsgrad else None
    steps = torch.tensor([0, 5, 17], device=DEV, dtype=dtype)
    mask = torch.tensor([1, 0, 1], dtype=torch.uint8, device=DEV)
    eps = 1e-4 if dtype == torch.float16 else 1e-8
    hyp = [torch.tensor(h, device=DEV, dtype=torch.float32).to(dtype) for h in
           ([1e-2, 3e-3, 5e-2], [0.9, 0.8, 0.95], [0.999, 0.99, 0.9999], [eps] * 3, [1e-2] * 3)]
    want = _fused_rows_adam(p, gr, m, v, mx, steps, hyp, mask, amsgrad, adamw, maximize)
    frozen = [t[1].clone() for t in (p, m, v)]
    flags = (TS_BUMP_STEPS | (TS_AMSGRAD if amsgrad else 0) | (TS_ADAMW if adamw else 0)
             | (TS_MAXIMIZE if maximize else 0))
    bufs = [p, gr, m, v] + ([mx] if amsgrad else [])
    assert abi_step("adam", bufs, steps, hyp, mask, flags, dtype=dtype, workspace=workspace) == 0
    for name, got, w in (("params", p, want[0]), ("exp_avgs", m, want[1]),
                         ("exp_avg_sqs", v, want[2]), ("max_exp_avg_sqs", mx, want[3])):
        if got is None:
            continue
        for r in (0, 2):
            _same(f"{name}[{r}]", got[r], w[r])
    for t, f in zip((p, m, v), frozen):
        _same("frozen row", t[1], f)


@pytest.mark.parametrize("layout", ["small", "large", "strided"])
@pytest.mark.parametrize("dtype,amsgrad", [
    (torch.float32, False), (torch.float32, True), (torch.float16, False),
    (torch.bfloat16, False), (torch.float64, False)], ids=str)
def test_adam_constants_per_wavefront_match_workspace(dtype, amsgrad, layout):
    """Without a workspace the streaming and element drivers derive a
    replica's step size and sqrt(v) divisor once per wavefront, the two pow and
    the two divides spread over even and odd lanes; with one, the preparation
    launch derives them one thread per replica. Both must give the same bits
    for every replica: 512 replicas, each with its own lr, betas (up to
    1 - 1e-7) and step count (1 to 2^24 - 1), in MALL-resident and large
    streaming launches and with strided parameters (the element driver)."""
    R = 512
    bpe = torch.finfo(dtype).bits // 8 * (5 if amsgrad else 4)
    T = _large_T(R, bpe) if layout == "large" else 1003
    g = torch.Generator(device=DEV).manual_seed(R + T)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)  # noqa: E731
    ops = [rnd(), rnd(), rnd(), rnd().abs()] + ([rnd().abs()] if amsgrad else [])
    # strided: the parameters every other element of a (R, 2T) buffer (a
    # clone of such a view would be contiguous, so copies re-take the view)
    base = None
    if layout == "strided":
        base = torch.randn(R, 2 * T, device=DEV, generator=g, dtype=dtype)
        ops[0] = base[:, ::2]

    def copy(t, i):
        return base.clone()[:, ::2] if base is not None and i == 0 else t.clone()

    u = lambda: torch.rand(R, device=DEV, generator=g, dtype=torch.float64)  # noqa: E731
    steps = torch.floor(torch.exp(u() * math.log(2.0 ** 24 - 1))).clamp_(1, 2 ** 24 - 1)
    steps[:4] = torch.tensor([1.0, 2.0, 3.0, 2.0 ** 24 - 1], dtype=torch.float64)
    beta1 = 1 - torch.exp(u() * math.log(1e-7) * 0.5 - 0.1)
    beta2 = 1 - torch.exp(u() * math.log(1e-7))
    lr = torch.exp(math.log(1e-5) + u() * math.log(1e4))
    eps = torch.full((R,), 1e-4 if dtype == torch.float16 else 1e-8, dtype=torch.float64,
                     device=DEV)
    wd = u() * 1e-2
    hyp = [h.to(dtype) for h in (lr, beta1, beta2, eps, wd)]
    steps = steps.to(dtype)
    mask = (torch.rand(R, device=DEV, generator=g) < 0.9).to(torch.uint8)
    flags = TS_AMSGRAD if amsgrad else 0
    got = [copy(t, i) for i, t in enumerate(ops)]
    assert abi_step("adam", got, steps, hyp, mask, flags, dtype=dtype, workspace=False) == 0
    want = [copy(t, i) for i, t in enumerate(ops)]
    assert abi_step("adam", want, steps, hyp, mask, flags, dtype=dtype, workspace=True) == 0
    assert got[0].stride(1) == (2 if layout == "strided" else 1)
    for name, a, b in zip(("params", "grads", "exp_avgs", "exp_avg_sqs", "max_exp_avg_sqs"),
                          got, want):
        _same(name, a, b)
    assert not torch.equal(got[0], ops[0])


@pytest.mark.filterwarnings("ignore:`is_first_step` argument has no effect")
@pytest.mark.parametrize("dtype,has_buf,nesterov", [
    (torch.float32, True, True), (torch.float32, True, False), (torch.float32, False, False),
    (torch.float16, True, True), (torch.float64, True, False)], ids=str)
def test_large_sgd_rows_bit_identical_to_aten(dtype, has_buf, nesterov):
    R = 3
    bpe = torch.finfo(dtype).bits // 8 * (3 if has_buf else 2)
    T = _large_T(R, bpe, extra=1)
    g = torch.Generator(device=DEV).manual_seed(T + 1)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)  # noqa: E731
    p, gr = rnd(), rnd()
    mb = rnd() if has_buf else None
    steps = torch.tensor([0, 3, 6], device=DEV, dtype=dtype)  # row 0: first step
    mask = torch.tensor([1, 1, 0], dtype=torch.uint8, device=DEV)
    hyp = [torch.tensor(h, device=DEV, dtype=torch.float32).to(dtype) for h in
           ([1e-2, 3e-2, 2e-2], [0.9 if has_buf else 0.0] * 3, [0.1 if has_buf else 0.0] * 3,
            [1e-2] * 3)]
    want_p, want_b = p.clone(), mb.clone() if has_buf else None
    for r in range(2):
        torch._fused_sgd_([want_p[r]], [gr[r].clone()], [want_b[r]] if has_buf else [],
                          weight_decay=hyp[3][r].item(), momentum=hyp[1][r].item(),
                          lr=hyp[0][r].item(), dampening=hyp[2][r].item(), nesterov=nesterov,
                          maximize=False, is_first_step=steps[r].item() + 1 == 1,
                          grad_scale=None, found_inf=None)
    flags = TS_BUMP_STEPS | (TS_NESTEROV if nesterov else 0)
    assert abi_step("sgd", [p, gr, mb], steps, hyp, mask, flags, dtype=dtype) == 0
    for r in range(3):
        _same(f"params[{r}]", p[r], want_p[r])
        if has_buf:
            _same(f"momentum_buffers[{r}]", mb[r], want_b[r])


@pytest.mark.parametrize("workspace", [False, True], ids=["no_ws", "ws"])
@pytest.mark.parametrize("dtype,extra", [
    (torch.float32, 3), (torch.float64, 3), (torch.bfloat16, 3), (torch.float16, 3),
    (torch.float16, 4)], ids=str)
def test_large_adagrad_rows_bit_identical_to_aten(dtype, extra, workspace):
    """float16 twice: with ragged rows (torch's element path, the state sum
    rounded twice) and with rows a multiple of 4 long (its vector path,
    rounded once)."""
    R = 3
    T = _large_T(R, torch.finfo(dtype).bits // 8 * 3, extra)
    assert dtype != torch.float16 or (T % 4 == 0) == (extra == 4)
    g = torch.Generator(device=DEV).manual_seed(T + 2)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)  # noqa: E731
    p, gr, s = rnd(), rnd(), rnd().abs()
    steps = torch.tensor([0, 40, 7], device=DEV, dtype=dtype)
    mask = torch.tensor([1, 1, 0], dtype=torch.uint8, device=DEV)
    hyp = [torch.tensor(h, device=DEV, dtype=torch.float32).to(dtype) for h in
           ([1e-2, 3e-2, 2e-2], [1e-2] * 3, [1e-2] * 3, [1e-10] * 3)]
    want_p, want_s = p.clone(), s.clone()
    for r in range(2):
        st = (steps[r].float() + 1).reshape(())
        torch._fused_adagrad_([want_p[r]], [gr[r].clone()], [want_s[r]], [st],
                              lr=hyp[0][r].item(), lr_decay=hyp[1][r].item(),
                              weight_decay=hyp[2][r].item(), eps=hyp[3][r].item(),
                              maximize=False, grad_scale=None, found_inf=None)
    assert abi_step("adagrad", [p, gr, s], steps, hyp, mask, TS_BUMP_STEPS, dtype=dtype,
                    workspace=workspace) == 0
    for r in range(3):
        _same(f"params[{r}]", p[r], want_p[r])
        _same(f"state_sums[{r}]", s[r], want_s[r])


@pytest.mark.parametrize("op,workspace", _op_ws(["adam", "sgd", "adagrad", "adagrad_f32"]))
def test_large_float32_and_bf16_state_match_oracle(op, workspace):
    """float32 params with float32 and with bfloat16 optimizer state, large
    launches, against the oracle (bfloat16 state: the float32 step, then
    nearest-even rounding); the float32 Adagrad variant against the oracle's
    CPU form, which it reproduces."""
    kind = "adagrad" if op == "adagrad_f32" else op
    nstate = {"adam": 2, "sgd": 1, "adagrad": 1}[kind]
    for state_bf16 in (False, True):
        R = 3
        T = _large_T(R, 8 + nstate * (2 if state_bf16 else 4), extra=2)
        c = dict(op=kind, R=R, T=T, amsgrad=False, maximize=False, decoupled=False, wd=1e-2,
                 momentum="mixed", dampening=0.1, nesterov=True, lr_decay=1e-2, eps=1e-10,
                 hypers="distinct", mask="one_frozen", steps0=[0, 4, 9], nsteps=1, seed=T)
        x = C.make_inputs(c, state_bf16)
        names = _operand_names(c, x)
        want = C.run_oracle(c, O.CPU if op == "adagrad_f32" else O.DEVICE, state_bf16=state_bf16)
        sdt = torch.bfloat16 if state_bf16 else torch.float32
        dev = {k: torch.from_numpy(x[k].copy()).to(DEV) for k in names if k != "g"}
        dev["g"] = torch.from_numpy(x["grads"][0].copy()).to(DEV)
        for k in names[2:]:
            dev[k] = dev[k].to(sdt)
        steps = torch.from_numpy(x["steps"].copy()).to(DEV)
        mask = torch.from_numpy(x["mask"].astype(np.uint8)).to(DEV)
        hyp = [torch.from_numpy(x[k].copy()).to(DEV) for k in _hyper_names(c)]
        flags = (TS_BUMP_STEPS | (TS_STATE_BF16 if state_bf16 else 0) | _flags(c)
                 | (TS_ADAGRAD_F32 if op == "adagrad_f32" else 0))
        assert abi_step(kind, [dev[k] for k in names], steps, hyp, mask, flags,
                        workspace=workspace) == 0
        for k in names:
            if k == "g":
                continue
            got = dev[k].float().cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want[k].view(np.uint32)), (k, state_bf16)
        assert np.array_equal(steps.cpu().numpy(), want["steps"])

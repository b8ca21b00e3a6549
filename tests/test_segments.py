"""The gradient scatter fused into the update (``churten::*`` ops).

The reference's step is ``state._consolidated_grads.update_(grads)`` -- one
copy per parameter into the ``(N, T)`` gradient buffer -- followed by the fused
update (src/torchstrap/optimizer/grad_transform.py:29-30). The segmented ops
must leave every column exactly as that pair would: the GPU tests compare the
two bit for bit (the consolidated update itself is pinned to the oracle and to
torch's fused optimizers elsewhere), over aligned and ragged layouts, gaps,
more segments than one launch holds, strided and row-broadcast gradients,
strided state buffers, frozen replicas, every flag combination and all four
dtypes. The CPU tests cover the CPU key, validation and the ``State`` /
``apply_gradient`` plumbing.
"""

from __future__ import annotations

from copy import deepcopy

import pytest
import torch
from torch.nn import Linear, ReLU, Sequential

import churten_amd.kernels as K
from churten_amd.optimizer import SGD, Adagrad, Adam
from churten_amd.state import State

DTYPES = [torch.float32, torch.float64, torch.float16, torch.bfloat16]
INT_VIEW = {torch.float32: torch.int32, torch.float64: torch.int64,
            torch.float16: torch.int16, torch.bfloat16: torch.int16}


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(INT_VIEW[a.dtype]),
                       b.contiguous().view(INT_VIEW[b.dtype]))


# ---------------------------------------------------------------------------
# layouts
# ---------------------------------------------------------------------------
def layout(kind: str, seed: int):
    """(parameter shapes, column offsets, T)."""
    g = torch.Generator().manual_seed(seed)
    ri = lambda lo, hi: int(torch.randint(lo, hi, (), generator=g))  # noqa: E731
    if kind == "state":        # the State layout: packed from 0, pad to a multiple of 4
        shapes = [(10, 5), (10,), (1, 10), (1,)]
        gaps = [0, 0, 0, 0]
    elif kind == "ragged":     # odd offsets and gaps between parameters
        shapes = [(7,), (3, 5), (1,), (33, 3), (2, 2, 2)]
        gaps = [1, 2, 0, 3, 5]
    elif kind == "many":       # more segments than one launch table holds
        shapes = [(ri(1, 40),) for _ in range(150)]
        gaps = [ri(0, 2) for _ in range(150)]
    elif kind == "big":        # segments spanning several tiles
        shapes = [(3000, 2), (5,), (1025,), (4096,)]
        gaps = [0, 0, 0, 3]
    else:
        raise ValueError(kind)
    cols, c = [], 0
    for s, gap in zip(shapes, gaps):
        c += gap
        cols.append(c)
        c += int(torch.tensor(s).prod())
    T = c + ri(0, 6)
    return shapes, cols, T


def make_grads(shapes, R, dtype, device, gen, strided: bool):
    """(R, *shape) gradients; with ``strided`` some are transposed views and
    some broadcast one row to all replicas (row stride 0)."""
    out = []
    for i, s in enumerate(shapes):
        if strided and len(s) == 2 and i % 2 == 0:
            t = torch.randn(R, s[1], s[0], generator=gen).to(device, dtype).transpose(1, 2)
        elif strided and i % 3 == 1:
            t = torch.randn(1, *s, generator=gen).to(device, dtype).expand(R, *s)
        else:
            t = torch.randn(R, *s, generator=gen).to(device, dtype)
        out.append(t)
    return out


def at_offset(t, off: int):
    """A copy of ``t`` whose storage starts ``off`` elements into a flat buffer
    (data off the 16-byte grid for off % 4 != 0)."""
    flat = torch.empty(t.numel() + off, dtype=t.dtype, device=t.device)
    out = flat[off:].view(t.shape)
    out.copy_(t)
    return out


def column_view(t, off: int):
    """A copy of the (R, T) ``t`` as columns [off, off + T) of an (R, T + off + 1)
    buffer: rows start ``off`` elements past a boundary and the row stride
    changes residue."""
    R, T = t.shape
    buf = torch.empty(R, T + off + 1, dtype=t.dtype, device=t.device)
    out = buf[:, off:off + T]
    out.copy_(t)
    return out


def scatter_reference(dst, grads, cols):
    for g, c in zip(grads, cols):
        n = g[0].numel()
        dst[:, c:c + n].copy_(g.reshape(g.shape[0], n))


# ---------------------------------------------------------------------------
# per-optimizer argument builders: ((R, T) state, (R,) vectors, flags)
# ---------------------------------------------------------------------------
VARIANTS = [
    ("adam", dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)),
    ("adam", dict(amsgrad=True, maximize=True, decoupled_weight_decay=False)),
    ("adam", dict(amsgrad=True, maximize=False, decoupled_weight_decay=True)),
    ("sgd", dict(nesterov=False, maximize=False, buffers=True)),
    ("sgd", dict(nesterov=True, maximize=True, buffers=True)),
    ("sgd", dict(nesterov=False, maximize=False, buffers=False)),
    ("adagrad", dict(maximize=False)),
    ("adagrad", dict(maximize=True)),
]


def vid(v):
    op, kw = v
    return op + "-" + "-".join(k for k, x in kw.items() if x)


def make_state(op, kw, R, T, dtype, device, gen, strided_state=False, state_dtype=None):
    """(params, [state buffers], steps, [hyperparameters], flags); the state
    buffers are in ``state_dtype`` (default: ``dtype``)."""
    def rt(positive=False, as_state=True):
        t = torch.randn(R, T, generator=gen).to(dtype)
        t = t.abs() if positive else t
        if as_state and state_dtype is not None:
            t = t.to(state_dtype)
        return _to_dev_strided(t, device) if strided_state else t.to(device)

    def vec(lo, hi):
        return (lo + (hi - lo) * torch.rand(R, generator=gen)).to(device, dtype)

    steps = torch.zeros(R, dtype=dtype, device=device)  # SGD: first step comes first
    if op == "adam":
        st = [rt(), rt(True), rt(True) if kw["amsgrad"] else None]
        hyp = [vec(1e-3, 1e-2), vec(0.8, 0.95), vec(0.99, 0.9999), vec(1e-8, 1e-6),
               vec(0.0, 1e-2)]
        flags = dict(kw)
    elif op == "sgd":
        st = [rt() if kw["buffers"] else None]
        mom = vec(0.5, 0.9) if kw["buffers"] else torch.zeros(R, dtype=dtype, device=device)
        damp = (torch.zeros(R, dtype=dtype, device=device) if kw["nesterov"]
                else vec(0.0, 0.2))
        hyp = [vec(1e-3, 1e-1), mom, damp, vec(0.0, 1e-2)]
        flags = dict(nesterov=kw["nesterov"], maximize=kw["maximize"])
    else:
        st = [rt(True)]
        hyp = [vec(1e-3, 1e-1), vec(0.0, 0.1), vec(0.0, 1e-2), vec(1e-10, 1e-8)]
        flags = dict(kw)
    return rt(as_state=False), st, steps, hyp, flags


def _to_dev_strided(t, device):
    R, T = t.shape
    b = torch.empty(T, R, dtype=t.dtype, device=device).t()
    b.copy_(t.to(device))
    return b


def dense_call(op, params, grads, st, steps, hyp, mask, flags):
    if op == "adam":
        return K.adam_step_(params, grads, st[0], st[1], st[2], steps, *hyp, mask, **flags)
    if op == "sgd":
        return K.sgd_step_(params, grads, st[0], steps, *hyp, mask, **flags)
    return K.adagrad_step_(params, grads, st[0], steps, *hyp, mask, **flags)


def segments_call(op, params, grads, cols, grads_out, st, steps, hyp, mask, flags):
    if op == "adam":
        return K.adam_step_segments_(params, grads, cols, grads_out, st[0], st[1], st[2],
                                     steps, *hyp, mask, **flags)
    if op == "sgd":
        return K.sgd_step_segments_(params, grads, cols, grads_out, st[0], steps, *hyp, mask,
                                    **flags)
    return K.adagrad_step_segments_(params, grads, cols, grads_out, st[0], steps, *hyp, mask,
                                    **flags)


def clone_all(xs):
    return [x.clone() if x is not None else None for x in xs]


def run_both(device, op, kw, kind, dtype, with_out, strided_grads, strided_state, seed,
             n_steps=2, state_dtype=None, offset=0):
    """Runs ``n_steps`` segmented steps and the same steps as scatter +
    consolidated update, from identical starting state; returns both. With
    ``offset`` the segmented call's (R, T) operands are ``column_view``s and its
    gradients start ``offset`` elements into their storage."""
    R = 5
    shapes, cols, T = layout(kind, seed)
    gen = torch.Generator().manual_seed(seed + 100)
    p, st, steps, hyp, flags = make_state(op, kw, R, T, dtype, device, gen, strided_state,
                                          state_dtype)
    mask = torch.tensor([True, False, True, True, False], device=device)
    G0 = torch.randn(R, T, generator=gen).to(device, dtype)  # stale gradient contents
    a = dict(p=p, st=st, steps=steps, G=G0.clone() if with_out else None)
    if offset:
        a["p"] = column_view(p, offset)
        a["st"] = [column_view(x, offset) if x is not None else None for x in st]
        if with_out:
            a["G"] = column_view(G0, offset)
    b = dict(p=p.clone(), st=clone_all(st), steps=steps.clone(),
             G=G0.clone() if with_out else torch.zeros_like(G0))
    if offset and op == "adagrad" and dtype == torch.float16:
        # float16 Adagrad rounds its state once on the rows torch's fused kernel
        # runs on its vector path (aligned rows) and twice elsewhere: the
        # consolidated update runs on the same layout, so its rows agree
        b["p"] = column_view(p, offset)
        b["st"] = [column_view(x, offset) if x is not None else None for x in st]
        if with_out:
            b["G"] = column_view(G0, offset)
    for _ in range(n_steps):
        grads = make_grads(shapes, R, dtype, device, gen, strided_grads)
        seg_grads = [at_offset(g, offset) for g in grads] if offset else grads
        # order of the table must not matter
        order = list(reversed(range(len(grads))))
        out = segments_call(op, a["p"], [seg_grads[i] for i in order], [cols[i] for i in order],
                            a["G"], a["st"], a["steps"], hyp, mask, flags)
        assert out.shape == () and out.item() == 0
        if not with_out:
            b["G"].zero_()
        scatter_reference(b["G"], grads, cols)
        dense_call(op, b["p"], b["G"], b["st"], b["steps"], hyp, mask, flags)
    return a, b


def assert_same(a, b, with_out):
    assert bits_equal(a["p"], b["p"]), "params"
    for i, (x, y) in enumerate(zip(a["st"], b["st"])):
        if x is not None:
            assert bits_equal(x, y), f"state {i}"
    assert bits_equal(a["steps"], b["steps"]), "steps"
    if with_out:
        assert bits_equal(a["G"], b["G"]), "grads_out"


# ---------------------------------------------------------------------------
# GPU: segmented == scatter + consolidated update, bit for bit
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
@pytest.mark.parametrize("kind", ["state", "ragged", "many", "big"])
@pytest.mark.parametrize("with_out", [True, False], ids=["grads_out", "no_out"])
def test_gpu_segments_match_scatter_then_update(variant, kind, with_out):
    op, kw = variant
    a, b = run_both("cuda", op, kw, kind, torch.float32, with_out, strided_grads=False,
                    strided_state=False, seed=11)
    torch.cuda.synchronize()
    assert_same(a, b, with_out)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_gpu_segments_dtypes_and_strided_grads(variant, dtype):
    op, kw = variant
    a, b = run_both("cuda", op, kw, "ragged", dtype, True, strided_grads=True,
                    strided_state=False, seed=5)
    torch.cuda.synchronize()
    assert_same(a, b, True)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
@pytest.mark.parametrize("kind", ["state", "ragged", "many"])
def test_gpu_segments_bf16_state(variant, kind):
    """bfloat16 optimizer state next to float32 params, segmented vs dense."""
    op, kw = variant
    a, b = run_both("cuda", op, kw, kind, torch.float32, True, strided_grads=True,
                    strided_state=False, seed=8, state_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert_same(a, b, True)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
@pytest.mark.parametrize("kind", ["state", "many"])
def test_gpu_segments_strided_state_buffers(variant, kind):
    """(R, T) operands that are transposed views: no vector access anywhere."""
    op, kw = variant
    a, b = run_both("cuda", op, kw, kind, torch.float32, True, strided_grads=True,
                    strided_state=True, seed=3)
    torch.cuda.synchronize()
    assert_same(a, b, True)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
@pytest.mark.parametrize("offset", [1, 2, 3])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_gpu_segments_misaligned_operands(variant, offset, dtype):
    """(R, T) operands whose rows start off the 16-byte grid, with a row stride
    of another residue, and gradients at odd element offsets: the vector walk
    follows each consolidated row's own boundaries."""
    op, kw = variant
    for kind, with_out in (("big", True), ("ragged", False)):
        a, b = run_both("cuda", op, kw, kind, dtype, with_out, strided_grads=False,
                        strided_state=False, seed=21 + offset, offset=offset)
        torch.cuda.synchronize()
        assert_same(a, b, with_out)


@pytest.mark.gpu
@pytest.mark.parametrize("offset", [1, 2, 3])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_gpu_scatter_misaligned_destination(offset, dtype):
    R = 5
    shapes, cols, T = layout("big", 4)
    gen = torch.Generator().manual_seed(offset)
    grads = [at_offset(g, offset) for g in make_grads(shapes, R, dtype, "cuda", gen, False)]
    want = torch.randn(R, T, generator=gen).to("cuda", dtype)
    got = column_view(want, offset)
    scatter_reference(want, grads, cols)
    K.scatter_grads_(got, grads, cols)
    torch.cuda.synchronize()
    assert bits_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["state", "ragged", "many", "big"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_gpu_scatter_matches_per_parameter_copies(kind, dtype):
    R = 4
    shapes, cols, T = layout(kind, 2)
    gen = torch.Generator().manual_seed(9)
    grads = make_grads(shapes, R, dtype, "cuda", gen, strided=True)
    want = torch.randn(R, T, generator=gen).to("cuda", dtype)
    got = want.clone()
    scatter_reference(want, grads, cols)
    K.scatter_grads_(got, grads[::-1], cols[::-1])
    torch.cuda.synchronize()
    assert bits_equal(got, want)


@pytest.mark.gpu
def test_gpu_segments_reject_overlap_without_side_effects():
    R, T = 2, 16
    p = torch.zeros(R, T, device="cuda")
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    steps = torch.zeros(R, device="cuda")
    hyp = [torch.full((R,), x, device="cuda") for x in (1e-3, 0.9, 0.999, 1e-8, 0.0)]
    mask = torch.ones(R, dtype=torch.bool, device="cuda")
    g = [torch.ones(R, 8, device="cuda"), torch.ones(R, 4, device="cuda")]
    with pytest.raises(RuntimeError, match="overlaps"):
        K.adam_step_segments_(p, g, [0, 6], None, m, v, None, steps, *hyp, mask,
                              amsgrad=False, maximize=False, decoupled_weight_decay=True)
    with pytest.raises(RuntimeError, match="outside"):
        K.scatter_grads_(p, g, [0, 14])
    torch.cuda.synchronize()
    assert steps.tolist() == [0.0, 0.0] and not p.any()


# ---------------------------------------------------------------------------
# GPU: the fused training step through State / apply_gradient
# ---------------------------------------------------------------------------
def _net(device):
    torch.manual_seed(0)
    return Sequential(Linear(5, 10), ReLU(), Linear(10, 3), ReLU(), Linear(3, 1)).to(device)


def _grad_dicts(state, n, device, seed):
    g = torch.Generator().manual_seed(seed)
    # param_meta holds the stacked (N, *shape)
    return [{name: torch.randn(*shape, generator=g).to(device)
             for name, shape, _, _ in state.param_meta} for _ in range(n)]


OPTIMIZERS = [
    (Adam, dict(lr=1e-2, weight_decay=1e-2, amsgrad=True)),
    (SGD, dict(lr=1e-2, momentum=0.9, nesterov=True)),
    (SGD, dict(lr=1e-2)),
    (Adagrad, dict(lr=1e-2, lr_decay=1e-3, initial_accumulator_value=0.1)),
]


def _fused_vs_scatter(device, opt_cls, kw, keep_grads=True):
    net = _net(device)
    fused = State.from_models([deepcopy(net) for _ in range(4)])
    opt_cls.init(fused, **kw)
    fused.active_mask[2] = False
    plain = deepcopy(fused)
    for grads in _grad_dicts(fused, 3, device, 4):
        opt_cls.apply_gradient(fused, grads, keep_grads=keep_grads)
        plain._consolidated_grads.update_(grads)
        opt_cls.update(plain)
    return fused, plain


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
@pytest.mark.parametrize("opt_cls,kw", OPTIMIZERS, ids=lambda x: getattr(x, "__name__", ""))
def test_apply_gradient_fused_equals_scatter_then_update(device, opt_cls, kw):
    fused, plain = _fused_vs_scatter(device, opt_cls, kw)
    assert bits_equal(fused.params, plain.params)
    assert bits_equal(fused.grads, plain.grads)
    for k, v in plain.optimizer_state.items():
        if isinstance(v, torch.Tensor):
            assert bits_equal(fused.optimizer_state[k], v), k


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
def test_keep_grads_false_leaves_the_gradient_buffer(device):
    fused, plain = _fused_vs_scatter(device, Adam, dict(lr=1e-2), keep_grads=False)
    assert bits_equal(fused.params, plain.params)
    assert not fused.grads.any()


# ---------------------------------------------------------------------------
# CPU key, validation, plumbing
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
@pytest.mark.parametrize("with_out", [True, False], ids=["grads_out", "no_out"])
def test_cpu_segments_match_scatter_then_update(variant, with_out):
    op, kw = variant
    a, b = run_both("cpu", op, kw, "ragged", torch.float32, with_out, strided_grads=True,
                    strided_state=False, seed=1)
    assert_same(a, b, with_out)


@pytest.mark.parametrize("variant", VARIANTS, ids=vid)
def test_cpu_segments_bf16_state(variant):
    op, kw = variant
    a, b = run_both("cpu", op, kw, "ragged", torch.float32, True, strided_grads=True,
                    strided_state=False, seed=2, state_dtype=torch.bfloat16)
    assert_same(a, b, True)


@pytest.mark.parametrize("kind", ["state", "ragged", "many"])
def test_cpu_scatter_matches_per_parameter_copies(kind):
    shapes, cols, T = layout(kind, 0)
    gen = torch.Generator().manual_seed(1)
    grads = make_grads(shapes, 3, torch.float32, "cpu", gen, strided=True)
    want = torch.randn(3, T, generator=gen)
    got = want.clone()
    scatter_reference(want, grads, cols)
    K.scatter_grads_(got, grads, cols)
    assert torch.equal(got, want)


def test_segment_validation_errors():
    p = torch.zeros(2, 16)
    one = lambda n, r=2: torch.ones(r, n)  # noqa: E731
    with pytest.raises(RuntimeError, match="overlaps"):
        K.scatter_grads_(p, [one(8), one(4)], [0, 7])
    with pytest.raises(RuntimeError, match="outside"):
        K.scatter_grads_(p, [one(8)], [9])
    with pytest.raises(RuntimeError, match="outside"):
        K.scatter_grads_(p, [one(1)], [-1])
    with pytest.raises(RuntimeError, match="leading dimension"):
        K.scatter_grads_(p, [one(4, r=3)], [0])
    with pytest.raises(RuntimeError, match="dtype"):
        K.scatter_grads_(p, [one(4).double()], [0])
    with pytest.raises(RuntimeError, match="column offsets"):
        K.scatter_grads_(p, [one(4)], [0, 4])
    # empty gradients never overlap anything
    K.scatter_grads_(p, [one(8), one(0), one(8)], [0, 4, 8])
    assert torch.equal(p, torch.ones(2, 16))


def test_fake_kernels_on_meta():
    m = lambda *s: torch.empty(*s, device="meta")  # noqa: E731
    mask = torch.empty(3, dtype=torch.bool, device="meta")
    out = K.adam_step_segments_(m(3, 8), [m(3, 2, 2)], [0], None, m(3, 8), m(3, 8), None,
                                m(3), m(3), m(3), m(3), m(3), m(3), mask, amsgrad=False,
                                maximize=False, decoupled_weight_decay=True)
    assert out.shape == () and out.device.type == "meta"
    out = K.sgd_step_segments_(m(3, 8), [m(3, 4)], [4], m(3, 8), None, m(3), m(3), m(3),
                               m(3), m(3), mask, nesterov=False, maximize=False)
    assert out.shape == ()
    out = K.adagrad_step_segments_(m(3, 8), [m(3, 4)], [4], None, m(3, 8), m(3), m(3), m(3),
                                   m(3), m(3), mask, maximize=False)
    assert out.shape == ()


def test_apply_gradient_falls_back_to_the_scatter_when_needed(monkeypatch):
    """Partial dicts, broadcast gradients and subclasses that override update
    take the scatter + update path."""
    calls = []
    real = Adam.update_segments.__func__

    def spy(cls, *a):
        calls.append(cls)
        return real(cls, *a)

    monkeypatch.setattr(Adam, "update_segments", classmethod(spy))
    state = State.from_models([_net("cpu") for _ in range(2)])
    Adam.init(state, lr=1e-2)
    full = _grad_dicts(state, 1, "cpu", 0)[0]
    Adam.apply_gradient(state, full)
    assert calls == [Adam]
    partial = dict(list(full.items())[:2])
    Adam.apply_gradient(state, partial)
    shared = {k: v[0] for k, v in full.items()}  # (*shape): broadcast over replicas
    Adam.apply_gradient(state, shared)
    assert calls == [Adam]
    assert torch.equal(state._consolidated_grads["0.weight"][1], full["0.weight"][0])

    class MyAdam(Adam):
        @classmethod
        def init(cls, state, **kw):
            return Adam.init(state, **kw)

        @classmethod
        def update(cls, state, **kw):
            calls.append("custom")
            return Adam.update(state, **kw)

    MyAdam.apply_gradient(state, full)
    assert calls == [Adam, "custom"]


def test_state_gradient_scatter_uses_one_launch_or_copies():
    state = State.from_models([_net("cpu") for _ in range(3)])
    grads = _grad_dicts(state, 1, "cpu", 3)[0]
    state._consolidated_grads.update_(grads)
    for name, shape, off, n in state.param_meta:
        assert torch.equal(state.grads[:, off:off + n], grads[name].reshape(3, n))
    # a float64 gradient is converted by the per-name path
    state._consolidated_grads.update_({"0.bias": torch.ones(3, 10, dtype=torch.float64)})
    assert torch.equal(state._consolidated_grads["0.bias"], torch.ones(3, 10))


# ---------------------------------------------------------------------------
# torch.library.opcheck: schema / alias annotations, fake kernels, dispatch
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
def test_opcheck_churten_ops(device):
    R, T = 3, 24
    g = torch.Generator().manual_seed(0)
    rnd = lambda *s: torch.randn(*s, generator=g).to(device)  # noqa: E731
    vec = lambda x: torch.full((R,), x, device=device)  # noqa: E731
    mask = torch.tensor([True, False, True], device=device)
    grads, cols = [rnd(R, 2, 5), rnd(R, 7)], [0, 12]
    torch.library.opcheck(torch.ops.churten.scatter_grads_.default,
                          (torch.zeros(R, T, device=device), grads, cols))
    torch.library.opcheck(
        torch.ops.churten.adam_step_segments_.default,
        (rnd(R, T), grads, cols, torch.zeros(R, T, device=device), rnd(R, T), rnd(R, T).abs(),
         None, vec(1.0), vec(1e-2), vec(0.9), vec(0.999), vec(1e-8), vec(0.0), mask, False,
         False, True))
    torch.library.opcheck(
        torch.ops.churten.sgd_step_segments_.default,
        (rnd(R, T), grads, cols, None, rnd(R, T), vec(2.0), vec(1e-2), vec(0.9), vec(0.0),
         vec(0.0), mask, True, False))
    torch.library.opcheck(
        torch.ops.churten.adagrad_step_segments_.default,
        (rnd(R, T), grads, cols, None, rnd(R, T).abs(), vec(1.0), vec(1e-2), vec(0.0),
         vec(0.0), vec(1e-10), mask, False, True))
    torch.library.opcheck(
        torch.ops.churten.adagrad_step_f32_.default,
        (rnd(R, T), rnd(R, T), rnd(R, T).abs(), vec(1.0), vec(1e-2), vec(0.0), vec(0.0),
         vec(1e-10), mask, False))

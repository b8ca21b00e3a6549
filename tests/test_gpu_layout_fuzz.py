"""Seeded random layouts through every driver, bit for bit against contiguous
buffers.

The drivers pick their access pattern from the operands' strides and
alignment (streaming rows with a per-row head tile before the first boundary
of the tile size, replica-minor columns, element-wise otherwise; per-parameter
gradients at any column offset). Every choice must give the bits the
contiguous layout gives, since all drivers share one element update. These
cases draw the layout at random -- row width, column offset inside a wider
buffer, row padding, transposed storage, mixed layouts across operands,
parameter dtype, bfloat16 state, optimizer and flags, frozen replicas -- and
compare each against the same step on contiguous copies.

One exception follows torch: float16 Adagrad rounds the state sum once on rows
that torch's fused kernel runs on its vector path and twice elsewhere, so each
of its rows is compared with contiguous copies whose rows take the same path
(the plain copies, or copies one element off alignment).
"""

from __future__ import annotations

import math
import random

import pytest
import torch

import churten_amd.kernels as K

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
INT_VIEW = {torch.float32: torch.int32, torch.float64: torch.int64,
            torch.float16: torch.int16, torch.bfloat16: torch.int16}


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(INT_VIEW[a.dtype]), b.contiguous().view(INT_VIEW[b.dtype]))


def placed(t: torch.Tensor, kind: str, off: int, pad: int) -> torch.Tensor:
    """The (R, T) values of ``t`` in a given storage layout."""
    R, T = t.shape
    if kind == "rows":          # columns [off, off + T) of an (R, T + off + pad) buffer
        buf = torch.empty(R, T + off + pad, dtype=t.dtype, device=t.device)
        v = buf[:, off:off + T]
    elif kind == "cols":        # a (T, R + pad) buffer seen as (R, T)
        buf = torch.empty(T, R + pad, dtype=t.dtype, device=t.device)
        v = buf[:, :R].t()
    else:                       # every other column of a wider buffer
        buf = torch.empty(R, 2 * T + off, dtype=t.dtype, device=t.device)
        v = buf[:, off:off + 2 * T:2]
    v.copy_(t)
    return v


def vector_rows(ops) -> torch.Tensor:
    """Per row of (R, T) operands, ATen's vector-path condition: the length a
    multiple of 4, unit inner stride, row pointers aligned to 4 elements."""
    R = ops[0].shape[0]
    return torch.tensor([all(t.shape[1] % 4 == 0 and t.stride(1) == 1 and
                             t[r].data_ptr() % (4 * t.element_size()) == 0 for t in ops)
                         for r in range(R)], device=DEV)


def draw(rng: random.Random):
    op = rng.choice(["adam", "adam_ams", "adamw", "sgd", "sgd_nesterov", "sgd_nobuf", "adagrad",
                     "adagrad_f32"])
    dtype = rng.choice([torch.float32, torch.float32, torch.float64, torch.float16,
                        torch.bfloat16])
    if op == "adagrad_f32" and dtype == torch.float64:
        dtype = torch.float32
    bf16_state = dtype == torch.float32 and op != "sgd_nobuf" and rng.random() < 0.3
    R = rng.choice([1, 2, 3, 5, 8, 17, 64, 65])
    T = rng.choice([1, 3, 4, 7, 63, 64, 65, 255, 257, 1000, 2049, 4103])
    kinds = rng.choice([("rows",), ("cols",), ("step",), ("rows", "cols"), ("rows", "step")])
    return dict(op=op, dtype=dtype, bf16_state=bf16_state, R=R, T=T, kinds=kinds,
                off=rng.randrange(0, 130), pad=rng.randrange(0, 70), seed=rng.randrange(1 << 30))


def run_case(c):
    g = torch.Generator(device=DEV).manual_seed(c["seed"])
    R, T, dt = c["R"], c["T"], c["dtype"]
    sdt = torch.bfloat16 if c["bf16_state"] else dt
    rnd = lambda dtype=dt: torch.randn(R, T, device=DEV, generator=g).to(dtype)  # noqa: E731
    pos = lambda dtype=dt: rnd(dtype).abs()  # noqa: E731
    vec = lambda lo, hi: (lo + (hi - lo) * torch.rand(R, device=DEV, generator=g)).to(dt)  # noqa
    mask = torch.rand(R, device=DEV, generator=g) < 0.75
    op = c["op"]
    if op.startswith("adam"):
        ams = op == "adam_ams"
        bufs = [rnd(), rnd(), rnd(sdt), pos(sdt)] + ([pos(sdt)] if ams else [])
        steps = torch.randint(1, 20, (R,), device=DEV, generator=g).to(dt)
        hyp = [vec(1e-3, 1e-2), vec(0.8, 0.95), vec(0.99, 0.9999), vec(1e-8, 1e-6), vec(0, 1e-2)]
        kw = dict(amsgrad=ams, maximize=bool(c["seed"] & 1), decoupled_weight_decay=op == "adamw")

        def step(b, s):
            K.adam_step_(b[0], b[1], b[2], b[3], b[4] if ams else None, s, *hyp, mask, **kw)
    elif op.startswith("sgd"):
        has_buf = op != "sgd_nobuf"
        bufs = [rnd(), rnd()] + ([rnd(sdt)] if has_buf else [])
        steps = torch.randint(0, 3, (R,), device=DEV, generator=g).to(dt)
        mom = vec(0.5, 0.9) if has_buf else torch.zeros(R, device=DEV, dtype=dt)
        nest = op == "sgd_nesterov"
        damp = torch.zeros(R, device=DEV, dtype=dt) if nest else vec(0, 0.2)
        hyp = [vec(1e-3, 1e-1), mom, damp, vec(0, 1e-2)]

        def step(b, s):
            K.sgd_step_(b[0], b[1], b[2] if has_buf else None, s, *hyp, mask, nesterov=nest,
                        maximize=bool(c["seed"] & 1))
    else:
        bufs = [rnd(), rnd(), pos(sdt)]
        steps = torch.randint(1, 20, (R,), device=DEV, generator=g).to(dt)
        hyp = [vec(1e-3, 1e-1), vec(0, 0.1), vec(0, 1e-2), vec(1e-10, 1e-8)]
        f = K.adagrad_step_f32_ if op == "adagrad_f32" else K.adagrad_step_

        def step(b, s):
            f(b[0], b[1], b[2], s, *hyp, mask, maximize=bool(c["seed"] & 1))
    kinds = c["kinds"]
    # operands differ in offset (rows: other 16-byte phases) and padding (cols:
    # other column strides)
    view = [placed(t, kinds[i % len(kinds)], c["off"] + i, c["pad"] + 3 * i)
            for i, t in enumerate(bufs)]
    dense = [t.clone() for t in bufs]
    s_view, s_dense = steps.clone(), steps.clone()
    for _ in range(2):
        step(view, s_view)
        step(dense, s_dense)
    if op == "adagrad" and dt == torch.float16:
        # the same rows of the element path: row stride T + 4, one element in
        off_path = [placed(t, "rows", 1, 3) for t in bufs]
        s_off = steps.clone()
        for _ in range(2):
            step(off_path, s_off)
        on = vector_rows(view).view(R, 1)
        dense = [torch.where(on, b, e) for b, e in zip(dense, off_path)]
    torch.cuda.synchronize()
    assert torch.equal(s_view, s_dense)
    for i, (a, b) in enumerate(zip(view, dense)):
        assert same_bits(a, b), f"operand {i}"


CASES = [draw(random.Random(1000 + i)) for i in range(240)]


@pytest.mark.parametrize("c", CASES, ids=lambda c: (
    f"{c['op']}-{str(c['dtype'])[6:]}{'-bf16s' if c['bf16_state'] else ''}-R{c['R']}-T{c['T']}-"
    f"{'+'.join(c['kinds'])}-o{c['off']}-p{c['pad']}"))
def test_random_layout_matches_contiguous(c):
    run_case(c)


def _wide(rng: random.Random):
    """Replica counts past one column-driver replica block (256), narrow rows."""
    c = draw(rng)
    c["R"] = rng.choice([257, 300, 512, 1000, 1024, 1030, 2048, 4096])
    c["T"] = rng.choice([1, 3, 33, 64, 65, 129, 300])
    return c


WIDE_CASES = [_wide(random.Random(400000 + i)) for i in range(80)]


@pytest.mark.parametrize("c", WIDE_CASES, ids=lambda c: (
    f"{c['op']}-{str(c['dtype'])[6:]}{'-bf16s' if c['bf16_state'] else ''}-R{c['R']}-T{c['T']}-"
    f"{'+'.join(c['kinds'])}-o{c['off']}-p{c['pad']}"))
def test_random_layout_many_replicas_matches_contiguous(c):
    run_case(c)


def _seg_case(rng: random.Random):
    dtype = rng.choice([torch.float32, torch.float32, torch.float64, torch.float16,
                        torch.bfloat16])
    bf16_state = dtype == torch.float32 and rng.random() < 0.4
    n = rng.randrange(1, 9)
    shapes = [tuple(rng.choice([1, 2, 3, 5, 31, 64, 129, 300]) for _ in range(rng.randrange(1, 3)))
              for _ in range(n)]
    gaps = [rng.randrange(0, 5) for _ in range(n)]
    return dict(dtype=dtype, bf16_state=bf16_state, shapes=shapes, gaps=gaps,
                R=rng.choice([2, 5, 9]), off=rng.randrange(0, 70), tail=rng.randrange(0, 9),
                with_out=rng.random() < 0.5, goff=rng.randrange(0, 4), seed=rng.randrange(1 << 30))


SEG_CASES = [_seg_case(random.Random(5000 + i)) for i in range(80)]


@pytest.mark.parametrize("c", SEG_CASES, ids=lambda c: (
    f"{str(c['dtype'])[6:]}{'-bf16s' if c['bf16_state'] else ''}-n{len(c['shapes'])}-R{c['R']}-"
    f"o{c['off']}-g{c['goff']}{'-out' if c['with_out'] else ''}"))
def test_random_segment_layout_matches_scatter_then_update(c):
    """Adam over per-parameter gradients at random column offsets, gradients at
    random storage offsets, (R, T) operands at a random column offset: equal to
    the scatter followed by the dense update, bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(c["seed"])
    R, dt = c["R"], c["dtype"]
    sdt = torch.bfloat16 if c["bf16_state"] else dt
    cols, col = [], 0
    for s, gap in zip(c["shapes"], c["gaps"]):
        col += gap
        cols.append(col)
        col += math.prod(s)
    T = col + c["tail"]
    rnd = lambda dtype=dt: torch.randn(R, T, device=DEV, generator=g).to(dtype)  # noqa: E731
    p, m, v, G0 = rnd(), rnd(sdt), rnd(sdt).abs(), rnd()
    steps = torch.randint(1, 9, (R,), device=DEV, generator=g).to(dt)
    hyp = [torch.full((R,), x, device=DEV, dtype=dt) for x in (1e-2, 0.9, 0.999, 1e-8, 1e-2)]
    mask = torch.rand(R, device=DEV, generator=g) < 0.7
    kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
    grads = []
    for s in c["shapes"]:
        t = torch.randn(R, *s, device=DEV, generator=g).to(dt)
        flat = torch.empty(t.numel() + c["goff"], device=DEV, dtype=dt)
        tv = flat[c["goff"]:].view(t.shape)
        tv.copy_(t)
        grads.append(tv)
    a = [placed(t, "rows", c["off"], 3) for t in (p, m, v)]
    a_G = placed(G0, "rows", c["off"], 3) if c["with_out"] else None
    b = [t.clone() for t in (p, m, v)]
    b_G = G0.clone() if c["with_out"] else torch.zeros_like(G0)
    s_a, s_b = steps.clone(), steps.clone()
    K.adam_step_segments_(a[0], grads, cols, a_G, a[1], a[2], None, s_a, *hyp, mask, **kw)
    for t, c0 in zip(grads, cols):
        n = t[0].numel()
        b_G[:, c0:c0 + n].copy_(t.reshape(R, n))
    K.adam_step_(b[0], b_G, b[1], b[2], None, s_b, *hyp, mask, **kw)
    torch.cuda.synchronize()
    assert torch.equal(s_a, s_b)
    for i, (x, y) in enumerate(zip(a, b)):
        assert same_bits(x, y), f"operand {i}"
    if c["with_out"]:
        assert same_bits(a_G, b_G), "grads_out"

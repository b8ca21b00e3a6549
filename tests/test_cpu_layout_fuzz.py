"""Seeded random layouts through the CPU dispatch key, bit for bit against the
oracle's CPU formulation.

The reference's CPU kernels (src/torchstrap/kernels/csrc/cpu/adam.cpp:263-269,
sgd.cpp, adagrad.cpp) take an 8-lane vector body plus a scalar tail only when
every (R, T) operand has unit inner stride, and the scalar formulation for the
whole row otherwise; rows are cut into 16384-element chunks
(cpu/consolidated.h:26) so the tail sits only at the end of a row. These cases
draw the layout at random -- row width across chunk boundaries, column offset
inside a wider buffer, transposed storage, every-other-column views, mixed
layouts across operands, strided per-replica inputs, bfloat16 state, optimizer
and flags, frozen replicas -- run two steps through ``torch.ops.torchstrap.*``
on CPU tensors, and compare every output with ``oracle.*_step(CPU, ...,
unit_stride=...)`` on contiguous copies, where ``unit_stride`` is what the
operands' strides select. bfloat16 state is widened to a row-major float32
copy, so for it only the params' and grads' strides decide.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

import churten_amd.kernels  # noqa: F401
from oracle import oracle as O

OPS = ["adam", "adam_ams", "adamw", "sgd", "sgd_nesterov", "sgd_nobuf", "adagrad"]


def placed(t: torch.Tensor, kind: str, off: int, pad: int) -> torch.Tensor:
    """The (R, T) values of ``t`` in a given storage layout."""
    R, T = t.shape
    if kind == "rows":          # columns [off, off + T) of an (R, T + off + pad) buffer
        v = torch.empty(R, T + off + pad, dtype=t.dtype)[:, off:off + T]
    elif kind == "cols":        # a (T, R + pad) buffer seen as (R, T)
        v = torch.empty(T, R + pad, dtype=t.dtype)[:, :R].t()
    else:                       # every other column of a wider buffer
        v = torch.empty(R, 2 * T + off, dtype=t.dtype)[:, off:off + 2 * T:2]
    v.copy_(t)
    return v


def placed_vec(x: np.ndarray, strided: bool, col: int) -> torch.Tensor:
    """An (R,) per-replica input, contiguous or a column of an (R, 3) matrix."""
    t = torch.from_numpy(x.copy())
    if not strided:
        return t
    buf = torch.zeros(len(x), 3, dtype=t.dtype)
    buf[:, col] = t
    return buf[:, col]


def draw(rng: random.Random):
    op = rng.choice(OPS)
    return dict(
        op=op, bf16_state=op != "sgd_nobuf" and rng.random() < 0.25,
        R=rng.choice([1, 2, 3, 5, 8, 17]),
        T=rng.choice([1, 7, 8, 9, 63, 64, 1000, 16383, 16384, 16391, 32775, 40000]),
        kinds=rng.choice([("rows",), ("cols",), ("step",), ("rows", "cols"), ("rows", "step"),
                          ("cols", "rows")]),
        off=rng.randrange(0, 40), pad=rng.randrange(0, 9), vec_strided=rng.random() < 0.3,
        maximize=rng.random() < 0.5, seed=rng.randrange(1 << 30))


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def bf16_values(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(a).to(torch.bfloat16).float().numpy()


def run_case(c):
    rs = np.random.RandomState(c["seed"] & 0x7FFFFFFF)
    R, T, op = c["R"], c["T"], c["op"]
    rnd = lambda: rs.standard_normal((R, T)).astype(np.float32)  # noqa: E731
    pos = lambda: np.abs(rnd())  # noqa: E731
    vec = lambda lo, hi: (lo + (hi - lo) * rs.random_sample(R)).astype(np.float32)  # noqa: E731
    mask = rs.random_sample(R) < 0.75
    sb = c["bf16_state"]
    if op.startswith("adam"):
        ams = op == "adam_ams"
        names = ["p", "g", "m", "v"] + (["mx"] if ams else [])
        arrs = [rnd(), rnd(), rnd(), pos()] + ([pos()] if ams else [])
        steps = rs.randint(0, 20, R).astype(np.float32)
        hyp = [vec(1e-3, 1e-2), vec(0.8, 0.95), vec(0.99, 0.9999), vec(1e-8, 1e-6), vec(0, 1e-2)]
        kw = dict(amsgrad=ams, maximize=c["maximize"], decoupled_weight_decay=op == "adamw")

        def product(t, s, h, mk):
            torch.ops.torchstrap.adam_step_(t[0], t[1], t[2], t[3], t[4] if ams else None, s,
                                            *h, mk, **kw)

        def oracle(a, s, unit):
            O.adam_step(O.CPU, a[0], a[1], a[2], a[3], a[4] if ams else None, s, *hyp, mask,
                        unit_stride=unit, state_bf16=sb, **kw)
    elif op.startswith("sgd"):
        buf = op != "sgd_nobuf"
        nest = op == "sgd_nesterov"
        names = ["p", "g"] + (["mb"] if buf else [])
        arrs = [rnd(), rnd()] + ([rnd()] if buf else [])
        steps = rs.randint(0, 3, R).astype(np.float32)
        mom = vec(0.5, 0.9) if buf else np.zeros(R, np.float32)
        damp = np.zeros(R, np.float32) if nest else vec(0, 0.2)
        hyp = [vec(1e-3, 1e-1), mom, damp, vec(0, 1e-2)]

        def product(t, s, h, mk):
            torch.ops.torchstrap.sgd_step_(t[0], t[1], t[2] if buf else None, s, *h, mk,
                                           nesterov=nest, maximize=c["maximize"])

        def oracle(a, s, unit):
            O.sgd_step(O.CPU, a[0], a[1], a[2] if buf else None, s, *hyp, mask, nesterov=nest,
                       maximize=c["maximize"], unit_stride=unit, state_bf16=sb)
    else:
        names = ["p", "g", "s"]
        arrs = [rnd(), rnd(), pos()]
        steps = rs.randint(0, 20, R).astype(np.float32)
        hyp = [vec(1e-3, 1e-1), vec(0, 0.1), vec(0, 1e-2), vec(1e-10, 1e-8)]

        def product(t, s, h, mk):
            torch.ops.torchstrap.adagrad_step_(t[0], t[1], t[2], s, *h, mk,
                                               maximize=c["maximize"])

        def oracle(a, s, unit):
            O.adagrad_step(O.CPU, a[0], a[1], a[2], s, *hyp, mask, maximize=c["maximize"],
                           unit_stride=unit, state_bf16=sb)
    if sb:                      # state starts bfloat16-valued
        arrs = arrs[:2] + [bf16_values(a) for a in arrs[2:]]
    kinds = c["kinds"]
    views = []
    for i, a in enumerate(arrs):
        t = torch.from_numpy(a.copy())
        if sb and i >= 2:
            t = t.to(torch.bfloat16)
        # operands differ in offset and padding
        views.append(placed(t, kinds[i % len(kinds)], c["off"] + i, c["pad"] + 3 * i))
    decide = views[:2] if sb else views
    unit = all(v.stride(1) == 1 for v in decide)
    vs = c["vec_strided"]
    s_t = placed_vec(steps, vs, 1)
    h_t = [placed_vec(h, vs, i % 3) for i, h in enumerate(hyp)]
    m_t = placed_vec(mask, vs, 2)
    ref = [a.copy() for a in arrs]
    s_ref = steps.copy()
    for _ in range(2):
        product(views, s_t, h_t, m_t)
        oracle(ref, s_ref, unit)
    np.testing.assert_array_equal(s_t.numpy(), s_ref)
    for name, v, r, a0 in zip(names, views, ref, arrs):
        got = v.float().contiguous().numpy()
        bad = np.flatnonzero(bits(got) != bits(r))
        assert bad.size == 0, (
            f"{name}: {bad.size} elements differ (unit_stride={unit}), first at "
            f"{np.unravel_index(bad[0], got.shape)}: {got.flat[bad[0]]!r} vs {r.flat[bad[0]]!r}")
        frozen = ~mask
        assert np.array_equal(bits(got[frozen]), bits(a0[frozen])), f"{name}: frozen row changed"


CASES = [draw(random.Random(9000 + i)) for i in range(160)]


@pytest.mark.parametrize("c", CASES, ids=lambda c: (
    f"{c['op']}{'-bf16s' if c['bf16_state'] else ''}-R{c['R']}-T{c['T']}-"
    f"{'+'.join(c['kinds'])}-o{c['off']}-p{c['pad']}{'-vs' if c['vec_strided'] else ''}"))
def test_cpu_random_layout_matches_oracle_cpu_form(c):
    run_case(c)

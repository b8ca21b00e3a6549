"""Operator semantics on the GPU: freeze/thaw, vmap, layouts, edge cases,
errors, dtypes and torch.library registration.

Mirrors the reference's tiers 3-5 (test/optimizer/test_inplace_*_masking.py,
test_inplace_*_vmap.py, test_cpu_cuda_*_parity.py's opcheck) on the MI355X.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.func import vmap

import churten_amd.kernels as K
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def full(R, x, dtype=torch.float32):
    return torch.full((R,), x, device=DEV, dtype=dtype)


def adam_args(R, T, amsgrad=False, seed=0, steps=2.0, dtype=torch.float32):
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g).to(dtype)  # noqa: E731
    st = [rnd(), rnd(), rnd().abs(), rnd().abs(), rnd().abs() if amsgrad else None]
    return st + [full(R, steps, dtype), full(R, 1e-2, dtype), full(R, 0.9, dtype),
                 full(R, 0.999, dtype), full(R, 1e-8, dtype), full(R, 1e-2, dtype)]


# ---------------------------------------------------------------------------
# freeze semantics (reference test_inplace_adam_masking.py:50-111)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("inactive", [[], [2], [0, 3], [0, 1, 2, 3, 4]])
@pytest.mark.parametrize("amsgrad", [False, True])
def test_adam_frozen_rows_bit_identical(inactive, amsgrad):
    R, T = 5, 4 * 6 + 6 + 3 + 3
    a = adam_args(R, T, amsgrad, seed=7)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    mask[inactive] = False
    before = [t.clone() if t is not None else None for t in a]
    K.adam_step_(*a, mask, amsgrad=amsgrad, maximize=False, decoupled_weight_decay=True)
    torch.cuda.synchronize()
    act = mask.nonzero().flatten()
    frz = (~mask).nonzero().flatten()
    for i in (0, 2, 3, 4, 5):
        if a[i] is None:
            continue
        assert torch.equal(a[i][frz], before[i][frz]), f"arg {i} frozen rows changed"
        if len(act) and i != 4:
            assert not torch.equal(a[i][act], before[i][act]), f"arg {i} active rows unchanged"


def test_adam_step0_freeze_never_reads_state():
    """A replica frozen at step 0 would give 1 - beta^0 = 0 and NaN if computed;
    its rows (even NaN-filled ones) must stay untouched and NaN-free elsewhere."""
    R, T = 3, 64
    a = adam_args(R, T, steps=0.0)
    a[0][1] = float("nan")
    mask = torch.tensor([True, False, True], device=DEV)
    K.adam_step_(*a, mask, amsgrad=False, maximize=False, decoupled_weight_decay=False)
    torch.cuda.synchronize()
    assert torch.isnan(a[0][1]).all()
    assert torch.isfinite(a[0][[0, 2]]).all()
    assert a[5].tolist() == [1.0, 0.0, 1.0]


def test_sgd_frozen_at_step0_then_thawed_gets_buf_equal_grad():
    """Reference test_inplace_sgd_masking.py:102-140: a replica frozen before its
    first step keeps a pristine buffer; on thaw its first step has buf == grad."""
    R, T = 3, 52
    g = torch.Generator(device=DEV).manual_seed(3)
    p = torch.randn(R, T, device=DEV, generator=g)
    mb = torch.randn(R, T, device=DEV, generator=g)
    steps = torch.zeros(R, device=DEV)
    hyp = (full(R, 1e-2), full(R, 0.9), full(R, 0.0), full(R, 0.0))
    mask = torch.tensor([True, False, True], device=DEV)
    mb_before = mb.clone()
    for _ in range(2):
        grad = torch.randn(R, T, device=DEV, generator=g)
        K.sgd_step_(p, grad, mb, steps, *hyp, mask, nesterov=False, maximize=False)
    assert torch.equal(mb[1], mb_before[1])
    assert steps.tolist() == [2.0, 0.0, 2.0]
    grad = torch.randn(R, T, device=DEV, generator=g)
    K.sgd_step_(p, grad, mb, steps, *hyp, torch.ones(R, dtype=torch.bool, device=DEV),
                nesterov=False, maximize=False)
    torch.cuda.synchronize()
    assert torch.equal(mb[1], grad[1])
    assert steps.tolist() == [3.0, 1.0, 3.0]


def test_sgd_momentum0_replica_is_plain_sgd():
    """A momentum-0 replica inside a buffered call: buf = grad, p -= lr * grad."""
    R, T = 2, 1000
    g = torch.Generator(device=DEV).manual_seed(4)
    p = torch.randn(R, T, device=DEV, generator=g)
    mb = torch.randn(R, T, device=DEV, generator=g)
    steps = torch.full((R,), 5.0, device=DEV)
    grad = torch.randn(R, T, device=DEV, generator=g)
    p0 = p.clone()
    K.sgd_step_(p, grad, mb, steps, full(R, 0.25), torch.tensor([0.0, 0.9], device=DEV),
                full(R, 0.0), full(R, 0.0), torch.ones(R, dtype=torch.bool, device=DEV),
                nesterov=False, maximize=False)
    torch.cuda.synchronize()
    assert torch.equal(mb[0], grad[0])
    assert torch.equal(p[0], p0[0] - 0.25 * grad[0])  # lr a power of 2: exact


@pytest.mark.parametrize("nesterov", [True, False], ids=["nesterov", "plain"])
def test_sgd_momentum0_replica_with_dampening(nesterov):
    """BASELINE config 3's combination (dampening 0.1, nesterov) on momentum-0
    replicas inside a buffered call; ATen's fused SGD cannot express a
    per-replica momentum of 0 next to buffered ones, so the values come from
    the mathematics (reference cuda/sgd.cu:117-130 with momentum 0, in double):
    - after its first step the buffer is fma(0, buf, (1-d)*g) = (1-d)*g, exact
      in double ((1-d) has at most 28 significant bits, g 24), so the stored
      buffer is RN32((1-d)*g);
    - on its first step the buffer is g;
    - the parameter moves by lr times g (nesterov: g + 0*buf) or times the
      buffer narrowed to float (no nesterov: ATen assigns it to the float
      gradient); with lr a power of 2 that product is exact and p - lr*x is
      rounded to double and then to float, as computed here.
    Beside them: a momentum-0.9 replica and a frozen momentum-0 replica."""
    R, T = 4, 1000
    d = 0.1
    g = torch.Generator(device=DEV).manual_seed(14)
    p = torch.randn(R, T, device=DEV, generator=g)
    mb = torch.randn(R, T, device=DEV, generator=g)
    grad = torch.randn(R, T, device=DEV, generator=g)
    steps = torch.tensor([5.0, 0.0, 3.0, 2.0], device=DEV)  # replica 1 takes its first step
    mask = torch.tensor([True, True, True, False], device=DEV)
    p0, mb0 = p.clone(), mb.clone()
    K.sgd_step_(p, grad, mb, steps, full(R, 0.25), torch.tensor([0.0, 0.0, 0.9, 0.0], device=DEV),
                full(R, d), full(R, 0.0), mask, nesterov=nesterov, maximize=False)
    torch.cuda.synchronize()
    one_minus_d = 1.0 - torch.tensor(d, dtype=torch.float32).double()  # exact in double
    buf64 = one_minus_d * grad[0].double()  # exact in double
    assert torch.equal(mb[0], buf64.float())
    assert torch.equal(mb[1], grad[1])
    step0 = grad[0].double() if nesterov else buf64.float().double()
    assert torch.equal(p[0], (p0[0].double() - 0.25 * step0).float())
    assert torch.equal(p[1], (p0[1].double() - 0.25 * grad[1].double()).float())
    assert torch.equal(p[3], p0[3]) and torch.equal(mb[3], mb0[3])
    assert steps.tolist() == [6.0, 1.0, 4.0, 2.0]
    # the forms a kernel could plausibly compute instead are distinguishable here
    assert not torch.equal(mb[0], grad[0])  # dampening ignored on momentum-0 rows
    d32 = torch.tensor(1.0 - d, dtype=torch.float32, device=DEV)
    assert not torch.equal(mb[0], d32 * grad[0])  # (1 - d) rounded to float first


@pytest.mark.parametrize("lr_decay", [0.0, 0.5])
def test_adagrad_thawed_step_matches_never_frozen(lr_decay):
    """Reference test_inplace_adagrad_masking.py:91-131: a frozen replica's clock
    does not advance (no lr decay while frozen), so its first step after thawing
    is bit-equal to the first step of a replica that was never frozen."""
    T = 45
    g = torch.Generator(device=DEV).manual_seed(6)
    p_init = torch.randn(T, device=DEV, generator=g)
    s_init = torch.rand(T, device=DEV, generator=g)
    grad = torch.randn(T, device=DEV, generator=g)
    hyp = lambda R: (full(R, 1e-2), full(R, lr_decay), full(R, 1e-2), full(R, 1e-10))  # noqa
    # never frozen: one replica, one step
    pa, sa, stepa = p_init.view(1, T).clone(), s_init.view(1, T).clone(), torch.zeros(1, device=DEV)
    K.adagrad_step_(pa, grad.view(1, T), sa, stepa, *hyp(1),
                    torch.ones(1, dtype=torch.bool, device=DEV), maximize=False)
    # replica 1 frozen for three calls while replica 0 trains, then thawed
    pb = torch.stack([torch.randn(T, device=DEV, generator=g), p_init])
    sb = torch.stack([torch.rand(T, device=DEV, generator=g), s_init])
    stepb = torch.zeros(2, device=DEV)
    for _ in range(3):
        K.adagrad_step_(pb, torch.randn(2, T, device=DEV, generator=g), sb, stepb, *hyp(2),
                        torch.tensor([True, False], device=DEV), maximize=False)
    assert torch.equal(pb[1], p_init) and stepb.tolist() == [3.0, 0.0]
    K.adagrad_step_(pb, torch.stack([grad, grad]), sb, stepb, *hyp(2),
                    torch.ones(2, dtype=torch.bool, device=DEV), maximize=False)
    torch.cuda.synchronize()
    assert stepb.tolist() == [4.0, 1.0]
    assert torch.equal(pb[1], pa[0]) and torch.equal(sb[1], sa[0])


# ---------------------------------------------------------------------------
# vmap (reference test_inplace_adam_vmap.py)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("amsgrad", [False, True])
def test_adam_outer_vmap_matches_direct_call(amsgrad):
    B, T = 3, 33
    g = torch.Generator(device=DEV).manual_seed(8)
    mk = lambda: torch.randn(B, T, device=DEV, generator=g)  # noqa: E731
    base = [mk(), mk(), mk().abs(), mk().abs(), mk().abs(), torch.zeros(B, device=DEV)]
    lr = torch.linspace(5e-3, 5e-2, B, device=DEV)
    hyp = [lr, full(B, 0.9), full(B, 0.999), full(B, 1e-8), full(B, 1e-2)]
    mask = torch.ones(B, dtype=torch.bool, device=DEV)
    v_state = [t.clone() for t in base]
    d_state = [t.clone() for t in base]

    def one(p, gr, m, v, mx, s, lr, b1, b2, eps, wd, msk):
        return K.adam_step_(p.unsqueeze(0), gr.unsqueeze(0), m.unsqueeze(0), v.unsqueeze(0),
                            mx.unsqueeze(0) if amsgrad else None, s.view(1), lr.view(1),
                            b1.view(1), b2.view(1), eps.view(1), wd.view(1),
                            msk.view(1).to(torch.bool), amsgrad=amsgrad, maximize=False,
                            decoupled_weight_decay=True)

    vmap(one, in_dims=(0,) * 12)(*v_state, *hyp, mask)
    K.adam_step_(*d_state[:4], d_state[4] if amsgrad else None, d_state[5], *hyp, mask,
                 amsgrad=amsgrad, maximize=False, decoupled_weight_decay=True)
    torch.cuda.synchronize()
    for a, b in zip(v_state, d_state):
        assert torch.equal(a, b)


def test_sgd_vmap_batch_dim_1_is_strided():
    """in_dims=1 makes the rule's movedim produce a strided (B, T) view."""
    B, T = 4, 20
    g = torch.Generator(device=DEV).manual_seed(9)
    p_tb = torch.randn(T, B, device=DEV, generator=g)
    mb_tb = torch.randn(T, B, device=DEV, generator=g)
    gr_tb = torch.randn(T, B, device=DEV, generator=g)
    steps = torch.full((B,), 3.0, device=DEV)
    p_d, mb_d = p_tb.t().contiguous(), mb_tb.t().contiguous()
    steps_d = steps.clone()
    hyp = (torch.linspace(1e-3, 1e-2, B, device=DEV), full(B, 0.9), full(B, 0.1),
           full(B, 1e-2))
    mask = torch.ones(B, dtype=torch.bool, device=DEV)

    def one(p, gr, mb, s, lr, mom, damp, wd, msk):
        return K.sgd_step_(p.unsqueeze(0), gr.unsqueeze(0), mb.unsqueeze(0), s.view(1),
                           lr.view(1), mom.view(1), damp.view(1), wd.view(1),
                           msk.view(1), nesterov=False, maximize=False)

    vmap(one, in_dims=(1, 1, 1, 0, 0, 0, 0, 0, 0))(p_tb, gr_tb, mb_tb, steps, *hyp, mask)
    K.sgd_step_(p_d, gr_tb.t().contiguous(), mb_d, steps_d, *hyp, mask, nesterov=False,
                maximize=False)
    torch.cuda.synchronize()
    assert torch.equal(p_tb.t(), p_d) and torch.equal(mb_tb.t(), mb_d)
    assert torch.equal(steps, steps_d)


def test_adagrad_vmap_unbatched_scalar_hypers_broadcast():
    B, T = 3, 16
    g = torch.Generator(device=DEV).manual_seed(10)
    p, s = torch.randn(B, T, device=DEV, generator=g), torch.rand(B, T, device=DEV, generator=g)
    gr = torch.randn(B, T, device=DEV, generator=g)
    steps = torch.zeros(B, device=DEV)
    p2, s2, steps2 = p.clone(), s.clone(), steps.clone()
    lr = torch.tensor(1e-2, device=DEV)

    def one(p, gr, s, st):
        return K.adagrad_step_(p.unsqueeze(0), gr.unsqueeze(0), s.unsqueeze(0), st.view(1),
                               lr, lr * 0, lr * 0, lr * 0 + 1e-10,
                               torch.ones((), dtype=torch.bool, device=DEV), maximize=False)

    vmap(one)(p, gr, s, steps)
    K.adagrad_step_(p2, gr, s2, steps2, full(B, 1e-2), full(B, 0.0), full(B, 0.0),
                    full(B, 1e-10), torch.ones(B, dtype=torch.bool, device=DEV),
                    maximize=False)
    torch.cuda.synchronize()
    assert torch.equal(p, p2) and torch.equal(s, s2) and torch.equal(steps, steps2)


# ---------------------------------------------------------------------------
# edge cases and layouts
# ---------------------------------------------------------------------------
def test_return_is_fresh_zero_scalar():
    a = adam_args(2, 8)
    out = K.adam_step_(*a, torch.ones(2, dtype=torch.bool, device=DEV), amsgrad=False,
                       maximize=False, decoupled_weight_decay=True)
    assert out.shape == () and out.dtype == torch.float32 and out.device.type == "cuda"
    assert out.item() == 0.0
    assert all(out.data_ptr() != t.data_ptr() for t in a if t is not None)


@pytest.mark.parametrize("R,T", [(0, 16), (3, 0), (0, 0)])
def test_empty_state_still_bumps_steps(R, T):
    a = adam_args(R, T)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    out = K.adam_step_(*a, mask, amsgrad=False, maximize=False, decoupled_weight_decay=True)
    torch.cuda.synchronize()
    assert out.item() == 0.0
    assert a[5].tolist() == [3.0] * R
    s = torch.zeros(R, device=DEV)
    K.sgd_step_(torch.zeros(R, T, device=DEV), torch.zeros(R, T, device=DEV), None, s,
                full(R, 1.0), full(R, 0.0), full(R, 0.0), full(R, 0.0), mask, nesterov=False,
                maximize=False)
    K.adagrad_step_(torch.zeros(R, T, device=DEV), torch.zeros(R, T, device=DEV),
                    torch.zeros(R, T, device=DEV), s, full(R, 1.0), full(R, 0.0),
                    full(R, 0.0), full(R, 1e-10), mask, maximize=False)
    assert s.tolist() == [2.0] * R


@pytest.mark.parametrize("T", [1, 2, 3, 5, 1023, 1024, 1025, 4097])
def test_odd_widths_bit_exact_to_oracle(T):
    R = 3
    g = torch.Generator(device=DEV).manual_seed(T)
    a = adam_args(R, T, amsgrad=True, seed=T)
    mask = torch.tensor([True, False, True], device=DEV)
    host = [t.cpu().numpy().copy() if t is not None else None for t in a]
    grad = a[1]
    K.adam_step_(*a, mask, amsgrad=True, maximize=False, decoupled_weight_decay=True)
    torch.cuda.synchronize()
    O.adam_step(O.DEVICE, host[0], host[1], host[2], host[3], host[4], host[5], host[6],
                host[7], host[8], host[9], host[10], mask.cpu().numpy(), amsgrad=True,
                decoupled_weight_decay=True)
    for i in (0, 2, 3, 4, 5):
        assert np.array_equal(a[i].cpu().numpy().view(np.uint32), host[i].view(np.uint32)), i
    del g, grad


@pytest.mark.parametrize("offset,extra", [(1, 1), (2, 3), (3, 2), (0, 5), (1, 0), (4, 1),
                                          (17, 3), (40, 0), (63, 2)])
@pytest.mark.parametrize("T", [5, 30, 64, 1023, 2050])
def test_misaligned_row_views_bit_exact(offset, extra, T):
    """Column-slice views whose rows start off a 16- or 256-byte boundary (a
    different one on every row when the row stride is not a multiple of 4 or
    64): the streaming driver's per-row head/tail handling gives the same bits
    as contiguous buffers, also for rows shorter than the head; views whose
    operands disagree on the 16-byte boundary (here: grads offset differently)
    take the element path, same bits again."""
    R = 5
    big = adam_args(R, T + offset + extra, amsgrad=True, seed=T + offset)
    view = [t[:, offset:offset + T] if t is not None and t.dim() == 2 else t for t in big]
    odd_g = adam_args(R, T + 3, seed=99)[1][:, (offset + 1) % 4:(offset + 1) % 4 + T]
    dense = [t.clone().contiguous() if t is not None else None for t in view]
    mixed = [t.clone() if t is not None else None for t in dense]
    mixed[1] = odd_g.clone()
    odd_view = [t.clone() if t is not None else None for t in view]
    odd_view[1] = odd_g
    mask = torch.tensor([True, False, True, True, True], device=DEV)
    kw = dict(amsgrad=True, maximize=True, decoupled_weight_decay=False)
    K.adam_step_(*view, mask, **kw)
    K.adam_step_(*dense, mask, **kw)
    K.adam_step_(*odd_view, mask, **kw)
    K.adam_step_(*mixed, mask, **kw)
    torch.cuda.synchronize()
    for i in (0, 2, 3, 4, 5):
        assert torch.equal(view[i], dense[i]), i
        assert torch.equal(odd_view[i], mixed[i]), i


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("offset", [1, 6, 31, 127])
def test_misaligned_row_views_other_dtypes_bit_exact(dtype, offset):
    """As above for the other parameter types: rows start at offsets of up to
    127 elements from a 256-byte boundary."""
    R, T = 5, 1500
    big = adam_args(R, T + offset + 3, seed=offset, dtype=dtype)
    view = [t[:, offset:offset + T] if t is not None and t.dim() == 2 else t for t in big]
    dense = [t.clone().contiguous() if t is not None else None for t in view]
    mask = torch.tensor([True, True, False, True, True], device=DEV)
    kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
    K.adam_step_(*view, mask, **kw)
    K.adam_step_(*dense, mask, **kw)
    torch.cuda.synchronize()
    for i in (0, 2, 3, 5):
        assert torch.equal(view[i], dense[i]), i


@pytest.mark.parametrize("T", [3, 700, 1024, 1029, 4100])
@pytest.mark.parametrize("offset", [0, 1, 255, 256, 1021, 1024, 2047, 3071, 4095])
def test_views_at_every_tile_phase_match_oracle(offset, T):
    """The streaming driver's tiles start on the row's boundaries of the tile
    size (up to 4096 float32 elements); a head tile per row takes what lies
    before the first one. Column views at offsets across that whole range,
    rows whose widths are below, at and above a tile, with the row stride
    moving every row to another phase: each element against the oracle."""
    R = 4
    big = adam_args(R, offset + T + 37, amsgrad=True, seed=offset * 7 + T)
    view = [t[:, offset:offset + T] if t is not None and t.dim() == 2 else t for t in big]
    mask = torch.tensor([True, True, False, True], device=DEV)
    host = [t.contiguous().cpu().numpy().copy() if t is not None else None for t in view]
    kw = dict(amsgrad=True, maximize=False, decoupled_weight_decay=True)
    K.adam_step_(*view, mask, **kw)
    torch.cuda.synchronize()
    O.adam_step(O.DEVICE, *host[:11], mask.cpu().numpy(), **kw)
    for i in (0, 2, 3, 4, 5):
        got = view[i].contiguous().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), host[i].view(np.uint32)), i
    untouched = big[0][:, :offset], big[0][:, offset + T:]
    ref = adam_args(R, offset + T + 37, amsgrad=True, seed=offset * 7 + T)[0]
    assert torch.equal(untouched[0], ref[:, :offset])
    assert torch.equal(untouched[1], ref[:, offset + T:])


@pytest.mark.parametrize("offset", [0, 3, 511, 4099, 8191])
def test_bf16_views_at_every_tile_phase_bit_exact_to_aten(offset):
    """As above for bfloat16 parameters (8 elements per pack, tiles of up to
    8192 elements), against torch's fused Adam on each active row, with
    hyperparameters exact in 16 bits."""
    R, T = 3, 5000
    dtype = torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(offset)
    W = offset + T + 13
    rnd = lambda: torch.randn(R, W, device=DEV, generator=g).to(dtype)  # noqa: E731
    big = [rnd(), rnd(), rnd().abs(), rnd().abs()]
    p, gr, m, v = (t[:, offset:offset + T] for t in big)
    lr, b1, b2, eps, wd = 2.0**-7, 0.875, 1 - 2.0**-7, 2.0**-14, 2.0**-6
    mask = torch.tensor([True, False, True], device=DEV)
    ref = [[t[r].clone() for t in (p, m, v)] for r in range(R)]
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    for r in (0, 2):
        torch._fused_adam_([ref[r][0]], [gr[r].clone()], [ref[r][1]], [ref[r][2]], [],
                           [torch.tensor(1.0, device=DEV)], lr=lr, beta1=b1, beta2=b2,
                           weight_decay=wd, eps=eps, amsgrad=False, maximize=False,
                           grad_scale=None, found_inf=None)
    K.adam_step_(p, gr, m, v, None, steps, *(full(R, x, dtype) for x in (lr, b1, b2, eps, wd)),
                 mask, amsgrad=False, maximize=False, decoupled_weight_decay=False)
    torch.cuda.synchronize()
    for r in range(R):
        for got, want in zip((p[r], m[r], v[r]), ref[r]):
            assert torch.equal(got, want), r


@pytest.mark.parametrize("R,T", [(2500, 300), (2500, 600), (2500, 1100), (2500, 1700),
                                 (1500, 4100), (700, 110_000)])
def test_many_rows_land_on_their_own_tiles(R, T):
    """A streaming workgroup finds its row by dividing its index by the tiles
    per row (a multiply and shifts with host-computed constants). Many rows and
    1, 2, 3, 4, 9 and 430 tiles per row (the last a launch beyond the MALL):
    sampled rows, the first and last included, equal the oracle's, and frozen
    ones stay bit-identical."""
    a = adam_args(R, T, seed=R + T)
    mask = torch.arange(R, device=DEV) % 7 != 3
    rows = sorted({0, 1, 2, 3, R // 2, R // 2 + 1, R - 2, R - 1, 10, 17})
    host = [t[rows].cpu().numpy().copy() if t is not None else None for t in a]
    before = [t[rows].clone() if t is not None else None for t in a]
    kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
    K.adam_step_(*a, mask, **kw)
    torch.cuda.synchronize()
    m = mask[rows].cpu().numpy()
    O.adam_step(O.DEVICE, *host[:11], m, **kw)
    for i in (0, 2, 3):
        got = a[i][rows]
        for k in range(len(rows)):
            if m[k]:
                assert np.array_equal(got[k].cpu().numpy().view(np.uint32),
                                      host[i][k].view(np.uint32)), (i, rows[k])
            else:
                assert torch.equal(got[k], before[i][k]), (i, rows[k])


@pytest.mark.parametrize("large", [False, True], ids=["small", "large"])
@pytest.mark.parametrize("op", ["adam", "sgd", "adagrad"])
@pytest.mark.parametrize("offset", [0, 1, 2, 3, 5])
def test_mask_views_at_every_byte_offset(offset, op, large):
    """The streaming driver reads a replica's active byte as part of the
    aligned 4-byte word that holds it (Adam and Adagrad beyond the MALL, SGD
    with momentum at every size; Adam's MALL-resident shape keeps a vector
    load). Masks that are views starting 0-3 bytes into such a word, with rows
    of every residue mod 4, must give each replica its own byte: frozen rows
    bit-identical, active rows equal to the oracle's."""
    R = 11
    bytes_per_elem = 16 if op == "adam" else 12  # params, grads and state, float32
    T = (300 * 2**20) // (bytes_per_elem * R) // 4 * 4 + 4 if large else 1030
    g = torch.Generator(device=DEV).manual_seed(offset + 31)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g)  # noqa: E731
    pattern = [True, False, True, True, False, False, True, False, True, True, False]
    big = torch.zeros(R + 8, dtype=torch.bool, device=DEV)
    big[offset:offset + R] = torch.tensor(pattern, device=DEV)
    mask = big[offset:offset + R]
    assert mask.data_ptr() % 4 == offset % 4
    if op == "adam":
        a = [rnd(), rnd(), rnd().abs(), rnd().abs(), None, full(R, 2.0), full(R, 1e-2),
             full(R, 0.9), full(R, 0.999), full(R, 1e-8), full(R, 1e-2)]
        kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
        state, n_in, run, ref = (0, 2, 3), 11, K.adam_step_, O.adam_step
    elif op == "sgd":
        a = [rnd(), rnd(), rnd(), full(R, 3.0), full(R, 1e-2), full(R, 0.9), full(R, 0.1),
             full(R, 1e-3)]
        kw = dict(nesterov=True, maximize=False)
        state, n_in, run, ref = (0, 2), 8, K.sgd_step_, O.sgd_step
    else:
        a = [rnd(), rnd(), rnd().abs(), full(R, 2.0), full(R, 1e-2), full(R, 1e-3),
             full(R, 1e-3), full(R, 1e-10)]
        kw = dict(maximize=False)
        state, n_in, run, ref = (0, 2), 8, K.adagrad_step_, O.adagrad_step
    steps = 5 if op == "adam" else 3
    rows = [0, 1, 2, 3, 4, 7, 10]
    host = [t[rows].cpu().numpy().copy() if t is not None else None for t in a]
    before = [t.clone() if t is not None else None for t in a]
    run(*a, mask, **kw)
    torch.cuda.synchronize()
    ref(O.DEVICE, *host[:n_in], np.array([pattern[r] for r in rows]), **kw)
    for i in state:
        for k, r in enumerate(rows):
            if pattern[r]:
                got = a[i][r].cpu().numpy()
                assert np.array_equal(got.view(np.uint32), host[i][k].view(np.uint32)), (i, r)
            else:
                assert torch.equal(a[i][r], before[i][r]), (i, r)
    assert torch.equal(a[steps], before[steps] + mask.float())


@pytest.mark.parametrize("op", ["sgd", "adagrad", "adam-bf16"])
def test_ragged_rows_other_policies_bit_exact(op):
    """Rows of width T = 4k + 3 in one contiguous (R, T) allocation (every row
    starts at a different 16-byte phase) against the same rows padded to 4k + 4."""
    R, T = 6, 4099
    g = torch.Generator(device=DEV).manual_seed(5)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g)  # noqa: E731
    pad = lambda t: torch.nn.functional.pad(t, (0, 1))  # noqa: E731
    mask = torch.tensor([True, True, False, True, True, True], device=DEV)
    if op == "sgd":
        ragged = [rnd(), rnd(), rnd(), torch.ones(R, device=DEV)]
        hyp = [full(R, 1e-2), full(R, 0.9), full(R, 0.1), full(R, 1e-3)]
        run = lambda a: K.sgd_step_(a[0], a[1], a[2], a[3], *hyp, mask, nesterov=False,  # noqa
                                    maximize=False)
    elif op == "adagrad":
        ragged = [rnd(), rnd(), rnd().abs(), torch.ones(R, device=DEV)]
        hyp = [full(R, 1e-2), full(R, 1e-3), full(R, 1e-3), full(R, 1e-10)]
        run = lambda a: K.adagrad_step_(a[0], a[1], a[2], a[3], *hyp, mask,  # noqa
                                        maximize=False)
    else:
        ragged = [rnd(), rnd(), rnd().to(torch.bfloat16), rnd().abs().to(torch.bfloat16),
                  torch.ones(R, device=DEV)]
        hyp = [full(R, 1e-2), full(R, 0.9), full(R, 0.999), full(R, 1e-8), full(R, 1e-2)]
        run = lambda a: K.adam_step_(a[0], a[1], a[2], a[3], None, a[4], *hyp, mask,  # noqa
                                     amsgrad=False, maximize=False, decoupled_weight_decay=True)
    padded = [pad(t) if t.dim() == 2 else t.clone() for t in ragged]
    run(ragged)
    run(padded)
    torch.cuda.synchronize()
    for a, b in zip(ragged, padded):
        want = b[:, :T] if b.dim() == 2 else b
        assert torch.equal(a, want)


def _replica_minor(t: torch.Tensor, pad: int) -> torch.Tensor:
    """The (R, T) values as a view of a (T, R + pad) buffer: unit replica stride."""
    R, T = t.shape
    back = torch.empty(T, R + pad, dtype=t.dtype, device=t.device)
    view = back[:, :R].t()
    view.copy_(t)
    return view


@pytest.mark.parametrize("op", ["adam-amsgrad", "adamw", "sgd-nesterov", "sgd-first", "sgd-mixed",
                                "adagrad", "adagrad-f32", "adam-bf16", "adam-f64", "adam-f16",
                                "adam-bf16p"])
@pytest.mark.parametrize("R,T", [(2, 1), (3, 1000), (64, 33), (100, 517), (257, 40), (600, 9),
                                 (1024, 5), (1030, 7), (2052, 3)])
@pytest.mark.parametrize("pad", [0, 3])
def test_replica_minor_views_bit_exact(op, R, T, pad):
    """Operands with unit replica stride ((T, R) buffers, optionally padded, seen
    as (R, T): what an outer vmap over a non-leading dimension hands over) take
    the column driver: the same bits as contiguous buffers, frozen replicas
    untouched. Replica counts cover one and several replica blocks, packs cut
    by the last replica, and (sgd-mixed) replicas on their first step next to
    others that read their momentum buffer."""
    g = torch.Generator(device=DEV).manual_seed(R * 1000 + T)
    dt = {"adam-f64": torch.float64, "adam-f16": torch.float16,
          "adam-bf16p": torch.bfloat16}.get(op, torch.float32)
    st_dt = torch.bfloat16 if op == "adam-bf16" else dt
    rnd = lambda dtype=dt: torch.randn(R, T, device=DEV, generator=g).to(dtype)  # noqa: E731
    pos = lambda dtype=dt: rnd(dtype).abs()  # noqa: E731
    vec = lambda lo, hi: (lo + (hi - lo) * torch.rand(R, device=DEV, generator=g)).to(dt)  # noqa
    mask = torch.rand(R, device=DEV, generator=g) < 0.7
    mask[0] = False
    steps = torch.randint(0 if op == "sgd-first" else 1, 50, (R,), device=DEV,
                          generator=g).to(dt)
    if op == "sgd-first":
        steps.zero_()
    if op == "sgd-mixed":
        steps = torch.randint(0, 2, (R,), device=DEV, generator=g).to(dt)
    if op.startswith("adam"):
        ams = op == "adam-amsgrad"
        bufs = [rnd(), rnd(), rnd(st_dt), pos(st_dt)] + ([pos(st_dt)] if ams else [])
        hyp = [vec(1e-3, 1e-2), vec(0.8, 0.95), vec(0.99, 0.9999), vec(1e-8, 1e-6),
               vec(0.0, 1e-2)]
        kw = dict(amsgrad=ams, maximize=op == "adam-bf16",
                  decoupled_weight_decay=op != "adam-amsgrad")

        def run(b, s):
            K.adam_step_(b[0], b[1], b[2], b[3], b[4] if ams else None, s, *hyp, mask, **kw)
    elif op.startswith("sgd"):
        bufs = [rnd(), rnd(), rnd()]
        hyp = [vec(1e-3, 1e-1), vec(0.5, 0.9), torch.zeros(R, device=DEV), vec(0.0, 1e-2)]

        def run(b, s):
            K.sgd_step_(b[0], b[1], b[2], s, *hyp, mask, nesterov=True, maximize=False)
    else:
        bufs = [rnd(), rnd(), pos()]
        hyp = [vec(1e-3, 1e-1), vec(0.0, 0.1), vec(0.0, 1e-2), vec(1e-10, 1e-8)]
        f = K.adagrad_step_f32_ if op == "adagrad-f32" else K.adagrad_step_

        def run(b, s):
            f(b[0], b[1], b[2], s, *hyp, mask, maximize=True)
    view = [_replica_minor(t, pad) for t in bufs]
    dense = [t.clone() for t in bufs]
    before = [t.clone() for t in bufs]
    s_view, s_dense = steps.clone(), steps.clone()
    run(view, s_view)
    run(dense, s_dense)
    torch.cuda.synchronize()
    assert torch.equal(s_view, s_dense)
    for i, (a, b) in enumerate(zip(view, dense)):
        assert torch.equal(a, b), i
        assert torch.equal(a[~mask], before[i][~mask]), i


@pytest.mark.parametrize("R,pad", [(64, 0), (256, 0), (300, 0), (1024, 0), (1024, 32), (1024, 3),
                                   (2048, 0)])
@pytest.mark.parametrize("frozen", [(), (70, 71, 75), (0, 1000)])
def test_replica_minor_access_paths(R, pad, frozen):
    """The column driver's access variants on one launch: wavefronts whose
    replicas are all active next to ones with frozen replicas, one and several
    replica blocks per column, with line-aligned column strides (pad 0 / 32)
    and without (pad 3, R = 300), every workgroup order. Bit for bit against
    contiguous buffers; frozen replicas untouched."""
    T = 77
    frozen = [r for r in frozen if r < R]
    a = adam_args(R, T, seed=R + pad)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    mask[frozen] = False
    view = [_replica_minor(t, pad) for t in a[:4]]
    dense = [t.clone() for t in a[:4]]
    before = [t.clone() for t in a[:4]]
    s_view, s_dense = a[5].clone(), a[5].clone()
    kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
    for _ in range(2):
        K.adam_step_(*view, None, s_view, *a[6:], mask, **kw)
        K.adam_step_(*dense, None, s_dense, *a[6:], mask, **kw)
    torch.cuda.synchronize()
    assert torch.equal(s_view, s_dense)
    for i, (x, y) in enumerate(zip(view, dense)):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32)), i
        assert torch.equal(x[~mask], before[i][~mask]), i


@pytest.mark.parametrize("amsgrad", [False, True])
def test_replica_minor_step0_freeze_with_workspace(amsgrad):
    """Replicas frozen before their first step keep step 0, where the bias
    corrections would divide by 1 - beta^0 = 0. The operator's preparation
    launch writes workspace constants for active replicas only, and the column
    driver's threads for a frozen replica exit before reading constants or any
    operand: with NaN in the frozen replicas' state, their columns stay
    bit-identical and the active replicas get the bits of contiguous buffers.
    (That the frozen replicas' workspace entries are never written is checked
    through the C ABI with a NaN-filled workspace, in test_gpu_abi.py.)"""
    R, T = 70, 45
    a = adam_args(R, T, amsgrad, seed=11, steps=0.0)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    mask[[0, 33, 69]] = False
    for t in a[2:5]:
        if t is not None:
            t[~mask] = float("nan")
    ops = [t for t in a[:5] if t is not None]
    view = [_replica_minor(t, 0) for t in ops]
    dense = [t.clone() for t in ops]
    before = [t.clone() for t in ops]
    s_view, s_dense = a[5].clone(), a[5].clone()
    kw = dict(amsgrad=amsgrad, maximize=False, decoupled_weight_decay=False)
    mx = lambda b: b[4] if amsgrad else None  # noqa: E731
    for _ in range(2):
        K.adam_step_(*view[:4], mx(view), s_view, *a[6:], mask, **kw)
        K.adam_step_(*dense[:4], mx(dense), s_dense, *a[6:], mask, **kw)
    torch.cuda.synchronize()
    assert torch.equal(s_view, s_dense)
    assert s_view[~mask].eq(0).all() and s_view[mask].eq(2).all()
    for i, (x, y) in enumerate(zip(view, dense)):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32)), i
        assert torch.equal(x[~mask].view(torch.int32), before[i][~mask].view(torch.int32)), i


def test_noncontiguous_and_foreign_dtype_side_inputs():
    """(R,) inputs may be strided or float64 and steps float64, mask float:
    normalised like the reference (to the param dtype / bool)."""
    R, T = 3, 40
    a = adam_args(R, T, seed=13)
    b = [t.clone() if t is not None else None for t in a]
    wide = torch.stack([a[6], a[6]], 1)[:, 0]  # strided lr view
    assert not wide.is_contiguous()
    b_steps = b[5].double()
    K.adam_step_(*a[:6], wide, *a[7:], torch.tensor([1.0, 0.0, 1.0], device=DEV),
                 amsgrad=False, maximize=False, decoupled_weight_decay=True)
    K.adam_step_(*b[:5], b_steps, *(t.double() for t in b[6:]),
                 torch.tensor([True, False, True], device=DEV), amsgrad=False,
                 maximize=False, decoupled_weight_decay=True)
    torch.cuda.synchronize()
    for i in (0, 2, 3):
        assert torch.equal(a[i], b[i])
    assert a[5].tolist() == b_steps.tolist() == [3.0, 2.0, 3.0]


# ---------------------------------------------------------------------------
# errors (reference: RuntimeError from TORCH_CHECK)
# ---------------------------------------------------------------------------
def test_errors_are_runtime_errors():
    R, T = 2, 8
    a = adam_args(R, T)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
    with pytest.raises(RuntimeError, match="2-D"):
        K.adam_step_(a[0][0], *a[1:], mask, **kw)
    with pytest.raises(RuntimeError, match="amsgrad=True requires max_exp_avg_sqs"):
        K.adam_step_(*a, mask, amsgrad=True, maximize=False, decoupled_weight_decay=True)
    with pytest.raises(RuntimeError, match="grads"):
        K.adam_step_(a[0], a[1][:, :4], *a[2:], mask, **kw)
    with pytest.raises(RuntimeError, match="lr"):
        K.adam_step_(*a[:6], full(R + 1, 1e-3), *a[7:], mask, **kw)
    with pytest.raises(RuntimeError, match="lr"):
        K.adam_step_(*a[:6], torch.full((R,), 1e-3), *a[7:], mask, **kw)
    with pytest.raises(RuntimeError, match="nesterov=True requires momentum_buffers"):
        K.sgd_step_(a[0], a[1], None, a[5], *a[6:10], mask, nesterov=True, maximize=False)
    with pytest.raises(RuntimeError, match="65535"):
        big = torch.zeros(65536, 1, device=DEV)
        r = torch.zeros(65536, device=DEV)
        K.sgd_step_(big, big, None, r, r, r, r, r, r.bool(), nesterov=False, maximize=False)
    with pytest.raises(RuntimeError, match="dtype"):
        K.adam_step_(a[0], a[1].double(), *a[2:], mask, **kw)


# ---------------------------------------------------------------------------
# registration
# ---------------------------------------------------------------------------
def test_opcheck_all_ops():
    R, T = 3, 8
    mask = torch.tensor([True, False, True], device=DEV)
    U = lambda x: full(R, x)  # noqa: E731
    rn = lambda: torch.randn(R, T, device=DEV)  # noqa: E731
    torch.library.opcheck(
        torch.ops.torchstrap.adam_step_.default,
        (rn(), rn(), rn().abs(), rn().abs(), None, torch.zeros(R, device=DEV), U(1e-2),
         U(0.9), U(0.999), U(1e-8), U(1e-2), mask),
        dict(amsgrad=False, maximize=False, decoupled_weight_decay=True))
    torch.library.opcheck(
        torch.ops.torchstrap.sgd_step_.default,
        (rn(), rn(), rn(), torch.zeros(R, device=DEV), U(1e-2), U(0.9), U(0.0), U(0.0), mask),
        dict(nesterov=True, maximize=False))
    torch.library.opcheck(
        torch.ops.torchstrap.sgd_step_.default,
        (rn(), rn(), None, torch.zeros(R, device=DEV), U(1e-2), U(0.0), U(0.0), U(0.0), mask),
        dict(nesterov=False, maximize=False))
    torch.library.opcheck(
        torch.ops.torchstrap.adagrad_step_.default,
        (rn(), rn(), rn().abs(), torch.zeros(R, device=DEV), U(1e-2), U(0.0), U(0.0),
         U(1e-10), mask),
        dict(maximize=False))


# ---------------------------------------------------------------------------
# other parameter dtypes (the reference dispatches fp32/fp64/fp16/bf16)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("amsgrad", [False, True])
def test_adam_fp64_bit_exact_to_aten(amsgrad):
    R, T = 2, 77
    g = torch.Generator(device=DEV).manual_seed(14)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=torch.float64)  # noqa
    p, m, v, mx = rnd(), rnd().abs(), rnd().abs(), rnd().abs()
    ref = [[t[r].clone() for t in (p, m, v, mx)] for r in range(R)]
    steps = torch.zeros(R, device=DEV, dtype=torch.float64)
    lr = torch.tensor([1e-2, 3e-3], device=DEV, dtype=torch.float64)
    h = [full(R, x, torch.float64) for x in (0.9, 0.999, 1e-8, 1e-2)]
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    for k in range(3):
        grad = rnd()
        for r in range(R):
            torch._fused_adamw_([ref[r][0]], [grad[r].clone()], [ref[r][1]], [ref[r][2]],
                                [ref[r][3]] if amsgrad else [],
                                [torch.tensor(float(k + 1), device=DEV)], lr=lr[r].item(),
                                beta1=0.9, beta2=0.999, weight_decay=1e-2, eps=1e-8,
                                amsgrad=amsgrad, maximize=False, grad_scale=None,
                                found_inf=None)
        K.adam_step_(p, grad, m, v, mx if amsgrad else None, steps, lr, *h, mask,
                     amsgrad=amsgrad, maximize=False, decoupled_weight_decay=True)
    torch.cuda.synchronize()
    for r in range(R):
        for got, want in zip((p[r], m[r], v[r]), ref[r][:3]):
            assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_adam_16bit_bit_exact_to_aten_with_representable_hypers(dtype):
    """Hyperparameters are carried in the param dtype (reference to_hyper); with
    values exact in 16 bits the element math must equal torch's, bit for bit."""
    R, T = 2, 64
    g = torch.Generator(device=DEV).manual_seed(15)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g).to(dtype)  # noqa: E731
    p, m, v = rnd(), rnd().abs(), rnd().abs()
    ref = [[t[r].clone() for t in (p, m, v)] for r in range(R)]
    lr, b1, b2, eps, wd = 2.0**-7, 0.875, 1 - 2.0**-7, 2.0**-14, 2.0**-6
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    for k in range(3):
        grad = rnd()
        for r in range(R):
            torch._fused_adam_([ref[r][0]], [grad[r].clone()], [ref[r][1]], [ref[r][2]], [],
                               [torch.tensor(float(k + 1), device=DEV)], lr=lr, beta1=b1,
                               beta2=b2, weight_decay=wd, eps=eps, amsgrad=False,
                               maximize=False, grad_scale=None, found_inf=None)
        K.adam_step_(p, grad, m, v, None, steps, *(full(R, x, dtype) for x in (lr, b1, b2, eps, wd)),
                     mask, amsgrad=False, maximize=False, decoupled_weight_decay=False)
    torch.cuda.synchronize()
    for r in range(R):
        for got, want in zip((p[r], m[r], v[r]), ref[r]):
            assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16, torch.bfloat16])
def test_sgd_adagrad_other_dtypes_close_to_fp32(dtype):
    R, T = 2, 100
    tol = {torch.float64: 1e-6, torch.float16: 2e-3, torch.bfloat16: 2e-2}[dtype]
    g = torch.Generator(device=DEV).manual_seed(16)
    base = [torch.randn(R, T, device=DEV, generator=g) for _ in range(3)]
    for op in ("sgd", "adagrad"):
        outs = []
        for dt in (torch.float32, dtype):
            p, gr, x = (t.to(dt).clone() for t in base)
            x = x.abs()
            steps = torch.zeros(R, device=DEV, dtype=dt)
            mask = torch.ones(R, dtype=torch.bool, device=DEV)
            if op == "sgd":
                K.sgd_step_(p, gr, x, steps, full(R, 0.125, dt), full(R, 0.5, dt),
                            full(R, 0.0, dt), full(R, 0.0, dt), mask, nesterov=True,
                            maximize=False)
            else:
                K.adagrad_step_(p, gr, x, steps, full(R, 0.125, dt), full(R, 0.0, dt),
                                full(R, 0.0, dt), full(R, 2.0**-14, dt), mask, maximize=False)
            outs.append((p.float(), x.float()))
        torch.cuda.synchronize()
        for a, b in zip(*outs):
            torch.testing.assert_close(b, a, atol=tol, rtol=tol)

"""Bit-exact parity with torch's own fused optimizers on the MI355X.

Mirrors the reference's tier-1 gate (test/optimizer/test_aten_fused_parity.py,
test_aten_sgd_parity.py, test_aten_adagrad_parity.py): for the case ATen can
express -- one replica, its own float32 hyperparameters -- the operator must
agree with ``torch._fused_adam_`` / ``_fused_adamw_`` / ``_fused_sgd_`` /
``_fused_adagrad_`` to the bit, on params, every moment and the step counter.
Here the whole ensemble is checked at once: each active replica row against
its own ATen call, with distinct per-replica hyperparameters.
"""

from __future__ import annotations

import itertools

import pytest
import torch

import churten_amd.kernels as K

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def f32(x):
    return torch.tensor(x, dtype=torch.float32).item()


def same(name, a, b):
    if not torch.equal(a, b):
        n = (a != b).sum().item()
        d = (a - b).abs().max().item()
        raise AssertionError(f"{name}: {n}/{a.numel()} elements differ, max {d:.3e}")


def _vecs(R, *rows, dtype=torch.float32):
    """float32-rounded hyperparameters, in the parameter dtype."""
    return [torch.tensor(r[:R], device=DEV, dtype=torch.float32).to(dtype) for r in rows]


# float64 parameters: the products inside the update are inexact there, so these
# cases also pin which multiply-adds torch's build fuses. 16-bit parameters: the
# update narrows a double expression to the float math value and that to the
# storage type, two roundings that must not be folded into one (long rows hit
# the half-way cases). torch runs rows whose length is a multiple of 4 on its
# vector path and the others element by element, two separately compiled
# bodies: 262144-element rows (four of its 65536-element chunks) take the first
# at length, 70001-element rows the second.
DTYPES = [torch.float32, torch.float64, torch.float16, torch.bfloat16]
ROWS = [64, 45, 70001, 262144]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("T", ROWS)
@pytest.mark.parametrize("amsgrad,maximize,decoupled,wd",
                         list(itertools.product([False, True], [False, True],
                                                [False, True], [0.0, 1e-2])))
def test_adam_rows_bit_identical_to_aten(T, amsgrad, maximize, decoupled, wd, dtype, R=3):
    g = torch.Generator(device=DEV).manual_seed(T)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)
    p, m, v, mx = rnd(), rnd().abs(), rnd().abs(), rnd().abs()
    lr, b1, b2, eps = _vecs(R, [1e-2, 3e-3, 5e-2], [0.9, 0.8, 0.95],
                            [0.999, 0.99, 0.9999], [1e-8, 1e-6, 1e-7], dtype=dtype)
    wdv = torch.full((R,), f32(wd), device=DEV, dtype=dtype)
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    ref = [[t[r].clone() for t in (p, m, v, mx)] + [torch.zeros((), device=DEV)]
           for r in range(R)]
    fused = torch._fused_adamw_ if decoupled else torch._fused_adam_
    for _ in range(3):
        grad = rnd()
        for r in range(R):
            pr, mr, vr, xr, sr = ref[r]
            sr += 1
            fused([pr], [grad[r].clone()], [mr], [vr], [xr] if amsgrad else [], [sr],
                  lr=lr[r].item(), beta1=b1[r].item(), beta2=b2[r].item(),
                  weight_decay=wdv[r].item(), eps=eps[r].item(), amsgrad=amsgrad,
                  maximize=maximize, grad_scale=None, found_inf=None)
        K.adam_step_(p, grad, m, v, mx if amsgrad else None, steps, lr, b1, b2, eps,
                     wdv, mask, amsgrad=amsgrad, maximize=maximize,
                     decoupled_weight_decay=decoupled)
    torch.cuda.synchronize()
    for r in range(R):
        same(f"params[{r}]", p[r], ref[r][0])
        same(f"exp_avgs[{r}]", m[r], ref[r][1])
        same(f"exp_avg_sqs[{r}]", v[r], ref[r][2])
        if amsgrad:
            same(f"max_exp_avg_sqs[{r}]", mx[r], ref[r][3])
        assert steps[r].item() == ref[r][4].item() == 3


# torch warns that is_first_step means nothing without momentum buffers.
@pytest.mark.filterwarnings("ignore:`is_first_step` argument has no effect")
@pytest.mark.parametrize("T", ROWS)
@pytest.mark.parametrize("momentum,dampening,wd,nesterov,maximize", [
    c for c in itertools.product([0.0, 0.9], [0.0, 0.3], [0.0, 1e-2], [False, True],
                                 [False, True])
    if not (c[3] and c[0] == 0.0)])  # nesterov needs momentum buffers
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_sgd_rows_bit_identical_to_aten(T, momentum, dampening, wd, nesterov,
                                        maximize, dtype, R=2):
    g = torch.Generator(device=DEV).manual_seed(T + 1)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)
    p = rnd()
    has_buf = momentum != 0.0
    mb = rnd() if has_buf else None
    (lr,) = _vecs(R, [1e-2, 3e-2], dtype=dtype)
    mom = torch.full((R,), f32(momentum), device=DEV, dtype=dtype)
    damp = torch.full((R,), f32(dampening), device=DEV, dtype=dtype)
    wdv = torch.full((R,), f32(wd), device=DEV, dtype=dtype)
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    ref = [(p[r].clone(), mb[r].clone() if has_buf else None) for r in range(R)]
    for it in range(3):
        grad = rnd()
        for r in range(R):
            torch._fused_sgd_([ref[r][0]], [grad[r].clone()],
                              [ref[r][1]] if has_buf else [], weight_decay=wdv[r].item(),
                              momentum=mom[r].item(), lr=lr[r].item(),
                              dampening=damp[r].item(), nesterov=nesterov,
                              maximize=maximize, is_first_step=it == 0,
                              grad_scale=None, found_inf=None)
        K.sgd_step_(p, grad, mb, steps, lr, mom, damp, wdv, mask, nesterov=nesterov,
                    maximize=maximize)
    torch.cuda.synchronize()
    for r in range(R):
        same(f"params[{r}]", p[r], ref[r][0])
        if has_buf:
            same(f"momentum_buffers[{r}]", mb[r], ref[r][1])
    assert torch.equal(steps, torch.full((R,), 3.0, device=DEV, dtype=steps.dtype))


# BASELINE config 3's combination in one call: per-replica momentum
# {0.5, 0.9, 0.99} and a momentum-0 replica next to buffered ones, dampening
# 0.1 with nesterov, replicas on their first step next to later ones, and a
# frozen replica. Each buffered row against its own torch._fused_sgd_ call
# (is_first_step from that row's bumped step); the momentum-0 row's params
# against the buffer-less ATen step, which is what nesterov and a zero
# momentum reduce to (its buffer, which ATen does not keep, is checked against
# the oracle by the golden-case tests).
@pytest.mark.filterwarnings("ignore:`is_first_step` argument has no effect")
@pytest.mark.parametrize("T", [45, 70001, 262144])
@pytest.mark.parametrize("maximize,wd", [(False, 0.0), (True, 1e-2)])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_sgd_config3_flags_bit_identical_to_aten(T, maximize, wd, dtype):
    R = 6
    g = torch.Generator(device=DEV).manual_seed(T + 3)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)
    p, mb = rnd(), rnd()
    (lr, mom) = _vecs(R, [1e-2, 3e-2, 2e-2, 5e-3, 1e-2, 4e-2],
                      [0.5, 0.9, 0.99, 0.0, 0.9, 0.5], dtype=dtype)
    damp = torch.full((R,), f32(0.1), device=DEV, dtype=dtype)
    wdv = torch.full((R,), f32(wd), device=DEV, dtype=dtype)
    steps = torch.tensor([0, 3, 0, 1, 7, 0], device=DEV, dtype=torch.float32).to(dtype)
    mask = torch.tensor([1, 1, 1, 1, 1, 0], dtype=torch.bool, device=DEV)
    p0, mb0 = p.clone(), mb.clone()
    ref = [(p[r].clone(), mb[r].clone()) for r in range(R)]
    ref_steps = steps.clone()
    for _ in range(3):
        grad = rnd()
        ref_steps += mask.to(dtype)
        for r in range(R):
            if not mask[r]:
                continue
            m_r = mom[r].item()
            torch._fused_sgd_([ref[r][0]], [grad[r].clone()], [ref[r][1]] if m_r != 0 else [],
                              weight_decay=wdv[r].item(), momentum=m_r, lr=lr[r].item(),
                              dampening=damp[r].item(), nesterov=m_r != 0, maximize=maximize,
                              is_first_step=bool(ref_steps[r].item() == 1),
                              grad_scale=None, found_inf=None)
        K.sgd_step_(p, grad, mb, steps, lr, mom, damp, wdv, mask, nesterov=True,
                    maximize=maximize)
    torch.cuda.synchronize()
    for r in range(R):
        if not mask[r]:
            same(f"frozen params[{r}]", p[r], p0[r])
            same(f"frozen momentum_buffers[{r}]", mb[r], mb0[r])
            continue
        same(f"params[{r}]", p[r], ref[r][0])
        if mom[r].item() != 0:
            same(f"momentum_buffers[{r}]", mb[r], ref[r][1])
    assert torch.equal(steps, ref_steps)


@pytest.mark.parametrize("T", ROWS)
@pytest.mark.parametrize("lr_decay,wd,eps,maximize", list(itertools.product(
    [0.0, 1e-2], [0.0, 1e-2], [1e-10, 1e-6], [False, True])))
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_adagrad_rows_bit_identical_to_aten(T, lr_decay, wd, eps, maximize, dtype, R=2):
    g = torch.Generator(device=DEV).manual_seed(T + 2)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g, dtype=dtype)
    p, s = rnd(), rnd().abs()
    (lr,) = _vecs(R, [1e-2, 3e-2], dtype=dtype)
    lrd = torch.full((R,), f32(lr_decay), device=DEV, dtype=dtype)
    wdv = torch.full((R,), f32(wd), device=DEV, dtype=dtype)
    ev = torch.full((R,), f32(eps), device=DEV, dtype=dtype)
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    ref = [(p[r].clone(), s[r].clone(), torch.zeros((), device=DEV)) for r in range(R)]
    for _ in range(3):
        grad = rnd()
        for r in range(R):
            pr, sr, st = ref[r]
            st += 1
            torch._fused_adagrad_([pr], [grad[r].clone()], [sr], [st], lr=lr[r].item(),
                                  lr_decay=lrd[r].item(), weight_decay=wdv[r].item(),
                                  eps=ev[r].item(), maximize=maximize, grad_scale=None,
                                  found_inf=None)
        K.adagrad_step_(p, grad, s, steps, lr, lrd, wdv, ev, mask, maximize=maximize)
    torch.cuda.synchronize()
    for r in range(R):
        same(f"params[{r}]", p[r], ref[r][0])
        same(f"state_sums[{r}]", s[r], ref[r][1])
        assert steps[r].item() == ref[r][2].item() == 3


def test_adam_matches_torch_optim_fused_end_to_end():
    """N independent torch.optim.AdamW(fused=True) vs one consolidated call."""
    R, shapes = 4, [(32, 16), (32,), (10, 32), (10,)]
    torch.manual_seed(0)
    models = [[torch.randn(*s, device=DEV, requires_grad=True) for s in shapes]
              for _ in range(R)]
    # The consolidated state carries float32 hyperparameters, so torch.optim
    # gets the same float32 values (as the reference's parity test does).
    opts = [torch.optim.AdamW(ps, lr=f32(1e-3), betas=(f32(0.9), f32(0.999)),
                              eps=f32(1e-8), weight_decay=f32(1e-2), fused=True)
            for ps in models]
    flat = torch.stack([torch.cat([t.detach().reshape(-1) for t in ps]) for ps in models])
    T = flat.shape[1]
    m, v = torch.zeros_like(flat), torch.zeros_like(flat)
    steps = torch.zeros(R, device=DEV)
    full = lambda x: torch.full((R,), f32(x), device=DEV)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    for _ in range(4):
        grads = [[torch.randn_like(t) for t in ps] for ps in models]
        for ps, gs, opt in zip(models, grads, opts):
            for t, gt in zip(ps, gs):
                t.grad = gt.clone()
            opt.step()
        gflat = torch.stack([torch.cat([gt.reshape(-1) for gt in gs]) for gs in grads])
        K.adam_step_(flat, gflat, m, v, None, steps, full(1e-3), full(0.9), full(0.999),
                     full(1e-8), full(1e-2), mask, amsgrad=False, maximize=False,
                     decoupled_weight_decay=True)
    torch.cuda.synchronize()
    want = torch.stack([torch.cat([t.detach().reshape(-1) for t in ps]) for ps in models])
    assert flat.shape == (R, T)
    same("params", flat, want)

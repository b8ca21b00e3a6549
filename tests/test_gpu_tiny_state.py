"""Adam and Adagrad rows against torch's fused kernels, bit for bit, with
optimizer state that sends the kernels' square roots down both of their paths:
values at and below 2^-96 (zero, subnormal, just under and over the threshold)
mixed with ordinary ones inside wavefronts, next to rows whose first half holds
ordinary values only. Gradients are zero wherever the state is tiny, so the
square root's input stays tiny after the update. Every dtype, small launches
and launches past the MALL-resident size (the two streaming shapes)."""

from __future__ import annotations

import pytest
import torch

import churten_amd.kernels as K

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
LEVELS = [0.0, 1e-40, 2.0 ** -100, 2.0 ** -97, 2.0 ** -95, 1e-8, 1.0, 1e4]
ORDINARY = (5, 6)  # indices of ordinary magnitudes in LEVELS


def _bits(t):
    return t.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


def same(name, a, b):
    if not torch.equal(_bits(a), _bits(b)):
        n = (_bits(a) != _bits(b)).sum().item()
        raise AssertionError(f"{name}: {n}/{a.numel()} elements differ")


def _state(R, T, g, dtype):
    """Per element one of LEVELS; the first half of each row ordinary only.
    Returns the values and the mask of ordinary elements."""
    idx = torch.randint(0, len(LEVELS), (R, T), generator=g, device=DEV)
    ordinary = torch.randint(ORDINARY[0], ORDINARY[1] + 1, (R, T), generator=g, device=DEV)
    idx[:, : T // 2] = ordinary[:, : T // 2]
    vals = torch.tensor(LEVELS, device=DEV)[idx]
    return vals.to(dtype), (idx >= ORDINARY[0]) & (idx <= ORDINARY[1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("amsgrad", [False, True])
@pytest.mark.parametrize("R,T", [(3, 4096), (4, 8 << 20)], ids=["small", "large"])
def test_adam_tiny_state_bit_identical_to_aten(R, T, amsgrad, dtype):
    g = torch.Generator(device=DEV).manual_seed(T + amsgrad)
    p = torch.randn(R, T, device=DEV, generator=g).to(dtype)
    m = torch.randn(R, T, device=DEV, generator=g).to(dtype)
    v, ordinary = _state(R, T, g, dtype)
    mx, _ = _state(R, T, g, dtype)
    lr = torch.tensor([1e-2, 3e-3, 5e-2, 1e-3][:R], device=DEV).to(dtype)
    b1 = torch.tensor([0.9, 0.8, 0.95, 0.9][:R], device=DEV).to(dtype)
    b2 = torch.tensor([0.999, 0.99, 0.9999, 0.999][:R], device=DEV).to(dtype)
    eps = torch.tensor([1e-8, 1e-6, 1e-7, 1e-8][:R], device=DEV).to(dtype)
    wd = torch.zeros(R, device=DEV, dtype=dtype)
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    ref = [[t[r].clone() for t in (p, m, v, mx)] + [torch.zeros((), device=DEV)]
           for r in range(R)]
    for _ in range(2):
        grad = (torch.randn(R, T, device=DEV, generator=g) * ordinary).to(dtype)
        for r in range(R):
            pr, mr, vr, xr, sr = ref[r]
            sr += 1
            torch._fused_adam_([pr], [grad[r].clone()], [mr], [vr], [xr] if amsgrad else [],
                               [sr], lr=lr[r].item(), beta1=b1[r].item(), beta2=b2[r].item(),
                               weight_decay=0.0, eps=eps[r].item(), amsgrad=amsgrad,
                               maximize=False, grad_scale=None, found_inf=None)
        K.adam_step_(p, grad, m, v, mx if amsgrad else None, steps, lr, b1, b2, eps, wd, mask,
                     amsgrad=amsgrad, maximize=False, decoupled_weight_decay=False)
    torch.cuda.synchronize()
    for r in range(R):
        same(f"params[{r}]", p[r], ref[r][0])
        same(f"exp_avgs[{r}]", m[r], ref[r][1])
        same(f"exp_avg_sqs[{r}]", v[r], ref[r][2])
        if amsgrad:
            same(f"max_exp_avg_sqs[{r}]", mx[r], ref[r][3])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("R,T", [(3, 4096), (4, 8 << 20)], ids=["small", "large"])
def test_adagrad_tiny_state_bit_identical_to_aten(R, T, dtype):
    g = torch.Generator(device=DEV).manual_seed(T + 7)
    p = torch.randn(R, T, device=DEV, generator=g).to(dtype)
    s, ordinary = _state(R, T, g, dtype)
    lr = torch.tensor([1e-2, 3e-2, 5e-3, 1e-2][:R], device=DEV).to(dtype)
    lrd = torch.zeros(R, device=DEV, dtype=dtype)
    wd = torch.zeros(R, device=DEV, dtype=dtype)
    eps = torch.full((R,), 1e-10, device=DEV).to(dtype)
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    ref = [(p[r].clone(), s[r].clone(), torch.zeros((), device=DEV)) for r in range(R)]
    for _ in range(2):
        grad = (torch.randn(R, T, device=DEV, generator=g) * ordinary).to(dtype)
        for r in range(R):
            pr, sr, st = ref[r]
            st += 1
            torch._fused_adagrad_([pr], [grad[r].clone()], [sr], [st], lr=lr[r].item(),
                                  lr_decay=0.0, weight_decay=0.0, eps=eps[r].item(),
                                  maximize=False, grad_scale=None, found_inf=None)
        K.adagrad_step_(p, grad, s, steps, lr, lrd, wd, eps, mask, maximize=False)
    torch.cuda.synchronize()
    for r in range(R):
        same(f"params[{r}]", p[r], ref[r][0])
        same(f"state_sums[{r}]", s[r], ref[r][1])

"""Twenty-step trajectories against torch's fused kernels, bit for bit.

The ATen parity sweep runs three steps. Here every optimizer runs twenty, so
the bias corrections, Adagrad's lr decay and the moments' growth move through
many step counts, on rows long enough for torch's vector path (262144
elements, four of its 65536-element chunks) and rows of 262147 elements that
it runs element by element, in all four dtypes. Gradients mix
ordinary values with exact zeros and subnormal values of the dtype (an eighth
and a quarter of its smallest normal), so moments underflow, stay zero, and
restart; each row has its own hyperparameters. Every replica row is compared after every
step: params and every state buffer, the steps counter at the end.
"""

from __future__ import annotations

import pytest
import torch

import churten_amd.kernels as K

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
STEPS = 20
DTYPES = [torch.float32, torch.float64, torch.float16, torch.bfloat16]
INT = {torch.float32: torch.int32, torch.float64: torch.int64, torch.float16: torch.int16,
       torch.bfloat16: torch.int16}


def same(name, a, b):
    if not torch.equal(a.view(INT[a.dtype]), b.view(INT[b.dtype])):
        n = int((a.view(INT[a.dtype]) != b.view(INT[b.dtype])).sum())
        raise AssertionError(f"{name}: {n}/{a.numel()} elements differ")


def grads(gen, R, T, dtype):
    """Ordinary values, with a tenth exact zeros and a tenth subnormal ones."""
    g = torch.randn(R, T, generator=gen, device=DEV)
    kind = torch.randint(0, 10, (R, T), generator=gen, device=DEV)
    tiny = torch.finfo(dtype).smallest_normal * 2.0 ** -3
    g = torch.where(kind == 0, torch.zeros_like(g), g)
    g = torch.where(kind == 1, g.sign() * tiny * (1 + kind.float()), g)
    return g.to(dtype)


def vec(vals, dtype):
    return torch.tensor(vals, device=DEV, dtype=torch.float32).to(dtype)


CASES = [
    ("adam", dict(amsgrad=False, maximize=False, decoupled=False)),
    ("adam", dict(amsgrad=True, maximize=True, decoupled=True)),
    ("sgd", dict(nesterov=True, dampening=0.0)),
    ("sgd", dict(nesterov=False, dampening=0.3)),
    ("adagrad", dict(maximize=False)),
    ("adagrad", dict(maximize=True)),
]


@pytest.mark.parametrize("T", [262144, 262147], ids=["vector-rows", "element-rows"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("op,kw", CASES, ids=lambda c: c if isinstance(c, str) else
                         "-".join(k for k, v in c.items() if v))
def test_twenty_steps_bit_identical_to_aten(op, kw, dtype, T):
    R = 2
    gen = torch.Generator(device=DEV).manual_seed(T + {"adam": 1, "sgd": 2, "adagrad": 3}[op])
    p = torch.randn(R, T, generator=gen, device=DEV).to(dtype)
    steps = torch.zeros(R, device=DEV, dtype=dtype)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    if op == "adam":
        m = torch.zeros(R, T, device=DEV, dtype=dtype)
        v = torch.zeros(R, T, device=DEV, dtype=dtype)
        mx = torch.zeros(R, T, device=DEV, dtype=dtype) if kw["amsgrad"] else None
        lr, b1, b2 = vec([1e-3, 3e-2], dtype), vec([0.9, 0.8], dtype), vec([0.999, 0.99], dtype)
        eps = vec([1e-8 if dtype not in (torch.float16,) else 1e-4, 1e-6], dtype)
        wd = vec([0.0, 1e-2], dtype)
        state = [m, v] + ([mx] if mx is not None else [])
    elif op == "sgd":
        buf = torch.zeros(R, T, device=DEV, dtype=dtype)
        lr, mom = vec([1e-2, 5e-2], dtype), vec([0.9, 0.5], dtype)
        damp = vec([kw["dampening"]] * R, dtype)
        wd = vec([1e-2, 0.0], dtype)
        state = [buf]
    else:
        s = torch.rand(R, T, generator=gen, device=DEV).to(dtype)
        lr, lrd = vec([1e-2, 3e-2], dtype), vec([0.0, 1e-2], dtype)
        wd, eps = vec([0.0, 1e-2], dtype), vec([1e-10, 1e-6], dtype)
        state = [s]
    ref = [[t[r].clone() for t in [p] + state] + [torch.zeros((), device=DEV)]
           for r in range(R)]
    for k in range(STEPS):
        g = grads(gen, R, T, dtype)
        if op == "adam":
            K.adam_step_(p, g, state[0], state[1], mx, steps, lr, b1, b2, eps, wd, mask,
                         amsgrad=kw["amsgrad"], maximize=kw["maximize"],
                         decoupled_weight_decay=kw["decoupled"])
        elif op == "sgd":
            K.sgd_step_(p, g, state[0], steps, lr, mom, damp, wd, mask,
                        nesterov=kw["nesterov"], maximize=False)
        else:
            K.adagrad_step_(p, g, state[0], steps, lr, lrd, wd, eps, mask,
                            maximize=kw["maximize"])
        for r in range(R):
            row = ref[r]
            st = row[-1]
            st += 1
            gr = g[r].clone()
            if op == "adam":
                fn = torch._fused_adamw_ if kw["decoupled"] else torch._fused_adam_
                fn([row[0]], [gr], [row[1]], [row[2]], [row[3]] if kw["amsgrad"] else [], [st],
                   lr=lr[r].item(), beta1=b1[r].item(), beta2=b2[r].item(),
                   weight_decay=wd[r].item(), eps=eps[r].item(), amsgrad=kw["amsgrad"],
                   maximize=kw["maximize"], grad_scale=None, found_inf=None)
            elif op == "sgd":
                torch._fused_sgd_([row[0]], [gr], [row[1]], weight_decay=wd[r].item(),
                                  momentum=mom[r].item(), lr=lr[r].item(),
                                  dampening=damp[r].item(), nesterov=kw["nesterov"],
                                  maximize=False, is_first_step=(k == 0), grad_scale=None,
                                  found_inf=None)
            else:
                torch._fused_adagrad_([row[0]], [gr], [row[1]], [st], lr=lr[r].item(),
                                      lr_decay=lrd[r].item(), weight_decay=wd[r].item(),
                                      eps=eps[r].item(), maximize=kw["maximize"],
                                      grad_scale=None, found_inf=None)
        torch.cuda.synchronize()
        for r in range(R):
            same(f"step {k + 1} params[{r}]", p[r], ref[r][0])
            for i, t in enumerate(state):
                same(f"step {k + 1} state {i} [{r}]", t[r], ref[r][1 + i])
    assert steps.tolist() == [float(STEPS)] * R

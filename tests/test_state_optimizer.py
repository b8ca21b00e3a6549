"""The callers of the operators: the consolidated State and the Adam / SGD /
Adagrad GradientTransformations, end to end.

Mirrors the reference's tier-6 and layout tests (test/optimizer/test_state.py,
test_state_sgd.py, test_state_adagrad.py, test/test_consolidation_alignment.py):
an ensemble of N identical replicas trained through ``apply_gradient`` must
track a single copy of the model trained with ``torch.optim`` step for step,
the (N, T) width is padded to a multiple of 4, and the pad lanes stay exactly
zero through training. Every test runs on the CPU key; the ``gpu`` variants run
the same loop on the MI355X, where the Adam and SGD ensembles, stepped on the
same gradients, must equal ``torch.optim.*(fused=True)`` bit for bit.
"""

from __future__ import annotations

from copy import deepcopy

import pytest
import torch
from torch.func import functional_call, grad_and_value, vmap
from torch.nn import Linear, ReLU, Sequential
from torch.nn.functional import binary_cross_entropy_with_logits

from churten_amd.optimizer import SGD, Adagrad, Adam, GradientTransformation
from churten_amd.state import _CONSOLIDATION_ALIGNMENT, State

DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]


def f32(x):
    return torch.tensor(x, dtype=torch.float32).item()


def make_net(device="cpu"):
    torch.manual_seed(0)
    return Sequential(Linear(5, 10), ReLU(), Linear(10, 1)).to(device)


def ensemble(net, n):
    return State.from_models([deepcopy(net) for _ in range(n)])


def grad_fn(net):
    base = deepcopy(net).to("meta")

    def loss_fn(params, buffers, x, y):
        return binary_cross_entropy_with_logits(functional_call(base, (params, buffers), (x,)), y)

    return vmap(grad_and_value(loss_fn, argnums=0), in_dims=(0, 0, None, None))


def data(device):
    g = torch.Generator().manual_seed(1)
    x = torch.rand(10, 5, generator=g).to(device)
    y = torch.cat([torch.zeros(5, 1), torch.ones(5, 1)]).to(device)
    return x, y


def run_pair(device, opt_cls, opt_kwargs, torch_opt, n=3, steps=5, shared_grads=False):
    """Trains the ensemble and one reference copy. With ``shared_grads`` the
    reference is stepped on replica 0's gradients (so the comparison isolates
    the optimizer: the ensemble's vmapped backward and the reference's
    ``.backward()`` need not agree to the last bit on the GPU)."""
    net = make_net(device)
    state = ensemble(net, n)
    opt_cls.init(state, **opt_kwargs)
    ref = deepcopy(net)
    opt = torch_opt(ref.parameters())
    x, y = data(device)
    gl = grad_fn(net)
    for _ in range(steps):
        grads, _ = gl(state.params_dict, state.buffers_dict, x, y)
        opt_cls.apply_gradient(state, grads)
        opt.zero_grad(set_to_none=True)
        if shared_grads:
            for name, p in ref.named_parameters():
                p.grad = grads[name][0].detach().clone()
        else:
            binary_cross_entropy_with_logits(ref(x), y).backward()
        opt.step()
    return state, dict(ref.named_parameters())


@pytest.mark.parametrize("device", DEVICES)
def test_adam_ensemble_tracks_torch_adamw(device):
    hyp = dict(lr=f32(1e-2), betas=(f32(0.9), f32(0.999)), eps=f32(1e-8),
               weight_decay=f32(1e-2))
    fused = device == "cuda"
    state, ref = run_pair(
        device, Adam, dict(lr=hyp["lr"], beta1=hyp["betas"][0], beta2=hyp["betas"][1],
                           eps=hyp["eps"], weight_decay=hyp["weight_decay"]),
        lambda ps: torch.optim.AdamW(ps, fused=fused, **hyp), shared_grads=fused)
    for name, want in ref.items():
        for r in range(3):
            got = state.params_dict[name][r]
            if fused and r == 0:
                assert torch.equal(got, want.detach()), name
            else:
                torch.testing.assert_close(got, want.detach(), rtol=1e-5, atol=1e-6)
    assert state.optimizer_state["state_steps"].tolist() == [5.0] * 3


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("nesterov", [False, True])
def test_sgd_ensemble_tracks_torch_sgd(device, nesterov):
    hyp = dict(lr=f32(5e-2), momentum=f32(0.9), weight_decay=f32(1e-3))
    fused = device == "cuda"
    state, ref = run_pair(device, SGD, dict(nesterov=nesterov, **hyp),
                          lambda ps: torch.optim.SGD(ps, nesterov=nesterov, fused=fused, **hyp),
                          shared_grads=fused)
    for name, want in ref.items():
        for r in range(3):
            got = state.params_dict[name][r]
            if fused and r == 0:
                assert torch.equal(got, want.detach()), name
            else:
                torch.testing.assert_close(got, want.detach(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("device", DEVICES)
def test_adagrad_ensemble_tracks_torch_adagrad(device):
    hyp = dict(lr=f32(5e-2), lr_decay=f32(1e-2), weight_decay=f32(1e-3),
               initial_accumulator_value=0.1, eps=f32(1e-10))
    state, ref = run_pair(device, Adagrad, hyp, lambda ps: torch.optim.Adagrad(ps, **hyp))
    for name, want in ref.items():
        for r in range(3):
            torch.testing.assert_close(state.params_dict[name][r], want.detach(),
                                       rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# layout (reference test_consolidation_alignment.py)
# ---------------------------------------------------------------------------
class Buffered(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = Linear(4, 8)
        self.register_buffer("scale", torch.ones(5))

    def forward(self, x):
        return self.lin(x) * self.scale[0]


def test_width_is_padded_and_offsets_never_cover_the_pad():
    state = State.from_models([Sequential(Linear(4, 8), ReLU(), Linear(8, 1)) for _ in range(3)])
    raw = sum(n for _, _, _, n in state.param_meta)
    assert raw == 49
    assert state.params.shape == (3, 52) and 52 % _CONSOLIDATION_ALIGNMENT == 0
    assert max(off + n for _, _, off, n in state.param_meta) == raw
    assert not state.params[:, raw:].any()
    assert state.buffers.shape == (3, 0) and state.buffer_meta == []


def test_buffers_are_padded_and_views_alias():
    state = State.from_models([Buffered() for _ in range(2)])
    assert state.buffers.shape == (2, 8)
    assert torch.equal(state.buffers_dict["scale"], torch.ones(2, 5))
    state.params_dict["lin.bias"].fill_(3.0)
    assert torch.equal(state.params[:, 32:40], torch.full((2, 8), 3.0))
    state._consolidated_grads.update_({"lin.weight": torch.ones(2, 8, 4)})
    assert torch.equal(state.grads[:, :32], torch.ones(2, 32))
    assert not state.grads[:, 32:].any()


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("opt_cls,kw", [
    (Adam, dict(lr=1e-2, weight_decay=1e-2)),
    (SGD, dict(lr=1e-2, momentum=0.9, weight_decay=1e-2)),
    (Adagrad, dict(lr=1e-2, weight_decay=1e-2, initial_accumulator_value=0.1)),
])
def test_pad_lanes_stay_zero_after_steps(device, opt_cls, kw):
    net = Sequential(Linear(4, 8), ReLU(), Linear(8, 1)).to(device)
    state = State.from_models([Sequential(Linear(4, 8), ReLU(), Linear(8, 1)).to(device)
                               for _ in range(3)])
    opt_cls.init(state, **kw)
    x, y = torch.randn(3, 16, 4, device=device), torch.randn(3, 16, 1, device=device)
    base = deepcopy(net).to("meta")

    def loss(params, buffers, x, y):
        return ((functional_call(base, (params, buffers), (x,)) - y) ** 2).mean()

    gl = vmap(grad_and_value(loss, argnums=0), in_dims=(0, 0, 0, 0))
    for _ in range(5):
        grads, _ = gl(state.params_dict, state.buffers_dict, x, y)
        opt_cls.apply_gradient(state, grads)
    assert state.optimizer_state["state_steps"].tolist() == [5.0] * 3
    for name, buf in [("params", state.flat_params), ("grads", state.flat_grads)] + [
            (k, v) for k, v in state.optimizer_state.items()
            if isinstance(v, torch.Tensor) and v.dim() == 2 and k != "state_sums"]:
        assert not buf[:, 49:].any(), f"{name} pad lanes are not zero"


# ---------------------------------------------------------------------------
# optimizer construction
# ---------------------------------------------------------------------------
def test_gradient_transformation_requires_init_and_update():
    with pytest.raises(TypeError, match="init"):
        GradientTransformation("NoInit", (), {"update": lambda s: s})
    with pytest.raises(TypeError, match="update"):
        GradientTransformation("NoUpdate", (), {"init": lambda s: s})


def test_sgd_nesterov_validation():
    state = ensemble(make_net(), 2)
    with pytest.raises(ValueError, match="Nesterov"):
        SGD.init(state, lr=1e-2, momentum=0.0, nesterov=True)
    with pytest.raises(ValueError, match="Nesterov"):
        SGD.init(state, lr=1e-2, momentum=0.9, dampening=0.1, nesterov=True)
    SGD.init(state, lr=1e-2, momentum=torch.tensor([0.0, 0.9]), nesterov=True)
    assert "momentum_buffers" in state.optimizer_state


def test_sgd_without_momentum_allocates_no_buffer():
    state = ensemble(make_net(), 2)
    SGD.init(state, lr=1e-2)
    assert "momentum_buffers" not in state.optimizer_state
    assert state.optimizer_state["has_momentum"] is False


def test_per_replica_hyperparameters_and_flags():
    state = ensemble(make_net(), 3)
    Adam.init(state, lr=torch.tensor([1e-3, 1e-2, 1e-1]), amsgrad=True, maximize=True,
              decoupled_weight_decay=False)
    opt = state.optimizer_state
    assert opt["lr"].dtype == torch.float32 and opt["lr"].tolist() == pytest.approx([1e-3, 1e-2, 1e-1])
    assert opt["max_exp_avg_sqs"].shape == state.params.shape
    assert opt["amsgrad"] is True and opt["maximize"] is True
    assert opt["decoupled_weight_decay"] is False
    assert opt["state_steps"].tolist() == [0.0] * 3


def test_adagrad_initial_accumulator_fills_pad_lanes_too():
    state = ensemble(make_net(), 2)
    Adagrad.init(state, initial_accumulator_value=0.25)
    assert torch.equal(state.optimizer_state["state_sums"],
                       torch.full_like(state.params, 0.25))


def test_frozen_replica_does_not_move():
    state = ensemble(make_net(), 3)
    Adam.init(state, lr=1e-2)
    state.active_mask[1] = False
    before = state.params[1].clone()
    x, y = data("cpu")
    grads, _ = grad_fn(make_net())(state.params_dict, state.buffers_dict, x, y)
    Adam.apply_gradient(state, grads)
    assert torch.equal(state.params[1], before)
    assert state.optimizer_state["state_steps"].tolist() == [1.0, 0.0, 1.0]


# ---------------------------------------------------------------------------
# bfloat16 optimizer state (an extension; float32 params)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("opt_cls,kw,keys", [
    (Adam, dict(lr=1e-2, amsgrad=True), ("exp_avgs", "exp_avg_sqs", "max_exp_avg_sqs")),
    (SGD, dict(lr=5e-2, momentum=0.9, nesterov=True), ("momentum_buffers",)),
    (Adagrad, dict(lr=5e-2, initial_accumulator_value=0.1), ("state_sums",)),
])
def test_bf16_state_ensemble_tracks_float32_state(device, opt_cls, kw, keys):
    net = make_net(device)
    x, y = data(device)
    gl = grad_fn(net)
    runs = {}
    for sd in (None, torch.bfloat16):
        state = ensemble(net, 2)
        opt_cls.init(state, state_dtype=sd, **kw)
        for _ in range(5):
            grads, _ = gl(state.params_dict, state.buffers_dict, x, y)
            opt_cls.apply_gradient(state, grads)
        runs[sd] = state
    lo, hi = runs[torch.bfloat16], runs[None]
    for k in keys:
        assert lo.optimizer_state[k].dtype == torch.bfloat16
        assert hi.optimizer_state[k].dtype == torch.float32
    assert lo.params.dtype == torch.float32
    torch.testing.assert_close(lo.params, hi.params, rtol=0, atol=2e-3)
    assert lo.params.shape[1] == 72 and not lo.params[:, 71:].any()  # pad lane stays zero

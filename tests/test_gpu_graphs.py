"""The operators under HIP graph capture.

Small ensembles are launch-bound, and the MI355X way to remove launch overhead
is to capture the training step in a graph and replay it. The operators
enqueue only kernels on the current stream (no host synchronisation, no memset
nodes, the zero result from torch's caching allocator), so they can be
captured. Each test replays the graph several times, with eager work and
synchronisations between replays, and checks every replay bit for bit against
the same sequence run eagerly.
"""

from __future__ import annotations

import pytest
import torch

import churten_amd.kernels as K

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
R, T = 6, 4 * 1000 + 12


def _adam_state(seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g)  # noqa: E731
    p, m, v = rnd(), rnd().abs(), rnd().abs()
    hyp = [torch.full((R,), x, device=DEV) for x in (1e-2, 0.9, 0.999, 1e-8, 1e-2)]
    steps = torch.zeros(R, device=DEV)
    mask = torch.tensor([True, True, False, True, True, False], device=DEV)
    return [p, None, m, v, None, steps, *hyp, mask]


def _clone(args):
    return [a.clone() if isinstance(a, torch.Tensor) else a for a in args]


def _run(args, grad):
    args[1] = grad
    return K.adam_step_(*args, amsgrad=False, maximize=False, decoupled_weight_decay=True)


@pytest.mark.parametrize("segmented", [False, True])
def test_adam_step_replays_match_eager(segmented):
    torch.manual_seed(0)
    grads = [torch.randn(R, T, device=DEV) for _ in range(4)]
    eager = _adam_state(1)
    graphed = _clone(eager)
    static_grad = torch.zeros(R, T, device=DEV)
    cols = [0, 4000]
    parts = [static_grad[:, :4000], static_grad[:, 4000:]]

    def step(args):
        if segmented:
            return torch.ops.churten.adam_step_segments_(
                args[0], parts, cols, None, args[2], args[3], None, *args[5:],
                amsgrad=False, maximize=False, decoupled_weight_decay=True)
        return _run(args, static_grad)

    # warm up on a side stream, as torch's capture guide requires
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    warm = _clone(eager)
    with torch.cuda.stream(s):
        static_grad.copy_(grads[0])
        step(warm)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step(graphed)
    for i, gr in enumerate(grads):
        static_grad.copy_(gr)
        graph.replay()
        torch.cuda.synchronize()
        if segmented:
            ref = torch.ops.churten.adam_step_segments_(
                eager[0], [gr[:, :4000], gr[:, 4000:]], cols, None, eager[2], eager[3], None,
                *eager[5:], amsgrad=False, maximize=False, decoupled_weight_decay=True)
        else:
            ref = _run(eager, gr.clone())
        torch.cuda.synchronize()
        for k in (0, 2, 3, 5):
            assert torch.equal(graphed[k], eager[k]), (i, k)
        assert out.item() == 0 and ref.item() == 0
    assert graphed[5].tolist() == [4.0, 4.0, 0.0, 4.0, 4.0, 0.0]


def test_sgd_and_adagrad_replays_match_eager():
    torch.manual_seed(1)
    g = torch.Generator(device=DEV).manual_seed(2)
    rnd = lambda: torch.randn(R, T, device=DEV, generator=g)  # noqa: E731
    p1, b1, p2, s2 = rnd(), rnd(), rnd(), rnd().abs()
    steps1, steps2 = torch.zeros(R, device=DEV), torch.zeros(R, device=DEV)
    mask = torch.ones(R, dtype=torch.bool, device=DEV)
    # hyperparameters exist before capture: nothing is allocated or filled in the graph
    hs = [torch.full((R,), x, device=DEV) for x in (1e-2, 0.9, 0.0, 1e-3)]
    ha = [torch.full((R,), x, device=DEV) for x in (1e-2, 1e-3, 1e-3, 1e-10)]
    eager = [t.clone() for t in (p1, b1, steps1, p2, s2, steps2)]
    static_grad = torch.zeros(R, T, device=DEV)

    def step(p1, b1, steps1, p2, s2, steps2, grad):
        K.sgd_step_(p1, grad, b1, steps1, *hs, mask, nesterov=True, maximize=False)
        K.adagrad_step_(p2, grad, s2, steps2, *ha, mask, maximize=False)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(*[t.clone() for t in (p1, b1, steps1, p2, s2, steps2)], static_grad)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(p1, b1, steps1, p2, s2, steps2, static_grad)
    for i in range(4):
        gr = torch.randn(R, T, device=DEV)
        static_grad.copy_(gr)
        graph.replay()
        torch.cuda.synchronize()
        step(*eager, gr)
        torch.cuda.synchronize()
        for a, b in zip((p1, b1, steps1, p2, s2, steps2), eager):
            assert torch.equal(a, b), i

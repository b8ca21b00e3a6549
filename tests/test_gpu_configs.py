"""BASELINE.json's five configurations at their real sizes.

Configs 1-4 (up to 64 x 545,100) are checked whole: every element of every
row, after one step, bit-identical to the oracle's device formulation (frozen
rows included: they must come back unchanged). Config 5 (128 x 25,171,968,
52 GB of state) is checked through size-independent properties: frozen rows
unchanged bit for bit, the step counters, and windows of active rows -- at the
start, the middle and the very end of the buffers, where element offsets pass
2^31 -- bit-identical to the oracle run on the same window.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import churten_amd.kernels  # noqa: F401
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _np(t):
    return None if t is None else t.detach().cpu().numpy().copy()


def _oracle_call(op, host, kw):
    if op == "adam":
        O.adam_step(O.DEVICE, *host, **kw)
    elif op == "sgd":
        O.sgd_step(O.DEVICE, *host, **kw)
    else:
        O.adagrad_step(O.DEVICE, *host, **kw)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_config_one_step_bit_exact(cfg):
    op, args, kw, _ = bench.make_config(cfg)
    host = [_np(t) for t in args]
    getattr(torch.ops.torchstrap, f"{op}_step_")(*args, **kw)
    torch.cuda.synchronize()
    _oracle_call(op, host, kw)
    for i, (t, h) in enumerate(zip(args, host)):
        if t is None or i == 1:
            continue
        got = _np(t)
        if got.dtype == np.bool_:
            continue
        assert np.array_equal(got.view(np.uint32), h.view(np.uint32)), f"config {cfg} arg {i}"


def test_config5_properties():
    op, args, kw, nbytes = bench.make_config(5)
    p, gr, m, v, _, steps = args[:6]
    mask = args[11]
    R, T = p.shape
    assert (R, T) == (128, 25171968) and R * T > 2**31
    frozen = (~mask).nonzero().flatten()
    active = mask.nonzero().flatten().tolist()
    assert len(frozen) > 0 and len(active) > 0
    keep = [t[frozen].clone() for t in (p, m, v)]
    windows = [(active[0], 0), (active[len(active) // 2], T // 2 - 2048),
               (active[-1], T - 4096)]
    hyp = [_np(t) for t in args[6:11]]
    before = []
    for r, t0 in windows:
        before.append([_np(t[r : r + 1, t0 : t0 + 4096]) for t in (p, gr, m, v)]
                      + [_np(steps[r : r + 1])] + [h[r : r + 1].copy() for h in hyp])
    steps0 = _np(steps)
    torch.ops.torchstrap.adam_step_(*args, **kw)
    torch.cuda.synchronize()
    for t, k in zip((p, m, v), keep):
        assert torch.equal(t[frozen], k)
    want_steps = steps0 + _np(mask).astype(np.float32)
    assert np.array_equal(_np(steps), want_steps)
    for (r, t0), b in zip(windows, before):
        pw, gw, mw, vw, sw, *hw = b
        O.adam_step(O.DEVICE, pw, gw, mw, vw, None, sw, *hw, np.ones(1, bool), **kw)
        for name, t, want in (("p", p, pw), ("m", m, mw), ("v", v, vw)):
            got = _np(t[r : r + 1, t0 : t0 + 4096])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (
                f"row {r} window {t0}: {name}")


def test_config5_segmented_update_equals_dense():
    """The 12 per-parameter gradients of config 5's transformer block, read in
    place by the segmented update (consolidated gradient refilled on the way),
    give the same state, bit for bit, over all 52 GB, as the dense update."""
    op, args, kw, _ = bench.make_config(5)
    p, gr, m, v, mx, steps, *hyp = args
    twin = [t.clone() for t in (p, m, v, steps)]
    cols, grads, c = [], [], 0
    for shape in bench.BLOCK_LAYOUT:
        n = int(np.prod(shape))
        cols.append(c)
        grads.append(gr[:, c:c + n])  # (R, n) views with row stride T
        c += n
    gout = torch.zeros_like(gr)
    torch.ops.torchstrap.adam_step_(p, gr, m, v, None, steps, *hyp, **kw)
    torch.ops.churten.adam_step_segments_(twin[0], grads, cols, gout, twin[1], twin[2], None,
                                          twin[3], *hyp, **kw)
    torch.cuda.synchronize()
    for name, a, b in (("params", p, twin[0]), ("exp_avgs", m, twin[1]),
                       ("exp_avg_sqs", v, twin[2]), ("steps", steps, twin[3])):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
    assert torch.equal(gout, gr)


def test_config5_bf16_state_windows():
    """Config 5 with bfloat16 moments: frozen rows untouched, windows of active
    rows (past the 2^31-element mark too) bit-identical to the oracle's float32
    step followed by nearest-even rounding."""
    op, args, kw, _ = bench.make_config(5)
    p, gr, m, v, mx, steps, *hyp = args
    mask = hyp[-1]
    mb, vb = m.to(torch.bfloat16), v.to(torch.bfloat16)
    del m, v
    R, T = p.shape
    active = mask.nonzero().flatten().tolist()
    frozen = (~mask).nonzero().flatten()
    windows = [(active[0], 0), (active[-1], T - 4096)]
    before = [[_np(t[r:r + 1, t0:t0 + 4096].float()) for t in (p, gr, mb, vb)] for r, t0 in windows]
    hyp_np = [_np(t) for t in hyp[:-1]]
    steps0 = _np(steps)
    keep = [t[frozen].clone() for t in (p, mb, vb)]
    torch.ops.torchstrap.adam_step_(p, gr, mb, vb, None, steps, *hyp, **kw)
    torch.cuda.synchronize()
    for t, k in zip((p, mb, vb), keep):
        assert torch.equal(t[frozen], k)
    for (r, t0), (pw, gw, mw, vw) in zip(windows, before):
        sw = steps0[r:r + 1].copy()
        O.adam_step(O.DEVICE, pw, gw, mw, vw, None, sw, *[h[r:r + 1].copy() for h in hyp_np],
                    np.ones(1, bool), state_bf16=True, **kw)
        for name, t, want in (("p", p, pw), ("m", mb, mw), ("v", vb, vw)):
            got = _np(t[r:r + 1, t0:t0 + 4096].float())
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (r, t0, name)


def test_single_row_past_2_31_elements():
    """One replica row of 2^31 + 4099 elements (34 GB of Adam state): element
    indices inside a row pass 2^31 and the row is ragged. Windows at the
    start, across 2^31 and at the very end equal the oracle; the same step with
    the gradient as one per-parameter segment equals the dense step, bit for
    bit, over the whole row."""
    T = 2**31 + 4099
    g = torch.Generator(device="cuda").manual_seed(31)
    p = torch.randn(1, T, device="cuda", generator=g).mul_(0.02)
    gr = torch.randn(1, T, device="cuda", generator=g).mul_(1e-3)
    m = torch.randn(1, T, device="cuda", generator=g).mul_(1e-3)
    v = torch.rand(1, T, device="cuda", generator=g).mul_(1e-4)
    steps = torch.full((1,), 7.0, device="cuda")
    hyp = [torch.full((1,), x, device="cuda") for x in (1e-3, 0.9, 0.999, 1e-8, 1e-2)]
    mask = torch.ones(1, dtype=torch.bool, device="cuda")
    kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=True)
    windows = [0, 2**31 - 2048, T - 4096]
    before = [[_np(t[:, t0:t0 + 4096]) for t in (p, gr, m, v)] for t0 in windows]
    twin = [t.clone() for t in (p, m, v)]
    steps2 = steps.clone()
    torch.ops.torchstrap.adam_step_(p, gr, m, v, None, steps, *hyp, mask, **kw)
    torch.ops.churten.adam_step_segments_(twin[0], [gr], [0], None, twin[1], twin[2], None,
                                          steps2, *hyp, mask, **kw)
    torch.cuda.synchronize()
    for name, a, b in (("params", p, twin[0]), ("exp_avgs", m, twin[1]),
                       ("exp_avg_sqs", v, twin[2])):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
    del twin
    hw = [_np(h) for h in hyp]
    for t0, (pw, gw, mw, vw) in zip(windows, before):
        O.adam_step(O.DEVICE, pw, gw, mw, vw, None, np.full(1, 7.0, np.float32), *hw,
                    np.ones(1, bool), **kw)
        for name, t, want in (("p", p, pw), ("m", m, mw), ("v", v, vw)):
            got = _np(t[:, t0:t0 + 4096])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} @ {t0}"

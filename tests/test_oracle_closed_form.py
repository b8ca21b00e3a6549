"""The oracle against what the mathematics fixes, independently of any golden file.

Each check is chosen so that a plausible restatement mistake fails it: a
swapped beta1/beta2, a missing bias correction, eps inside the sqrt, a wrong
sign under maximize, weight decay applied to the wrong quantity, the step bump
after instead of before, a frozen row touched, dampening applied on a first
step, lr_decay applied with the wrong step offset.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O

F = np.float32
FORMS = [O.DEVICE, O.CPU]


def vec(R, x):
    return np.full(R, x, dtype=F)


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("maximize", [False, True])
def test_adam_first_step_is_lr_times_sign(form, maximize):
    """From zero moments the bias-corrected first step is lr * g / (|g| + eps)."""
    R, T = 2, 257
    r = rng(1)
    p = r.standard_normal((R, T)).astype(F)
    g = r.standard_normal((R, T)).astype(F)
    m = np.zeros((R, T), F)
    v = np.zeros((R, T), F)
    steps = np.zeros(R, F)
    lr, b1, b2, eps = np.array([1e-2, 3e-3], F), vec(R, 0.9), vec(R, 0.999), vec(R, 1e-8)
    p0 = p.copy()
    O.adam_step(form, p, g, m, v, None, steps, lr, b1, b2, eps, vec(R, 0.0),
                np.ones(R, bool), maximize=maximize, decoupled_weight_decay=False)
    sgn = -1.0 if maximize else 1.0
    want = p0 - sgn * lr[:, None] * g / (np.abs(g) + 1e-8)
    np.testing.assert_allclose(p, want, rtol=0, atol=3e-8)
    c1 = 1 - np.float64(F(0.9))  # the betas are float32 values
    c2 = 1 - np.float64(F(0.999))
    np.testing.assert_allclose(m, sgn * c1 * g.astype(np.float64), rtol=2e-6)
    np.testing.assert_allclose(v, c2 * g.astype(np.float64) ** 2, rtol=2e-6)
    assert steps.tolist() == [1.0, 1.0]


@pytest.mark.parametrize("form", FORMS)
def test_adam_matches_float64_textbook_over_steps(form):
    """Several steps against Adam / AdamW as published (Kingma & Ba; decoupled
    weight decay as Loshchilov & Hutter), in float64, with distinct betas."""
    R, T, K = 3, 96, 6
    r = rng(2)
    p = r.standard_normal((R, T)).astype(F)
    m = np.abs(r.standard_normal((R, T))).astype(F) * 0
    v = np.zeros((R, T), F)
    lr = np.array([1e-3, 5e-3, 2e-2], F)
    b1 = np.array([0.9, 0.8, 0.95], F)
    b2 = np.array([0.999, 0.99, 0.9999], F)
    eps = np.array([1e-8, 1e-6, 1e-7], F)
    wd = np.array([0.0, 1e-2, 5e-2], F)
    steps = np.zeros(R, F)
    P, M, V = (x.astype(np.float64) for x in (p, m, v))
    for k in range(1, K + 1):
        g = r.standard_normal((R, T)).astype(F)
        O.adam_step(form, p, g, m, v, None, steps, lr, b1, b2, eps, wd, np.ones(R, bool),
                    decoupled_weight_decay=True)
        L, B1, B2, E, W = (x.astype(np.float64)[:, None] for x in (lr, b1, b2, eps, wd))
        P = P * (1 - L * W)
        M = B1 * M + (1 - B1) * g
        V = B2 * V + (1 - B2) * g.astype(np.float64) ** 2
        mhat = M / (1 - B1**k)
        P = P - L * mhat / (np.sqrt(V) / np.sqrt(1 - B2**k) + E)
    np.testing.assert_allclose(p, P, rtol=1e-5, atol=1e-6)
    assert steps.tolist() == [K] * R


@pytest.mark.parametrize("form", FORMS)
def test_adam_l2_weight_decay_enters_the_gradient(form):
    """Non-decoupled decay: zero grad, zero moments -> update driven by wd * p."""
    R, T = 1, 64
    p = np.linspace(-1, 1, T, dtype=F)[None].copy()
    g = np.zeros((R, T), F)
    m, v = np.zeros((R, T), F), np.zeros((R, T), F)
    p0 = p.copy()
    O.adam_step(form, p, g, m, v, None, np.zeros(R, F), vec(R, 1e-2), vec(R, 0.9),
                vec(R, 0.999), vec(R, 1e-8), vec(R, 0.5), np.ones(R, bool),
                decoupled_weight_decay=False)
    gw = 0.5 * p0.astype(np.float64)
    want = p0 - 1e-2 * gw / (np.abs(gw) + 1e-8)
    np.testing.assert_allclose(p, want, atol=3e-8)


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("amsgrad", [False, True])
def test_frozen_rows_untouched_even_at_step0(form, amsgrad):
    R, T = 3, 40
    r = rng(3)
    st = [r.standard_normal((R, T)).astype(F) for _ in range(5)]
    st[0][1] = np.nan
    before = [x.copy() for x in st]
    steps = np.array([0, 0, 7], F)
    mask = np.array([True, False, False])
    O.adam_step(form, st[0], st[1], st[2], np.abs(st[3]), np.abs(st[4]), steps,
                vec(R, 1e-2), vec(R, 0.9), vec(R, 0.999), vec(R, 1e-8), vec(R, 0.0), mask,
                amsgrad=amsgrad)
    assert np.isnan(st[0][1]).all()
    np.testing.assert_array_equal(st[0][2], before[0][2])
    np.testing.assert_array_equal(st[2][1:], before[2][1:])
    assert steps.tolist() == [1.0, 0.0, 7.0]
    assert np.isfinite(st[0][0]).all()


@pytest.mark.parametrize("form", FORMS)
def test_zero_pad_lanes_stay_zero(form):
    """Zero param, zero grad, zero state is a fixed point of all three updates."""
    R, T = 2, 16
    z = lambda: np.zeros((R, T), F)  # noqa: E731
    p, m, v, mx = z(), z(), z(), z()
    O.adam_step(form, p, z(), m, v, mx, vec(R, 4), vec(R, 1e-2), vec(R, 0.9), vec(R, 0.999),
                vec(R, 1e-8), vec(R, 1e-2), np.ones(R, bool), amsgrad=True)
    assert not p.any() and not m.any() and not v.any() and not mx.any()
    p, mb = z(), z()
    O.sgd_step(form, p, z(), mb, vec(R, 3), vec(R, 1e-2), vec(R, 0.9), vec(R, 0.1),
               vec(R, 1e-2), np.ones(R, bool), nesterov=True)
    assert not p.any() and not mb.any()
    p, s = z(), z()
    O.adagrad_step(form, p, z(), s, vec(R, 3), vec(R, 1e-2), vec(R, 1e-3), vec(R, 1e-2),
                   vec(R, 1e-10), np.ones(R, bool))
    assert not p.any() and not s.any()


@pytest.mark.parametrize("form", FORMS)
def test_sgd_first_step_and_momentum_recursion(form):
    """First step: buf = g (dampening not applied); then buf = mom*buf + (1-d)*g."""
    R, T = 2, 33
    r = rng(4)
    p = r.standard_normal((R, T)).astype(F)
    mb = r.standard_normal((R, T)).astype(F)
    steps = np.zeros(R, F)
    mom, damp, lr = vec(R, 0.5), vec(R, 0.25), vec(R, 0.125)
    g1 = r.standard_normal((R, T)).astype(F)
    p0 = p.copy()
    O.sgd_step(form, p, g1, mb, steps, lr, mom, damp, vec(R, 0.0), np.ones(R, bool))
    np.testing.assert_array_equal(mb, g1)
    np.testing.assert_array_equal(p, (p0 - 0.125 * g1).astype(F))
    g2 = r.standard_normal((R, T)).astype(F)
    p1 = p.copy()
    O.sgd_step(form, p, g2, mb, steps, lr, mom, damp, vec(R, 0.0), np.ones(R, bool))
    want_buf = 0.5 * g1.astype(np.float64) + 0.75 * g2
    np.testing.assert_allclose(mb, want_buf, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(p, p1 - 0.125 * want_buf, rtol=1e-6, atol=1e-7)
    assert steps.tolist() == [2.0, 2.0]


@pytest.mark.parametrize("form", FORMS)
def test_sgd_nesterov_and_maximize(form):
    R, T = 1, 20
    r = rng(5)
    p = r.standard_normal((R, T)).astype(F)
    mb = r.standard_normal((R, T)).astype(F)
    g = r.standard_normal((R, T)).astype(F)
    steps = np.full(R, 4, F)  # not a first step
    p0, b0 = p.copy(), mb.copy()
    O.sgd_step(form, p, g, mb, steps, vec(R, 0.25), vec(R, 0.5), vec(R, 0.0), vec(R, 0.0),
               np.ones(R, bool), nesterov=True, maximize=True)
    gg = -g.astype(np.float64)
    buf = 0.5 * b0 + gg
    np.testing.assert_allclose(mb, buf, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(p, p0 - 0.25 * (gg + 0.5 * buf), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("form", FORMS)
def test_adagrad_steps_and_lr_decay(form):
    """s += g^2; p -= lr / (1 + (k-1) lr_decay) * g / (sqrt(s) + eps)."""
    R, T, K = 2, 50, 4
    r = rng(6)
    p = r.standard_normal((R, T)).astype(F)
    s = np.full((R, T), 0.1, F)
    lrd = np.array([0.0, 0.5], F)
    P, S = p.astype(np.float64), s.astype(np.float64)
    steps = np.zeros(R, F)
    for k in range(1, K + 1):
        g = r.standard_normal((R, T)).astype(F)
        O.adagrad_step(form, p, g, s, steps, vec(R, 1e-2), lrd, vec(R, 0.0), vec(R, 1e-10),
                       np.ones(R, bool))
        S = S + g.astype(np.float64) ** 2
        clr = 1e-2 / (1 + (k - 1) * lrd.astype(np.float64))[:, None]
        P = P - clr * g / (np.sqrt(S) + 1e-10)
    np.testing.assert_allclose(s, S, rtol=1e-6)
    np.testing.assert_allclose(p, P, rtol=1e-5, atol=1e-6)
    assert steps.tolist() == [K, K]


def test_device_and_cpu_forms_differ_only_by_rounding():
    """The two formulations are different roundings of one update."""
    import cases as C

    for c in C.adam_cases()[:16] + C.sgd_cases()[:8] + C.adagrad_cases()[:8]:
        a = C.run_oracle(c, O.DEVICE)
        b = C.run_oracle(c, O.CPU)
        for k in a:
            np.testing.assert_allclose(a[k], b[k], rtol=1e-5, atol=1e-5, err_msg=k)

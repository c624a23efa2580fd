"""Pins the fp64 selective-scan oracle (CPU only).

Independent checks:
  * central finite differences of the oracle's forward for every input it
    returns a gradient for (full BPTT, all controller cases, both input modes);
  * PyTorch float64 autograd of a separate time-major restatement
    (oracle/torch_ref.py), which also covers TBPTT(1), where finite
    differences do not apply;
  * closed forms: DC gain gamma/(gamma - i(1-gamma)theta) for constant input,
    impulse response, zero heads == static ZOH two-tap coefficients
    (reference tests/test_selective_rqf.py:320-337), sigmoid write gate at
    0 / +-1000 logits (:554-583), series continuity at |a| = 1e-4.
"""

import cmath
import math

import numpy as np
import pytest
import torch

from oracle import oracle, torch_ref
from tests.helpers import crandn
from tests.selective_cases import CASES, case_id, make_inputs, to_torch


def _loss(inp, z, gy, gx):
    raw, act = oracle.selective_fwd(z, inp)
    return np.real(np.vdot(gy, raw)) + np.real(np.vdot(gx, act))


def _perturbed(inp, field, idx, delta):
    arr = getattr(inp, field).copy()
    arr[idx] += delta
    d = dict(inp.__dict__)
    d[field] = arr
    return oracle.SelectiveInputs(**d)


@pytest.mark.parametrize("prospective", [False, True])
@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_gradients_match_finite_differences(case, prospective):
    rng = np.random.default_rng(abs(hash(case_id(case))) % 2**32)
    F, B, T = 4, 2, 9
    inp = make_inputs(F, B, T, case, rng, prospective=prospective)
    z, gy, gx = crandn(rng, F, B, T), crandn(rng, F, B, T), crandn(rng, F, B, T)
    dz, dzw, dg, dd, dw, dbias, dtheta = oracle.selective_bwd(z, inp, gy, gx)
    np.testing.assert_array_equal(dz, dzw)
    h = 1e-6

    def fd_scalar(field, idx):
        lp = _loss(_perturbed(inp, field, idx, h), z, gy, gx)
        lm = _loss(_perturbed(inp, field, idx, -h), z, gy, gx)
        return (lp - lm) / (2 * h)

    def close(fd, an, what):
        assert abs(fd - an) <= 2e-6 * (1 + abs(fd)), (what, fd, an)

    for f in range(F):
        close(fd_scalar("bias", f), dbias[f], ("bias", f))
        close(fd_scalar("theta", f), dtheta[f], ("theta", f))
    probe = [(0, 0, 0), (1, 1, 4), (F - 1, 0, T - 1), (2, 1, 1)]
    for idx in probe:
        for unit, comp in ((1.0, np.real), (1j, np.imag)):
            zp, zm = z.copy(), z.copy()
            zp[idx] += unit * h
            zm[idx] -= unit * h
            fd = (_loss(inp, zp, gy, gx) - _loss(inp, zm, gy, gx)) / (2 * h)
            close(fd, comp(dz[idx]), ("z", idx, unit))
        if dg is not None:
            close(fd_scalar("gamma_logits", idx), dg[idx], ("g", idx))
        if dw is not None:
            close(fd_scalar("write_logits", idx), dw[idx], ("w", idx))
    if dd is not None:
        G = inp.warp_logits.shape[0]
        for idx in [(0, 0, 0), (G - 1, 1, 5), (0, 1, T - 1)]:
            close(fd_scalar("warp_logits", idx), dd[idx], ("d", idx))


def _torch_grads(inp, z, gy, gx, truncated, lag_detached):
    """float64 autograd of the restatement; returns grads of (z, g, d, w, bias, theta)."""
    ti = to_torch(inp, dtype=torch.float64)
    leaves = [ti.gamma_logits, ti.warp_logits, ti.write_logits, ti.bias, ti.theta]
    for v in leaves:
        v.requires_grad_(True)
    zt = torch.as_tensor(z).requires_grad_(True)
    lag = zt.detach() if lag_detached else zt
    raw = torch_ref.selective_scan(zt, ti, truncated=truncated, z_lag=lag)
    act = torch_ref.split_relu(raw)
    loss = (torch.as_tensor(gy).conj() * raw).real.sum() + (torch.as_tensor(gx).conj() * act).real.sum()
    grads = torch.autograd.grad(loss, [zt, *leaves], allow_unused=True)
    return [None if g is None else g.numpy() for g in grads]


@pytest.mark.parametrize("truncated", [False, True])
@pytest.mark.parametrize("prospective", [False, True])
@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_gradients_match_torch_autograd(case, prospective, truncated):
    rng = np.random.default_rng(7 + len(case_id(case)))
    F, B, T = 5, 2, 12
    gh = prospective and case["gamma"] and not case.get("log_shift")
    inp = make_inputs(F, B, T, case, rng, prospective=prospective, gamma_horizon=gh)
    z, gy, gx = crandn(rng, F, B, T), crandn(rng, F, B, T), crandn(rng, F, B, T)
    raw, act = oracle.selective_fwd(z, inp)
    ti = to_torch(inp, dtype=torch.float64)
    raw_t = torch_ref.selective_scan(torch.as_tensor(z), ti)
    np.testing.assert_allclose(raw, raw_t.numpy(), rtol=1e-12, atol=1e-12)
    dz, dzw, dg, dd, dw, dbias, dtheta = oracle.selective_bwd(z, inp, gy, gx, truncated=truncated)
    # TBPTT(1): the lag tap's gradient reaches W (dzw) only; x sees dz.
    g_w = _torch_grads(inp, z, gy, gx, truncated, lag_detached=False)
    g_x = _torch_grads(inp, z, gy, gx, truncated, lag_detached=True) if truncated else g_w
    tol = dict(rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(dzw, g_w[0], **tol)
    np.testing.assert_allclose(dz, g_x[0], **tol)
    for got, want in ((dg, g_w[1]), (dd, g_w[2]), (dw, g_w[3])):
        if got is None:
            assert want is None or not np.any(want)
        else:
            np.testing.assert_allclose(got, want, **tol)
    np.testing.assert_allclose(dbias, g_w[4], **tol)
    np.testing.assert_allclose(dtheta, g_w[5], **tol)


def test_dc_gain_closed_form():
    """Constant drive, zero logits: y -> gamma / (gamma - i(1-gamma)theta)."""
    rng = np.random.default_rng(11)
    F, B, T = 6, 1, 4000
    case = dict(gamma=True, write=True, warp="grouped", log_shift=False, write_sigmoid=True)
    inp = make_inputs(F, B, T, case, rng, prospective=True)
    inp.theta[:] = np.linspace(0.1, 2.5, F)
    gamma = np.linspace(0.15, 0.9, F)
    inp.bias[:] = np.log((gamma - inp.minimum) / inp.span) - np.log1p(-(gamma - inp.minimum) / inp.span)
    for name in ("gamma_logits", "warp_logits", "write_logits"):
        getattr(inp, name)[:] = 0
    raw, _ = oracle.selective_fwd(np.ones((F, B, T), complex), inp)
    expect = gamma / (gamma - 1j * (1 - gamma) * inp.theta)
    np.testing.assert_allclose(raw[:, 0, -1], expect, rtol=1e-10)


def test_impulse_response_closed_form():
    """z = delta: y0 = p, y1 = A p + n, y_t = A^{t-1} (A p + n) (constant coefficients)."""
    rng = np.random.default_rng(12)
    F, B, T = 3, 1, 30
    case = dict(gamma=False, write=True, warp="none", log_shift=False, write_sigmoid=True)
    inp = make_inputs(F, B, T, case, rng, prospective=True)
    inp.write_logits[:] = 0
    z = np.zeros((F, B, T), complex)
    z[:, :, 0] = 1
    raw, _ = oracle.selective_fwd(z, inp)
    A, p, n = oracle.selective_coefficients(inp, F, B, T)
    t = np.arange(1, T)
    expect1 = (A[:, 0, 0] * p[:, 0, 0] + n[:, 0, 0])[:, None] * A[:, 0, 0][:, None] ** (t - 1)
    np.testing.assert_allclose(raw[:, 0, 0], p[:, 0, 0], rtol=1e-14)
    np.testing.assert_allclose(raw[:, 0, 1:], expect1, rtol=1e-12)


@pytest.mark.parametrize("mode", ["tau", "gamma", "horizon"])
def test_zero_heads_equal_static_two_tap(mode):
    """Zero logits reduce to the static ZOH taps (cmath restatement of filter.py:630-646)."""
    rng = np.random.default_rng(13)
    F, B, T = 5, 2, 4
    case = dict(gamma=True, write=True, warp="global", log_shift=False, write_sigmoid=True)
    inp = make_inputs(F, B, T, case, rng, prospective=True, gamma_horizon=mode == "gamma",
                      horizon=0.7 if mode == "horizon" else None)
    for name in ("gamma_logits", "warp_logits", "write_logits"):
        getattr(inp, name)[:] = 0
    A, p, n = oracle.selective_coefficients(inp, F, B, T)
    sig = 1 / (1 + np.exp(-inp.bias))
    gamma = inp.minimum + inp.span * sig
    for f in range(F):
        a = inp.step[f] * complex(-gamma[f], (1 - gamma[f]) * inp.theta[f])
        c1 = cmath.exp(a)
        ratio = 1 / gamma[f] if mode == "gamma" else inp.horizon[f]
        tap0 = gamma[f] * inp.step[f] * (cmath.exp(a) - 1) / a + gamma[f] * ratio * c1
        tap1 = -gamma[f] * ratio * c1
        np.testing.assert_allclose(A[f], c1, rtol=1e-13)
        np.testing.assert_allclose(p[f], tap0, rtol=1e-12)
        np.testing.assert_allclose(n[f], tap1, rtol=1e-13)
    c1o, t0o, t1o = oracle.zoh_two_tap(gamma, inp.theta, inp.step,
                                       1 / gamma if mode == "gamma" else inp.horizon)
    np.testing.assert_allclose(c1o, A[:, 0, 0], rtol=1e-14)
    np.testing.assert_allclose(t0o, p[:, 0, 0], rtol=1e-13)
    np.testing.assert_allclose(t1o, n[:, 0, 0], rtol=1e-14)


def test_sigmoid_write_gate_unit_gain_and_saturation():
    rng = np.random.default_rng(14)
    F, B, T = 4, 2, 20
    on = dict(gamma=True, write=True, warp="none", log_shift=False, write_sigmoid=True)
    off = dict(on, write=False)
    inp_on = make_inputs(F, B, T, on, rng, write_max=3.0)
    inp_off = oracle.SelectiveInputs(**dict(inp_on.__dict__, write_logits=np.zeros((0, B, T)),
                                            options=(True, False, False) + inp_on.options[3:8]
                                            + (False,) + inp_on.options[9:]))
    z = crandn(rng, F, B, T)
    base, _ = oracle.selective_fwd(z, inp_off)
    for logit, scale in ((0.0, 1.0), (-1000.0, 0.0), (1000.0, 3.0)):
        inp_on.write_logits[:] = logit
        raw, _ = oracle.selective_fwd(z, inp_on)
        np.testing.assert_allclose(raw, scale * base, rtol=1e-12, atol=1e-300)
    del off


def test_exprel_series_is_continuous_at_threshold():
    """phi just below / above |a| = 1e-4 agree (series vs expm1 branch)."""
    F, B, T = 2, 1, 1
    for eta in (1e-4 * (1 - 1e-9), 1e-4 * (1 + 1e-9)):
        inp = make_inputs(F, B, T, dict(gamma=False, write=True, warp="none", log_shift=False,
                                        write_sigmoid=True), np.random.default_rng(0),
                          prospective=False, eta=eta)
        inp.bias[:] = 1.0  # gamma = 1: a = -eta (real)
        inp.write_logits[:] = 0
        _, p, _ = oracle.selective_coefficients(inp, F, B, T)
        a = -eta
        np.testing.assert_allclose(p[0, 0, 0] / eta, math.expm1(a) / a, rtol=1e-13)


def test_collapsed_and_tiny_poles_stay_finite():
    rng = np.random.default_rng(15)
    F, B, T = 3, 2, 10
    case = dict(gamma=False, write=True, warp="none", log_shift=False, write_sigmoid=True)
    for eta, bias, theta in ((20000.0, 0.5, 1.0), (0.2, math.exp(-70), math.exp(-50))):
        inp = make_inputs(F, B, T, case, rng, eta=eta)
        inp.bias[:] = bias
        inp.theta[:] = theta
        z, gy, gx = crandn(rng, F, B, T), crandn(rng, F, B, T), crandn(rng, F, B, T)
        raw, act = oracle.selective_fwd(z, inp)
        out = oracle.selective_bwd(z, inp, gy, gx)
        assert np.all(np.isfinite(raw))
        for g in out:
            if g is not None:
                assert np.all(np.isfinite(g))


def test_frequency_band_clamp_and_clipped_gradients():
    """Global warp with a band bound (reference tests/test_selective_rqf.py:458-503):
    the effective frequency angle(A) / ((1 - gamma) eta) equals
    clamp(theta * exp(c tanh d), lo, hi), and a clipped step passes no gradient
    to the warp logit or to theta."""
    F, B = 1, 1
    c = math.log(4.0)
    lo, hi = 0.3, 1.2
    theta = math.sqrt(lo * hi)
    case = dict(gamma=False, write=False, warp="global", log_shift=False, write_sigmoid=True)
    for d, clipped in ((-2.0, True), (0.1, False), (2.0, True)):
        inp = make_inputs(F, B, 1, case, np.random.default_rng(0), prospective=False,
                          warp_scale=c, eta=0.2)
        inp.bias[:] = 0.2  # gamma (no gamma head: bias is gamma)
        inp.theta[:] = theta
        inp.theta_minimum[:] = lo
        inp.theta_maximum[:] = hi
        inp.warp_logits[:] = d
        A, _, _ = oracle.selective_coefficients(inp, F, B, 1)
        eff = np.angle(A[0, 0, 0]) / ((1 - 0.2) * 0.2)
        np.testing.assert_allclose(eff, min(max(theta * math.exp(c * math.tanh(d)), lo), hi),
                                   rtol=1e-13)
        z = np.array([[[1.0 + 0.5j]]])
        _, _, _, dd, _, _, dtheta = oracle.selective_bwd(z, inp, np.array([[[0.3 - 1j]]]), None)
        if clipped:
            assert dd[0, 0, 0] == 0.0 and dtheta[0] == 0.0
        else:
            assert dd[0, 0, 0] != 0.0 and dtheta[0] != 0.0


def test_log_shift_gamma_limits():
    """log_shift link: gamma = exp(bias + c tanh g) reaches exp(bias +- c) at
    saturated logits (reference tests/test_selective_rqf.py:372-397), read back
    from the pole radius |A| = exp(-gamma eta)."""
    F, B, T = 3, 1, 3
    c = math.log(1.25)
    case = dict(gamma=True, write=False, warp="none", log_shift=True, write_sigmoid=True)
    inp = make_inputs(F, B, T, case, np.random.default_rng(1), prospective=False,
                      gamma_scale=c, eta=0.3)
    inp.gamma_logits[:, :, 0] = 1000.0
    inp.gamma_logits[:, :, 1] = -1000.0
    inp.gamma_logits[:, :, 2] = 0.0
    A, _, _ = oracle.selective_coefficients(inp, F, B, T)
    gamma = -np.log(np.abs(A[:, 0, :])) / 0.3
    np.testing.assert_allclose(gamma[:, 0], np.exp(inp.bias + c), rtol=1e-12)
    np.testing.assert_allclose(gamma[:, 1], np.exp(inp.bias - c), rtol=1e-12)
    np.testing.assert_allclose(gamma[:, 2], np.exp(inp.bias), rtol=1e-12)

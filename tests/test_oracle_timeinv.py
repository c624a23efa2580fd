"""Pins the fp64 oracle of the time-invariant scans (CPU only).

Each check is independent of the oracle's own loop: closed forms, a brute
force convolution, the adjoint identity of a linear map, central finite
differences, and the fused-vs-materialised drive identity the reference's
parity tests use (tests/test_scan_backends_parity.py:74-106).
"""

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import crandn


def _coeffs(rng, F):
    mag = rng.uniform(0.8, 0.99, F)
    return mag * np.exp(1j * rng.uniform(0, 2 * np.pi, F)), 0.1 * crandn(rng, F), 0.5 * crandn(rng, F)


def test_impulse_response_closed_form():
    rng = np.random.default_rng(0)
    F, T = 5, 40
    c1, c2, _ = _coeffs(rng, F)
    u = np.zeros((1, T, F), complex)
    u[0, 0, :] = 1
    y = oracle.twotap_fwd(c1, c2, None, u)
    t = np.arange(T)[:, None]
    np.testing.assert_allclose(y[0], c2 * c1 ** t, rtol=1e-13, atol=1e-15)


def test_step_response_closed_form():
    rng = np.random.default_rng(1)
    F, T = 4, 50
    c1, c2, _ = _coeffs(rng, F)
    y = oracle.twotap_fwd(c1, c2, None, np.ones((2, T, F), complex))
    t = np.arange(T)[:, None]
    expect = c2 * (1 - c1 ** (t + 1)) / (1 - c1)
    np.testing.assert_allclose(y[1], expect, rtol=1e-12)


@pytest.mark.parametrize("layout", [oracle.BTF, oracle.FBT])
def test_two_tap_equals_brute_force_convolution(layout):
    rng = np.random.default_rng(2)
    B, T, F = 3, 33, 6
    c1, k0, k1 = _coeffs(rng, F)
    x_btf = crandn(rng, B, T, F)
    x = x_btf if layout == oracle.BTF else x_btf.transpose(2, 0, 1).copy()
    y = oracle.twotap_fwd(c1, k0, k1, x, layout=layout)
    y_btf = y if layout == oracle.BTF else y.transpose(1, 2, 0)
    xprev = np.concatenate([np.zeros((B, 1, F)), x_btf[:, :-1]], axis=1)
    drive = k0 * x_btf + k1 * xprev
    t = np.arange(T)
    kernel = c1[None, None, :] ** (t[:, None, None] - t[None, :, None])  # (t, s, F)
    causal = (t[:, None] >= t[None, :])[:, :, None]
    expect = np.einsum("tsf,bsf->btf", np.where(causal, kernel, 0), drive)
    np.testing.assert_allclose(y_btf, expect, rtol=1e-12, atol=1e-12)


def test_fused_two_tap_equals_materialised_drive():
    rng = np.random.default_rng(3)
    B, T, F = 2, 70, 5
    c1, k0, k1 = _coeffs(rng, F)
    x = crandn(rng, B, T, F)
    drive = k0 * x
    drive[:, 1:] += k1 * x[:, :-1]
    np.testing.assert_allclose(oracle.twotap_fwd(c1, k0, k1, x),
                               oracle.twotap_fwd(c1, np.ones(F), None, drive), rtol=1e-13)


@pytest.mark.parametrize("layout", [oracle.BTF, oracle.FBT])
def test_adjoint_dot_product_identity(layout):
    """Re<gy, J v> == Re<J^H gy, v> for the linear map x -> y."""
    rng = np.random.default_rng(4)
    B, T, F = 2, 45, 3
    c1, k0, k1 = _coeffs(rng, F)
    shape = (B, T, F) if layout == oracle.BTF else (F, B, T)
    v, gy = crandn(rng, *shape), crandn(rng, *shape)
    y = oracle.twotap_fwd(c1, k0, k1, v, layout=layout)
    gx, *_ = oracle.twotap_bwd(c1, k0, k1, v, y, gy, layout=layout)
    lhs = np.real(np.vdot(gy, y))
    rhs = np.real(np.vdot(gx, v))
    assert abs(lhs - rhs) <= 1e-11 * abs(lhs)


@pytest.mark.parametrize("mask_act", [False, True])
def test_coefficient_gradients_by_finite_differences(mask_act):
    rng = np.random.default_rng(5)
    B, T, F = 2, 21, 3
    c1, k0, k1 = _coeffs(rng, F)
    x, gy = crandn(rng, F, B, T), crandn(rng, F, B, T)

    def loss(c1_, k0_, k1_, x_):
        y, a = oracle.twotap_fwd(c1_, k0_, k1_, x_, layout=oracle.FBT, act=True)
        return np.real(np.vdot(gy, a if mask_act else y))

    y = oracle.twotap_fwd(c1, k0, k1, x, layout=oracle.FBT)
    gx, gc1, gk0, gk1 = oracle.twotap_bwd(c1, k0, k1, x, y, gy, layout=oracle.FBT,
                                          mask_act=mask_act)
    h = 1e-6
    for name, arr, grad in (("c1", c1, gc1), ("k0", k0, gk0), ("k1", k1, gk1)):
        for f in range(F):
            for unit, comp in ((1.0, np.real), (1j, np.imag)):
                args = {"c1": c1, "k0": k0, "k1": k1}
                plus = {k: v.copy() for k, v in args.items()}
                minus = {k: v.copy() for k, v in args.items()}
                plus[name][f] += unit * h
                minus[name][f] -= unit * h
                fd = (loss(plus["c1"], plus["k0"], plus["k1"], x)
                      - loss(minus["c1"], minus["k0"], minus["k1"], x)) / (2 * h)
                assert abs(fd - comp(grad[f])) <= 1e-6 * (1 + abs(fd)), (name, f, unit)
    for idx in [(0, 0, 0), (1, 1, 7), (2, 0, T - 1)]:
        for unit, comp in ((1.0, np.real), (1j, np.imag)):
            xp, xm = x.copy(), x.copy()
            xp[idx] += unit * h
            xm[idx] -= unit * h
            fd = (loss(c1, k0, k1, xp) - loss(c1, k0, k1, xm)) / (2 * h)
            assert abs(fd - comp(gx[idx])) <= 1e-6 * (1 + abs(fd)), idx


def test_layouts_agree():
    rng = np.random.default_rng(6)
    B, T, F = 3, 17, 4
    c1, k0, k1 = _coeffs(rng, F)
    x = crandn(rng, B, T, F)
    gy = crandn(rng, B, T, F)
    y = oracle.twotap_fwd(c1, k0, k1, x)
    yf = oracle.twotap_fwd(c1, k0, k1, x.transpose(2, 0, 1).copy(), layout=oracle.FBT)
    np.testing.assert_allclose(yf.transpose(1, 2, 0), y, rtol=1e-14)
    g1 = oracle.twotap_bwd(c1, k0, k1, x, y, gy)
    g2 = oracle.twotap_bwd(c1, k0, k1, x.transpose(2, 0, 1).copy(), yf,
                           gy.transpose(2, 0, 1).copy(), layout=oracle.FBT)
    np.testing.assert_allclose(g2[0].transpose(1, 2, 0), g1[0], rtol=1e-13)
    for a, b in zip(g1[1:], g2[1:]):
        np.testing.assert_allclose(a, b, rtol=1e-12)


def test_empty_and_single_step():
    c1, k0 = np.array([0.5 + 0.1j]), np.array([2.0 + 0j])
    assert oracle.twotap_fwd(c1, k0, None, np.zeros((0, 5, 1), complex)).shape == (0, 5, 1)
    y = oracle.twotap_fwd(c1, k0, None, np.full((1, 1, 1), 3 + 1j))
    np.testing.assert_allclose(y.ravel(), [6 + 2j])

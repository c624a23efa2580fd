"""Pins the fp64 multi-oscillator oracle (oracle/rqf_oracle.c: orc_mosc_*).

The reference defines the fused multi-oscillator scan as the same result as
its unfused path: expand the input over the oscillators, run one complex scan
per oscillator, and sum the oscillators with their C-weights
(rqf_models/backbones/rqf/block.py:599-630 `_c_weighted_sum`,
:766-785 `_scan_standard_fallback`).  The single-oscillator scan oracle is
pinned by tests/test_oracle_timeinv.py, so composing it pins the fused one;
the gradients are checked against the composition's adjoint and against
central finite differences in the conjugate-Wirtinger convention
(grad = dL/dRe + i dL/dIm) that the reference's kernels produce.
"""

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import crandn


def _problem(rng, B, T, F, N):
    c1 = rng.uniform(0.7, 0.99, F * N) * np.exp(1j * rng.uniform(0, 2 * np.pi, F * N))
    c2 = 0.5 * crandn(rng, F * N)
    cw = crandn(rng, F * N)
    u = crandn(rng, B, T, F)
    return c1, c2, cw, u


def _composed(c1, c2, cw, u, N):
    B, T, F = u.shape
    xs = oracle.twotap_fwd(c1, c2, None, np.repeat(u, N, axis=2))  # (B,T,F*N)
    return (xs.reshape(B, T, F, N) * cw.reshape(F, N)).sum(-1), xs


@pytest.mark.parametrize("B,T,F,N", [(2, 37, 3, 1), (2, 37, 3, 2), (1, 50, 4, 3), (3, 9, 2, 8)])
def test_forward_is_expand_scan_weighted_sum(B, T, F, N):
    rng = np.random.default_rng(B * 100 + T + N)
    c1, c2, cw, u = _problem(rng, B, T, F, N)
    y, yabs = oracle.mosc_fwd(c1, c2, cw, u, N)
    want, _ = _composed(c1, c2, cw, u, N)
    assert np.max(np.abs(y - want)) <= 1e-12 * np.max(np.abs(want))
    assert np.max(np.abs(yabs - np.abs(want))) <= 1e-12 * np.max(np.abs(want))


def test_no_weights_single_oscillator_is_the_plain_scan():
    rng = np.random.default_rng(3)
    c1, c2, _, u = _problem(rng, 2, 40, 5, 1)
    y, yabs = oracle.mosc_fwd(c1, c2, None, u, 1)
    want = oracle.twotap_fwd(c1, c2, None, u)
    assert np.max(np.abs(y - want)) <= 1e-13 * np.max(np.abs(want))
    assert np.max(np.abs(yabs - np.abs(want))) <= 1e-13 * np.max(np.abs(want))


@pytest.mark.parametrize("N", [1, 2, 4])
def test_backward_is_the_composed_adjoint(N):
    rng = np.random.default_rng(10 + N)
    B, T, F = 2, 33, 3
    c1, c2, cw, u = _problem(rng, B, T, F, N)
    gy = crandn(rng, B, T, F)
    gu, gc1, gc2, gcw = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    _, xs = _composed(c1, c2, cw, u, N)
    # cotangent on oscillator n's state: conj(cw_n) gy
    gx_osc = np.repeat(gy, N, axis=2) * np.conj(np.tile(cw, 1))[None, None, :]
    gxe, gc1_w, gc2_w, _ = oracle.twotap_bwd(c1, c2, None, np.repeat(u, N, axis=2), xs, gx_osc)
    gu_w = gxe.reshape(B, T, F, N).sum(-1)
    gcw_w = (np.repeat(gy, N, axis=2) * np.conj(xs)).sum((0, 1))
    for got, want in ((gu, gu_w), (gc1, gc1_w), (gc2, gc2_w), (gcw, gcw_w)):
        assert np.max(np.abs(got - want)) <= 1e-11 * np.max(np.abs(want))


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(7)
    B, T, F, N = 1, 12, 2, 3
    c1, c2, cw, u = _problem(rng, B, T, F, N)
    G = crandn(rng, B, T, F)

    def loss(c1_, c2_, cw_, u_):
        y, _ = oracle.mosc_fwd(c1_, c2_, cw_, u_, N)
        return float(np.real(np.sum(np.conj(G) * y)))

    gu, gc1, gc2, gcw = oracle.mosc_bwd(c1, c2, cw, u, G, N)
    h = 1e-6

    def fd(arr, idx, which):
        def bump(delta):
            a = arr.copy()
            a[idx] += delta
            args = {"c1": c1, "c2": c2, "cw": cw, "u": u}
            args[which] = a
            return loss(args["c1"], args["c2"], args["cw"], args["u"])
        dr = (bump(h) - bump(-h)) / (2 * h)
        di = (bump(1j * h) - bump(-1j * h)) / (2 * h)
        return dr + 1j * di

    for which, arr, grad in (("c1", c1, gc1), ("c2", c2, gc2), ("cw", cw, gcw)):
        for idx in range(F * N):
            assert abs(fd(arr, idx, which) - grad[idx]) <= 1e-6 * (1 + abs(grad[idx])), (which, idx)
    for idx in [(0, 0, 0), (0, 5, 1), (0, T - 1, 0)]:
        assert abs(fd(u, idx, "u") - gu[idx]) <= 1e-6 * (1 + abs(gu[idx])), idx

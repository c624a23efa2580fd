"""The exchanged-order coefficient sums the (B,T,F) and multi-oscillator
backward kernels evaluate, checked on the CPU against the oracle's reference
form.

The reference pairs the adjoint at step t with the state at t-1
(chunked_scan_kernel.py:286-299 and :491-503; triton_scan_kernel.py:2370-2404).
The kernels instead sum against the input, with the adjoint's C1 tangent
``h[r] = conj(C1) h[r+1] + g[r+1]`` for grad_C1 (csrc/timeinv.hip
``btf_bwd_final_kernel``, csrc/multiosc.hip ``mosc_bwd_final_kernel``).  Here
that scheme is restated in numpy fp64, segmented the way the kernels run it:

* a local pass per segment from a zero pair;
* the fold of the later segments' pairs with ``(P g, P h + len P' g)``;
* a final pass per segment.

It is compared with the oracle, whose sums follow the reference's pairing.
Segment lengths cover 1 step, ragged last segments and one segment.  A wrong
carry term, a transposed conjugate or an off-by-one in the tangent changes
the result at the 1e-1 level.
"""

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import crandn


def _segments(T, L):
    return [(s, min(T, s + L)) for s in range(0, T, L)]


def _adjoint_pairs(ac, g_in, L, tangent_carry=True):
    """Per segment, the (g, h) pair entering from its end: local passes from a
    zero pair, then the fold over the later segments (full segments only
    carry).  ``tangent_carry=False`` drops the fold's len * P' * g term."""
    T = g_in.shape[1]
    segs = _segments(T, L)
    starts = []
    for tb, te in segs:
        g = np.zeros(g_in[:, 0].shape, complex)
        h = np.zeros_like(g)
        for t in range(te - 1, tb - 1, -1):
            h = ac * h + g
            g = ac * g + g_in[:, t]
        starts.append((g, h))
    P, Pm = ac ** L, ac ** (L - 1)
    entering = [None] * len(segs)
    E = np.zeros_like(starts[0][0])
    H = np.zeros_like(E)
    for s in range(len(segs) - 1, -1, -1):
        entering[s] = (E, H)
        E, H = P * E + starts[s][0], P * H + tangent_carry * L * Pm * E + starts[s][1]
    return segs, entering


def twotap_grads_exchanged(c1, k0, k1, x, gy, L, tangent_carry=True):
    """(gx, gc1, gk0, gk1) of the (B,T,F) two-tap scan, the kernels' way: no
    forward state is read."""
    ac = np.conj(c1)
    k1v = np.zeros_like(c1) if k1 is None else k1
    segs, entering = _adjoint_pairs(ac, gy, L, tangent_carry)
    gx = np.zeros_like(x)
    s1 = np.zeros(c1.shape, complex)
    s0 = np.zeros_like(s1)
    s2 = np.zeros_like(s1)
    for (tb, te), (g, h) in zip(segs, entering):
        for t in range(te - 1, tb - 1, -1):
            xp = x[:, t - 1] if t > 0 else np.zeros_like(x[:, 0])
            h_new = ac * h + g
            g_new = ac * g + gy[:, t]
            gx[:, t] = np.conj(k0) * g_new + np.conj(k1v) * g
            d = k0 * x[:, t] + k1v * xp
            s1 += (np.conj(d) * h_new).sum(0)
            s0 += (np.conj(x[:, t]) * g_new).sum(0)
            s2 += (np.conj(xp) * g_new).sum(0)
            g, h = g_new, h_new
    return gx, s1, s0, (None if k1 is None else s2)


def mosc_grads_exchanged(c1, c2, cw, u, gy, N, L):
    """(gu, gc1, gc2, gcw) of the multi-oscillator scan, the kernels' way."""
    B, T, F = u.shape
    a = c1.reshape(F, N)
    w = cw.reshape(F, N)
    g2 = c2.reshape(F, N)
    gy_n = np.repeat(gy[..., None], N, axis=-1)  # (B, T, F, N)
    segs, entering = _adjoint_pairs(np.conj(a), gy_n, L)
    gu = np.zeros(u.shape, complex)
    q = np.zeros((F, N), complex)
    r = np.zeros_like(q)
    hw = np.conj(w * g2)
    for (tb, te), (e, f) in zip(segs, entering):
        for t in range(te - 1, tb - 1, -1):
            f = np.conj(a) * f + e
            e = np.conj(a) * e + gy_n[:, t]
            gu[:, t] = (hw * e).sum(-1)
            q += (np.conj(u[:, t, :, None]) * e).sum(0)
            r += (np.conj(u[:, t, :, None]) * f).sum(0)
    gc1 = (np.conj(w * g2) * r).ravel()
    return gu, gc1, (np.conj(w) * q).ravel(), (np.conj(g2) * q).ravel()


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


def _coefs(rng, n):
    c1 = rng.uniform(0.6, 0.99, n) * np.exp(1j * rng.uniform(-np.pi, np.pi, n))
    return c1, crandn(rng, n), crandn(rng, n)


@pytest.mark.parametrize("prospective", [False, True])
@pytest.mark.parametrize("T,L", [(37, 1), (37, 5), (37, 37), (64, 16), (50, 64)])
def test_twotap_exchanged_sums_match_the_reference_form(prospective, T, L):
    rng = np.random.default_rng(T * 100 + L + prospective)
    B, F = 2, 3
    c1, k0, k1 = _coefs(rng, F)
    if not prospective:
        k1 = None
    x = crandn(rng, B, T, F)
    gy = crandn(rng, B, T, F)
    y = oracle.twotap_fwd(c1, k0, k1, x)
    want = oracle.twotap_bwd(c1, k0, k1, x, y, gy)
    got = twotap_grads_exchanged(c1, k0, k1, x, gy, L)
    for name, gv, wv in zip(("gx", "gc1", "gk0", "gk1"), got, want):
        if wv is None:
            assert gv is None
            continue
        assert _rel(gv, wv) < 1e-12, name


@pytest.mark.parametrize("N", [1, 3, 4])
@pytest.mark.parametrize("T,L", [(29, 1), (29, 4), (29, 29), (40, 16)])
def test_multi_osc_exchanged_sums_match_the_reference_form(N, T, L):
    rng = np.random.default_rng(T * 10 + L + N)
    B, F = 2, 3
    c1, c2, cw = _coefs(rng, F * N)
    u = crandn(rng, B, T, F)
    gy = crandn(rng, B, T, F)
    want = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    got = mosc_grads_exchanged(c1, c2, cw, u, gy, N, L)
    for name, gv, wv in zip(("gu", "gc1", "gc2", "gcw"), got, want):
        assert _rel(gv, wv) < 1e-12, name


def test_a_dropped_carry_term_is_caught():
    """The fold's len * P' * g term is what carries the tangent across
    segments: without it grad_C1 is wrong at the 1e-1 level."""
    rng = np.random.default_rng(7)
    B, T, F = 2, 40, 3
    c1, k0, k1 = _coefs(rng, F)
    x, gy = crandn(rng, B, T, F), crandn(rng, B, T, F)
    want = oracle.twotap_bwd(c1, k0, k1, x, oracle.twotap_fwd(c1, k0, k1, x), gy)[1]
    assert _rel(twotap_grads_exchanged(c1, k0, k1, x, gy, 8)[1], want) < 1e-12
    got = twotap_grads_exchanged(c1, k0, k1, x, gy, 8, tangent_carry=False)[1]
    assert _rel(got, want) > 1e-2

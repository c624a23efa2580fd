"""Pins the fp64 selective oracle against vectors written by the reference's own code.

tests/golden/selective_golden.npz holds, for every controller case x
{plain, prospective} x {full BPTT, TBPTT(1)}, the inputs, the coefficients
(A, gated p, gated n), the outputs (raw, act) and the autograd gradients of
the reference's `selective_coefficients` / `reference_layer_scan`
(rqf_models/ops/selective_scan.py:26-104), computed in float64 by
tests/golden/make_selective_golden.py.  The oracle must reproduce them to
near machine precision; the drive GEMM and its gradients are formed here the
way `_SelectiveLayerScan` does (selective_scan.py:108-160).
"""

import os

import numpy as np
import pytest

from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "selective_golden.npz")
RTOL = 1e-10


def _load():
    with np.load(GOLDEN, allow_pickle=False) as f:
        data = {k: f[k] for k in f.files}
    return data


DATA = _load()
CASES = [str(c) for c in DATA["cases"]]


def _rel(got, want):
    got, want = np.asarray(got), np.asarray(want)
    scale = max(np.max(np.abs(want)), 1e-300)
    return float(np.max(np.abs(got - want)) / scale) if want.size else 0.0


def _inputs(key):
    g = lambda name: DATA[f"{key}/{name}"]  # noqa: E731
    o = g("options")
    options = (bool(o[0]), bool(o[1]), bool(o[2]), bool(o[3]), float(o[4]), float(o[5]),
               bool(o[6]), bool(o[7]), bool(o[8]), float(o[9]), float(o[10]), bool(o[11]))
    groups = g("groups")
    return oracle.SelectiveInputs(
        gamma_logits=g("gamma_logits"), warp_logits=g("warp_logits"),
        write_logits=g("write_logits"), bias=g("bias"), theta=g("theta"),
        groups=groups if groups.size else None, minimum=g("minimum"), span=g("span"),
        step=g("step"), horizon=g("horizon"), theta_minimum=g("theta_minimum"),
        theta_maximum=g("theta_maximum"), options=options,
    )


def test_fixture_covers_the_option_matrix():
    assert len(CASES) == 76
    assert {c.split("|")[1] for c in CASES} == {"p0", "p1"}
    assert {c.split("|")[2] for c in CASES} == {"t0", "t1"}


@pytest.mark.parametrize("key", CASES)
def test_oracle_reproduces_reference_vectors(key):
    I, F, B, T, G = (int(v) for v in DATA["shape"])
    g = lambda name: DATA[f"{key}/{name}"]  # noqa: E731
    inp = _inputs(key)
    truncated = key.endswith("t1")
    x, W = g("x"), g("W")
    z = (W @ x.reshape(I, B * T)).reshape(F, B, T)

    A, p, n = oracle.selective_coefficients(inp, F, B, T)
    raw, act = oracle.selective_fwd(z, inp)
    dz, dzw, dg, dd, dw, dbias, dtheta = oracle.selective_bwd(
        z, inp, g("cot_raw"), g("cot_act"), truncated=truncated)
    dx = (W.conj().T @ dz.reshape(F, B * T)).reshape(I, B, T)
    dW = dzw.reshape(F, B * T) @ x.reshape(I, B * T).conj().T

    errs = {
        "A": _rel(A, g("A")), "p": _rel(p, g("p")), "n": _rel(n, g("n")),
        "raw": _rel(raw, g("raw")), "act": _rel(act, g("act")),
        "dx": _rel(dx, g("dx")), "dW": _rel(dW, g("dW")),
        "dbias": _rel(dbias, g("dbias")), "dtheta": _rel(dtheta, g("dtheta")),
    }
    for name, got in (("dgamma_logits", dg), ("dwarp_logits", dd), ("dwrite_logits", dw)):
        want = g(name)
        if got is None:
            assert want.size == 0 or not np.any(want), name
        else:
            errs[name] = _rel(got, want)
    bad = {k: v for k, v in errs.items() if not v <= RTOL}
    assert not bad, bad

"""Selective-scan option matrix and seeded inputs shared by CPU and GPU tests.

The option matrix follows the reference's CONTROLLER_CASES
(tests/test_selective_rqf.py:35-59): every combination of gamma / write /
warp heads with both gamma links, plus the affine write link.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import torch

from oracle import oracle


def controller_cases():
    cases = []
    for gamma, write, warp in itertools.product((False, True), (False, True),
                                                ("none", "global", "grouped")):
        if not gamma and not write and warp == "none":
            continue
        links = ("sigmoid", "log_shift") if gamma else ("sigmoid",)
        for link in links:
            cases.append(dict(gamma=gamma, write=write, warp=warp, log_shift=link == "log_shift",
                              write_sigmoid=True))
    cases.append(dict(gamma=False, write=True, warp="none", log_shift=False, write_sigmoid=False))
    cases.append(dict(gamma=True, write=True, warp="global", log_shift=False, write_sigmoid=False))
    return cases


CASES = controller_cases()


def case_id(c):
    return "g{}{}-w{}{}-{}".format(
        int(c["gamma"]), "L" if c.get("log_shift") else "S", int(c["write"]),
        "S" if c.get("write_sigmoid", True) else "A", c["warp"])


def make_inputs(F, B, T, case, rng, *, prospective=True, gamma_horizon=False, G=3,
                logit_scale=1.0, warp_scale=math.log(1.25), gamma_scale=math.log(1.25),
                write_max=2.0, eta=0.2, horizon=None, bound_warp=True):
    """numpy fp64 SelectiveInputs (oracle mirror of SelectiveScanInputs)."""
    n_warp = {"none": 0, "global": 1, "grouped": min(G, F)}[case["warp"]]
    theta = np.exp(rng.uniform(np.log(0.02), np.log(3.0), F))
    gamma = np.clip(theta / (1 + theta), 0.02, 0.98)
    lo = np.full(F, 1e-3)
    span = np.full(F, 1 - 2e-3)
    if case["gamma"] and case.get("log_shift"):
        bias = np.log(gamma) - gamma_scale
    elif case["gamma"]:
        bias = np.log((gamma - lo) / span) - np.log1p(-(gamma - lo) / span)
    else:
        bias = gamma
    hor = np.ones(F) if horizon is None else np.full(F, float(horizon))
    ranks = np.argsort(np.argsort(theta, kind="stable"), kind="stable")
    groups = (ranks * n_warp // F).astype(np.int64) if n_warp else None

    def logits(rows):
        return logit_scale * rng.standard_normal((rows, B, T))

    wsig = bool(case["write"] and case.get("write_sigmoid", True))
    options = (
        bool(case["gamma"]), n_warp > 0, bool(case["write"]), bool(case.get("log_shift", False)),
        float(gamma_scale), float(warp_scale), bool(prospective), bool(gamma_horizon), wsig,
        float(write_max), -math.log(write_max - 1), bool(n_warp > 0 and bound_warp),
    )
    return oracle.SelectiveInputs(
        gamma_logits=logits(F) if case["gamma"] else np.zeros((0, B, T)),
        warp_logits=logits(n_warp) if n_warp else np.zeros((0, B, T)),
        write_logits=(0.5 * logits(F) if not wsig else logits(F)) if case["write"]
        else np.zeros((0, B, T)),
        bias=bias, theta=theta, groups=groups, minimum=lo, span=span,
        step=np.full(F, float(eta)), horizon=hor,
        theta_minimum=np.full(F, 0.015), theta_maximum=np.full(F, 2 * math.pi),
        options=options,
    )


def to_torch(inp, device="cpu", dtype=torch.float32):
    """torch SelectiveScanInputs-like tuple (fields as the reference)."""
    from prospective_rqf_amd.selective_scan import SelectiveScanInputs

    def t(a):
        return torch.as_tensor(np.ascontiguousarray(a), dtype=dtype, device=device)

    return SelectiveScanInputs(
        t(inp.gamma_logits), t(inp.warp_logits), t(inp.write_logits), t(inp.bias), t(inp.theta),
        None if inp.groups is None else torch.as_tensor(inp.groups, dtype=torch.int64,
                                                        device=device),
        t(inp.minimum), t(inp.span), t(inp.step), t(inp.horizon), t(inp.theta_minimum),
        t(inp.theta_maximum), inp.options,
    )


def rounded_to_f32(inp):
    """The same inputs with every float rounded to fp32 (what the GPU sees)."""
    def r(a):
        return np.asarray(a, dtype=np.float32).astype(np.float64)

    return oracle.SelectiveInputs(
        r(inp.gamma_logits), r(inp.warp_logits), r(inp.write_logits), r(inp.bias), r(inp.theta),
        inp.groups, r(inp.minimum), r(inp.span), r(inp.step), r(inp.horizon),
        r(inp.theta_minimum), r(inp.theta_maximum),
        tuple(float(np.float32(v)) if isinstance(v, float) else v for v in inp.options),
    )


def from_torch(inp):
    """oracle.SelectiveInputs (fp64 numpy) holding exactly the fp32 values of a
    torch ``SelectiveScanInputs`` (e.g. one built by ``workloads.selective_inputs``)."""

    def npy(v):
        return v.detach().cpu().to(torch.float64).numpy()

    _, B, T = inp.gamma_logits.shape if inp.options[0] else inp.write_logits.shape

    def logits(v, on):
        return npy(v) if on and v is not None and v.numel() else np.zeros((0, B, T))

    return oracle.SelectiveInputs(
        logits(inp.gamma_logits, inp.options[0]), logits(inp.warp_logits, inp.options[1]),
        logits(inp.write_logits, inp.options[2]), npy(inp.bias), npy(inp.theta),
        None if inp.groups is None else inp.groups.detach().cpu().numpy().astype(np.int64),
        npy(inp.minimum), npy(inp.span), npy(inp.step), npy(inp.horizon),
        npy(inp.theta_minimum), npy(inp.theta_maximum),
        tuple(float(np.float32(v)) if isinstance(v, float) else v for v in inp.options),
    )

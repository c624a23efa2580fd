"""Writes tests/golden/selective_golden.npz from the reference's own code.

Run in the build container only (it imports the reference from
/root/reference, which exists nowhere else):

    python tests/golden/make_selective_golden.py

What it pins: the reference's selective coefficient map and serial layer scan
(rqf_models/ops/selective_scan.py:26-104, `selective_coefficients` and
`reference_layer_scan`), in float64, for every controller case of
tests/selective_cases.py x {plain, prospective} x {full BPTT, TBPTT(1)}:
  * inputs: logits, per-channel parameters, warp groups, options, x, W and
    the cotangents on raw and act;
  * outputs: A, gated p, gated n, raw, act;
  * gradients of L = Re<cot_raw, raw> + Re<cot_act, act> with respect to x, W,
    the three logit tensors, bias and theta (PyTorch autograd, conjugate
    Wirtinger convention).
The file holds data only (numpy arrays, no pickled objects).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REFERENCE = "/root/reference"

SHAPE = dict(I=2, F=4, B=2, T=12, G=2)
SEED = 1234


def main():
    sys.path.insert(0, ROOT)
    sys.path.insert(0, REFERENCE)
    from rqf_models.ops.selective_scan import (  # noqa: E402  (reference code)
        SelectiveScanInputs,
        reference_layer_scan,
        selective_coefficients,
    )

    from tests.selective_cases import CASES, case_id, make_inputs  # noqa: E402

    I, F, B, T, G = (SHAPE[k] for k in "IFBTG")
    out = {"shape": np.array([I, F, B, T, G], np.int64)}
    rng = np.random.default_rng(SEED)
    names = []
    for case in CASES:
        for prospective in (False, True):
            for truncated in (False, True):
                key = f"{case_id(case)}|p{int(prospective)}|t{int(truncated)}"
                names.append(key)
                inp = make_inputs(F, B, T, case, rng, prospective=prospective, G=G)
                x = rng.standard_normal((I, B, T)) + 1j * rng.standard_normal((I, B, T))
                W = 0.5 * (rng.standard_normal((F, I)) + 1j * rng.standard_normal((F, I)))
                cot_raw = rng.standard_normal((F, B, T)) + 1j * rng.standard_normal((F, B, T))
                cot_act = rng.standard_normal((F, B, T)) + 1j * rng.standard_normal((F, B, T))

                t64 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.float64)  # noqa: E731
                leaves = [t64(inp.gamma_logits), t64(inp.warp_logits), t64(inp.write_logits),
                          t64(inp.bias), t64(inp.theta)]
                for v in leaves:
                    v.requires_grad_(True)
                groups = None if inp.groups is None else torch.as_tensor(inp.groups)
                sin = SelectiveScanInputs(
                    leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], groups,
                    t64(inp.minimum), t64(inp.span), t64(inp.step), t64(inp.horizon),
                    t64(inp.theta_minimum), t64(inp.theta_maximum), tuple(inp.options))
                xt = torch.as_tensor(x).requires_grad_(True)
                Wt = torch.as_tensor(W).requires_grad_(True)
                raw, act = reference_layer_scan(xt, Wt, sin, truncated=truncated, activate=True,
                                                write_raw=True)
                loss = ((torch.as_tensor(cot_raw).conj() * raw).real.sum()
                        + (torch.as_tensor(cot_act).conj() * act).real.sum())
                grads = torch.autograd.grad(loss, [xt, Wt, *leaves], allow_unused=True)
                with torch.no_grad():
                    A, p, n = selective_coefficients(sin)

                rec = {
                    "gamma_logits": inp.gamma_logits, "warp_logits": inp.warp_logits,
                    "write_logits": inp.write_logits, "bias": inp.bias, "theta": inp.theta,
                    "groups": np.zeros(0, np.int64) if inp.groups is None else inp.groups,
                    "minimum": inp.minimum, "span": inp.span, "step": inp.step,
                    "horizon": inp.horizon, "theta_minimum": inp.theta_minimum,
                    "theta_maximum": inp.theta_maximum,
                    "options": np.array([float(o) for o in inp.options], np.float64),
                    "x": x, "W": W, "cot_raw": cot_raw, "cot_act": cot_act,
                    "A": A.numpy(), "p": p.numpy(), "n": n.numpy(),
                    "raw": raw.detach().numpy(), "act": act.detach().numpy(),
                }
                gnames = ("dx", "dW", "dgamma_logits", "dwarp_logits", "dwrite_logits", "dbias",
                          "dtheta")
                shapes = (x.shape, W.shape, inp.gamma_logits.shape, inp.warp_logits.shape,
                          inp.write_logits.shape, inp.bias.shape, inp.theta.shape)
                for gname, g, shp in zip(gnames, grads, shapes):
                    rec[gname] = np.zeros(shp) if g is None else g.detach().numpy()
                for k, v in rec.items():
                    out[f"{key}/{k}"] = np.asarray(v)
    out["cases"] = np.array(names)
    path = os.path.join(HERE, "selective_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(names)} cases, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()

"""Writes tests/golden/controller_golden.npz from the reference's own controller.

Run in the build container only (it imports the reference from
/root/reference, which exists nowhere else):

    python tests/golden/make_controller_golden.py

What it pins: ``SelectiveController`` construction and ``forward``
(rqf_models/backbones/rqf/selective.py:100-278) on the reference's own
``RQF`` filter module (rqf_models/backbones/rqf/filter.py), i.e. how the
selector heads and the filter's log-space parameters become the
``SelectiveScanInputs`` the selective kernels consume:
  * the bias logit under the interior and straight-through clamps and the
    log-shift link, the modulus gamma features;
  * the parameter projection construction triggers (interior margin, log
    headroom, Nyquist-bounded frequency band, optional stability band);
  * the warp-group ranks, the horizon broadcast (None / scalar / per-filter
    prospective_tau), the theta band and the 12-entry options tuple;
  * float32 and float64 filters (the controller's compute dtype).
Per case it stores the filter state before construction, the heads, the
source and the call arguments (inputs), and the filter state after
construction and every field of the returned inputs (outputs).  It also
stores the error messages of invalid settings.  Data only: numpy arrays and
JSON text, no pickled objects.
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = "/root/reference"
OUT = os.path.join(HERE, "controller_golden.npz")

N_IN, B, T = 3, 2, 5
SAMP = 16000.0

# Filter modules: (name, F, float64, constructor kwargs).  The "wide" band
# reaches past Nyquist (pi*tau/dt) so the band projection moves log_theta.
FILTERS = [
    ("recipe", 8, False, dict(tau=5.0 / SAMP, dt=1.0 / SAMP, seq_duration=1.0)),
    ("band", 6, False, dict(tau=1e-3, dt=1.0 / SAMP, min_gamma=0.05, max_gamma=0.5,
                            min_freq=10.0, max_freq=12000.0)),
    ("band64", 6, True, dict(tau=1e-3, dt=1.0 / SAMP, min_gamma=0.05, max_gamma=0.5,
                             min_freq=10.0, max_freq=12000.0)),
    ("stable", 5, False, dict(tau=2e-3, dt=1.0 / SAMP, min_gamma=0.01, max_gamma=0.9,
                              min_freq=20.0, max_freq=2000.0, clamp_gamma=True)),
]

CONFIGS = [
    dict(),
    dict(gamma_edge="st_clamp", write_control=True, write_link="affine",
         frequency_warp="global", warp_bound="none"),
    dict(write_control=True, frequency_warp="grouped", num_groups=4),
    dict(gamma_link="log_shift", gamma_features="modulus", frequency_warp="grouped",
         num_groups=2, write_control=True, write_max=3.0),
    dict(gamma_control=False, write_control=True, frequency_warp="grouped", num_groups=3),
    dict(gamma_edge_margin=0.05, frequency_warp="grouped", num_groups=5, write_control=True,
         write_link="affine", max_log_scale=math.log(4.0)),
    dict(gamma_link="log_shift", gamma_max_log_scale=math.log(1.5), frequency_warp="global"),
    dict(gamma_features="modulus", gamma_edge="st_clamp", frequency_warp="grouped",
         num_groups=2, warp_bound="none"),
]

# (prospective, mode, prospective_tau) with the tau values as multiples of the filter's tau.
CALLS = [(True, "tau", None), (False, "tau", None), (True, "gamma", None),
         (True, "gamma", 0.5), (True, "tau", "per_filter")]

INVALID = [
    dict(gamma_link="bogus"),
    dict(num_groups=0),
    dict(write_max=1.0),
    dict(gamma_edge_margin=0.5),
    dict(max_log_scale=-1.0),
    dict(gamma_control=False, gamma_link="log_shift"),
    dict(gamma_control=False),
    dict(gamma_control=1),
]
# Valid settings the controller's constructor rejects for a filter: (filter, config).
CTOR_INVALID = [
    ("band", dict(frequency_warp="grouped", num_groups=7)),
    ("band", dict(gamma_link="log_shift", gamma_max_log_scale=math.log(20.0))),
]


def main():
    sys.path.insert(0, REFERENCE)
    from rqf_models.backbones.rqf.filter import RQF  # noqa: E402  (reference code)
    from rqf_models.backbones.rqf.selective import (  # noqa: E402
        SelectiveController,
        SelectiveRQFConfig,
    )

    out = {}
    meta = []

    def make_filter(fname, seed):
        _, F, f64, kw = next(f for f in FILTERS if f[0] == fname)
        torch.manual_seed(seed)
        rqf = RQF(num_filters=F, param_space="log", discretization="zoh", learn_tau=False, **kw)
        return rqf.double() if f64 else rqf

    def state(rqf):
        return {
            "log_tau": rqf.log_tau.detach().numpy().copy(),
            "log_gamma": rqf.log_gamma.detach().numpy().copy(),
            "log_theta": rqf.log_theta.detach().numpy().copy(),
            "min_gamma": rqf._min_gamma.numpy().copy(),
            "max_gamma": rqf._max_gamma.numpy().copy(),
            "min_freq": rqf._min_freq.numpy().copy(),
            "max_freq": rqf._max_freq.numpy().copy(),
        }

    case = 0
    for fi, (fname, F, f64, kw) in enumerate(FILTERS):
        for ci, cfg in enumerate(CONFIGS):
            groups = cfg.get("num_groups", 4)
            if cfg.get("frequency_warp") == "grouped" and groups > F:
                continue
            # Two of the call variants per (filter, settings) pair, rotating.
            for k in ((fi + ci) % len(CALLS), (fi + ci + 2) % len(CALLS)):
                prospective, mode, ptau = CALLS[k]
                seed = 1000 * fi + 10 * ci + k
                rqf = make_filter(fname, seed)
                pre = state(rqf)
                config = SelectiveRQFConfig(**cfg)
                ctl = SelectiveController(N_IN, rqf, config)
                post = state(rqf)
                gen = torch.Generator().manual_seed(seed)
                for name in ("W_gamma", "W_write", "W_delta"):
                    head = getattr(ctl, name)
                    if head is not None:
                        with torch.no_grad():
                            head.copy_(0.4 * torch.randn(head.shape, generator=gen))
                source = torch.complex(torch.randn(N_IN, B, T, generator=gen),
                                       torch.randn(N_IN, B, T, generator=gen))
                tau = rqf.tau.detach()
                if ptau is None:
                    prospective_tau = None
                elif ptau == "per_filter":
                    prospective_tau = [float(v) for v in (0.25 + 0.1 * torch.arange(F)) * tau]
                else:
                    prospective_tau = float(ptau * tau[0])
                inp = ctl(source, rqf, prospective=prospective, mode=mode,
                          prospective_tau=prospective_tau)
                p = f"c{case}/"
                for key, v in pre.items():
                    out[p + "pre_" + key] = v
                for key, v in post.items():
                    out[p + "post_" + key] = v
                for name in ("W_gamma", "W_write", "W_delta"):
                    head = getattr(ctl, name)
                    if head is not None:
                        out[p + name] = head.detach().numpy().copy()
                out[p + "source_re"] = source.real.numpy().copy()
                out[p + "source_im"] = source.imag.numpy().copy()
                for name in ("gamma_logits", "warp_logits", "write_logits", "bias", "theta",
                             "minimum", "span", "step", "horizon", "theta_minimum",
                             "theta_maximum"):
                    out[p + "out_" + name] = getattr(inp, name).detach().numpy().copy()
                if inp.groups is not None:
                    out[p + "out_groups"] = inp.groups.numpy().copy()
                out[p + "out_options"] = np.array([float(v) for v in inp.options], np.float64)
                meta.append(dict(case=case, filter=fname, config=cfg, prospective=prospective,
                                 mode=mode, prospective_tau=prospective_tau,
                                 dt=float(rqf.dt), float64=f64,
                                 clamp_gamma=bool(kw.get("clamp_gamma", False))))
                case += 1

    errors = []
    for cfg in INVALID:
        try:
            SelectiveRQFConfig(**cfg)
        except (ValueError, TypeError) as exc:
            errors.append(dict(config=cfg, where="config", type=type(exc).__name__, message=str(exc)))
        else:
            raise AssertionError(f"reference accepted {cfg}")
    for fname, cfg in CTOR_INVALID:
        rqf = make_filter(fname, 7)
        try:
            SelectiveController(N_IN, rqf, SelectiveRQFConfig(**cfg))
        except ValueError as exc:
            errors.append(dict(config=cfg, filter=fname, where="controller", type="ValueError",
                               message=str(exc)))
        else:
            raise AssertionError(f"reference accepted {fname} {cfg}")

    out["meta"] = np.array(json.dumps(dict(cases=meta, errors=errors, n_in=N_IN, B=B, T=T)))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {case} cases, {len(errors)} error cases")


if __name__ == "__main__":
    main()

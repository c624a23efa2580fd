"""Synthetic workloads of the benchmark configurations (seeded, no datasets).

Per-channel parameters follow the reference's resonant "paper recipe"
(rqf_models/backbones/rqf/filter.py:250-262, 330-358, 371-377):

* theta = 2*pi*f*tau log-uniform in [log(2*pi*tau/seq_duration), log(2*pi)]
* gamma = theta/(1+theta) (critical damping), gamma bounds [1e-6, 1-1e-6],
  projected to the interior margin (selective.py:126-136, filter.py:398-400)
* eta = dt/tau, horizon = 1 (prospective_tau None)
* theta band [2*pi*f_min*tau, min(2*pi*f_max*tau, pi*tau/dt)] with
  f_min = 1/seq_duration, f_max = 1/tau
* warp groups = rank(theta) * G // F (selective.py:164-165)
* sigmoid gamma link: bias = logit((gamma - lo)/span) (selective.py:227-236)

The selective scan inputs are assembled by the restated selective controller
(``selective_controller``) from that filter state.

ZOH two-tap coefficients for the static (non-selective) scans follow
``RQF.compute_two_tap_coefficients`` (filter.py:630-646).
"""

from __future__ import annotations

import math

import torch

from prospective_rqf_amd.selective_controller import (
    FilterState,
    SelectiveController,
    SelectiveRQFConfig,
)
from prospective_rqf_amd.selective_scan import SelectiveScanInputs

LN_1_25 = math.log(1.25)


def recipe_params(F: int, *, samp: float, tau: float, seq_duration: float, margin: float = 1e-3,
                  max_freq_factor: float = 1.0, generator: torch.Generator | None = None,
                  dtype=torch.float64):
    """Per-channel (theta, gamma, eta, lo, span, theta_lo, theta_hi) in fp64.

    theta is log-uniform in [2*pi*tau/seq_duration, 2*pi*max_freq_factor]
    (filter_max_freq_factor of filter.py:330-345)."""
    dt = 1.0 / samp
    lo_t = math.log(2 * math.pi * tau / seq_duration)
    hi_t = math.log(2 * math.pi * max_freq_factor)
    theta = torch.exp(lo_t + torch.rand(F, generator=generator, dtype=dtype) * (hi_t - lo_t))
    lo, hi = 1e-6, 1.0 - 1e-6
    span = hi - lo
    gamma = (theta / (1 + theta)).clamp(lo + margin * span, hi - margin * span)
    theta_lo = torch.full((F,), 2 * math.pi * (1.0 / seq_duration) * tau, dtype=dtype)
    theta_hi = torch.full((F,), min(2 * math.pi * (1.0 / tau) * tau, math.pi * tau / dt),
                          dtype=dtype)
    eta = torch.full((F,), dt / tau, dtype=dtype)
    return dict(theta=theta, gamma=gamma, eta=eta, lo=torch.full((F,), lo, dtype=dtype),
                span=torch.full((F,), span, dtype=dtype), theta_lo=theta_lo, theta_hi=theta_hi)


def zoh_two_tap(gamma, theta, eta, ratio):
    """(C1, tap0, tap1) of the impulse-ZOH prospective recurrence (filter.py:630-646)."""
    a = torch.complex(-gamma * eta, (1 - gamma) * theta * eta)
    C1 = torch.exp(a)
    small = a.abs() < 1e-4
    safe = torch.where(small, torch.ones_like(a), a)
    phi = torch.where(small, 1 + a * (0.5 + a * (1 / 6 + a / 24)), torch.expm1(a) / safe)
    extra = gamma * ratio * C1
    return C1, gamma * eta * phi + extra, -extra


def recipe_filter(F: int, *, samp: float, tau: float, seq_duration: float,
                  max_freq_factor: float = 1.0, generator: torch.Generator | None = None,
                  dtype=torch.float32) -> FilterState:
    """Log-space filter state of the resonant recipe (filter.py:250-262, 330-361):
    log_theta log-uniform as in :func:`recipe_params`, critical-damping gamma
    clamped into [1e-6, 1 - 1e-6], f_min = 1/seq_duration, f_max = 1/tau."""
    p = recipe_params(F, samp=samp, tau=tau, seq_duration=seq_duration, margin=0.0,
                      max_freq_factor=max_freq_factor, generator=generator)
    full = lambda v: torch.full((F,), v, dtype=dtype)  # noqa: E731
    return FilterState(
        log_tau=torch.log(full(tau)), log_gamma=torch.log(p["gamma"].to(dtype)),
        log_theta=torch.log(p["theta"]).to(dtype), min_gamma=full(1e-6),
        max_gamma=full(1.0 - 1e-6), min_freq=full(1.0 / seq_duration),
        max_freq=1.0 / full(tau), dt=1.0 / samp)


def selective_inputs(F, B, T, *, G=8, gamma=True, write=True, warp="grouped", log_shift=False,
                     prospective=True, gamma_horizon=False, write_sigmoid=True, write_max=2.0,
                     gamma_scale=LN_1_25, warp_scale=LN_1_25, bound_warp=True, samp=16000.0,
                     tau=5.0 / 16000.0, seq_duration=1.0, logit_std=1.0, device="cpu", seed=0):
    """SelectiveScanInputs of a recipe filter with N(0, logit_std^2) head logits.

    Every field but the logits comes from the selective controller
    (``selective_controller.SelectiveController``, the restatement of
    selective.py:100-278 pinned against the reference's own): the filter
    projection at construction, the bias logit, warp-group ranks, theta band,
    horizon and options.  The logits stand in for the head GEMM's output."""
    g = torch.Generator().manual_seed(seed)
    rqf = recipe_filter(F, samp=samp, tau=tau, seq_duration=seq_duration, generator=g)
    config = SelectiveRQFConfig(
        gamma_control=bool(gamma), gamma_link="log_shift" if log_shift else "sigmoid",
        gamma_max_log_scale=float(gamma_scale), write_control=bool(write),
        write_link="sigmoid" if write_sigmoid else "affine", write_max=float(write_max),
        frequency_warp=warp, warp_bound="band" if bound_warp else "none",
        num_groups=G if warp == "grouped" else 4, max_log_scale=float(warp_scale))
    ctl = SelectiveController(1, rqf, config)
    n_warp = config.warp_groups

    def logits(rows):
        return (logit_std * torch.randn(rows, B, T, generator=g)).float()

    inp = ctl.assemble(logits(F) if gamma else torch.empty(0, B, T),
                       logits(n_warp) if n_warp else torch.empty(0, B, T),
                       logits(F) if write else torch.empty(0, B, T), rqf,
                       prospective=bool(prospective), mode="gamma" if gamma_horizon else "tau",
                       prospective_tau=None)
    move = lambda v: None if v is None else v.to(device)  # noqa: E731
    return SelectiveScanInputs(*(move(v) for v in inp[:-1]), inp.options)


def randn_c64(*shape, generator=None, device="cpu"):
    re = torch.randn(*shape, generator=generator)
    im = torch.randn(*shape, generator=generator)
    return torch.complex(re, im).to(device)


def raw_waveform(B, T, *, samp=16000.0, generator=None):
    """Sum of 3 random sinusoids in [50, 4000] Hz plus N(0, 0.05^2), clipped to [-1, 1]."""
    t = torch.arange(T, dtype=torch.float64) / samp
    f = 50 + (4000 - 50) * torch.rand(B, 3, 1, generator=generator, dtype=torch.float64)
    ph = 2 * math.pi * torch.rand(B, 3, 1, generator=generator, dtype=torch.float64)
    x = torch.sin(2 * math.pi * f * t + ph).sum(1) / 3
    x = x + 0.05 * torch.randn(B, T, generator=generator, dtype=torch.float64)
    return x.clamp(-1, 1).float()


def static_two_tap(F, *, samp=16000.0, tau=5.0 / 16000.0, seq_duration=1.0, max_freq_factor=1.0,
                   seed=0, device="cpu"):
    """(C1, tap0, tap1) complex64 per channel for the static prospective RQF."""
    g = torch.Generator().manual_seed(seed)
    p = recipe_params(F, samp=samp, tau=tau, seq_duration=seq_duration, margin=0.0,
                      max_freq_factor=max_freq_factor, generator=g)
    c1, t0, t1 = zoh_two_tap(p["gamma"], p["theta"], p["eta"], torch.ones_like(p["gamma"]))
    return tuple(v.to(torch.complex64).to(device) for v in (c1, t0, t1))

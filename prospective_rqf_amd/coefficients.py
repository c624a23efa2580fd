"""RQF filter coefficients from the filter module's parameters (caller side of the scans).

The scans take per-channel complex coefficients; in the reference they come from
``RQF.compute_coefficients`` / ``RQF.compute_two_tap_coefficients``
(rqf_models/backbones/rqf/filter.py:451-664) over the parameter reads
``tau`` (:414-421), ``gamma`` (:424-436) and ``freq`` (:438-449).  This module
restates those formulas so that parameters read from a packaged checkpoint (or any
state dict) can drive the HIP scans without the reference's model classes.

Continuous-time filter per channel (filter.py:466-471): ``alpha = gamma/tau``,
``lambda = -alpha + i*2*pi*f*(1-gamma)``, drive ``alpha*(u + tau_p*du/dt)`` with the
look-ahead ``tau_p = rho*tau`` (rho = 1 in "tau" mode, 1/gamma in "gamma" mode,
prospective_tau/tau when given).  With ``h = dt``, ``x = lambda*h``, ``eta = h/tau``,
``phi(x) = (e^x-1)/x`` and ``psi(x) = (e^x-1-x)/x^2``:

* ZOH single tap:   C1 = e^x, C2 = gamma*eta*phi
* Euler single tap: C1 = 1 + x, C2 = gamma*eta
* bilinear:         C1 = (1+x/2)/(1-x/2), C2 = gamma*eta/(1-x/2)
* ZOH two-tap (impulse-prospective): tap0 = gamma*eta*phi + gamma*rho*C1, tap1 = -gamma*rho*C1
* Euler two-tap:    tap0 = gamma*eta + gamma*rho, tap1 = -gamma*rho
* FOH two-tap:      tap0 = gamma*eta*psi (+ gamma*rho*phi),
                    tap1 = gamma*eta*(phi-psi) (- gamma*rho*phi)

Evaluation is in float64 whatever the parameter dtype (the reference evaluates in
the parameters' float32 and casts to complex64 before the scan); results are
returned as ``out_dtype`` (complex64 by default, the dtype the scans take).
``phi`` and ``psi`` use a cancellation-free complex ``expm1`` and, for ``psi`` at
small ``|x|``, its Taylor series, so they are accurate to a few ulp of float64 at
every argument; the reference's float32 thresholds (filter.py:21-85) only change
the float32 rounding.
"""

from __future__ import annotations

import math
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import torch

_DISCRETIZATIONS = ("euler", "zoh", "bilinear", "foh")
_PSI_SERIES_BELOW = 0.125  # |x| below which psi is summed from its series
_PSI_TERMS = 14             # x^k/(k+2)! for k < 14: remainder < 0.125^14/16! at the bound


def expm1_complex(x: torch.Tensor) -> torch.Tensor:
    """e^x - 1 for complex ``x`` without cancellation in the real part.

    Re(e^{a+ib} - 1) = expm1(a)*cos(b) - 2*sin(b/2)^2, Im = e^a*sin(b)."""
    a, b = x.real, x.imag
    re = torch.expm1(a) * torch.cos(b) - 2.0 * torch.sin(0.5 * b) ** 2
    im = torch.exp(a) * torch.sin(b)
    return torch.complex(re, im)


def phi_complex(x: torch.Tensor) -> torch.Tensor:
    """(e^x - 1)/x, with the limit 1 at x = 0 (filter.py:21-50)."""
    zero = x == 0
    safe = torch.where(zero, torch.ones_like(x), x)
    return torch.where(zero, torch.ones_like(x), expm1_complex(safe) / safe)


def psi_complex(x: torch.Tensor) -> torch.Tensor:
    """(e^x - 1 - x)/x^2, with the limit 1/2 at x = 0 (filter.py:53-85)."""
    small = x.abs() < _PSI_SERIES_BELOW
    # Series sum_k x^k/(k+2)!, Horner from the top term.
    series = torch.zeros_like(x)
    for k in reversed(range(_PSI_TERMS)):
        series = series * x + 1.0 / math.factorial(k + 2)
    safe = torch.where(small, torch.ones_like(x), x)
    direct = (expm1_complex(safe) - safe) / (safe * safe)
    return torch.where(small, series, direct)


@dataclass
class RQFParams:
    """Per-channel parameters of one RQF filter module (``filter.py:168-360``).

    ``param_space="sigmoid"`` reads ``gamma_param``/``freq_param`` through the
    sigmoid into [min, max] (filter.py:424-449); ``"log"`` reads ``log_gamma`` and
    ``log_theta`` (theta = 2*pi*f*tau).  ``dt`` is ``1/samp_frequency``
    (block.py:350)."""

    log_tau: torch.Tensor
    dt: float
    discretization: str = "euler"
    clamp_gamma: bool = False
    param_space: str = "sigmoid"
    gamma_param: torch.Tensor | None = None
    freq_param: torch.Tensor | None = None
    min_gamma: torch.Tensor | None = None
    max_gamma: torch.Tensor | None = None
    min_freq: torch.Tensor | None = None
    max_freq: torch.Tensor | None = None
    log_gamma: torch.Tensor | None = None
    log_theta: torch.Tensor | None = None

    def __post_init__(self):
        if self.discretization not in _DISCRETIZATIONS:
            raise ValueError(f"discretization must be one of {_DISCRETIZATIONS}, "
                             f"got {self.discretization!r}")
        if self.param_space not in ("sigmoid", "log"):
            raise ValueError(f"param_space must be 'sigmoid' or 'log', got {self.param_space!r}")
        need = (("gamma_param", "freq_param", "min_gamma", "max_gamma", "min_freq", "max_freq")
                if self.param_space == "sigmoid" else ("log_gamma", "log_theta"))
        missing = [n for n in need if getattr(self, n) is None]
        if missing:
            raise ValueError(f"{self.param_space} parameters need {missing}")

    @classmethod
    def from_state_dict(cls, state: Mapping[str, torch.Tensor], prefix: str, *, dt: float,
                        discretization: str, clamp_gamma: bool) -> RQFParams:
        """Read the leaves and bound buffers an RQF module stores under ``prefix``
        (e.g. ``"encoder.blocks.0.rqf_fwd."``): ``log_tau`` plus either the sigmoid
        leaves with ``_min/_max_gamma``, ``_min/_max_freq`` or ``log_gamma``/``log_theta``."""
        def get(name):
            t = state.get(prefix + name)
            return None if t is None else t.detach().to("cpu", torch.float64)

        log_space = prefix + "log_theta" in state
        return cls(log_tau=get("log_tau"), dt=float(dt), discretization=discretization,
                   clamp_gamma=bool(clamp_gamma), param_space="log" if log_space else "sigmoid",
                   gamma_param=get("gamma_param"), freq_param=get("freq_param"),
                   min_gamma=get("_min_gamma"), max_gamma=get("_max_gamma"),
                   min_freq=get("_min_freq"), max_freq=get("_max_freq"),
                   log_gamma=get("log_gamma"), log_theta=get("log_theta"))

    def _f64(self, t):
        return t.detach().to(torch.float64)

    @property
    def tau(self) -> torch.Tensor:
        return torch.exp(self._f64(self.log_tau))

    @property
    def gamma(self) -> torch.Tensor:
        if self.param_space == "log":
            return torch.exp(self._f64(self.log_gamma))
        lo, hi = self._f64(self.min_gamma), self._f64(self.max_gamma)
        return lo + (hi - lo) * torch.sigmoid(self._f64(self.gamma_param))

    @property
    def freq(self) -> torch.Tensor:
        if self.param_space == "log":
            return torch.exp(self._f64(self.log_theta)) / (2 * math.pi * self.tau)
        lo, hi = self._f64(self.min_freq), self._f64(self.max_freq)
        return lo + (hi - lo) * torch.sigmoid(self._f64(self.freq_param))

    def effective_gamma(self) -> torch.Tensor:
        """gamma, projected into [1 - 1/sqrt(1+(w*tau)^2), w*tau/(1+w*tau)] when
        ``clamp_gamma`` is set (filter.py:461-465, 595-599), w = 2*pi*f."""
        gamma = self.gamma
        if not self.clamp_gamma:
            return gamma
        wt = 2 * math.pi * self.freq * self.tau
        lo = 1 - 1 / torch.sqrt(1 + wt * wt)
        hi = wt / (1 + wt)
        return torch.minimum(torch.maximum(gamma, lo), hi)  # torch.clamp(min=lo, max=hi)

    def pole(self):
        """(gamma_eff, x = lambda*dt, eta = dt/tau), all float64 / complex128."""
        tau, freq = self.tau, self.freq
        gamma = self.effective_gamma()
        lam = torch.complex(-gamma / tau, 2 * math.pi * freq * (1.0 - gamma))
        return gamma, lam * self.dt, self.dt / tau


def _rho(params: RQFParams, gamma: torch.Tensor, mode: str, prospective_tau) -> torch.Tensor:
    if prospective_tau is None:
        return torch.ones_like(gamma) if mode == "tau" else 1.0 / gamma
    tau_p = torch.as_tensor(prospective_tau, dtype=torch.float64)
    return tau_p / params.tau


def compute_coefficients(params: RQFParams, out_dtype=torch.complex64):
    """(C1, C2) of the single-tap recurrence ``x[t] = C1*x[t-1] + C2*u[t]``
    (filter.py:451-508).  FOH has no single-tap form and raises."""
    gamma, x, eta = params.pole()
    d = params.discretization
    if d == "euler":
        c1 = 1.0 + x
        c2 = (gamma * eta).to(torch.complex128)
    elif d == "zoh":
        c1 = torch.exp(x)
        c2 = gamma * eta * phi_complex(x)
    elif d == "bilinear":
        den = 1.0 - 0.5 * x
        c1 = (1.0 + 0.5 * x) / den
        c2 = gamma * eta / den
    else:
        raise NotImplementedError("discretization='foh' requires a two-tap update; call "
                                  "compute_two_tap_coefficients(prospective=...) instead.")
    return c1.to(out_dtype), c2.to(out_dtype)


def compute_two_tap_coefficients(params: RQFParams, prospective: bool = True, mode: str = "tau",
                                 prospective_tau: float | Sequence[float] | torch.Tensor | None = None,
                                 out_dtype=torch.complex64):
    """(C1, tap0, tap1) of ``y[n+1] = C1*y[n] + tap0*u[n] + tap1*u[n-1]``
    (filter.py:510-664).  Same errors as the reference: a mode other than "tau" or
    "gamma" raises ValueError; bilinear, and non-prospective Euler/ZOH, raise
    NotImplementedError."""
    if mode not in ("tau", "gamma"):
        raise ValueError(f"mode must be one of ('tau', 'gamma'), got {mode!r}")
    d = params.discretization
    if d == "bilinear":
        raise NotImplementedError("Two-tap update is not defined for bilinear discretization. "
                                  "Use 'euler', 'zoh', or 'foh'.")
    if d in ("euler", "zoh") and not prospective:
        which = "Euler" if d == "euler" else "ZOH"
        raise NotImplementedError(f"Non-prospective {which} uses the single-tap recurrence; "
                                  "call compute_coefficients() instead.")
    gamma, x, eta = params.pole()
    ge = gamma * eta
    g_rho = gamma * _rho(params, gamma, mode, prospective_tau)
    if d == "euler":
        c1 = 1.0 + x
        tap0 = (ge + g_rho).to(torch.complex128)
        tap1 = (-g_rho).to(torch.complex128)
    elif d == "zoh":
        c1 = torch.exp(x)
        tap0 = ge * phi_complex(x) + g_rho * c1
        tap1 = -g_rho * c1
    else:
        c1 = torch.exp(x)
        phi, psi = phi_complex(x), psi_complex(x)
        tap0 = ge * psi
        tap1 = ge * (phi - psi)
        if prospective:
            tap0 = tap0 + g_rho * phi
            tap1 = tap1 - g_rho * phi
    return c1.to(out_dtype), tap0.to(out_dtype), tap1.to(out_dtype)


def compute_prospective_taps(params: RQFParams, mode: str = "tau", prospective_tau=None,
                             out_dtype=torch.complex64):
    """Alias of ``compute_two_tap_coefficients(prospective=True)`` (filter.py:666-686)."""
    return compute_two_tap_coefficients(params, True, mode, prospective_tau, out_dtype)

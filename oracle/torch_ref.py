"""PyTorch restatement of the reference's CPU path for the scan backends.

TEST INFRASTRUCTURE ONLY (used by tests/ and by bench.py's ``cpu_baseline``
leg; never by the product package).  Two uses:

* in float64 with autograd it is the independent gradient check of the C
  oracle's hand-derived adjoints (torch supplies the conjugate-Wirtinger
  convention the reference's autograd uses);
* in float32 it is the timed CPU baseline: the same full-tensor coefficient
  math and per-step Python loop under autograd that the reference runs on CPU.

Followed line by line in behaviour (not copied):
  selective_coefficients  rqf_models/ops/selective_scan.py:26-68
  reference_layer_scan    rqf_models/ops/selective_scan.py:71-104 (after the drive GEMM)
  _sequential_scan_cpu    rqf_models/ops/scan.py:252-287
  _apply_prospective_taps rqf_models/backbones/rqf/block.py:644-682
"""

from __future__ import annotations

import torch


def selective_coefficients(inputs, F, B, T):
    """(A, gated p, gated n), each (F,B,T) complex, from torch SelectiveScanInputs-like fields."""
    gl, dl, wl = inputs.gamma_logits, inputs.warp_logits, inputs.write_logits
    o = inputs.options
    gamma = inputs.bias[:, None, None]
    if o[0]:
        if o[3]:
            gamma = torch.exp(gamma + o[4] * torch.tanh(gl))
        else:
            gamma = inputs.minimum[:, None, None] + inputs.span[:, None, None] * torch.sigmoid(gamma + gl)
    theta = inputs.theta[:, None, None]
    if o[1]:
        theta = theta * torch.exp(o[5] * torch.tanh(dl)[inputs.groups])
        if o[11]:
            theta = torch.clamp(theta, inputs.theta_minimum[:, None, None],
                                inputs.theta_maximum[:, None, None])
    eta = inputs.step[:, None, None]
    a = torch.complex(-gamma * eta, (1 - gamma) * theta * eta)
    A = torch.exp(a)
    small = a.abs() < 1e-4
    safe = torch.where(small, torch.ones_like(a), a)
    phi = torch.where(small, 1 + a * (0.5 + a * (1 / 6 + a / 24)), torch.expm1(a) / safe)
    p = gamma * eta * phi
    n = torch.zeros_like(p)
    if o[6]:
        ratio = 1 / gamma if o[7] else inputs.horizon[:, None, None]
        extra = ratio * gamma * A
        p, n = p + extra, -extra
    if o[2]:
        gate = o[9] * torch.sigmoid(wl + o[10]) if o[8] else 1 + wl
        p, n = p * gate, n * gate
    shape = (F, B, T)
    return A.expand(shape), p.expand(shape), n.expand(shape)


def selective_scan(z, inputs, *, truncated=False, z_lag=None):
    """Serial selective recurrence on the drive ``z`` (F,B,T): returns ``raw``.

    ``z_lag`` is the lag-tap source (``W @ x.detach()`` in TBPTT(1)); defaults to ``z``.
    """
    F, B, T = z.shape
    lag = z if z_lag is None else z_lag
    A, p, n = selective_coefficients(inputs, F, B, T)
    prev = z.new_zeros((F, B))
    values = []
    for t in range(T):
        prev = A[..., t] * (prev.detach() if truncated else prev) + p[..., t] * z[..., t]
        if t and inputs.options[6]:
            prev = prev + n[..., t] * lag[..., t - 1]
        values.append(prev)
    if not values:
        return z.new_zeros((F, B, 0))
    return torch.stack(values, dim=-1)


def split_relu(y):
    return torch.complex(y.real.relu(), y.imag.relu())


def sequential_scan(C1, C2, u):
    """x[t] = C1 x[t-1] + C2 u[t] on (B,T,F), serial over t.

    Like the reference, each step's state is written into a preallocated
    output by slice assignment (so autograd cost matches the reference's)."""
    B, T, F = u.shape
    prev = torch.zeros(B, F, dtype=u.dtype, device=u.device)
    out = torch.empty(B, T, F, dtype=u.dtype, device=u.device)
    for t in range(T):
        prev = C1 * prev + C2 * u[:, t, :]
        out[:, t, :] = prev
    return out


def prospective_drive(u, tap0, tap1, time_dim=1):
    """drive[t] = tap0 u[t] + tap1 u[t-1] with u[-1] = 0 along ``time_dim``."""
    delayed = torch.cat(
        [torch.zeros_like(u.narrow(time_dim, 0, 1)), u.narrow(time_dim, 0, u.shape[time_dim] - 1)],
        dim=time_dim,
    )
    if time_dim == 1:  # (B,T,F): taps broadcast on the last axis
        return tap0 * u + tap1 * delayed
    return tap0[:, None, None] * u + tap1[:, None, None] * delayed


def fbt_scan(C1, tap0, tap1, z):
    """Two-tap scan in (F,B,T) layout, serial over t."""
    drive = prospective_drive(z, tap0, tap1, time_dim=2)
    F, B, T = z.shape
    prev = torch.zeros(F, B, dtype=z.dtype, device=z.device)
    outs = []
    for t in range(T):
        prev = C1[:, None] * prev + drive[..., t]
        outs.append(prev)
    return torch.stack(outs, dim=-1) if outs else z.new_zeros((F, B, 0))

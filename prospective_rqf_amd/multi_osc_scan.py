"""Multi-oscillator scans with C-weight reduction, and the fused ``|y|`` readout.

Mirrors the reference's fused multi-oscillator family in
rqf_models/ops/triton_scan_kernel.py:

* ``_sequential_scan_multi_osc_forward_raw`` / ``_forward_abs_raw``
  (:1942-2087), ``_sequential_scan_multi_osc_backward_raw`` (:2280-2410),
  ``_SequentialScanMultiOscFunction`` / ``_triton_sequential_scan_multi_osc``
  (:2413-2520);
* the real-input twins ``_sequential_scan_multi_osc_real_forward_raw`` /
  ``_forward_abs_raw`` / ``_backward_real_raw`` and
  ``_SequentialScanMultiOscRealFunction`` / ``_triton_sequential_scan_multi_osc_real``
  (:2624-3079);
* ``_triton_parallel_scan_multi_osc`` (:4106-4140): the same equation, so the
  same kernels;
* the single-oscillator ``|y|`` scans ``_sequential_scan_forward_abs_raw_block_f``
  (:507) and ``_sequential_scan_real_forward_abs_raw_block_f`` (:1531) used by
  ``scan.sequential_scan_abs``.

Per filter f with N oscillators (coefficient index ``f*N + n``)::

    x_n[t] = C1_n x_n[t-1] + C2_n u[t]
    y[t]   = sum_n cw_n x_n[t]          cw = c_weights[:, 0] + 1j*c_weights[:, 1]

The kernels are ``rqf_multi_osc_fwd`` / ``rqf_multi_osc_bwd`` of librqf_hip.so;
any N >= 1 (the reference pads N to a power of two, triton_scan_kernel.py:1855-1900;
the kernels run the oscillators in chunks of up to four).  Gradients follow the reference's kernels: ``grad_C1 = sum d
conj(x[t-1])``, ``grad_C2 = sum d conj(u)``, ``grad_u = sum_n conj(C2_n) d_n``
(its real part for real ``u``) and ``grad_c_weights = (Re, Im) of
sum grad_y conj(x_n)``, with ``d_n[t] = conj(C1_n) d_n[t+1] + conj(cw_n)
grad_y[t]``.  The kernels evaluate all three coefficient sums in the
adjoint's reverse sweep, against ``u``, after exchanging the order of
summation (same values; no forward state and no per-step state tensor).  Unlike the reference, the
coefficient gradients are reduced in a fixed order (no atomics), so repeated
calls agree bit for bit.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from prospective_rqf_amd import _lib

MAX_OSC = 1 << 20  # a bound on the C ABI's argument, not on the kernels


def _c64(t: torch.Tensor) -> torch.Tensor:
    if t.dtype is torch.complex64 and t.is_contiguous() and not t.is_conj():
        return t  # the common case, without a conversion call
    if not t.is_complex():
        t = t.to(torch.cfloat)
    return t.to(torch.complex64).resolve_conj().contiguous()


def _f32(t: torch.Tensor) -> torch.Tensor:
    if t.is_complex():
        raise ValueError("expected a real input tensor")
    return t.to(torch.float32).contiguous()


def _like(grad: torch.Tensor | None, param: torch.Tensor) -> torch.Tensor | None:
    """Gradient in the parameter's dtype (a real coefficient gets the real part)."""
    if grad is None:
        return None
    if not param.is_complex():
        return grad.real.to(param.dtype)
    return grad.to(param.dtype)


def _cw_complex(c_weights: torch.Tensor) -> torch.Tensor:
    """(F*N, 2) real C-weights -> (F*N,) complex64 (interleaved view)."""
    if c_weights.dim() != 2 or c_weights.shape[1] != 2:
        raise ValueError(f"c_weights must have shape (scan_filters, 2), got {tuple(c_weights.shape)}")
    return torch.view_as_complex(c_weights.detach().to(torch.float32).contiguous())


def _check(u: torch.Tensor, C1: torch.Tensor, C2: torch.Tensor, num_osc: int) -> tuple[int, int, int]:
    if u.dim() != 3:
        raise ValueError(f"expected (batch, time, filters) input, got shape {tuple(u.shape)}")
    if not 1 <= num_osc <= MAX_OSC:
        raise ValueError(f"num_osc must be in [1, {MAX_OSC}], got {num_osc}")
    B, T, F = u.shape
    if C1.shape != (F * num_osc,) or C2.shape != (F * num_osc,):
        raise ValueError(f"C1/C2 must have shape ({F * num_osc},) for {F} filters x {num_osc} "
                         f"oscillators, got {tuple(C1.shape)}, {tuple(C2.shape)}")
    return B, T, F


def _forward(C1, C2, u, cw, num_osc, *, real: bool, absolute: bool):
    C1, C2 = _c64(C1), _c64(C2)
    u = _f32(u) if real else _c64(u)
    cw = None if cw is None else _c64(cw)
    B, T, F = _check(u, C1, C2, num_osc)
    if cw is not None and cw.shape != (F * num_osc,):
        raise ValueError(f"C-weights must cover {F * num_osc} oscillators, got {tuple(cw.shape)}")
    _lib.require_device(C1, C2, u, cw)
    out = torch.empty(B, T, F, device=u.device,
                      dtype=torch.float32 if absolute else torch.complex64)
    lib = _lib.load()
    n = lib.rqf_multi_osc_workspace(B, T, F, num_osc, 0)
    ws = _lib.workspace(n, u.device)
    _lib.check(
        lib.rqf_multi_osc_fwd(_lib.ptr(C1), _lib.ptr(C2), _lib.ptr(cw), _lib.ptr(u), int(real),
                              _lib.ptr(out), int(absolute), B, T, F, num_osc, _lib.ptr(ws), n,
                              _lib.stream_of(u)),
        "rqf_multi_osc_fwd",
    )
    return out


def _backward(C1, C2, u, c_weights, grad_output, num_osc, *, real: bool, compute_grad_C1=True,
              compute_grad_C2=True, compute_grad_u=True, compute_grad_cw=True):
    if not (compute_grad_C1 or compute_grad_C2 or compute_grad_u or compute_grad_cw):
        return None, None, None, None
    C1, C2 = _c64(C1), _c64(C2)
    u = _f32(u) if real else _c64(u)
    cw = _c64(_cw_complex(c_weights))
    grad_output = _c64(grad_output)
    B, T, F = _check(u, C1, C2, num_osc)
    if cw.shape != (F * num_osc,):
        raise ValueError(f"c_weights must cover {F * num_osc} oscillators, got "
                         f"{tuple(c_weights.shape)}")
    if grad_output.shape != (B, T, F):
        raise ValueError(f"grad_output must have shape {(B, T, F)}, got "
                         f"{tuple(grad_output.shape)}")
    _lib.require_device(C1, C2, u, cw, grad_output)
    dev = u.device
    grad_u = torch.empty_like(u) if compute_grad_u else None
    gc1 = torch.empty(F * num_osc, dtype=torch.complex64, device=dev) if compute_grad_C1 else None
    gc2 = torch.empty(F * num_osc, dtype=torch.complex64, device=dev) if compute_grad_C2 else None
    gcw = torch.empty(F * num_osc, dtype=torch.complex64, device=dev) if compute_grad_cw else None
    lib = _lib.load()
    n = lib.rqf_multi_osc_workspace(B, T, F, num_osc, 1)
    ws = _lib.workspace(n, dev)
    _lib.check(
        lib.rqf_multi_osc_bwd(_lib.ptr(C1), _lib.ptr(C2), _lib.ptr(cw), _lib.ptr(u), int(real),
                              _lib.ptr(grad_output), _lib.ptr(grad_u), _lib.ptr(gc1),
                              _lib.ptr(gc2), _lib.ptr(gcw), B, T, F, num_osc, _lib.ptr(ws), n,
                              _lib.stream_of(u)),
        "rqf_multi_osc_bwd",
    )
    grad_cw = None if gcw is None else torch.view_as_real(gcw).to(c_weights.dtype)
    return gc1, gc2, grad_u, grad_cw


# ----------------------------- complex input --------------------------------

def _sequential_scan_multi_osc_forward_raw(C1, C2, u, cw_real, cw_imag, num_osc):
    """Reduced complex output (B,T,F) of the fused multi-oscillator scan."""
    return _forward(C1, C2, u, torch.complex(cw_real.float(), cw_imag.float()), num_osc,
                    real=False, absolute=False)


def _sequential_scan_multi_osc_forward_abs_raw(C1, C2, u, cw_real, cw_imag, num_osc):
    """``|y|`` (B,T,F) real of the fused multi-oscillator scan (no autograd)."""
    return _forward(C1, C2, u, torch.complex(cw_real.float(), cw_imag.float()), num_osc,
                    real=False, absolute=True)


def _sequential_scan_multi_osc_backward_raw(C1, C2, u, c_weights, grad_output, num_osc, *,
                                            compute_grad_C1=True, compute_grad_C2=True,
                                            compute_grad_u=True, compute_grad_cw=True):
    """``(grad_C1, grad_C2, grad_u, grad_c_weights)``; entries not requested are None."""
    return _backward(C1, C2, u, c_weights, grad_output, num_osc, real=False,
                     compute_grad_C1=compute_grad_C1, compute_grad_C2=compute_grad_C2,
                     compute_grad_u=compute_grad_u, compute_grad_cw=compute_grad_cw)


class _SequentialScanMultiOscFunction(torch.autograd.Function):
    """Autograd boundary of the fused multi-oscillator scan (complex ``u``).

    Saves only (C1, C2, u, c_weights), as the reference does; the backward
    needs no forward state.
    """

    @staticmethod
    def forward(ctx, C1, C2, u, c_weights, num_osc):
        out = _forward(C1, C2, u, _cw_complex(c_weights), num_osc, real=False, absolute=False)
        ctx.save_for_backward(C1, C2, u, c_weights)
        ctx.num_osc = num_osc
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        C1, C2, u, c_weights = ctx.saved_tensors
        need_C1, need_C2, need_u, need_cw, _ = ctx.needs_input_grad
        gc1, gc2, gu, gcw = _backward(C1, C2, u, c_weights, grad_output, ctx.num_osc, real=False,
                                      compute_grad_C1=need_C1, compute_grad_C2=need_C2,
                                      compute_grad_u=need_u, compute_grad_cw=need_cw)
        if gu is not None and not u.is_complex():
            gu = gu.real
        return _like(gc1, C1), _like(gc2, C2), gu, gcw, None


def _triton_sequential_scan_multi_osc(C1, C2, u, c_weights, num_osc):
    """Fused multi-oscillator complex scan with C-weight reduction and autograd."""
    return _SequentialScanMultiOscFunction.apply(C1, C2, u, c_weights, num_osc)


def _triton_parallel_scan_multi_osc(C1, C2, u, c_weights, num_osc):
    """The reference's parallel-scan variant computes the same equation; the
    HIP kernels are already parallel over time segments."""
    return _SequentialScanMultiOscFunction.apply(C1, C2, u, c_weights, num_osc)


# ------------------------------- real input ---------------------------------

def _sequential_scan_multi_osc_real_forward_raw(C1, C2, u, c_weights, num_osc):
    """Real-input specialisation: the same equation with Im(u) = 0."""
    return _forward(C1, C2, u, _cw_complex(c_weights), num_osc, real=True, absolute=False)


def _sequential_scan_multi_osc_real_forward_abs_raw(C1, C2, u, c_weights, num_osc):
    """``|y|`` for real ``u`` (no autograd)."""
    return _forward(C1, C2, u, _cw_complex(c_weights), num_osc, real=True, absolute=True)


def _sequential_scan_multi_osc_backward_real_raw(C1, C2, u, c_weights, grad_output, num_osc, *,
                                                 compute_grad_C1=True, compute_grad_C2=True,
                                                 compute_grad_u=True, compute_grad_cw=True):
    """Real-input backward: ``grad_u`` is real."""
    return _backward(C1, C2, u, c_weights, grad_output, num_osc, real=True,
                     compute_grad_C1=compute_grad_C1, compute_grad_C2=compute_grad_C2,
                     compute_grad_u=compute_grad_u, compute_grad_cw=compute_grad_cw)


class _SequentialScanMultiOscRealFunction(torch.autograd.Function):
    """Autograd boundary of the real-input fused multi-oscillator scan."""

    @staticmethod
    def forward(ctx, C1, C2, u, c_weights, num_osc):
        if u.is_complex():
            raise ValueError("_SequentialScanMultiOscRealFunction expects real input")
        u = u.to(torch.float32)
        out = _forward(C1, C2, u, _cw_complex(c_weights), num_osc, real=True, absolute=False)
        ctx.save_for_backward(C1, C2, u, c_weights)
        ctx.num_osc = num_osc
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        C1, C2, u, c_weights = ctx.saved_tensors
        need_C1, need_C2, need_u, need_cw, _ = ctx.needs_input_grad
        gc1, gc2, gu, gcw = _backward(C1, C2, u, c_weights, grad_output, ctx.num_osc, real=True,
                                      compute_grad_C1=need_C1, compute_grad_C2=need_C2,
                                      compute_grad_u=need_u, compute_grad_cw=need_cw)
        return _like(gc1, C1), _like(gc2, C2), gu, gcw, None


def _triton_sequential_scan_multi_osc_real(C1, C2, u, c_weights, num_osc):
    """Fused multi-oscillator scan for real ``u`` with autograd."""
    if u.is_complex():
        raise ValueError("_triton_sequential_scan_multi_osc_real expects real input")
    return _SequentialScanMultiOscRealFunction.apply(C1, C2, u, c_weights, num_osc)


# -------------------------- single-oscillator |y| ---------------------------

def _sequential_scan_forward_abs_raw_block_f(C1, C2, u):
    """``|x|`` of x[t] = C1 x[t-1] + C2 u[t] for complex u (B,T,F), F = len(C1)."""
    if not u.is_complex():
        raise ValueError("_sequential_scan_forward_abs_raw_block_f expects complex input")
    return _forward(C1, C2, u, None, 1, real=False, absolute=True)


def _sequential_scan_real_forward_abs_raw_block_f(C1, C2, u):
    """``|x|`` of x[t] = C1 x[t-1] + C2 u[t] for real u (B,T,F)."""
    if u.is_complex():
        raise ValueError("_sequential_scan_real_forward_abs_raw_block_f expects real input")
    return _forward(C1, C2, u, None, 1, real=True, absolute=True)

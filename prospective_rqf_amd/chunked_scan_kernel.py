"""Time-invariant complex scans in the reference's ``(batch, time, filters)`` API.

Mirrors rqf_models/ops/chunked_scan_kernel.py: ``_pick_chunk`` (:28-41),
``_chunked_scan_forward_raw`` / ``_chunked_scan_backward_raw`` (:217-303),
``_ChunkedScanFunction`` / ``_triton_chunked_scan`` (:306-358) and the fused
two-tap prospective variant (:442-526).  The names are kept (including the
``_triton_`` prefix) so callers bind unchanged; the kernels are HIP
(``rqf_chunked_*`` in librqf_hip.so) and work on (B,T,F) directly, without
the reference's permute copies.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from prospective_rqf_amd import _lib

_CHUNK = 2048


def _pick_chunk(filters: int, batch: int) -> int:
    """The reference's chunk rule (kept for API compatibility; the HIP kernels
    size their own segments)."""
    programs = filters * batch
    if programs >= 256:
        return 512
    if programs >= 64:
        return 1024
    return _CHUNK


def _c64(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype is torch.complex64 and t.is_contiguous() and not t.is_conj():
        return t  # the common case, without a conversion call
    if not t.is_complex():
        t = t.to(torch.cfloat)
    return t.to(torch.complex64).resolve_conj().contiguous()


def _check_btf(u: torch.Tensor, *coefs: torch.Tensor) -> None:
    if u.dim() != 3:
        raise ValueError(f"expected (batch, time, filters) input, got shape {tuple(u.shape)}")
    for c in coefs:
        if c.shape != (u.shape[2],):
            raise ValueError(f"coefficients must have shape ({u.shape[2]},), got {tuple(c.shape)}")


def _check_like(u: torch.Tensor, **tensors) -> None:
    """Every named (B,T,F) tensor (None allowed) must have the input's shape."""
    for name, t in tensors.items():
        if t is not None and t.shape != u.shape:
            raise ValueError(f"{name} must have the input's shape {tuple(u.shape)}, "
                             f"got {tuple(t.shape)}")


_WS_BYTES: dict = {}


def _ws(B, T, F, device):
    """The backward's workspace (fp64 partial sums); its size per shape is
    asked of the library once."""
    n = _WS_BYTES.get((B, T, F))
    if n is None:
        n = _WS_BYTES[(B, T, F)] = _lib.load().rqf_btf_scan_workspace(B, T, F)
    return _lib.workspace(n, device), n


def _chunked_scan_forward_raw(C1, C2, u):
    """x[t] = C1 x[t-1] + C2 u[t] on (B,T,F); returns complex64 (B,T,F)."""
    C1, C2, u = _c64(C1), _c64(C2), _c64(u)
    _check_btf(u, C1, C2)
    _lib.require_device(C1, C2, u)
    B, T, F = u.shape
    out = torch.empty_like(u)
    # the single-pass forward needs no workspace
    _lib.check(
        _lib.load().rqf_chunked_scan_fwd(_lib.ptr(C1), _lib.ptr(C2), _lib.ptr(u), _lib.ptr(out),
                                         B, T, F, None, 0, _lib.stream_of(u)),
        "rqf_chunked_scan_fwd",
    )
    return out


def _chunked_scan_backward_raw(C1, C2, u, states, grad_output):
    """Adjoint of the chunked scan: ``(grad_C1, grad_C2, grad_u)``.

    ``states`` (the forward output the reference's kernel reads) is accepted for
    the reference's signature and may be None: the kernel evaluates
    ``grad_C1`` from ``u`` with the order of summation exchanged."""
    C1, C2, u, grad_output = (_c64(t) for t in (C1, C2, u, grad_output))
    _check_btf(u, C1, C2)
    _check_like(u, states=states, grad_output=grad_output)
    _lib.require_device(C1, C2, u, grad_output)
    B, T, F = u.shape
    grad_u = torch.empty_like(u)
    gc1 = torch.empty(F, dtype=torch.complex64, device=u.device)
    gc2 = torch.empty_like(gc1)
    ws, n = _ws(B, T, F, u.device)
    _lib.check(
        _lib.load().rqf_chunked_scan_bwd(
            _lib.ptr(C1), _lib.ptr(C2), _lib.ptr(u), None, _lib.ptr(grad_output),
            _lib.ptr(grad_u), _lib.ptr(gc1), _lib.ptr(gc2), B, T, F, _lib.ptr(ws), n,
            _lib.stream_of(u)),
        "rqf_chunked_scan_bwd",
    )
    return gc1, gc2, grad_u


class _ChunkedScanFunction(torch.autograd.Function):
    """Autograd wrapper: forward and adjoint both run on the HIP kernels."""

    @staticmethod
    def forward(ctx, C1, C2, u):
        C1, C2, u = _c64(C1), _c64(C2), _c64(u)
        output = _chunked_scan_forward_raw(C1, C2, u)
        # The reference also saves the output for its backward kernel
        # (chunked_scan_kernel.py:328); the HIP adjoint does not read it.
        ctx.save_for_backward(C1, C2, u)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        C1, C2, u = ctx.saved_tensors
        return _chunked_scan_backward_raw(C1, C2, u, None, grad_output)


def _triton_chunked_scan(C1, C2, u):
    """x[n] = C1 x[n-1] + C2 u[n] on (batch, time, filters); complex64 output."""
    return _ChunkedScanFunction.apply(C1, C2, u)


chunked_scan = _triton_chunked_scan


def _chunked_prospective_forward_raw(C1, tap0, tap1, x):
    C1, tap0, tap1, x = (_c64(t) for t in (C1, tap0, tap1, x))
    _check_btf(x, C1, tap0, tap1)
    _lib.require_device(C1, tap0, tap1, x)
    B, T, F = x.shape
    out = torch.empty_like(x)
    _lib.check(
        _lib.load().rqf_chunked_prospective_fwd(
            _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(out), B, T, F,
            None, 0, _lib.stream_of(x)),
        "rqf_chunked_prospective_fwd",
    )
    return out


def _chunked_prospective_backward_raw(C1, tap0, tap1, x, states, grad_output):
    """``(grad_C1, grad_tap0, grad_tap1, grad_x)`` of the two-tap scan.
    ``states``, the forward output the reference's autograd context saves
    (chunked_scan_kernel.py:486), is accepted and may be None: the kernel
    does not read it.  The reference's ``_ChunkedProspectiveScanFunction.backward``
    (chunked_scan_kernel.py:490-504) computes the same with a chunked adjoint
    scan and five pointwise passes; here one single-pass scan
    (``rqf_chunked_prospective_bwd``) produces grad_x and the three sums."""
    C1, tap0, tap1, x, grad_output = (_c64(t) for t in (C1, tap0, tap1, x, grad_output))
    _check_btf(x, C1, tap0, tap1)
    _check_like(x, states=states, grad_output=grad_output)
    _lib.require_device(C1, tap0, tap1, x, grad_output)
    B, T, F = x.shape
    grad_x = torch.empty_like(x)
    gc1 = torch.empty(F, dtype=torch.complex64, device=x.device)
    gt0 = torch.empty_like(gc1)
    gt1 = torch.empty_like(gc1)
    ws, n = _ws(B, T, F, x.device)
    _lib.check(
        _lib.load().rqf_chunked_prospective_bwd(
            _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), None,
            _lib.ptr(grad_output), _lib.ptr(grad_x), _lib.ptr(gc1), _lib.ptr(gt0),
            _lib.ptr(gt1), B, T, F, _lib.ptr(ws), n, _lib.stream_of(x)),
        "rqf_chunked_prospective_bwd",
    )
    return gc1, gt0, gt1, grad_x


class _ChunkedProspectiveScanFunction(torch.autograd.Function):
    """x_out[n] = C1 x_out[n-1] + tap0 x[n] + tap1 x[n-1], drive fused."""

    @staticmethod
    def forward(ctx, C1, tap0, tap1, x):
        C1, tap0, tap1, x = (_c64(t) for t in (C1, tap0, tap1, x))
        output = _chunked_prospective_forward_raw(C1, tap0, tap1, x)
        # The output is not saved: the HIP adjoint does not read it.
        ctx.save_for_backward(C1, tap0, tap1, x)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        C1, tap0, tap1, x = ctx.saved_tensors
        return _chunked_prospective_backward_raw(C1, tap0, tap1, x, None, grad_output)


def _triton_chunked_scan_prospective(C1, tap0, tap1, x):
    """Fused two-tap prospective scan on (batch, time, filters)."""
    return _ChunkedProspectiveScanFunction.apply(C1, tap0, tap1, x)


chunked_scan_prospective = _triton_chunked_scan_prospective

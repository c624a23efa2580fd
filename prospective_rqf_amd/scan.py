"""Dispatch surface of the time-invariant scans, honouring the reference's flags.

Mirrors rqf_models/ops/scan.py: the import-time flags (:38-70),
``sequential_scan`` (:290-378), ``sequential_scan_abs`` (:381-432) and
``parallel_scan`` (:435-529) for the scalar (``B is None``) case that the
HIP kernels serve.

Flags (read at import, like the reference):
  ORGANICS_SCAN_BACKEND=chunked|sequential  -> ``_SCAN_BACKEND``, ``_USE_CHUNKED``
  ORGANICS_DISABLE_TRITON=1                  -> ``_HAS_TRITON`` False
``_HAS_TRITON`` keeps the reference's name for "the accelerated kernels are
usable"; here that means librqf_hip.so is built and not disabled.
``_HAS_FBT_PROSPECTIVE`` mirrors the cells' import-time flag (pure.py:34-40):
the fused FBT / selective kernels are importable, which, as in the reference,
``ORGANICS_DISABLE_TRITON`` does not change.
``ORGANICS_RQF_FBT`` is read at call time by the callers (pure.py:143-144,
500-508), see :func:`fbt_enabled` and :func:`selective_use_kernel`.

Only HIP-device inputs on the chunked backend are served.  The reference's
CPU loop, PyTorch Blelloch scan, legacy sequential kernels and B-matrix
variant are not part of this backend: such calls raise instead of silently
running elsewhere.
"""

from __future__ import annotations

import os

import torch

from prospective_rqf_amd import _lib
from prospective_rqf_amd.chunked_scan_kernel import _triton_chunked_scan

_TRITON_DISABLED = os.environ.get("ORGANICS_DISABLE_TRITON", "0") == "1"
_SCAN_BACKEND = os.environ.get("ORGANICS_SCAN_BACKEND", "chunked").lower()
_USE_CHUNKED = _SCAN_BACKEND == "chunked"
try:
    _lib.load()
    _HAS_FBT_PROSPECTIVE = True
except (OSError, _lib.RQFError):
    _HAS_FBT_PROSPECTIVE = False
_HAS_TRITON = _HAS_FBT_PROSPECTIVE and not _TRITON_DISABLED


def selective_use_kernel() -> bool:
    """``use_kernel`` of the selective cells, read at call time
    (``_forward_selective``, pure.py:143-144): the chunked backend is selected
    and ``ORGANICS_RQF_FBT`` is not ``"0"``."""
    return _SCAN_BACKEND == "chunked" and os.environ.get("ORGANICS_RQF_FBT", "1") != "0"


def fbt_enabled(x: torch.Tensor | None = None) -> bool:
    """Whether the channel-outermost fused path applies (``_fbt_enabled``,
    pure.py:500-508): the fused kernels are available, ``x`` (when given) is a
    device tensor, the chunked backend is selected and ``ORGANICS_RQF_FBT`` is
    not ``"0"`` at call time.  The reference also requires every block to be
    FBT-eligible; that check belongs to the cell."""
    return (_HAS_FBT_PROSPECTIVE and (x is None or x.is_cuda) and selective_use_kernel())


def _prepare(C1, C2, u):
    """Type coercion and single-feature broadcast of the reference (scan.py:326-352)."""
    if not C1.is_complex():
        C1 = C1.to(torch.cfloat)
    if not C2.is_complex():
        C2 = C2.to(torch.cfloat)
    _, _, in_filters = u.shape
    num_filters = C1.shape[0]
    if in_filters == 1 and num_filters > 1:
        u = u.expand(-1, -1, num_filters)
    if not u.is_complex():
        u = u.to(torch.cfloat)
    return C1, C2, u


def _require_served(u, B):
    if B is not None:
        raise NotImplementedError("the B-matrix scan is not served by the HIP backend")
    if not (_HAS_TRITON and _USE_CHUNKED):
        raise RuntimeError(
            "HIP scan backend disabled (ORGANICS_DISABLE_TRITON=1, "
            "ORGANICS_SCAN_BACKEND != chunked, or librqf_hip.so not built)"
        )
    if not u.is_cuda:
        raise RuntimeError("sequential_scan/parallel_scan: HIP backend needs a device tensor")


def sequential_scan(C1, C2, u, B=None):
    """x[n] = C1 x[n-1] + C2 u[n] on (batch, time, filters) -> complex64."""
    _require_served(u, B)
    return _triton_chunked_scan(*_prepare(C1, C2, u))


def sequential_scan_abs(C1, C2, u, B=None):
    """``|sequential_scan(C1, C2, u)|`` as real (batch, time, filters) (scan.py:381-432).

    Without autograd the magnitude is fused into the scan's output store
    (``rqf_multi_osc_fwd`` with one oscillator and no C-weights), reading a
    real ``u`` as real.  When any input requires grad the reference composes
    ``sequential_scan(...).abs()``, and so does this.
    """
    _require_served(u, B)
    needs_grad = torch.is_grad_enabled() and (u.requires_grad or C1.requires_grad
                                              or C2.requires_grad)
    if needs_grad:
        return sequential_scan(C1, C2, u).abs()
    from prospective_rqf_amd.multi_osc_scan import (
        _sequential_scan_forward_abs_raw_block_f,
        _sequential_scan_real_forward_abs_raw_block_f,
    )

    if not C1.is_complex():
        C1 = C1.to(torch.cfloat)
    if not C2.is_complex():
        C2 = C2.to(torch.cfloat)
    _, _, in_filters = u.shape
    num_filters = C1.shape[0]
    if in_filters == 1 and num_filters > 1:
        u = u.expand(-1, -1, num_filters).contiguous()
    if u.is_complex():
        return _sequential_scan_forward_abs_raw_block_f(C1, C2, u)
    return _sequential_scan_real_forward_abs_raw_block_f(C1, C2, u)


def parallel_scan(C1, C2, u, B=None):
    """Same recurrence; the chunked kernel is itself a parallel scan (scan.py:505-509)."""
    _require_served(u, B)
    return _triton_chunked_scan(*_prepare(C1, C2, u))

"""Channel-outermost ``(filters, batch, time)`` two-tap prospective scans.

Mirrors rqf_models/ops/fbt_scan_kernel.py: ``_FBTProspectiveScan`` /
``fbt_prospective_scan`` (:245-357) and ``_FBTRecompute`` /
``fbt_recompute_scan`` (:575-689), same signatures and return values, on the
HIP kernels ``rqf_fbt_*``.

The recompute variant stores only the split-ReLU output plus the state that
enters every tile of 256 steps, and replays the tile in the backward; its
carry granularity is internal to the autograd context.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from prospective_rqf_amd import _lib


def _c64(t):
    if t.dtype is torch.complex64 and t.is_contiguous() and not t.is_conj():
        return t  # the common case, without a conversion call
    if not t.is_complex():
        t = t.to(torch.cfloat)
    return t.to(torch.complex64).resolve_conj().contiguous()


def _coefs(C1, tap0, tap1, filters):
    out = [_c64(c) for c in (C1, tap0, tap1)]
    for c in out:
        if c.shape != (filters,):
            raise ValueError(f"coefficients must have shape ({filters},), got {tuple(c.shape)}")
    return out


def _bwd_grads(F, device):
    return [torch.empty(F, dtype=torch.complex64, device=device) for _ in range(3)]


class _FBTProspectiveScan(torch.autograd.Function):
    """Two-tap prospective scan on (F,B,T); optional fused split-ReLU output."""

    @staticmethod
    def forward(ctx, C1, tap0, tap1, x_fbt, fuse_act):
        x = _c64(x_fbt)
        if x.dim() != 3:
            raise ValueError(f"expected (filters, batch, time) input, got shape {tuple(x.shape)}")
        filters, batch, time = x.shape
        C1, tap0, tap1 = _coefs(C1, tap0, tap1, filters)
        _lib.require_device(x, C1, tap0, tap1)
        raw = torch.empty_like(x)
        act = torch.empty_like(x) if fuse_act else None
        _lib.check(
            _lib.load().rqf_fbt_prospective_fwd(
                _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(raw),
                _lib.ptr(act), filters, batch, time, _lib.stream_of(x)),
            "rqf_fbt_prospective_fwd",
        )
        ctx.save_for_backward(C1, tap0, tap1, x, raw)
        ctx.fuse_act = fuse_act
        return act if fuse_act else raw

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        C1, tap0, tap1, x, raw = ctx.saved_tensors
        filters, batch, time = x.shape
        g = _c64(grad_output)
        if g.shape != x.shape:
            raise ValueError(f"grad_output must have the input's shape {tuple(x.shape)}, "
                             f"got {tuple(g.shape)}")
        _lib.require_device(g)
        grad_z = torch.empty_like(x)
        gc1, gt0, gt1 = _bwd_grads(filters, x.device)
        lib = _lib.load()
        n = lib.rqf_fbt_workspace(filters, batch, time)
        ws = _lib.workspace(n, x.device)
        _lib.check(
            lib.rqf_fbt_prospective_bwd(
                _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(raw),
                _lib.ptr(g), int(bool(ctx.fuse_act)), _lib.ptr(grad_z), _lib.ptr(gc1),
                _lib.ptr(gt0), _lib.ptr(gt1), filters, batch, time, _lib.ptr(ws), n,
                _lib.stream_of(x)),
            "rqf_fbt_prospective_bwd",
        )
        return gc1, gt0, gt1, grad_z, None


def fbt_prospective_scan(C1, tap0, tap1, x_fbt, fuse_act=False):
    """x_out[n] = C1 x_out[n-1] + tap0 x[n] + tap1 x[n-1] on (F,B,T).

    Returns the split-ReLU output when ``fuse_act``, else the raw state."""
    return _FBTProspectiveScan.apply(C1, tap0, tap1, x_fbt, fuse_act)


def fbt_recompute_forward_raw(C1, tap0, tap1, x, skip=None):
    """Kernel-only forward of :func:`fbt_recompute_scan`: ``(act, carry, coefs)``.

    ``skip`` (optional, same shape as ``x``) is added to ``act`` in the
    kernel's output store: the encoder's residual connection
    (pure.py:530-534) without a separate pass."""
    x = _c64(x)
    if x.dim() != 3:
        raise ValueError(f"expected (filters, batch, time) input, got shape {tuple(x.shape)}")
    filters, batch, time = x.shape
    C1, tap0, tap1 = _coefs(C1, tap0, tap1, filters)
    if skip is not None:
        if skip.shape != x.shape:
            raise ValueError(f"skip must have the drive's shape {tuple(x.shape)}, "
                             f"got {tuple(skip.shape)}")
        skip = _c64(skip)
    _lib.require_device(x, skip, C1)
    lib = _lib.load()
    nchunks = lib.rqf_fbt_carry_chunks(time)
    act = torch.empty_like(x)
    carry = torch.empty((filters * batch, max(nchunks, 1)), dtype=torch.complex64, device=x.device)
    if skip is None:
        rc = lib.rqf_fbt_recompute_fwd(
            _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(act),
            _lib.ptr(carry), filters, batch, time, _lib.stream_of(x))
    else:
        rc = lib.rqf_fbt_recompute_skip_fwd(
            _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(skip),
            _lib.ptr(act), _lib.ptr(carry), filters, batch, time, _lib.stream_of(x))
    _lib.check(rc, "rqf_fbt_recompute_fwd")
    return act, carry, (C1, tap0, tap1, x)


def fbt_recompute_backward_raw(C1, tap0, tap1, x, carry, grad_output):
    """Kernel-only backward of :func:`fbt_recompute_scan`: ``(gC1, gtap0, gtap1, gx)``.

    ``carry`` is the forward's ``(F*B, rqf_fbt_carry_chunks(T))`` entry-state
    tensor; every shape is checked before the launch."""
    x = _c64(x)
    if x.dim() != 3:
        raise ValueError(f"expected (filters, batch, time) input, got shape {tuple(x.shape)}")
    filters, batch, time = x.shape
    C1, tap0, tap1 = _coefs(C1, tap0, tap1, filters)
    g = _c64(grad_output)
    if g.shape != x.shape:
        raise ValueError(f"grad_output must have the input's shape {tuple(x.shape)}, "
                         f"got {tuple(g.shape)}")
    lib = _lib.load()
    want = (filters * batch, max(lib.rqf_fbt_carry_chunks(time), 1))
    if tuple(carry.shape) != want or carry.dtype != torch.complex64:
        raise ValueError(f"carry must be complex64 of shape {want}, got {carry.dtype} "
                         f"{tuple(carry.shape)}")
    carry = carry.contiguous()
    _lib.require_device(x, g, carry, C1)
    grad_z = torch.empty_like(x)
    gc1, gt0, gt1 = _bwd_grads(filters, x.device)
    n = lib.rqf_fbt_workspace(filters, batch, time)
    ws = _lib.workspace(n, x.device)
    _lib.check(
        lib.rqf_fbt_recompute_bwd(
            _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(carry),
            _lib.ptr(g), _lib.ptr(grad_z), _lib.ptr(gc1), _lib.ptr(gt0), _lib.ptr(gt1),
            filters, batch, time, _lib.ptr(ws), n, _lib.stream_of(x)),
        "rqf_fbt_recompute_bwd",
    )
    return gc1, gt0, gt1, grad_z


def fbt_recompute_backward_noalloc(C1, tap0, tap1, x, carry, grad_output, grad_z, grad_C1,
                                   grad_tap0, grad_tap1):
    """:func:`fbt_recompute_backward_raw` into caller-owned outputs, allocating
    nothing: ``rqf_fbt_recompute_bwd_noalloc`` keeps its partial sums in the
    library's static per-GPU scratch (at most ``F*B = 87381`` rows), so the
    call is usable where device allocation is not (graph capture, serving
    loops).  Every tensor must already be complex64, contiguous and on the
    device, with ``grad_z`` shaped like ``x`` and the three coefficient
    gradients shaped ``(F,)``; nothing is converted.  Calls that overlap on
    one GPU share the scratch and must be serialised by the caller."""
    tensors = dict(C1=C1, tap0=tap0, tap1=tap1, x=x, carry=carry, grad_output=grad_output,
                   grad_z=grad_z, grad_C1=grad_C1, grad_tap0=grad_tap0, grad_tap1=grad_tap1)
    for name, t in tensors.items():
        if t.dtype != torch.complex64 or not t.is_contiguous() or t.is_conj():
            raise ValueError(f"{name} must be a contiguous complex64 tensor without a "
                             "pending conjugation (nothing is converted here)")
    _lib.require_device(*tensors.values())
    if x.dim() != 3:
        raise ValueError(f"expected (filters, batch, time) input, got shape {tuple(x.shape)}")
    filters, batch, time = x.shape
    for name in ("C1", "tap0", "tap1", "grad_C1", "grad_tap0", "grad_tap1"):
        if tensors[name].shape != (filters,):
            raise ValueError(f"{name} must have shape ({filters},)")
    for name in ("grad_output", "grad_z"):
        if tensors[name].shape != x.shape:
            raise ValueError(f"{name} must have the input's shape {tuple(x.shape)}")
    lib = _lib.load()
    if tuple(carry.shape) != (filters * batch, max(lib.rqf_fbt_carry_chunks(time), 1)):
        raise ValueError("carry must be the forward's (F*B, rqf_fbt_carry_chunks(T)) entry states")
    _lib.check(
        lib.rqf_fbt_recompute_bwd_noalloc(
            _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(x), _lib.ptr(carry),
            _lib.ptr(grad_output), _lib.ptr(grad_z), _lib.ptr(grad_C1), _lib.ptr(grad_tap0),
            _lib.ptr(grad_tap1), filters, batch, time, _lib.stream_of(x)),
        "rqf_fbt_recompute_bwd_noalloc",
    )
    return grad_C1, grad_tap0, grad_tap1, grad_z


class _FBTRecompute(torch.autograd.Function):
    """Split-ReLU prospective scan that replays the raw state in the backward."""

    @staticmethod
    def forward(ctx, C1, tap0, tap1, x_fbt, skip=None):
        act, carry, (C1, tap0, tap1, x) = fbt_recompute_forward_raw(C1, tap0, tap1, x_fbt, skip)
        ctx.save_for_backward(C1, tap0, tap1, x, carry)
        ctx.has_skip = skip is not None
        return act

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        C1, tap0, tap1, x, carry = ctx.saved_tensors
        grads = fbt_recompute_backward_raw(C1, tap0, tap1, x, carry, grad_output)
        # act = split-ReLU(scan) + skip: the skip's gradient is the cotangent itself.
        return (*grads, grad_output if ctx.has_skip else None)


def fbt_recompute_scan(C1, tap0, tap1, x_fbt, skip=None):
    """Split-ReLU prospective scan; stores the output plus per-tile entry states.

    With ``skip`` (the layer input, same shape) the result is
    ``split-ReLU(scan) + skip``, the residual add fused into the kernel."""
    return _FBTRecompute.apply(C1, tap0, tap1, x_fbt, skip)


# ---------------------------------------------------------------------------
# Layer 0 on a real input: stacked real projection + recompute scan
# ---------------------------------------------------------------------------


def _pack_layer0(w_stacked):
    """Weights of ``z = A h`` for the MFMA projection GEMM: rows 2f and 2f+1 are
    ``Wr_f`` and ``Wi_f``, so the kernel writes complex row f of ``z``
    interleaved, as the recompute scan reads it."""
    from prospective_rqf_amd import projection

    f = w_stacked.shape[0] // 2
    a = torch.empty(2 * f, w_stacked.shape[1], dtype=torch.float32, device=w_stacked.device)
    a[0::2], a[1::2] = w_stacked[:f], w_stacked[f:]
    return projection._padded(a)


def _pack_layer0_dh(w_stacked):
    """Weights of ``grad_h = A [Re gz_0, Im gz_0, Re gz_1, ...]``: row k is
    ``(Wr[0,k], Wi[0,k], Wr[1,k], ...)``, i.e. ``grad_h = Re(W^H gz)``."""
    from prospective_rqf_amd import projection

    f = w_stacked.shape[0] // 2
    a = torch.empty(w_stacked.shape[1], 2 * f, dtype=torch.float32, device=w_stacked.device)
    a[:, 0::2], a[:, 1::2] = w_stacked[:f].T, w_stacked[f:].T
    return projection._padded(a)


# Widest real inputs whose input gradient, and whose weight gradient, the
# one-pass kernel (rqf_layer0_grads) serves.
_LAYER0_NARROW_H = 16
_LAYER0_NARROW_W = 2


def _layer0_grads(w, gz, h, need_w, need_h):
    """``(grad_w_stacked, grad_h)`` of ``z = (Wr + i Wi) h`` from ``gz`` (F, n):
    ``[Re gz; Im gz] h^T`` and ``Re(W^H gz)``.  One pass over ``gz`` where the
    input is narrow enough; otherwise the MFMA projection GEMM for ``grad_h``
    and a real split-K GEMM on ``gz``'s interleaved storage for the weights."""
    from prospective_rqf_amd import projection

    filters, cols = gz.shape
    width = h.shape[0]
    fused_h = need_h and width <= _LAYER0_NARROW_H
    fused_w = need_w and width <= _LAYER0_NARROW_W
    grad_w = grad_h = None
    if fused_h or fused_w:
        lib = _lib.load()
        if fused_h:
            grad_h = torch.empty(width, cols, dtype=torch.float32, device=gz.device)
        if fused_w:
            grad_w = torch.empty(2 * filters, width, dtype=torch.float32, device=gz.device)
        n = lib.rqf_layer0_grads_workspace(filters, width, cols) if fused_w else 0
        ws = _lib.workspace(n, gz.device)
        _lib.check(lib.rqf_layer0_grads(_lib.ptr(w), _lib.ptr(gz), _lib.ptr(h), _lib.ptr(grad_h),
                                        _lib.ptr(grad_w), filters, width, cols, _lib.ptr(ws), n,
                                        _lib.stream_of(gz)), "rqf_layer0_grads")
    if need_h and grad_h is None:
        grad_h = projection._proj_gemm(_pack_layer0_dh(w), gz, None, cols, 0, width,
                                       gz.device)[1]
    if need_w and grad_w is None:
        hx = torch.zeros(2 * width, 2 * cols, dtype=torch.float32, device=h.device)
        hx[:width, 0::2] = h
        hx[width:, 1::2] = h
        g = projection.weight_grad(torch.view_as_real(gz).reshape(filters, 2 * cols), hx)
        grad_w = torch.cat((g[:, :width], g[:, width:]))
    return grad_w, grad_h


class _Layer0RealScan(torch.autograd.Function):
    """Real-input layer-0 projection feeding the split-ReLU recompute scan
    (rqf_models/ops/fbt_scan_kernel.py:899-1002).

    The reference writes the stacked real GEMM ``[Wr; Wi] @ h`` to planar
    ``(zr, zi)`` buffers and runs planar twins of the recompute kernels.  Here,
    with one input feature (the raw waveform), the scan kernels form the drive
    ``z = (Wr + i Wi) x`` themselves (``rqf_fbt_layer0_fwd`` / ``_bwd``): no
    GEMM and no drive tensor.  Wider inputs go through the MFMA projection
    GEMM (``rqf_proj_gemm``), which writes ``z`` interleaved, so the ordinary
    recompute kernels consume it.  The backward reads ``grad_z``
    where the scan leaves it: ``grad_h = [Wr; Wi]^T [Re gz; Im gz]`` and
    ``grad_w_stacked = [Re gz; Im gz] h^T`` in one pass for narrow inputs
    (``rqf_layer0_grads``: up to 16 wide for grad_h, 2 for the weights, which
    covers the raw waveform), else a GEMM each."""

    @staticmethod
    def forward(ctx, w_stacked, h_real, C1, tap0, tap1, batch):
        from prospective_rqf_amd import projection

        if w_stacked.dim() != 2 or w_stacked.shape[0] % 2 or w_stacked.is_complex():
            raise ValueError("w_stacked must be a real (2*num_filters, d_model) matrix, got "
                             f"{tuple(w_stacked.shape)} {w_stacked.dtype}")
        if h_real.dim() != 2 or h_real.is_complex() or h_real.shape[0] != w_stacked.shape[1]:
            raise ValueError(f"h_real must be a real ({w_stacked.shape[1]}, batch*time) matrix, "
                             f"got {tuple(h_real.shape)} {h_real.dtype}")
        batch = int(batch)
        if batch < 1 or h_real.shape[1] % batch:
            raise ValueError(f"batch {batch} does not divide the {h_real.shape[1]} columns")
        _lib.require_device(w_stacked, h_real)
        w = w_stacked.detach().to(torch.float32).contiguous()
        h = h_real.detach().to(torch.float32).contiguous()
        filters, cols = w.shape[0] // 2, h.shape[1]
        time = cols // batch
        if w.shape[1] == 1:
            # One input feature: the scan forms z = (Wr + i Wi) x itself.
            C1, tap0, tap1 = _coefs(C1, tap0, tap1, filters)
            _lib.require_device(C1)
            wz = torch.complex(w[:filters, 0], w[filters:, 0]).contiguous()
            lib = _lib.load()
            act = torch.empty(filters, batch, time, dtype=torch.complex64, device=h.device)
            carry = torch.empty((filters * batch, max(lib.rqf_fbt_carry_chunks(time), 1)),
                                dtype=torch.complex64, device=h.device)
            _lib.check(lib.rqf_fbt_layer0_fwd(
                _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(wz), _lib.ptr(h),
                _lib.ptr(act), _lib.ptr(carry), filters, batch, time, _lib.stream_of(h)),
                "rqf_fbt_layer0_fwd")
            ctx.save_for_backward(w, h, wz, carry, C1, tap0, tap1)
            ctx.fused = True
            return act
        z, _ = projection._proj_gemm(_pack_layer0(w), None, h, cols, filters, 0, h.device)
        z = z.view(filters, batch, time)
        act, carry, (C1, tap0, tap1, z) = fbt_recompute_forward_raw(C1, tap0, tap1, z)
        ctx.save_for_backward(w, h, z, carry, C1, tap0, tap1)
        ctx.fused = False
        return act

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_act):
        from prospective_rqf_amd import projection

        w, h, z, carry, C1, tap0, tap1 = ctx.saved_tensors
        filters, cols = w.shape[0] // 2, h.shape[1]
        if ctx.fused:  # z holds the drive weight wz; the scan forms the drive from h
            g = _c64(grad_act)
            batch = carry.shape[0] // filters
            if g.shape != (filters, batch, cols // batch):
                raise ValueError(f"grad_output must have shape {(filters, batch, cols // batch)}")
            lib = _lib.load()
            gz = torch.empty(filters, cols, dtype=torch.complex64, device=h.device)
            gc1, gt0, gt1 = _bwd_grads(filters, h.device)
            n = lib.rqf_fbt_workspace(filters, batch, cols // batch)
            ws = _lib.workspace(n, h.device)
            _lib.check(lib.rqf_fbt_layer0_bwd(
                _lib.ptr(C1), _lib.ptr(tap0), _lib.ptr(tap1), _lib.ptr(z), _lib.ptr(h),
                _lib.ptr(carry), _lib.ptr(g), _lib.ptr(gz), _lib.ptr(gc1), _lib.ptr(gt0),
                _lib.ptr(gt1), filters, batch, cols // batch, _lib.ptr(ws), n,
                _lib.stream_of(h)), "rqf_fbt_layer0_bwd")
        else:
            gc1, gt0, gt1, gz = fbt_recompute_backward_raw(C1, tap0, tap1, z, carry, grad_act)
        gz = gz.view(filters, cols)
        grad_w, grad_h = _layer0_grads(w, gz, h, ctx.needs_input_grad[0],
                                       ctx.needs_input_grad[1])
        return grad_w, grad_h, gc1, gt0, gt1, None


def fbt_layer0_real_scan(w_stacked, h_real, C1, tap0, tap1, batch):
    """Real-input layer-0 projection + split-ReLU prospective scan
    (rqf_models/ops/fbt_scan_kernel.py:1005-1032): ``(2F, D)`` real
    ``[Wr; Wi]``, ``(D, batch*time)`` real ``h``, complex ``(F,)`` coefficients;
    returns the complex ``(F, batch, time)`` activated output, equal up to fp32
    summation order to ``fbt_recompute_scan(C1, tap0, tap1, (Wr + i Wi) @ h)``."""
    return _Layer0RealScan.apply(w_stacked, h_real, C1, tap0, tap1, batch)

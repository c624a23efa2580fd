"""Host side of the fused selective scan: allocation and launch.

Mirrors ``selective_forward`` / ``selective_backward`` of the reference
(rqf_models/ops/selective_scan_kernel.py:491-561): same arguments, same
returned tensors and shapes.  The compute runs in ``librqf_hip.so``
(``rqf_selective_fwd`` / ``rqf_selective_bwd``).
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from prospective_rqf_amd import _lib


def _real_ptr(t: torch.Tensor | None):
    """Pointer to the interleaved (re, im) storage of a complex tensor."""
    if t is None:
        return None
    if t.is_conj():
        t = t.resolve_conj()
    return _lib.ptr(t)


# Validated warp-group tensors: id(caller's tensor) -> (weakref to it, its
# version counter, number of warp rows, device, device int64 copy, order).
# An entry counts only while the weak reference still resolves to the very
# tensor looked up and its version is unchanged, so a new tensor that reuses
# a freed tensor's id or address, or an in-place edit (through any view),
# is validated afresh.
_VALID_GROUPS: dict = {}


def _check_groups(groups: torch.Tensor, n_groups: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Validate the caller's ``groups`` tensor (F,) against ``n_groups`` warp rows.

    The kernels read ``warp_logits[groups[f]]``, so every entry must lie in
    ``[0, n_groups)``; otherwise ``ValueError`` is raised before any launch
    (the reference's controller builds them as ``rank * G // F``,
    rqf_models/backbones/rqf/selective.py:164-165).  Returns the int64 copy on
    ``device`` that the kernels read and the channel visiting order (stable
    argsort of the groups, int32) that keeps each group's channels adjacent.
    Both are cached per tensor object and version."""
    key = id(groups)
    hit = _VALID_GROUPS.get(key)
    if (hit is not None and hit[0]() is groups and hit[1] == groups._version
            and hit[2] == n_groups and hit[3] == device):
        return hit[4], hit[5]
    dev_groups = groups.to(device=device, dtype=torch.int64).contiguous()
    if dev_groups.numel():
        lo, hi = torch.aminmax(dev_groups)
        if int(lo) < 0 or int(hi) >= n_groups:
            raise ValueError(f"groups must index the {n_groups} warp-logit rows, "
                             f"got values in [{int(lo)}, {int(hi)}]")
    order = torch.argsort(dev_groups, stable=True).to(torch.int32).contiguous()
    for k in [k for k, v in _VALID_GROUPS.items() if v[0]() is None]:
        del _VALID_GROUPS[k]
    if len(_VALID_GROUPS) > 64:
        _VALID_GROUPS.clear()
    try:
        ref = weakref.ref(groups)
    except TypeError:  # not weak-referenceable: validate on every call
        return dev_groups, order
    _VALID_GROUPS[key] = (ref, groups._version, n_groups, device, dev_groups, order)
    return dev_groups, order


def inputs_struct(z: torch.Tensor, inputs) -> tuple[_lib.SelectiveInputsStruct, list]:
    """Pack ``SelectiveScanInputs`` into the C struct; returns (struct, keep-alive list)."""
    f, b, t = z.shape
    o = inputs.options
    has_gamma, has_warp, has_write = bool(o[0]), bool(o[1]), bool(o[2])

    dev = z.device

    def vec(v):
        if v.dtype is torch.float32 and v.device == dev and v.is_contiguous():
            return v  # the common case, without a conversion call
        return v.to(device=dev, dtype=torch.float32).contiguous()

    gl = vec(inputs.gamma_logits) if has_gamma else None
    dl = vec(inputs.warp_logits) if has_warp else None
    wl = vec(inputs.write_logits) if has_write else None
    params = [vec(getattr(inputs, n)) for n in (
        "bias", "theta", "minimum", "span", "step", "horizon", "theta_minimum", "theta_maximum")]
    for name, v, rows in (("gamma_logits", gl, f), ("write_logits", wl, f)):
        if v is not None and tuple(v.shape) != (rows, b, t):
            raise ValueError(f"{name} must have shape {(rows, b, t)}, got {tuple(v.shape)}")
    g = 0
    groups = order = None
    if dl is not None:
        if dl.dim() != 3 or tuple(dl.shape[1:]) != (b, t):
            raise ValueError(f"warp_logits must have shape (G, {b}, {t}), got {tuple(dl.shape)}")
        g = dl.shape[0]
        if g < 1:
            raise ValueError("the warp head needs at least one warp-logit row")
        if not isinstance(inputs.groups, torch.Tensor) or tuple(inputs.groups.shape) != (f,):
            raise ValueError("groups must be a (F,) index tensor when the warp head is on")
        if inputs.groups.is_complex() or inputs.groups.is_floating_point():
            raise ValueError("groups must be an integer index tensor")
        groups, order = _check_groups(inputs.groups, g, dev)
    for name, v in zip(("bias", "theta", "minimum", "span", "step", "horizon",
                        "theta_minimum", "theta_maximum"), params):
        if v.shape != (f,):
            raise ValueError(f"{name} must have shape ({f},), got {tuple(v.shape)}")
    s = _lib.SelectiveInputsStruct(
        f, b, t, g,
        *(None if v is None else v.data_ptr() for v in (gl, dl, wl)),
        *(v.data_ptr() for v in params),
        None if groups is None else groups.data_ptr(),
        int(has_gamma), int(has_warp), int(has_write), int(bool(o[3])),
        float(o[4]), float(o[5]),
        int(bool(o[6])), int(bool(o[7])), int(bool(o[8])),
        float(o[9]), float(o[10]),
        int(bool(o[11])),
        None if order is None else order.data_ptr(),
    )
    return s, [gl, dl, wl, groups, order, *params]


def _check_chunk(chunk) -> int:
    """The chunk must be a positive power of two (selective_scan.py:213-216)."""
    c = int(chunk)
    if c <= 0 or c & (c - 1):
        raise ValueError(f"chunk must be a positive power of two, got {chunk}")
    return c


def _check_drive(z) -> None:
    if z.dtype != torch.complex64:
        raise TypeError("the selective scan expects a complex64 drive")
    if z.dim() != 3:
        raise ValueError(f"expected a (filters, batch, time) drive, got shape {tuple(z.shape)}")


def _check_backward(z, entries, gy, gx, chunk) -> None:
    """Shapes the backward kernel reads through: every cotangent covers the
    drive's (F, B, T) and ``entries`` holds one complex64 state per (row,
    chunk), the forward's ``(F*B, ceil(T/chunk))`` (the reference takes the
    chunk count from ``entries.shape[1]``, selective_scan_kernel.py:545)."""
    f, b, t = z.shape
    for name, g in (("gy", gy), ("gx", gx)):
        if g is not None and tuple(g.shape) != (f, b, t):
            raise ValueError(f"{name} must have the drive's shape {(f, b, t)}, "
                             f"got {tuple(g.shape)}")
    want = (f * b, -(-t // chunk))
    if entries.dtype != torch.complex64 or tuple(entries.shape) != want:
        raise ValueError(f"entries must be complex64 of shape {want} (one state per row and "
                         f"chunk of {chunk}), got {entries.dtype} {tuple(entries.shape)}")


def selective_forward(z, inputs, activate, write_raw, chunk, skip=None):
    """Fused forward: returns ``(raw|None, act|None, entries)``.

    z: (F,B,T) complex64 drive.  entries: (F*B, ceil(T/chunk)) complex64 state
    entering each chunk (consumed by :func:`selective_backward`).  ``skip``
    (optional, like z) is added to both outputs in the kernel's stores: the
    encoder's residual connection (pure.py:486-496) without separate passes;
    entries stay the scan's own states.
    """
    _check_drive(z)
    chunk = _check_chunk(chunk)
    if not (activate or write_raw):
        raise ValueError("selective_forward needs activate or write_raw")
    if skip is not None and skip.shape != z.shape:
        raise ValueError(f"skip must have the drive's shape {tuple(z.shape)}, "
                         f"got {tuple(skip.shape)}")
    _lib.require_device(z, skip)
    z = z.resolve_conj().contiguous()
    if skip is not None:
        skip = skip.to(torch.complex64).resolve_conj().contiguous()
    f, b, t = z.shape
    nc = -(-t // chunk)
    raw = torch.empty_like(z) if write_raw else None
    act = torch.empty_like(z) if activate else None
    entries = torch.empty((f * b, nc), dtype=z.dtype, device=z.device)
    s, keep = inputs_struct(z, inputs)
    lib = _lib.load()
    if skip is None:
        rc = lib.rqf_selective_fwd(ctypes.byref(s), _real_ptr(z), chunk, _real_ptr(raw),
                                   _real_ptr(act), _real_ptr(entries), _lib.stream_of(z))
    else:
        rc = lib.rqf_selective_skip_fwd(ctypes.byref(s), _real_ptr(z), chunk, _real_ptr(skip),
                                        _real_ptr(raw), _real_ptr(act), _real_ptr(entries),
                                        _lib.stream_of(z))
    _lib.check(rc, "rqf_selective_fwd")
    del keep
    return raw, act, entries


def selective_backward(z, inputs, entries, gy, gx, activate, truncated, chunk):
    """Fused backward: ``(dz, dzw, dg|None, dd_group|None, dw|None, dbias, dtheta)``.

    ``dzw`` is the same tensor as ``dz`` unless ``truncated``.  Every shape
    is checked on the host before any launch (``ValueError``).
    """
    _check_drive(z)
    chunk = _check_chunk(chunk)
    _check_backward(z, entries, gy, gx, chunk)
    _lib.require_device(z, entries, gy, gx)
    z = z.resolve_conj().contiguous()
    f, b, t = z.shape
    o = inputs.options
    dz = torch.empty_like(z)
    dzw = torch.empty_like(z) if truncated else dz
    s, keep = inputs_struct(z, inputs)
    # The head gradients are consecutive row ranges of one buffer, in the
    # selector's head order (gamma, warp, write; selective.py:211-217), so the
    # projection backward reads them as one (rows, B*T) matrix without a copy.
    rows = (f if o[0] else 0, s.G if o[1] else 0, f if o[2] else 0)
    heads = torch.empty((sum(rows), b, t), dtype=torch.float32, device=z.device)
    dg, dd, dw = (heads[a:a + r] if r and o[i] else None
                  for i, (a, r) in enumerate(zip((0, rows[0], rows[0] + rows[1]), rows)))
    dbias = torch.empty(f, dtype=torch.float32, device=z.device)
    dtheta = torch.empty(f, dtype=torch.float32, device=z.device)
    gy = None if gy is None else gy.resolve_conj().to(torch.complex64).contiguous()
    gx = None if gx is None else gx.resolve_conj().to(torch.complex64).contiguous()
    entries = entries.contiguous()
    lib = _lib.load()
    nbytes = lib.rqf_selective_bwd_workspace(ctypes.byref(s), chunk)
    ws = _lib.workspace(nbytes, z.device)
    _lib.check(
        lib.rqf_selective_bwd(
            ctypes.byref(s), _real_ptr(z), _real_ptr(entries), chunk, _real_ptr(gy),
            _real_ptr(gx), int(bool(activate)), int(bool(truncated)), _real_ptr(dz),
            _real_ptr(dzw), _lib.ptr(dg), _lib.ptr(dd), _lib.ptr(dw), _lib.ptr(dbias),
            _lib.ptr(dtheta), _lib.ptr(ws), nbytes, _lib.stream_of(z),
        ),
        "rqf_selective_bwd",
    )
    del keep
    return dz, dzw, dg, dd, dw, dbias, dtheta

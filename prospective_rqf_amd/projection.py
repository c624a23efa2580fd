"""Projection GEMMs around the scans: drive ``z = W h`` and selector logits.

The reference computes these with plain ``torch.matmul`` calls:
``_SelectiveLayerScan`` (rqf_models/ops/selective_scan.py:117-118, 144-146),
``_SplitProjection`` (rqf_models/backbones/rqf/selective.py:78-97) and, through
autograd, the FBT stack's ``W_c @ h`` (rqf_models/backbones/rqf/pure.py:222-223).
Their weight gradients reduce over batch*time (~1e6 columns) into a small
(out, in) matrix.  A single GEMM of that shape has only a handful of output
tiles to spread over the 256 CUs.  On MI355X the complex64 one runs at
2.4 TFLOP/s: ``dz @ x.mH`` takes 222 ms at B=64, T=16000, H=256, against
2.8 ms for the scan's whole backward.  Here the reduction is split into
``splits`` batched GEMMs whose partial products are summed.  That takes 3.9 ms
there, and shortens every fp32 dot product, which also lowers the error.

The split weight gradients are plain library GEMMs (rocBLAS/hipBLASLt through
torch); only the reduction's shape is chosen here.  ``fused_forward`` and
``fused_dx`` run the hand-written MFMA kernel ``rqf_proj_gemm`` (csrc/proj.hip):
- the drive GEMM and the selector projection stacked into one real GEMM over
  the interleaved complex input, with no ``[Re; Im]`` copy;
- their input gradients likewise stacked, reading ``dz`` and the logit
  gradients where they lie.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

# Batched GEMMs the reduction is split into, and the least columns per split.
# Measured on MI355X for (out, in, batch*time) = (256, 256, 1.02e6):
# 16 -> 14.0 ms, 32 -> 7.0, 64 -> 3.9, 128 -> 4.0, 256 -> 4.6; at (48, 48, 5.1e5):
# 64 -> 1.78 ms, 128 -> 0.17, 256 -> 0.18.
WGRAD_SPLITS = 128
WGRAD_MIN_COLUMNS = 1024


def weight_grad(g: Tensor, x: Tensor, splits: int = WGRAD_SPLITS) -> Tensor:
    """``g @ x^H`` (``g @ x.T`` for real tensors) for ``g`` (M, N) and ``x`` (K, N),
    with the reduction over N split into at most ``splits`` batched GEMMs.

    The partial products are summed in a fixed order, so the result is
    deterministic.  The last ``N % splits`` columns, if any, go through one
    more GEMM."""
    if g.dim() != 2 or x.dim() != 2 or g.shape[1] != x.shape[1]:
        raise ValueError(f"weight_grad needs (M, N) and (K, N), got {tuple(g.shape)} and "
                         f"{tuple(x.shape)}")
    g = g.contiguous()
    x = x.contiguous()
    m, n = g.shape
    k_rows = x.shape[0]
    s = min(int(splits), n // WGRAD_MIN_COLUMNS)
    if s < 2:
        return g @ (x.mH if x.is_complex() else x.T)
    cols = n // s
    main = s * cols
    # (s, M, cols) and (s, K, cols) views: split j covers columns [j*cols, (j+1)*cols).
    a = g.as_strided((s, m, cols), (cols, n, 1))
    b = x.as_strided((s, k_rows, cols), (cols, n, 1))
    out = torch.bmm(a, b.mH if x.is_complex() else b.transpose(1, 2)).sum(0)
    if main < n:
        tail = x[:, main:]
        out = out + g[:, main:] @ (tail.mH if x.is_complex() else tail.T)
    return out


class _Projection(torch.autograd.Function):
    """``W @ h`` with the split weight gradient."""

    @staticmethod
    def forward(ctx, weight, h):
        ctx.save_for_backward(weight, h)
        with torch.autocast(h.device.type, enabled=False):
            return weight @ h

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        weight, h = ctx.saved_tensors
        dw = dh = None
        with torch.autocast(h.device.type, enabled=False):
            if ctx.needs_input_grad[0]:
                dw = weight_grad(grad, h)
            if ctx.needs_input_grad[1]:
                dh = (weight.mH if weight.is_complex() else weight.T) @ grad
        return dw, dh


def project(weight: Tensor, h: Tensor) -> Tensor:
    """``weight @ h`` for a 2-D ``h`` (in, batch*time), differentiable, with the
    split weight gradient.  Drop-in for the FBT stack's ``W_c @ h``
    (pure.py:222-223)."""
    return _Projection.apply(weight, h)


class _SplitProjection(torch.autograd.Function):
    """Mirror of the reference's ``_SplitProjection`` (selective.py:78-97):
    ``(weights @ v).split(sizes)``, with the split weight gradient."""

    @staticmethod
    def forward(ctx, v, weights, sizes):
        ctx.save_for_backward(v, weights)
        ctx.sizes = sizes
        ctx.set_materialize_grads(False)
        return (weights @ v).split(sizes)

    @staticmethod
    def backward(ctx, *grads):
        v, weights = ctx.saved_tensors
        grad = stacked([
            g if g is not None else v.new_zeros((n, v.shape[1]))
            for g, n in zip(grads, ctx.sizes)
            if n
        ])
        with torch.autocast(v.device.type, enabled=False):
            return weights.T @ grad, weight_grad(grad, v), None


def split_projection(v: Tensor, weights: Tensor, sizes) -> tuple[Tensor, ...]:
    """``(weights @ v).split(sizes)`` (selective.py:217), differentiable."""
    return _SplitProjection.apply(v, weights, tuple(sizes))


# ---------------------------------------------------------------------------
# Fused projections on MFMA (csrc/proj.hip, rqf_proj_gemm)
# ---------------------------------------------------------------------------

_PK, _PM = 16, 128  # the kernel's K stage and M tile


def _padded(a: Tensor) -> Tensor:
    """(M, K) fp32 weight rows -> the kernel's (k_pad, m_pad) k-major layout."""
    m, k = a.shape
    out = torch.zeros((k + _PK - 1) // _PK * _PK, (m + _PM - 1) // _PM * _PM,
                      dtype=torch.float32, device=a.device)
    out[:k, :m] = a.T
    return out


def pack_forward(weight: Tensor, heads: Tensor | None) -> Tensor:
    """A of ``[z; logits] = A [x_0.re, x_0.im, x_1.re, ...]``: rows 2f, 2f+1 give
    Re z_f, Im z_f of ``z = weight @ x``; then one row per selector head row j,
    ``heads[j] @ [Re x; Im x]`` (selective.py:205-217)."""
    f, d = weight.shape
    wr, wi = weight.real.float(), weight.imag.float()
    ml = 0 if heads is None else heads.shape[0]
    a = torch.empty(2 * f + ml, 2 * d, dtype=torch.float32, device=weight.device)
    a[0:2 * f:2, 0::2], a[0:2 * f:2, 1::2] = wr, -wi
    a[1:2 * f:2, 0::2], a[1:2 * f:2, 1::2] = wi, wr
    if ml:
        a[2 * f:, 0::2], a[2 * f:, 1::2] = heads[:, :d].float(), heads[:, d:].float()
    return _padded(a)


def pack_dx(weight: Tensor, heads: Tensor | None) -> Tensor:
    """A of ``dx = A [dz_0.re, dz_0.im, ..., g_0, g_1, ...]``: rows 2d, 2d+1 give
    Re, Im of ``weight.mH @ dz + complex(dv[:D], dv[D:])`` with ``dv = heads.T @ g``
    (selective_scan.py:144, selective.py:96)."""
    f, d = weight.shape
    wr, wi = weight.real.float(), weight.imag.float()
    ml = 0 if heads is None else heads.shape[0]
    a = torch.empty(2 * d, 2 * f + ml, dtype=torch.float32, device=weight.device)
    a[0::2, 0:2 * f:2], a[0::2, 1:2 * f:2] = wr.T, wi.T
    a[1::2, 0:2 * f:2], a[1::2, 1:2 * f:2] = -wi.T, wr.T
    if ml:
        a[0::2, 2 * f:], a[1::2, 2 * f:] = heads[:, :d].T.float(), heads[:, d:].T.float()
    return _padded(a)


def _proj_gemm(packed: Tensor, b_cplx: Tensor | None, b_real: Tensor | None, n: int,
               out_cplx_rows: int, out_real_rows: int, device, bias: Tensor | None = None,
               relu: bool = False):
    from prospective_rqf_amd import _lib

    lib = _lib.load()
    out_c = (torch.empty(out_cplx_rows, n, dtype=torch.complex64, device=device)
             if out_cplx_rows else None)
    out_r = (torch.empty(out_real_rows, n, dtype=torch.float32, device=device)
             if out_real_rows else None)
    a = _lib.ProjGemmArgs()
    a.weights, a.k_pad, a.m_pad = packed.data_ptr(), packed.shape[0], packed.shape[1]
    a.b_cplx = 0 if b_cplx is None else torch.view_as_real(b_cplx).data_ptr()
    a.b_cplx_rows = 0 if b_cplx is None else b_cplx.shape[0]
    a.b_real = 0 if b_real is None else b_real.data_ptr()
    a.b_real_rows = 0 if b_real is None else b_real.shape[0]
    a.n = n
    a.out_cplx = 0 if out_c is None else torch.view_as_real(out_c).data_ptr()
    a.out_cplx_rows = out_cplx_rows
    a.out_real = 0 if out_r is None else out_r.data_ptr()
    a.out_real_rows = out_real_rows
    a.out_real_bias = 0 if bias is None else bias.data_ptr()
    a.out_real_relu = int(bool(relu))
    _lib.check(lib.rqf_proj_gemm(ctypes.byref(a), _lib.stream_of(packed)), "rqf_proj_gemm")
    return out_c, out_r


def stacked(blocks: list) -> Tensor | None:
    """The row blocks as one (rows, N) tensor: their common storage when they are
    consecutive row ranges of one contiguous buffer (as ``selective_backward``
    allocates the logit gradients), else a concatenation."""
    blocks = [b for b in blocks if b is not None and b.shape[0]]
    if not blocks:
        return None
    flat = [b.reshape(b.shape[0], -1) if b.dim() != 2 else b for b in blocks]
    base = flat[0]
    storage = base.untyped_storage()
    same = all(b.is_contiguous() and b.dtype == base.dtype and b.shape[1] == base.shape[1]
               and b.untyped_storage().data_ptr() == storage.data_ptr() for b in flat)
    if same and all(flat[i + 1].data_ptr() == flat[i].data_ptr() + flat[i].numel() * flat[i].element_size()
                    for i in range(len(flat) - 1)):
        rows = sum(b.shape[0] for b in flat)
        return base.as_strided((rows, base.shape[1]), (base.shape[1], 1))
    return torch.cat(flat, 0)


def fused_forward(x: Tensor, weight: Tensor, heads: Tensor | None = None,
                  packed: Tensor | None = None):
    """``z = weight @ x`` (complex64, (F, N)) and ``heads @ [Re x; Im x]`` (fp32,
    (rows, N), or None) from one pass over ``x`` (D, N) complex64."""
    from prospective_rqf_amd import _lib

    _lib.require_device(x, weight, heads)
    if x.dtype != torch.complex64 or weight.dtype != torch.complex64:
        raise TypeError("fused_forward takes complex64 x and weight")
    x = x.resolve_conj().contiguous()
    if packed is None:
        packed = pack_forward(weight, heads)
    ml = 0 if heads is None else heads.shape[0]
    return _proj_gemm(packed, x, None, x.shape[1], weight.shape[0], ml, x.device)


def fused_dx(dz: Tensor, grads: list, weight: Tensor, heads: Tensor | None = None,
             packed: Tensor | None = None) -> Tensor:
    """``weight.mH @ dz + complex(dv[:D], dv[D:])``, ``dv = heads.T @ g`` with ``g``
    the fp32 row blocks ``grads`` stacked (rows summing to ``heads.shape[0]``), in
    one pass over ``dz`` (F, N) complex64 and ``g``.  Blocks that are consecutive
    row ranges of one buffer are read in place."""
    from prospective_rqf_amd import _lib

    _lib.require_device(dz, weight, heads, *grads)
    dz = dz.resolve_conj().contiguous()
    g = stacked([b.float() for b in grads])
    rows = 0 if g is None else g.shape[0]
    if heads is None and rows:
        raise ValueError("logit gradients given without selector heads")
    if heads is not None and rows != heads.shape[0]:
        raise ValueError("logit gradient rows must match the selector heads")
    if packed is None:
        packed = pack_dx(weight, heads)
    out, _ = _proj_gemm(packed, dz, g, dz.shape[1], weight.shape[1], 0, dz.device)
    return out

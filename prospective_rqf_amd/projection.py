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

These are plain library GEMMs (rocBLAS/hipBLASLt through torch); only the
reduction's shape is chosen here.
"""

from __future__ import annotations

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
        grad = torch.cat(
            [
                g if g is not None else v.new_zeros((n, v.shape[1]))
                for g, n in zip(grads, ctx.sizes)
                if n
            ]
        )
        with torch.autocast(v.device.type, enabled=False):
            return weights.T @ grad, weight_grad(grad, v), None


def split_projection(v: Tensor, weights: Tensor, sizes) -> tuple[Tensor, ...]:
    """``(weights @ v).split(sizes)`` (selective.py:217), differentiable."""
    return _SplitProjection.apply(v, weights, tuple(sizes))

"""Per-timestep ``[Re; Im]`` MLP readout on complex features.

Mirrors the head of the reference's ``ComplexReadoutClassifier``
(train.py:74-136).  Per time step the logits are
``W2 relu(W1 [Re f; Im f] + b1) + b2``, or ``W1 [Re f; Im f] + b1`` with no
hidden layer, and they are mean-pooled over time outside training.

It runs on the channel-outermost (F, B*T) features the FBT stack produces
(pure.py:510-536).  The reference first permutes them back to (B, T, F)
(pure.py:536) and concatenates real and imaginary parts (train.py:130); here
the first layer is one MFMA GEMM (``rqf_proj_gemm``) that reads the
interleaved complex features in place, with the bias and the ReLU fused into
its stores.  Dropout is the identity, as in evaluation; training with dropout
keeps the reference's module.
"""

from __future__ import annotations

import torch
from torch import Tensor

from prospective_rqf_amd.projection import _padded, _proj_gemm, weight_grad


def pack_hidden(w1: Tensor) -> Tensor:
    """A of ``W1 [Re f; Im f]`` over the interleaved K order (re f_0, im f_0, ...)."""
    h, f2 = w1.shape
    f = f2 // 2
    a = torch.empty(h, f2, dtype=torch.float32, device=w1.device)
    a[:, 0::2], a[:, 1::2] = w1[:, :f].float(), w1[:, f:].float()
    return _padded(a)


def pack_feature_grad(w1: Tensor) -> Tensor:
    """A of the feature gradient ``W1^T dh`` as complex rows: row 2f is its real
    part ``sum_h W1[h, f] dh_h``, row 2f + 1 its imaginary part
    ``sum_h W1[h, F + f] dh_h``."""
    h, f2 = w1.shape
    f = f2 // 2
    a = torch.empty(f2, h, dtype=torch.float32, device=w1.device)
    a[0::2], a[1::2] = w1[:, :f].T.float(), w1[:, f:].T.float()
    return _padded(a)


class _ComplexReadout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, w1, b1, w2, b2):
        n = feats.shape[1]
        relu = w2 is not None
        _, out = _proj_gemm(pack_hidden(w1), feats, None, n, 0, w1.shape[0], feats.device,
                            bias=b1.float().contiguous(), relu=relu)
        if relu:
            logits = torch.addmm(b2.float()[:, None], w2.float(), out)
        else:
            logits = out
        ctx.save_for_backward(feats, w1, w2, out if relu else None)
        return logits

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dlogits):
        feats, w1, w2, hidden = ctx.saved_tensors
        dlogits = dlogits.float().contiguous()
        dw2 = db2 = None
        if w2 is not None:
            dw2 = weight_grad(dlogits, hidden)
            db2 = dlogits.sum(1)
            dh = (w2.float().T @ dlogits).mul_(hidden > 0)
        else:
            dh = dlogits
        db1 = dh.sum(1)
        v = torch.cat((feats.real, feats.imag), 0)
        dw1 = weight_grad(dh, v)
        dfeats = None
        if ctx.needs_input_grad[0]:
            dfeats, _ = _proj_gemm(pack_feature_grad(w1), None, dh, feats.shape[1],
                                   feats.shape[0], 0, feats.device)
        return dfeats, dw1, db1, dw2, db2


def complex_readout(feats: Tensor, w1: Tensor, b1: Tensor, w2: Tensor | None = None,
                    b2: Tensor | None = None, pool: bool = True) -> Tensor:
    """Logits of the per-timestep readout on FBT-layout features.

    ``feats``: (F, B, T) complex64, channel outermost.  ``w1`` (H, 2F), ``b1`` (H)
    and, with a hidden layer, ``w2`` (C, H), ``b2`` (C), as ``nn.Linear`` stores
    them.  Returns (B, C) mean-pooled logits, or (B, T, C) with ``pool=False``
    (the per-step-loss training contract, train.py:131-134).
    """
    from prospective_rqf_amd import _lib

    _lib.require_device(feats, w1, b1, w2, b2)
    if feats.dtype != torch.complex64:
        raise TypeError("complex_readout takes complex64 features")
    if (w2 is None) != (b2 is None):
        raise ValueError("w2 and b2 go together")
    f, b, t = feats.shape
    if w1.shape[1] != 2 * f:
        raise ValueError(f"w1 has {w1.shape[1]} inputs for {f} complex features")
    logits = _ComplexReadout.apply(feats.resolve_conj().contiguous().reshape(f, b * t), w1, b1,
                                   w2, b2)
    logits = logits.reshape(-1, b, t)
    return logits.mean(-1).T if pool else logits.permute(1, 2, 0)

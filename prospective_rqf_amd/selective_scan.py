"""Selective scan autograd boundary on HIP devices.

Mirrors the kernel-side half of rqf_models/ops/selective_scan.py:
``SelectiveScanInputs`` (:10-23), ``_SelectiveLayerScan`` (:107-170) and the
eligible branch of ``selective_layer_scan`` (:173-227), with the HIP library
in place of the Triton kernels.

What is deliberately not here: the reference's PyTorch recurrence
(``reference_layer_scan``), which the reference runs for ineligible inputs
(CPU tensors, ``use_kernel=False``).  That path stays in the host framework;
this module raises for such inputs instead of substituting a slow copy, so a
kernel result can never silently come from PyTorch.
"""

from __future__ import annotations

from typing import NamedTuple

import torch
from torch import Tensor

from prospective_rqf_amd import _lib
from prospective_rqf_amd.projection import weight_grad
from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward


class SelectiveScanInputs(NamedTuple):
    """Same fields and order as the reference (rqf_models/ops/selective_scan.py:10-23)."""

    gamma_logits: Tensor
    warp_logits: Tensor
    write_logits: Tensor
    bias: Tensor
    theta: Tensor
    groups: Tensor | None
    minimum: Tensor
    span: Tensor
    step: Tensor
    horizon: Tensor
    theta_minimum: Tensor
    theta_maximum: Tensor
    options: tuple


def default_chunk(time: int) -> int:
    """``min(256, next_pow2(T))`` (rqf_models/ops/selective_scan.py:213-214)."""
    return min(256, 1 << max(0, int(time) - 1).bit_length())


class _SelectiveLayerScan(torch.autograd.Function):
    """Owns the drive GEMM so TBPTT(1) can send the lag cotangent to W only."""

    @staticmethod
    def forward(ctx, x, weight, *args):
        *tensors, options, truncated, activate, write_raw, chunk, skip = args
        inputs = SelectiveScanInputs(*tensors, options)
        f_in, batch, time = x.shape
        with torch.autocast(x.device.type, enabled=False):
            z = (weight @ x.reshape(f_in, batch * time)).reshape(-1, batch, time)
        raw, act, entries = selective_forward(z, inputs, activate, write_raw, chunk,
                                              skip=x if skip else None)
        ctx.save_for_backward(x, weight, z, entries, *tensors)
        ctx.options, ctx.truncated = options, truncated
        ctx.activate, ctx.chunk, ctx.skip = activate, chunk, skip
        ctx.set_materialize_grads(False)
        return raw, act

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_raw, grad_act):
        x, weight, z, entries, *tensors = ctx.saved_tensors
        inputs = SelectiveScanInputs(*tensors, ctx.options)
        dx_drive, dw_drive, dg, dd, dw, dbias, dtheta = selective_backward(
            z, inputs, entries, grad_raw, grad_act, ctx.activate, ctx.truncated, ctx.chunk
        )
        f_in = x.shape[0]
        with torch.autocast(x.device.type, enabled=False):
            dx = (weight.mH @ dx_drive.reshape(weight.shape[0], -1)).reshape_as(x)
            # The reference's single GEMM here (dw_drive @ x.mH) reduces over
            # batch*time into (out, in) and runs at ~2.4 TFLOP/s on MI355X.
            dweight = weight_grad(dw_drive.reshape(weight.shape[0], -1), x.reshape(f_in, -1))
        if ctx.skip:
            # raw + x and act + x: the skip passes both cotangents to x.
            for g in (grad_raw, grad_act):
                if g is not None:
                    dx = dx + g
        grads = (dx, dweight, dg, dd, dw, dbias, dtheta) + (None,) * 13
        return tuple(g if need else None for g, need in zip(grads, ctx.needs_input_grad))


def eligible(x: Tensor, weight: Tensor, inputs: SelectiveScanInputs, use_kernel: bool = True) -> bool:
    """The reference's eligibility rule (selective_scan.py:187-203) with the HIP
    library in place of ``import triton``."""
    return (
        use_kernel
        and x.is_cuda
        and x.dtype == torch.complex64
        and weight.dtype == torch.complex64
        and inputs.bias.dtype == torch.float32
        and x.shape[1] > 0
        and x.shape[-1] > 0
        and _lib.available()
    )


def selective_layer_scan(
    x: Tensor,
    weight: Tensor,
    inputs: SelectiveScanInputs,
    *,
    truncated: bool = False,
    activate: bool = True,
    write_raw: bool = True,
    use_kernel: bool = True,
    chunk: int | None = None,
    skip: bool = False,
) -> tuple[Tensor | None, Tensor | None]:
    """Complex ``(I,B,T)`` selective layer on the HIP kernels.

    Same signature, validation and return convention as the reference.  Inputs
    the kernels cannot serve raise ``RuntimeError``; the caller keeps its own
    ``reference_layer_scan`` for those (the reference routes them there,
    selective_scan.py:190-212).

    ``skip=True`` (not in the reference's signature) returns ``(raw + x,
    act + x)``: the encoder's residual connection (pure.py:486-496), added in
    the kernel's output stores.  It needs a square ``weight``.
    """
    if not activate and not write_raw:
        raise ValueError("selective scan requires at least one output")
    if skip and weight.shape[0] != x.shape[0]:
        raise ValueError("skip needs as many output channels as input channels")
    if not eligible(x, weight, inputs, use_kernel):
        raise RuntimeError(
            "selective_layer_scan: input not eligible for the HIP kernels (needs complex64 "
            "x/W on a HIP device, fp32 parameters, B>0, T>0, use_kernel=True and a built "
            "librqf_hip.so); route it to the reference implementation"
        )
    if chunk is None:
        chunk = default_chunk(x.shape[-1])
    if chunk < 1 or chunk & (chunk - 1):
        raise ValueError("chunk must be a positive power of two")
    tensors = [v.contiguous() if isinstance(v, Tensor) else v for v in inputs[:-1]]
    return _SelectiveLayerScan.apply(
        x.contiguous(), weight, *tensors, inputs.options, truncated, activate, write_raw, chunk,
        bool(skip)
    )

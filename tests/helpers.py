"""Numerics helpers shared by the tests."""

import json
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

# Parity bar: normwise max relative error of each output / gradient tensor
# against the fp64 oracle (north star: 1e-4 in fp32).
PARITY_RTOL = 1e-4


def relerr(actual, expected) -> float:
    """max|actual - expected| / max|expected| (0 when both are empty/zero)."""
    a = to_np(actual)
    e = to_np(expected)
    assert a.shape == e.shape, (a.shape, e.shape)
    if e.size == 0:
        return 0.0
    scale = float(np.max(np.abs(e)))
    diff = float(np.max(np.abs(a.astype(np.complex128) - e.astype(np.complex128))))
    if scale == 0.0:
        return diff
    return diff / scale


# Per-channel check of a per-channel gradient vector (dbias, dtheta, grad_C1,
# grad_tap, ...): each channel's error is measured against its own magnitude,
# floored at CHANNEL_FLOOR times the largest channel's, so a channel up to 100x
# below the largest is held to the bar relative to its own value (the
# normwise check alone would allow it 100x that).  The floor sits where fp32
# arithmetic puts it: each channel's gradient is a sum over B*T steps of
# products of the adjoint state, whose own fp32 error reaches ~1e-6 of the
# largest channel's gradient over the filters' memory.
CHANNEL_FLOOR = 1e-2
# The selective gradients dbias and dtheta carry factors that the reference's
# own formulas evaluate with cancellation in fp32: sigmoid'(x) = s (1 - s) as
# s -> 1 and (1 - gamma) as gamma -> 1 (selective_scan_kernel.py:441-447,
# selective_scan.py:40).  At the interior-gamma edges the reference's own
# fp32 arithmetic (its PyTorch path, restated in oracle/torch_ref.py) is
# 3e-4 - 9e-4 per channel from fp64 there, so the selective per-channel bar is
# 1e-3, or twice that fp32 restatement's own error where that is larger.
SELECTIVE_CHANNEL_RTOL = 1e-3


def chanerr(actual, expected, floor: float = CHANNEL_FLOOR) -> float:
    """max_f |a_f - e_f| / max(|e_f|, floor * max_f |e_f|) over the channels f.

    Arrays with more than one axis are compared per element (the first axis
    is the channel); 0 when both are empty or zero."""
    a = to_np(actual).astype(np.complex128).ravel()
    e = to_np(expected).astype(np.complex128).ravel()
    assert a.shape == e.shape, (a.shape, e.shape)
    if e.size == 0:
        return 0.0
    mag = np.abs(e)
    scale = np.maximum(mag, floor * float(mag.max()))
    diff = np.abs(a - e)
    if float(mag.max()) == 0.0:
        return float(diff.max())
    return float(np.max(diff / scale))


def to_np(t):
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.is_complex():
            return t.resolve_conj().to(torch.complex128).numpy()
        return t.to(torch.float64).numpy()
    return np.asarray(t)


def crandn(rng, *shape):
    return rng.standard_normal(shape) + 1j * rng.standard_normal(shape)


def load_checkpoint_params():
    """(records, arrays) of tests/golden/checkpoint_params.{json,npz}: one record per
    packaged checkpoint, per-channel RQF leaves flattened over (checkpoint, block)."""
    with open(os.path.join(GOLDEN, "checkpoint_params.json")) as f:
        records = json.load(f)
    arrays = np.load(os.path.join(GOLDEN, "checkpoint_params.npz"))
    return records, {k: arrays[k] for k in arrays.files}


def block_params(rec, arrays, block):
    """RQFParams of block ``block`` of checkpoint record ``rec``."""
    from prospective_rqf_amd.coefficients import RQFParams

    off, n = rec["blocks"][block]
    t = lambda k: torch.from_numpy(arrays[k][off:off + n].astype(np.float64))  # noqa: E731
    return RQFParams(log_tau=t("log_tau"), dt=rec["dt"], discretization=rec["discretization"],
                     clamp_gamma=rec["clamp_gamma"], gamma_param=t("gamma_param"),
                     freq_param=t("freq_param"), min_gamma=t("min_gamma"),
                     max_gamma=t("max_gamma"), min_freq=t("min_freq"), max_freq=t("max_freq"))


def block_coefficients(rec, arrays, block):
    """The complex64 coefficients block ``block`` feeds its scan, as complex128 numpy:
    (C1, tap0, tap1) for prospective models, (C1, C2, None) otherwise."""
    from prospective_rqf_amd.coefficients import compute_coefficients, compute_two_tap_coefficients

    p = block_params(rec, arrays, block)
    if rec["prospective"]:
        c = compute_two_tap_coefficients(p, True, rec["prospective_mode"], rec["prospective_tau"])
    else:
        c = compute_coefficients(p) + (None,)
    return tuple(None if v is None else v.numpy().astype(np.complex128) for v in c)


def cotangent_off_relu_kink(y_ref, gy, band=1e-4):
    """Zero the cotangent where the split-ReLU mask is decided by rounding.

    A masked backward (Re/Im of the cotangent pass where Re/Im of the raw state is
    > 0) is discontinuous in the state.  Where the fp64 state lies within float32
    rounding of zero, the kernel (whose recompute backward re-derives the state by
    replay) and the oracle may decide differently, and one such element moves a
    near-cancelling gradient like grad_z by up to ~10% normwise.  Zeroing the
    cotangent's component wherever the state's component lies within
    ``band * max|y_ref|`` of zero makes the result independent of those decisions
    while every other element still tests the kernel.  Returns (gy', count)."""
    y = np.asarray(y_ref)
    g = np.array(gy, dtype=np.complex128, copy=True)
    lim = band * (float(np.max(np.abs(y))) if y.size else 0.0)
    near_re, near_im = np.abs(y.real) <= lim, np.abs(y.imag) <= lim
    g = np.where(near_re, 0.0, g.real) + 1j * np.where(near_im, 0.0, g.imag)
    return g, int(near_re.sum() + near_im.sum())

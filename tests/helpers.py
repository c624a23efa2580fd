"""Numerics helpers shared by the tests."""

import numpy as np
import torch

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


def to_np(t):
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.is_complex():
            return t.resolve_conj().to(torch.complex128).numpy()
        return t.to(torch.float64).numpy()
    return np.asarray(t)


def crandn(rng, *shape):
    return rng.standard_normal(shape) + 1j * rng.standard_normal(shape)

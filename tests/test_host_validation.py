"""Host-side shape validation of the public entry points (no device needed).

Every kernel reads its inputs through the shapes the host passes it, so a
mismatched cotangent or state tensor must be rejected with ``ValueError``
before any launch.  The checks run before the device check, so CPU tensors
reach them here.  References: the reference's own entry points take the
chunk count from ``entries.shape[1]`` (selective_scan_kernel.py:545) and
validate the chunk and outputs (selective_scan.py:185-186,213-216).
"""

import numpy as np
import pytest
import torch

from prospective_rqf_amd import _lib
from prospective_rqf_amd import multi_osc_scan as mo
from prospective_rqf_amd.chunked_scan_kernel import (
    _chunked_prospective_backward_raw,
    _chunked_scan_backward_raw,
)
from prospective_rqf_amd.fbt_scan_kernel import fbt_prospective_scan, fbt_recompute_backward_raw
from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward
from tests.selective_cases import CASES, make_inputs, to_torch

F, B, T = 4, 2, 300
GROUPED = next(c for c in CASES if c["warp"] == "grouped" and c["gamma"] and c["write"])


def _sel():
    inp = to_torch(make_inputs(F, B, T, GROUPED, np.random.default_rng(0), G=2))
    z = torch.zeros(F, B, T, dtype=torch.complex64)
    return z, inp


def _cz(*shape):
    return torch.zeros(*shape, dtype=torch.complex64)


@pytest.mark.parametrize("bad", ["gy", "gx", "entries_rows", "entries_chunks", "entries_dtype",
                                 "chunk", "drive_dims"])
def test_selective_backward_rejects_mismatched_shapes(bad):
    z, inp = _sel()
    chunk = 128
    entries = _cz(F * B, -(-T // chunk))
    gy, gx = _cz(F, B, T), _cz(F, B, T)
    if bad == "gy":
        gy = _cz(F, B, T - 1)
    elif bad == "gx":
        gx = _cz(F, B + 1, T)
    elif bad == "entries_rows":
        entries = _cz(F * B - 1, -(-T // chunk))
    elif bad == "entries_chunks":
        entries = _cz(F * B, -(-T // 256))  # entries of another chunk size
    elif bad == "entries_dtype":
        entries = torch.zeros(F * B, -(-T // chunk), 2)
    elif bad == "chunk":
        chunk = 96
    else:
        z = _cz(F * B, T)
    with pytest.raises(ValueError):
        selective_backward(z, inp, entries, gy, gx, True, False, chunk)


@pytest.mark.parametrize("bad", ["chunk", "zero_chunk", "no_outputs", "skip"])
def test_selective_forward_rejects_bad_arguments(bad):
    z, inp = _sel()
    chunk, act, raw, skip = 256, True, True, None
    if bad == "chunk":
        chunk = 100
    elif bad == "zero_chunk":
        chunk = 0
    elif bad == "no_outputs":
        act = raw = False
    else:
        skip = _cz(F, B, T + 1)
    with pytest.raises(ValueError):
        selective_forward(z, inp, act, raw, chunk, skip=skip)


def test_selective_forward_rejects_a_non_complex_drive():
    _, inp = _sel()
    with pytest.raises(TypeError):
        selective_forward(torch.zeros(F, B, T), inp, True, True, 256)


@pytest.mark.parametrize("bad", ["grad", "carry_shape", "carry_dtype", "coef"])
def test_fbt_recompute_backward_rejects_mismatched_shapes(bad):
    c = _cz(F)
    x, g = _cz(F, B, T), _cz(F, B, T)
    carry = _cz(F * B, 2)  # rqf_fbt_carry_chunks(300) = 2 tiles of 256
    if bad == "grad":
        g = _cz(F, B, T + 1)
    elif bad == "carry_shape":
        carry = _cz(F * B, 3)
    elif bad == "carry_dtype":
        carry = torch.zeros(F * B, 2, 2)
    else:
        c = _cz(F + 1)
    with pytest.raises(ValueError):
        fbt_recompute_backward_raw(c, c, c, x, carry, g)


def test_fbt_prospective_rejects_bad_coefficients_and_rank():
    with pytest.raises(ValueError):
        fbt_prospective_scan(_cz(F + 1), _cz(F), _cz(F), _cz(F, B, T))
    with pytest.raises(ValueError):
        fbt_prospective_scan(_cz(F), _cz(F), _cz(F), _cz(F * B, T))


@pytest.mark.parametrize("fn", ["scan", "prospective"])
@pytest.mark.parametrize("bad", ["grad", "states", "coef"])
def test_chunked_backward_rejects_mismatched_shapes(fn, bad):
    c = _cz(F)
    u, g, states = _cz(B, T, F), _cz(B, T, F), None
    if bad == "grad":
        g = _cz(B, T - 1, F)
    elif bad == "states":
        states = _cz(B, T, F + 1)
    else:
        c = _cz(F - 1)
    with pytest.raises(ValueError):
        if fn == "scan":
            _chunked_scan_backward_raw(c, c, u, states, g)
        else:
            _chunked_prospective_backward_raw(c, c, c, u, states, g)


@pytest.mark.parametrize("bad", ["grad", "cw", "coef", "num_osc"])
def test_multi_osc_backward_rejects_mismatched_shapes(bad):
    n = 3
    c = _cz(F * n)
    cw = torch.zeros(F * n, 2)
    u, g = _cz(B, T, F), _cz(B, T, F)
    num_osc = n
    if bad == "grad":
        g = _cz(B, T, F + 1)
    elif bad == "cw":
        cw = torch.zeros(F * n - 1, 2)
    elif bad == "coef":
        c = _cz(F * n + 1)
    else:
        num_osc = 0
    with pytest.raises(ValueError):
        mo._sequential_scan_multi_osc_backward_raw(c, c, u, cw, g, num_osc)


def test_valid_arguments_pass_validation_and_reach_the_device_check():
    """The same calls with consistent shapes get past every shape check and
    stop at the device check (host tensors), so each rejection above is the
    shape check's."""
    from prospective_rqf_amd._lib import RQFError

    z, inp = _sel()
    chunk = 128
    entries = _cz(F * B, -(-T // chunk))
    c = _cz(F)
    calls = [
        lambda: selective_backward(z, inp, entries, _cz(F, B, T), _cz(F, B, T), True, False,
                                   chunk),
        lambda: selective_forward(z, inp, True, True, 256),
        lambda: fbt_recompute_backward_raw(c, c, c, _cz(F, B, T), _cz(F * B, 2), _cz(F, B, T)),
        lambda: fbt_prospective_scan(c, c, c, _cz(F, B, T)),
        lambda: _chunked_scan_backward_raw(c, c, _cz(B, T, F), None, _cz(B, T, F)),
        lambda: _chunked_prospective_backward_raw(c, c, c, _cz(B, T, F), None, _cz(B, T, F)),
        lambda: mo._sequential_scan_multi_osc_backward_raw(_cz(F * 3), _cz(F * 3), _cz(B, T, F),
                                                           torch.zeros(F * 3, 2), _cz(B, T, F),
                                                           3),
    ]
    for call in calls:
        with pytest.raises(RQFError):
            call()


class _OnDevice:
    """Stand-in for a device tensor: only what require_device reads."""

    is_cuda = True

    def __init__(self, index):
        self.index = index

    def get_device(self):
        return self.index


def test_device_check_rejects_mixed_and_non_current_devices(monkeypatch):
    """Inputs on two devices, or on a device that is not the current one, are
    refused before any pointer reaches a kernel; one device that is current
    passes, and None entries (absent optional inputs) are skipped."""
    monkeypatch.setattr(_lib, "_current_device", lambda: 0)
    _lib.require_device(_OnDevice(0), None, _OnDevice(0))
    with pytest.raises(_lib.RQFError, match="different devices"):
        _lib.require_device(_OnDevice(0), _OnDevice(1))
    with pytest.raises(_lib.RQFError, match="is current"):
        _lib.require_device(_OnDevice(1), None, _OnDevice(1))
    with pytest.raises(_lib.RQFError, match="HIP devices only"):
        _lib.require_device(_OnDevice(0), torch.zeros(1))

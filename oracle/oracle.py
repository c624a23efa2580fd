"""numpy front end of the fp64 CPU oracle (``rqf_oracle.c``).

TEST INFRASTRUCTURE ONLY.  ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it as the checker; the product package
``prospective_rqf_amd`` never imports it.

Complex arrays are numpy ``complex128``; real arrays ``float64``.  Layout codes:
``BTF`` is the reference's ``(batch, time, filters)`` API layout, ``FBT`` the
channel-outermost layout of the FBT and selective kernels.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librqf_oracle.so")
BTF, FBT = 0, 1

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a):
    return np.ascontiguousarray(a, dtype=np.complex128)


def _r(a):
    return np.ascontiguousarray(a, dtype=np.float64)


# --------------------------------------------------------------------------
# two-tap / time-invariant scan
# --------------------------------------------------------------------------


def twotap_fwd(c1, k0, k1, x, layout=BTF, act=False):
    """y[t] = c1 y[t-1] + k0 x[t] + k1 x[t-1]; ``k1=None`` is the plain C2 scan.

    Returns ``y`` (and the split-ReLU of it when ``act``)."""
    x = _c(x)
    if layout == BTF:
        B, T, F = x.shape
    else:
        F, B, T = x.shape
    c1, k0 = _c(c1), _c(k0)
    k1 = None if k1 is None else _c(k1)
    y = np.empty_like(x)
    out_act = np.empty_like(x) if act else None
    lib().orc_twotap_fwd(
        ctypes.c_int(layout), ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(F),
        _p(c1), _p(k0), _p(k1), _p(x), _p(y), _p(out_act),
    )
    return (y, out_act) if act else y


def twotap_bwd(c1, k0, k1, x, y, gy, layout=BTF, mask_act=False):
    """Adjoint of :func:`twotap_fwd`: returns ``(gx, gc1, gk0, gk1)``."""
    x, y, gy = _c(x), _c(y), _c(gy)
    if layout == BTF:
        B, T, F = x.shape
    else:
        F, B, T = x.shape
    c1, k0 = _c(c1), _c(k0)
    k1 = None if k1 is None else _c(k1)
    gx = np.empty_like(x)
    gc1 = np.empty(F, np.complex128)
    gk0 = np.empty(F, np.complex128)
    gk1 = np.empty(F, np.complex128) if k1 is not None else None
    lib().orc_twotap_bwd(
        ctypes.c_int(layout), ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(F),
        _p(c1), _p(k0), _p(k1), _p(x), _p(y), _p(gy), ctypes.c_int(int(mask_act)),
        _p(gx), _p(gc1), _p(gk0), _p(gk1),
    )
    return gx, gc1, gk0, gk1


# --------------------------------------------------------------------------
# multi-oscillator scan with C-weight reduction (BTF)
# --------------------------------------------------------------------------


def mosc_fwd(c1, c2, cw, u, num_osc):
    """``(y, |y|)`` of x_n[t] = c1_n x_n[t-1] + c2_n u[t], y = sum_n cw_n x_n
    (``cw=None``: y = x_0 with one oscillator).  ``u`` is (B,T,F)."""
    u = _c(u)
    B, T, F = u.shape
    c1, c2 = _c(c1), _c(c2)
    cw = None if cw is None else _c(cw)
    y = np.empty_like(u)
    yabs = np.empty(u.shape, np.float64)
    lib().orc_mosc_fwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(F),
                       ctypes.c_int64(num_osc), _p(c1), _p(c2), _p(cw), _p(u), _p(y), _p(yabs))
    return y, yabs


def mosc_bwd(c1, c2, cw, u, gy, num_osc):
    """Adjoint of :func:`mosc_fwd`: ``(gu, gc1, gc2, gcw)`` (gu complex (B,T,F);
    the coefficient gradients (F*N,) complex)."""
    u, gy = _c(u), _c(gy)
    B, T, F = u.shape
    c1, c2, cw = _c(c1), _c(c2), _c(cw)
    gu = np.empty_like(u)
    gc1 = np.empty(F * num_osc, np.complex128)
    gc2 = np.empty_like(gc1)
    gcw = np.empty_like(gc1)
    lib().orc_mosc_bwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(F),
                       ctypes.c_int64(num_osc), _p(c1), _p(c2), _p(cw), _p(u), _p(gy), _p(gu),
                       _p(gc1), _p(gc2), _p(gcw))
    return gu, gc1, gc2, gcw


# --------------------------------------------------------------------------
# selective scan
# --------------------------------------------------------------------------


class _SelStruct(ctypes.Structure):
    _fields_ = [
        ("F", ctypes.c_int64), ("B", ctypes.c_int64), ("T", ctypes.c_int64),
        ("G", ctypes.c_int64),
        ("gamma_logits", ctypes.c_void_p), ("warp_logits", ctypes.c_void_p),
        ("write_logits", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("theta", ctypes.c_void_p), ("minimum", ctypes.c_void_p),
        ("span", ctypes.c_void_p), ("step", ctypes.c_void_p), ("horizon", ctypes.c_void_p),
        ("theta_minimum", ctypes.c_void_p), ("theta_maximum", ctypes.c_void_p),
        ("groups", ctypes.c_void_p),
        ("has_gamma", ctypes.c_int32), ("has_warp", ctypes.c_int32),
        ("has_write", ctypes.c_int32), ("log_shift", ctypes.c_int32),
        ("gamma_scale", ctypes.c_double), ("warp_scale", ctypes.c_double),
        ("prospective", ctypes.c_int32), ("gamma_horizon", ctypes.c_int32),
        ("write_sigmoid", ctypes.c_int32),
        ("write_max", ctypes.c_double), ("write_bias", ctypes.c_double),
        ("bound_warp", ctypes.c_int32),
    ]


@dataclass
class SelectiveInputs:
    """numpy mirror of ``SelectiveScanInputs`` (rqf_models/ops/selective_scan.py:10-23).

    ``options`` is the reference's 12-tuple (rqf_models/backbones/rqf/selective.py:249-262):
    (has_gamma, has_warp, has_write, log_shift, gamma_scale, warp_scale,
    prospective, gamma_horizon, write_sigmoid, write_max, write_bias, bound_warp).
    """

    gamma_logits: np.ndarray  # (F|0, B, T)
    warp_logits: np.ndarray  # (G|0, B, T)
    write_logits: np.ndarray  # (F|0, B, T)
    bias: np.ndarray
    theta: np.ndarray
    groups: np.ndarray | None
    minimum: np.ndarray
    span: np.ndarray
    step: np.ndarray
    horizon: np.ndarray
    theta_minimum: np.ndarray
    theta_maximum: np.ndarray
    options: tuple

    def struct(self, F, B, T):
        o = self.options
        keep = [
            _r(self.gamma_logits), _r(self.warp_logits), _r(self.write_logits),
            _r(self.bias), _r(self.theta), _r(self.minimum), _r(self.span), _r(self.step),
            _r(self.horizon), _r(self.theta_minimum), _r(self.theta_maximum),
            None if self.groups is None else np.ascontiguousarray(self.groups, dtype=np.int64),
        ]
        s = _SelStruct(
            F, B, T, int(self.warp_logits.shape[0]) if o[1] else 0,
            *(_p(a) if a is not None and a.size else None for a in keep[:3]),
            *(_p(a) for a in keep[3:11]),
            _p(keep[11]),
            int(o[0]), int(o[1]), int(o[2]), int(o[3]), float(o[4]), float(o[5]),
            int(o[6]), int(o[7]), int(o[8]), float(o[9]), float(o[10]), int(o[11]),
        )
        return s, keep


def selective_coefficients(inputs: SelectiveInputs, F, B, T):
    s, keep = inputs.struct(F, B, T)
    A = np.empty((F, B, T), np.complex128)
    p = np.empty_like(A)
    n = np.empty_like(A)
    lib().orc_selective_coefficients(ctypes.byref(s), _p(A), _p(p), _p(n))
    return A, p, n


def selective_fwd(z, inputs: SelectiveInputs):
    """fp64 reference forward after the drive GEMM: returns ``(raw, act)``."""
    z = _c(z)
    F, B, T = z.shape
    s, keep = inputs.struct(F, B, T)
    raw = np.empty_like(z)
    act = np.empty_like(z)
    lib().orc_selective_fwd(ctypes.byref(s), _p(z), _p(raw), _p(act))
    return raw, act


def selective_bwd(z, inputs: SelectiveInputs, gy, gx, truncated=False):
    """fp64 reverse mode: ``(dz, dzw, dg|None, dd|None, dw|None, dbias, dtheta)``."""
    z = _c(z)
    F, B, T = z.shape
    s, keep = inputs.struct(F, B, T)
    gy = None if gy is None else _c(gy)
    gx = None if gx is None else _c(gx)
    o = inputs.options
    dz = np.empty_like(z)
    dzw = np.empty_like(z)
    dg = np.empty((F, B, T)) if o[0] else None
    G = int(inputs.warp_logits.shape[0]) if o[1] else 0
    dd = np.empty((G, B, T)) if o[1] else None
    dw = np.empty((F, B, T)) if o[2] else None
    dbias = np.empty(F)
    dtheta = np.empty(F)
    lib().orc_selective_bwd(
        ctypes.byref(s), _p(z), _p(gy), _p(gx), ctypes.c_int(int(truncated)),
        _p(dz), _p(dzw), _p(dg), _p(dd), _p(dw), _p(dbias), _p(dtheta),
    )
    return dz, dzw, dg, dd, dw, dbias, dtheta


def zoh_two_tap(gamma, theta, eta, ratio):
    """Static ZOH two-tap coefficients (rqf_models/backbones/rqf/filter.py:630-646)."""
    gamma, theta, eta, ratio = (_r(v) for v in (gamma, theta, eta, ratio))
    F = gamma.shape[0]
    c1 = np.empty(F, np.complex128)
    t0 = np.empty_like(c1)
    t1 = np.empty_like(c1)
    lib().orc_zoh_two_tap(ctypes.c_int64(F), _p(gamma), _p(theta), _p(eta), _p(ratio),
                          _p(c1), _p(t0), _p(t1))
    return c1, t0, t1

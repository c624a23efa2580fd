"""The scans at their largest accepted grids, and refusal one step past.

A dispatch counts its work-items in 32 bits, and a grid past 2^32 - 1 of
them runs truncated with no launch error.  So every entry point refuses such
a shape with RQF_ERR_ARG before launching (the bounds are in
include/rqf_scan.h), and its reductions over filters stride, so they take
any count.  At B = 1, T = 2:

* (B,T,F) chunked scan, F = 134217712 (8388607 blocks of 512 threads):
  x0 = C2 u0, x1 = C1 x0 + C2 u1; adjoint g1 = gy1, g0 = conj(C1) g1 + gy0,
  grad_u = conj(C2) g, grad_C2 = sum_t conj(u_t) g_t, grad_C1 = conj(x0) g1;
* multi-oscillator scan, N = 1 with C-weights, F = 67108848 (4194303 blocks
  of up to 1024 threads): y = cw C2 w, w0 = u0, w1 = C1 w0 + u1; e1 = gy1,
  e0 = conj(C1) e1 + gy0, grad_u = conj(cw C2) e, grad_C2 = conj(cw) Q,
  grad_cw = conj(C2) Q with Q = sum_t e_t conj(u_t), grad_C1 = conj(cw C2) R
  with R = e1 conj(u0);
* FBT prospective scan without the activation, F = 8388607 rows at B = 1
  (one 512-thread block per row in the forward), against the fp64 oracle.
  With the split-ReLU, 8.4 million rows hold states within float32 rounding
  of zero, whose mask then differs between the oracle's fp64 state and the
  kernel's fp32 one (seed 13 has one: -8.5e-9 against +2.3e-8), so the
  gradient is compared without the mask; the masked kernels share the
  grids.

These closed forms are the two-step recurrences written out, in float64 with
torch on the GPU.  The coefficient reductions run here over 8-134 million
filters, past the 2^20 blocks of their grid.  Bar: normwise max relative error
<= 1e-5 per tensor (two fp32 steps); the FBT case uses the suite's usual
parity bar against the oracle.
"""

import numpy as np
import pytest
import torch

from oracle import oracle
from prospective_rqf_amd import _lib
from prospective_rqf_amd import chunked_scan_kernel as ck
from prospective_rqf_amd import multi_osc_scan as mo
from prospective_rqf_amd.fbt_scan_kernel import fbt_prospective_scan
from tests.helpers import PARITY_RTOL, crandn, relerr

pytestmark = pytest.mark.gpu

RTOL = 1e-5
SLICE = 2**25


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    yield
    torch.cuda.empty_cache()


def _crand(*shape, gen):
    return torch.complex(torch.randn(*shape, device="cuda", generator=gen),
                         torch.randn(*shape, device="cuda", generator=gen))


def _coef(n, gen):
    mag = 0.5 + 0.49 * torch.rand(n, device="cuda", generator=gen)
    return torch.polar(mag, 6.283 * torch.rand(n, device="cuda", generator=gen))


def _d(t):
    return t.detach().to(torch.complex128)


def _err(got, want_fn, n):
    """Normwise max relative error of got (last axis n) against want_fn(lo, hi),
    slice by slice to bound the float64 temporaries."""
    num = den = 0.0
    for lo in range(0, n, SLICE):
        hi = min(n, lo + SLICE)
        w = want_fn(lo, hi)
        num = max(num, (_d(got[..., lo:hi]) - w).abs().max().item())
        den = max(den, w.abs().max().item())
    return num / den


def test_chunked_scan_at_grid_limit():
    F = ((2**32 - 1) // 512) * 16
    print(f"case: chunked scan at the grid limit B=1 T=2 F={F}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    C1 = _coef(F, gen).requires_grad_(True)
    C2 = _crand(F, gen=gen).requires_grad_(True)
    u = _crand(1, 2, F, gen=gen).requires_grad_(True)
    gy = _crand(1, 2, F, gen=gen)
    y = ck._triton_chunked_scan(C1, C2, u)
    y.backward(gy)
    torch.cuda.synchronize()

    def parts(lo, hi):
        c1, c2 = _d(C1[lo:hi]), _d(C2[lo:hi])
        uu, g = _d(u[0, :, lo:hi]), _d(gy[0, :, lo:hi])
        x0 = c2 * uu[0]
        g0 = c1.conj() * g[1] + g[0]
        return c1, c2, uu, x0, (g0, g[1])

    def want_y(lo, hi):
        c1, c2, uu, x0, _ = parts(lo, hi)
        return torch.stack([x0, c1 * x0 + c2 * uu[1]])[None]

    def want_gu(lo, hi):
        _, c2, _, _, (g0, g1) = parts(lo, hi)
        return torch.stack([c2.conj() * g0, c2.conj() * g1])[None]

    def want_gc1(lo, hi):
        _, _, _, x0, (_, g1) = parts(lo, hi)
        return x0.conj() * g1

    def want_gc2(lo, hi):
        _, _, uu, _, (g0, g1) = parts(lo, hi)
        return uu[0].conj() * g0 + uu[1].conj() * g1

    errs = {"y": _err(y, want_y, F), "grad_u": _err(u.grad, want_gu, F),
            "grad_C1": _err(C1.grad, want_gc1, F), "grad_C2": _err(C2.grad, want_gc2, F)}
    del y
    assert all(e <= RTOL for e in errs.values()), errs
    # one 16-filter block more is refused before any launch
    F1 = F + 16
    with pytest.raises(_lib.RQFError):
        ck._triton_chunked_scan(C1.detach()[:1].expand(F1).contiguous(),
                                C2.detach()[:1].expand(F1).contiguous(),
                                torch.zeros(1, 2, F1, dtype=torch.complex64, device="cuda"))


def test_multi_osc_at_grid_limit():
    F = ((2**32 - 1) // 1024) * 16
    print(f"case: multi-osc at the grid limit N=1 B=1 T=2 F={F}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(12)
    C1 = _coef(F, gen).requires_grad_(True)
    C2 = _crand(F, gen=gen).requires_grad_(True)
    cw = torch.randn(F, 2, device="cuda", generator=gen).requires_grad_(True)
    u = _crand(1, 2, F, gen=gen).requires_grad_(True)
    gy = _crand(1, 2, F, gen=gen)
    y = mo._triton_parallel_scan_multi_osc(C1, C2, u, cw, 1)
    y.backward(gy)
    torch.cuda.synchronize()

    def parts(lo, hi):
        c1, c2 = _d(C1[lo:hi]), _d(C2[lo:hi])
        w = torch.complex(cw[lo:hi, 0].double(), cw[lo:hi, 1].double()).detach()
        uu, g = _d(u[0, :, lo:hi]), _d(gy[0, :, lo:hi])
        e0 = c1.conj() * g[1] + g[0]
        q = e0 * uu[0].conj() + g[1] * uu[1].conj()
        return c1, c2, w, uu, (e0, g[1]), q

    def want_y(lo, hi):
        c1, c2, w, uu, _, _ = parts(lo, hi)
        return torch.stack([w * c2 * uu[0], w * c2 * (c1 * uu[0] + uu[1])])[None]

    def want_gu(lo, hi):
        _, c2, w, _, (e0, e1), _ = parts(lo, hi)
        h = (w * c2).conj()
        return torch.stack([h * e0, h * e1])[None]

    def want_gc1(lo, hi):
        _, c2, w, uu, (_, e1), _ = parts(lo, hi)
        return (w * c2).conj() * e1 * uu[0].conj()

    def want_gc2(lo, hi):
        _, _, w, _, _, q = parts(lo, hi)
        return w.conj() * q

    def want_gcw(lo, hi):
        _, c2, _, _, _, q = parts(lo, hi)
        return c2.conj() * q

    gcw = torch.complex(cw.grad[:, 0], cw.grad[:, 1])
    errs = {"y": _err(y, want_y, F), "grad_u": _err(u.grad, want_gu, F),
            "grad_C1": _err(C1.grad, want_gc1, F), "grad_C2": _err(C2.grad, want_gc2, F),
            "grad_cw": _err(gcw, want_gcw, F)}
    del y, gcw
    assert all(e <= RTOL for e in errs.values()), errs
    F1 = F + 16
    with pytest.raises((_lib.RQFError, ValueError)):
        mo._triton_parallel_scan_multi_osc(
            C1.detach()[:1].expand(F1).contiguous(), C2.detach()[:1].expand(F1).contiguous(),
            torch.zeros(1, 2, F1, dtype=torch.complex64, device="cuda"),
            cw.detach()[:1].expand(F1, 2).contiguous(), 1)


def test_fbt_prospective_at_row_limit():
    F, B, T = (2**32 - 1) // 512, 1, 2
    print(f"case: fbt prospective at the row limit F={F} B={B} T={T}", flush=True)
    rng = np.random.default_rng(13)
    mag = rng.uniform(0.5, 0.99, F)
    c1 = (mag * np.exp(1j * rng.uniform(0, 2 * np.pi, F))).astype(np.complex64)
    t0 = crandn(rng, F).astype(np.complex64)
    t1 = (0.5 * crandn(rng, F)).astype(np.complex64)
    z = crandn(rng, F, B, T).astype(np.complex64)
    gy = crandn(rng, F, B, T).astype(np.complex64)
    d = lambda a: a.astype(np.complex128)
    y_ref = oracle.twotap_fwd(d(c1), d(t0), d(t1), d(z), layout=oracle.FBT)
    gz_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(d(c1), d(t0), d(t1), d(z), y_ref,
                                                          d(gy), layout=oracle.FBT)
    dev = lambda a: torch.as_tensor(a, device="cuda").requires_grad_(True)
    C1, T0, T1, Z = dev(c1), dev(t0), dev(t1), dev(z)
    y = fbt_prospective_scan(C1, T0, T1, Z, fuse_act=False)
    y.backward(torch.as_tensor(gy, device="cuda"))
    for name, got, want in (("raw", y, y_ref), ("grad_z", Z.grad, gz_ref),
                            ("grad_C1", C1.grad, gc1_ref), ("grad_tap0", T0.grad, gt0_ref),
                            ("grad_tap1", T1.grad, gt1_ref)):
        err = relerr(got, want)
        assert err <= PARITY_RTOL, (name, err)
    del y
    with pytest.raises(_lib.RQFError):
        fbt_prospective_scan(C1.detach()[:1].expand(F + 1).contiguous(),
                             T0.detach()[:1].expand(F + 1).contiguous(),
                             T1.detach()[:1].expand(F + 1).contiguous(),
                             torch.zeros(F + 1, B, T, dtype=torch.complex64, device="cuda"),
                             fuse_act=False)

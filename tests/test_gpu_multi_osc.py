"""GPU parity of the multi-oscillator scans and the fused |y| readout.

Compares ``rqf_multi_osc_fwd`` / ``rqf_multi_osc_bwd`` (through the reference's
Python names) with the fp64 oracle, for complex and real inputs, 1 to 17
oscillators (more than 4 run in chunks of 4), sequence lengths below, at and
across the kernels' pass lengths (a block walks T in passes of 256 to 1024
steps; T = 3000 takes three or more), filter counts that leave a partial
16-filter group, and the autograd boundaries, including the ``needs_input_grad`` gating the
reference's kernels implement (triton_scan_kernel.py:2280-2410).  Bar:
normwise max relative error <= 1e-4 per output and gradient tensor.
"""

import numpy as np
import pytest
import torch

from oracle import oracle
from prospective_rqf_amd import multi_osc_scan as mo
from prospective_rqf_amd import scan as hip_scan
from tests.helpers import PARITY_RTOL, chanerr, crandn, relerr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _c64(a):
    return np.asarray(a, dtype=np.complex64).astype(np.complex128)


def _problem(rng, B, T, F, N, real):
    c1 = _c64(rng.uniform(0.7, 0.995, F * N) * np.exp(1j * rng.uniform(0, 2 * np.pi, F * N)))
    c2 = _c64(0.5 * crandn(rng, F * N))
    cw = _c64(crandn(rng, F * N))
    u = rng.standard_normal((B, T, F)) if real else crandn(rng, B, T, F)
    u = np.asarray(u, np.float32).astype(np.float64) if real else _c64(u)
    return c1, c2, cw, u


def _t(a, grad=False):
    if np.iscomplexobj(a):
        t = torch.as_tensor(a.astype(np.complex64), device="cuda")
    else:
        t = torch.as_tensor(a.astype(np.float32), device="cuda")
    return t.requires_grad_(grad)


def _cw_param(cw, grad=False):
    return torch.as_tensor(np.stack([cw.real, cw.imag], -1).astype(np.float32),
                           device="cuda").requires_grad_(grad)


# (2, 512, 19): passes that all lie inside [0, T), the last one included, for
# 2 to 4 oscillators (256-step backward passes), and one whole 512-step pass
# for one oscillator.
SHAPES = [(2, 1, 5), (2, 37, 3), (3, 256, 4), (2, 257, 3), (1, 1000, 2), (4, 3000, 64),
          (2, 600, 130), (2, 512, 19)]


@pytest.mark.parametrize("real", [False, True])
@pytest.mark.parametrize("N", [1, 2, 3, 4, 5, 8, 12, 17])
@pytest.mark.parametrize("shape", SHAPES)
def test_multi_osc_forward_backward(shape, N, real):
    B, T, F = shape
    print(f"case: multi-osc {shape} N={N} real={real}", flush=True)
    rng = np.random.default_rng(B * 1000 + T * 10 + F + N)
    c1, c2, cw, u = _problem(rng, B, T, F, N, real)
    gy = _c64(crandn(rng, B, T, F))
    y_ref, yabs_ref = oracle.mosc_fwd(c1, c2, cw, u, N)
    gu_ref, gc1_ref, gc2_ref, gcw_ref = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    C1, C2, U, CW = _t(c1, True), _t(c2, True), _t(u, True), _cw_param(cw, True)
    fn = mo._triton_sequential_scan_multi_osc_real if real else mo._triton_sequential_scan_multi_osc
    y = fn(C1, C2, U, CW, N)
    assert y.dtype == torch.complex64 and y.shape == (B, T, F)
    y.backward(_t(gy))
    gcw_got = CW.grad[:, 0].double() + 1j * CW.grad[:, 1].double()
    errs = {"y": relerr(y, y_ref), "gc1": relerr(C1.grad, gc1_ref),
            "gc2": relerr(C2.grad, gc2_ref), "gcw": relerr(gcw_got.cpu(), gcw_ref),
            "gu": relerr(U.grad, gu_ref.real if real else gu_ref),
            "gc1/channel": chanerr(C1.grad, gc1_ref), "gc2/channel": chanerr(C2.grad, gc2_ref),
            "gcw/channel": chanerr(gcw_got.cpu(), gcw_ref)}
    assert U.grad.dtype == U.dtype
    with torch.no_grad():
        if real:
            yabs = mo._sequential_scan_multi_osc_real_forward_abs_raw(C1, C2, U, CW, N)
        else:
            yabs = mo._sequential_scan_multi_osc_forward_abs_raw(C1, C2, U, CW[:, 0], CW[:, 1], N)
    assert yabs.dtype == torch.float32
    errs["|y|"] = relerr(yabs, yabs_ref)
    bad = {k: v for k, v in errs.items() if not v <= PARITY_RTOL}
    assert not bad, errs


@pytest.mark.parametrize("N,real", [(1, True), (2, True), (4, True), (1, False), (2, False),
                                    (4, False), (5, False)])
def test_more_filters_than_one_descriptor_range(N, real):
    """F above 65536: a pass of the forward no longer fits one 32-bit buffer
    range, so it runs with 64-bit addresses (the reference's grid has no
    filter limit, triton_scan_kernel.py:1991-2015).  Same checks as above,
    |y| included; T = 70 spans a ragged last pass."""
    B, T, F = 1, 70, 65536 + 40
    print(f"case: multi-osc wide rows {(B, T, F)} N={N} real={real}", flush=True)
    rng = np.random.default_rng(N + 7 * real)
    c1, c2, cw, u = _problem(rng, B, T, F, N, real)
    gy = _c64(crandn(rng, B, T, F))
    y_ref, yabs_ref = oracle.mosc_fwd(c1, c2, cw, u, N)
    gu_ref, gc1_ref, gc2_ref, gcw_ref = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    C1, C2, U, CW = _t(c1, True), _t(c2, True), _t(u, True), _cw_param(cw, True)
    fn = mo._triton_sequential_scan_multi_osc_real if real else mo._triton_sequential_scan_multi_osc
    y = fn(C1, C2, U, CW, N)
    y.backward(_t(gy))
    gcw_got = CW.grad[:, 0].double() + 1j * CW.grad[:, 1].double()
    errs = {"y": relerr(y, y_ref), "gc1": relerr(C1.grad, gc1_ref),
            "gc2": relerr(C2.grad, gc2_ref), "gcw": relerr(gcw_got.cpu(), gcw_ref),
            "gu": relerr(U.grad, gu_ref.real if real else gu_ref)}
    with torch.no_grad():
        if real:
            yabs = mo._sequential_scan_multi_osc_real_forward_abs_raw(C1, C2, U, CW, N)
        else:
            yabs = mo._sequential_scan_multi_osc_forward_abs_raw(C1, C2, U, CW[:, 0], CW[:, 1], N)
    errs["|y|"] = relerr(yabs, yabs_ref)
    bad = {k: v for k, v in errs.items() if not v <= PARITY_RTOL}
    assert not bad, errs


@pytest.mark.parametrize("F", [40, 65536 + 40])
@pytest.mark.parametrize("real", [False, True])
def test_scan_without_c_weights(F, real):
    """``rqf_multi_osc_fwd`` with no C-weights and N = 1 is the plain scan
    x[t] = C1 x[t-1] + C2 u[t] (complex output), or its magnitude; the Python
    names reach the magnitude (``sequential_scan_abs``), so the complex
    output is called through the C ABI.  Against the oracle's scan; narrow
    rows and rows past one 32-bit descriptor range."""
    from prospective_rqf_amd import _lib

    B, T = 2, 70
    print(f"case: multi-osc no C-weights F={F} real={real}", flush=True)
    rng = np.random.default_rng(F + real)
    c1 = _c64(rng.uniform(0.7, 0.995, F) * np.exp(1j * rng.uniform(0, 2 * np.pi, F)))
    c2 = _c64(0.5 * crandn(rng, F))
    u = rng.standard_normal((B, T, F)) if real else crandn(rng, B, T, F)
    u = np.asarray(u, np.float32).astype(np.float64) if real else _c64(u)
    want = oracle.twotap_fwd(c1, c2, None, np.asarray(u, np.complex128))
    C1, C2, U = _t(c1), _t(c2), _t(u)
    lib = _lib.load()
    for absolute in (False, True):
        out = torch.empty(B, T, F, device="cuda",
                          dtype=torch.float32 if absolute else torch.complex64)
        _lib.check(lib.rqf_multi_osc_fwd(_lib.ptr(C1), _lib.ptr(C2), None, _lib.ptr(U),
                                         int(real), _lib.ptr(out), int(absolute), B, T, F, 1,
                                         None, 0, _lib.stream_of(U)), "rqf_multi_osc_fwd")
        torch.cuda.synchronize()
        assert relerr(out, np.abs(want) if absolute else want) <= PARITY_RTOL, absolute


def test_needs_input_grad_gating_and_parallel_alias():
    rng = np.random.default_rng(5)
    B, T, F, N = 2, 300, 6, 4
    c1, c2, cw, u = _problem(rng, B, T, F, N, False)
    gy = _c64(crandn(rng, B, T, F))
    gu_ref, gc1_ref, gc2_ref, gcw_ref = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    # frozen recurrence: only u and the C-weights need gradients
    C1, C2, U, CW = _t(c1), _t(c2), _t(u, True), _cw_param(cw, True)
    y = mo._triton_parallel_scan_multi_osc(C1, C2, U, CW, N)
    y.backward(_t(gy))
    assert C1.grad is None and C2.grad is None
    assert relerr(U.grad, gu_ref) <= PARITY_RTOL
    gcw_got = CW.grad[:, 0].double() + 1j * CW.grad[:, 1].double()
    assert relerr(gcw_got.cpu(), gcw_ref) <= PARITY_RTOL
    # raw backward with only grad_C1 requested
    g = mo._sequential_scan_multi_osc_backward_raw(_t(c1), _t(c2), _t(u), _cw_param(cw), _t(gy),
                                                   N, compute_grad_C2=False, compute_grad_u=False,
                                                   compute_grad_cw=False)
    assert g[1] is None and g[2] is None and g[3] is None
    assert relerr(g[0], gc1_ref) <= PARITY_RTOL
    assert mo._sequential_scan_multi_osc_backward_raw(
        _t(c1), _t(c2), _t(u), _cw_param(cw), _t(gy), N, compute_grad_C1=False,
        compute_grad_C2=False, compute_grad_u=False, compute_grad_cw=False) == (None,) * 4


@pytest.mark.parametrize("real", [False, True])
@pytest.mark.parametrize("shape,N", [((2, 37, 3), 3), ((3, 2000, 40), 4), ((2, 600, 130), 8),
                                     ((2, 300, 20), 1), ((3, 257, 17), 2)])
def test_gradient_subsets_launch_their_own_variants(shape, N, real):
    """grad_u alone skips the adjoint's C1 tangent and the coefficient sums;
    the coefficient gradients alone skip grad_u.  Each variant runs the same
    arithmetic on what it computes: bit-identical to the full call, which is
    checked against the oracle."""
    B, T, F = shape
    print(f"case: multi-osc gradient subsets {shape} N={N} real={real}", flush=True)
    rng = np.random.default_rng(T + N)
    c1, c2, cw, u = _problem(rng, B, T, F, N, real)
    gy = _c64(crandn(rng, B, T, F))
    gu_ref, gc1_ref, gc2_ref, gcw_ref = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    if real:
        gu_ref = gu_ref.real
    C1, C2, U, CW, GY = _t(c1), _t(c2), _t(u), _cw_param(cw), _t(gy)
    full = mo._backward(C1, C2, U, CW, GY, N, real=real)
    want = (gc1_ref, gc2_ref, gu_ref, gcw_ref)
    for i, name in enumerate(("gc1", "gc2", "gu", "gcw")):
        got = full[i]
        if name == "gcw":
            got = got[:, 0].double() + 1j * got[:, 1].double()
        assert relerr(got, want[i]) <= PARITY_RTOL, name
    only_u = mo._backward(C1, C2, U, CW, GY, N, real=real, compute_grad_C1=False,
                          compute_grad_C2=False, compute_grad_cw=False)
    assert only_u[0] is None and only_u[1] is None and only_u[3] is None
    assert torch.equal(only_u[2], full[2])
    coefs = mo._backward(C1, C2, U, CW, GY, N, real=real, compute_grad_u=False)
    assert coefs[2] is None
    for i in (0, 1, 3):
        assert torch.equal(coefs[i], full[i])


def test_long_memory_filters_at_full_length():
    """Trained-filter magnitudes (|C1| up to 0.9996, ~2500-step memory) over
    T = 16000: the adjoint's C1 tangent grows like t |C1|^t, the regime where float32
    sums are least forgiving."""
    B, T, F, N = 2, 16000, 8, 4
    print(f"case: multi-osc long memory B={B} T={T} F={F} N={N}", flush=True)
    rng = np.random.default_rng(16000)
    r = np.concatenate([np.full(F * N // 2, 0.9996), rng.uniform(0.99, 0.9995, F * N // 2)])
    c1 = _c64(r * np.exp(1j * rng.uniform(-0.2, 0.2, F * N)))
    c2 = _c64(0.02 * crandn(rng, F * N))
    cw = _c64(crandn(rng, F * N))
    u = _c64(crandn(rng, B, T, F))
    gy = _c64(crandn(rng, B, T, F))
    y_ref, _ = oracle.mosc_fwd(c1, c2, cw, u, N)
    gu_ref, gc1_ref, gc2_ref, gcw_ref = oracle.mosc_bwd(c1, c2, cw, u, gy, N)
    C1, C2, U, CW = _t(c1, True), _t(c2, True), _t(u, True), _cw_param(cw, True)
    y = mo._triton_sequential_scan_multi_osc(C1, C2, U, CW, N)
    y.backward(_t(gy))
    gcw_got = CW.grad[:, 0].double() + 1j * CW.grad[:, 1].double()
    errs = {"y": relerr(y, y_ref), "gc1": relerr(C1.grad, gc1_ref),
            "gc2": relerr(C2.grad, gc2_ref), "gcw": relerr(gcw_got.cpu(), gcw_ref),
            "gu": relerr(U.grad, gu_ref),
            "gc1/channel": chanerr(C1.grad, gc1_ref), "gc2/channel": chanerr(C2.grad, gc2_ref),
            "gcw/channel": chanerr(gcw_got.cpu(), gcw_ref)}
    print("  " + " ".join(f"{k} {v:.1e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if not v <= PARITY_RTOL}
    assert not bad, errs


def test_forward_raw_names_match_the_autograd_path():
    rng = np.random.default_rng(9)
    B, T, F, N = 2, 500, 8, 2
    c1, c2, cw, u = _problem(rng, B, T, F, N, False)
    y_ref, _ = oracle.mosc_fwd(c1, c2, cw, u, N)
    CW = _cw_param(cw)
    y = mo._sequential_scan_multi_osc_forward_raw(_t(c1), _t(c2), _t(u), CW[:, 0], CW[:, 1], N)
    assert relerr(y, y_ref) <= PARITY_RTOL
    c1r, c2r, cwr, ur = _problem(rng, B, T, F, N, True)
    yr_ref, _ = oracle.mosc_fwd(c1r, c2r, cwr, ur, N)
    yr = mo._sequential_scan_multi_osc_real_forward_raw(_t(c1r), _t(c2r), _t(ur),
                                                        _cw_param(cwr), N)
    assert relerr(yr, yr_ref) <= PARITY_RTOL


@pytest.mark.parametrize("real", [False, True])
@pytest.mark.parametrize("in_f", [1, 16])
def test_sequential_scan_abs(real, in_f):
    rng = np.random.default_rng(11 + in_f)
    B, T, F = 3, 2000, 16
    c1 = _c64(rng.uniform(0.8, 0.999, F) * np.exp(1j * rng.uniform(0, np.pi, F)))
    c2 = _c64(0.3 * crandn(rng, F))
    u = rng.standard_normal((B, T, in_f)) if real else crandn(rng, B, T, in_f)
    u = np.asarray(u, np.float32).astype(np.float64) if real else _c64(u)
    ue = np.broadcast_to(u, (B, T, F))
    want = np.abs(oracle.twotap_fwd(c1, c2, None, ue.astype(np.complex128)))
    with torch.no_grad():
        got = hip_scan.sequential_scan_abs(_t(c1), _t(c2), _t(u))
    assert got.dtype == torch.float32 and got.shape == (B, T, F)
    assert relerr(got, want) <= PARITY_RTOL
    # with autograd the reference composes sequential_scan(...).abs()
    U = _t(u, True)
    got_g = hip_scan.sequential_scan_abs(_t(c1), _t(c2), U)
    assert got_g.requires_grad and relerr(got_g, want) <= PARITY_RTOL


def test_rejects_bad_oscillator_shapes_and_host_tensors():
    u = torch.zeros(1, 4, 2, dtype=torch.complex64, device="cuda")
    c = torch.zeros(2 * 9, dtype=torch.complex64, device="cuda")
    cw = torch.zeros(2 * 9, 2, device="cuda")
    with pytest.raises(ValueError):
        mo._triton_sequential_scan_multi_osc(c, c, u, cw, 0)
    with pytest.raises(ValueError):  # coefficients for 9 oscillators, 8 claimed
        mo._triton_sequential_scan_multi_osc(c, c, u, cw, 8)
    with pytest.raises(RuntimeError):
        mo._triton_sequential_scan_multi_osc(c.cpu()[:4], c.cpu()[:4], u.cpu(), cw.cpu()[:4], 2)


def test_empty_batch_and_time():
    c = torch.ones(6, dtype=torch.complex64, device="cuda")
    cw = torch.ones(6, 2, device="cuda", requires_grad=True)
    C1 = c.clone().requires_grad_(True)
    u = torch.zeros(0, 5, 3, dtype=torch.complex64, device="cuda", requires_grad=True)
    y = mo._triton_sequential_scan_multi_osc(C1, c, u, cw, 2)
    assert y.shape == (0, 5, 3)
    y.sum().abs().backward()
    assert torch.all(C1.grad == 0) and torch.all(cw.grad == 0)

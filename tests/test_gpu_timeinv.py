"""GPU parity of the time-invariant scans against the fp64 oracle.

Shapes follow the reference's backend parity tests
(tests/test_scan_backends_parity.py:55-106) plus chunk/tile edges.  Bar:
normwise max relative error <= 1e-4 per output and per gradient tensor.
"""

import numpy as np
import pytest
import torch

from oracle import oracle
from prospective_rqf_amd import scan as hip_scan
from prospective_rqf_amd.chunked_scan_kernel import (
    _triton_chunked_scan,
    _triton_chunked_scan_prospective,
)
from prospective_rqf_amd.fbt_scan_kernel import fbt_prospective_scan, fbt_recompute_scan
from tests.helpers import PARITY_RTOL, chanerr, crandn, relerr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _c64(a):
    return np.asarray(a, dtype=np.complex64).astype(np.complex128)


def _coeffs(rng, F):
    mag = rng.uniform(0.8, 0.99, F)
    c1 = _c64(mag * np.exp(1j * rng.uniform(0, 2 * np.pi, F)))
    return c1, _c64(0.1 * crandn(rng, F)), _c64(0.5 * crandn(rng, F))


def _dev(a):
    return torch.as_tensor(np.asarray(a, dtype=np.complex64), device="cuda").requires_grad_(True)


# T at and past 1024- and 2048-step edges (2048, 2049, 1025, 4352) and F past
# filter groups (130, 200).
@pytest.mark.parametrize("shape", [(4, 16000, 32), (2, 1023, 8), (2, 777, 16), (4, 161, 64),
                                   (1, 1, 3), (3, 17, 1), (2, 64, 130), (3, 2048, 64),
                                   (3, 2049, 64), (2, 1025, 200), (2, 4352, 128)])
def test_chunked_scan_matches_oracle(shape):
    B, T, F = shape
    print(f"case: chunked_scan {shape}", flush=True)
    rng = np.random.default_rng(B * 1000 + T + F)
    c1, c2, _ = _coeffs(rng, F)
    u = _c64(crandn(rng, B, T, F))
    gy = _c64(crandn(rng, B, T, F))
    y_ref = oracle.twotap_fwd(c1, c2, None, u)
    gu_ref, gc1_ref, gc2_ref, _ = oracle.twotap_bwd(c1, c2, None, u, y_ref, gy)
    C1, C2, U = _dev(c1), _dev(c2), _dev(u)
    y = _triton_chunked_scan(C1, C2, U)
    y.backward(torch.as_tensor(gy.astype(np.complex64), device="cuda"))
    for name, got, want in (("y", y, y_ref), ("grad_u", U.grad, gu_ref),
                            ("grad_C1", C1.grad, gc1_ref), ("grad_C2", C2.grad, gc2_ref)):
        err = relerr(got, want)
        assert err <= PARITY_RTOL, (name, err)
        if name.startswith(("grad_C", "grad_tap")):
            err = chanerr(got, want)
            assert err <= PARITY_RTOL, (name + "/channel", err)


@pytest.mark.parametrize("shape", [(3, 4096, 32), (2, 300, 5), (1, 2, 7), (2, 2304, 96)])
def test_chunked_prospective_matches_oracle(shape):
    B, T, F = shape
    print(f"case: chunked_prospective {shape}", flush=True)
    rng = np.random.default_rng(3 + T)
    c1, t0, t1 = _coeffs(rng, F)
    x = _c64(crandn(rng, B, T, F))
    gy = _c64(crandn(rng, B, T, F))
    y_ref = oracle.twotap_fwd(c1, t0, t1, x)
    gx_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(c1, t0, t1, x, y_ref, gy)
    C1, T0, T1, X = _dev(c1), _dev(t0), _dev(t1), _dev(x)
    y = _triton_chunked_scan_prospective(C1, T0, T1, X)
    y.backward(torch.as_tensor(gy.astype(np.complex64), device="cuda"))
    for name, got, want in (("y", y, y_ref), ("grad_x", X.grad, gx_ref),
                            ("grad_C1", C1.grad, gc1_ref), ("grad_tap0", T0.grad, gt0_ref),
                            ("grad_tap1", T1.grad, gt1_ref)):
        err = relerr(got, want)
        assert err <= PARITY_RTOL, (name, err)
        if name.startswith(("grad_C", "grad_tap")):
            err = chanerr(got, want)
            assert err <= PARITY_RTOL, (name + "/channel", err)


@pytest.mark.parametrize("variant", ["raw", "act", "recompute"])
@pytest.mark.parametrize("shape", [(16, 8, 3000), (5, 3, 1023), (4, 2, 512), (3, 2, 513),
                                   (2, 2, 1), (7, 3, 16000),
                                   # T a multiple of the 256-step tile: the row-block backward
                                   (3, 2, 4096), (5, 2, 1280), (2, 2, 256)])
def test_fbt_matches_oracle(variant, shape):
    F, B, T = shape
    print(f"case: fbt {variant} {shape}", flush=True)
    rng = np.random.default_rng(F * 7 + B * 3 + T)
    c1, t0, t1 = _coeffs(rng, F)
    z = _c64(crandn(rng, F, B, T))
    gy = _c64(crandn(rng, F, B, T))
    mask = variant != "raw"
    y_ref, act_ref = oracle.twotap_fwd(c1, t0, t1, z, layout=oracle.FBT, act=True)
    gz_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(c1, t0, t1, z, y_ref, gy,
                                                          layout=oracle.FBT, mask_act=mask)
    C1, T0, T1, Z = _dev(c1), _dev(t0), _dev(t1), _dev(z)
    if variant == "recompute":
        y = fbt_recompute_scan(C1, T0, T1, Z)
    else:
        y = fbt_prospective_scan(C1, T0, T1, Z, fuse_act=variant == "act")
    y.backward(torch.as_tensor(gy.astype(np.complex64), device="cuda"))
    out_ref = act_ref if mask else y_ref
    for name, got, want in (("out", y, out_ref), ("grad_z", Z.grad, gz_ref),
                            ("grad_C1", C1.grad, gc1_ref), ("grad_tap0", T0.grad, gt0_ref),
                            ("grad_tap1", T1.grad, gt1_ref)):
        err = relerr(got, want)
        assert err <= PARITY_RTOL, (name, err)
        if name.startswith(("grad_C", "grad_tap")):
            err = chanerr(got, want)
            assert err <= PARITY_RTOL, (name + "/channel", err)


@pytest.mark.parametrize("variant", ["raw", "act", "recompute"])
@pytest.mark.parametrize("T", [512, 513])
def test_fbt_rows_not_16_byte_aligned(variant, T):
    """A drive tensor that starts 8 bytes past a 16-byte boundary (a view at
    an odd complex offset): the kernels take their element-wise row forms,
    the row-block backward included (T = 512, a multiple of the 256-step
    tile)."""
    F, B = 3, 2
    print(f"case: fbt misaligned {variant} T={T}", flush=True)
    rng = np.random.default_rng(T + len(variant))
    c1, t0, t1 = _coeffs(rng, F)
    z = _c64(crandn(rng, F, B, T))
    gy = _c64(crandn(rng, F, B, T))
    mask = variant != "raw"
    y_ref, act_ref = oracle.twotap_fwd(c1, t0, t1, z, layout=oracle.FBT, act=True)
    gz_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(c1, t0, t1, z, y_ref, gy,
                                                          layout=oracle.FBT, mask_act=mask)
    buf = torch.zeros(F * B * T + 1, dtype=torch.complex64, device="cuda")
    buf[1:] = torch.as_tensor(z.astype(np.complex64).reshape(-1), device="cuda")
    Z = buf[1:].view(F, B, T).detach().requires_grad_(True)
    assert Z.data_ptr() % 16 == 8
    C1, T0, T1 = _dev(c1), _dev(t0), _dev(t1)
    if variant == "recompute":
        y = fbt_recompute_scan(C1, T0, T1, Z)
    else:
        y = fbt_prospective_scan(C1, T0, T1, Z, fuse_act=variant == "act")
    y.backward(torch.as_tensor(gy.astype(np.complex64), device="cuda"))
    for name, got, want in (("out", y, act_ref if mask else y_ref), ("grad_z", Z.grad, gz_ref),
                            ("grad_C1", C1.grad, gc1_ref), ("grad_tap0", T0.grad, gt0_ref),
                            ("grad_tap1", T1.grad, gt1_ref)):
        assert relerr(got, want) <= PARITY_RTOL, name


@pytest.mark.parametrize("is_complex", [False, True])
def test_dispatch_real_complex_and_single_feature(is_complex):
    print(f"case: dispatch complex={is_complex}", flush=True)
    rng = np.random.default_rng(4)
    F = 8
    c1, c2, _ = _coeffs(rng, F)
    for in_f in (F, 1):
        u = rng.standard_normal((2, 500, in_f))
        if is_complex:
            u = u + 1j * rng.standard_normal((2, 500, in_f))
        u = np.asarray(u, dtype=np.complex64 if is_complex else np.float32)
        ut = torch.as_tensor(u, device="cuda")
        y_ref = oracle.twotap_fwd(c1, c2, None, np.broadcast_to(u, (2, 500, F)).astype(np.complex128))
        for fn in (hip_scan.sequential_scan, hip_scan.parallel_scan):
            y = fn(torch.as_tensor(c1.astype(np.complex64), device="cuda"),
                   torch.as_tensor(c2.astype(np.complex64), device="cuda"), ut)
            assert y.dtype == torch.complex64 and y.shape == (2, 500, F)
            assert relerr(y, y_ref) <= PARITY_RTOL


def test_empty_inputs():
    c = torch.zeros(3, dtype=torch.complex64, device="cuda", requires_grad=True)
    z = torch.zeros(3, 0, 5, dtype=torch.complex64, device="cuda", requires_grad=True)
    y = fbt_recompute_scan(c, c, c, z)
    assert y.shape == (3, 0, 5)
    y.abs().sum().backward()
    assert float(c.grad.abs().sum()) == 0.0
    u = torch.zeros(0, 4, 3, dtype=torch.complex64, device="cuda", requires_grad=True)
    y2 = _triton_chunked_scan(c, c, u)
    y2.abs().sum().backward()
    assert u.grad.shape == u.shape

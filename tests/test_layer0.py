"""Layer 0 on a real input: ``fbt_layer0_real_scan`` (fbt_scan_kernel.py:899-1032).

GPU parity against an fp64 composition: ``z = (Wr + i Wi) h`` in float64,
the oracle's FBT two-tap scan with the split-ReLU mask and its adjoint
(``oracle.twotap_fwd`` / ``twotap_bwd``, pinned elsewhere against closed
forms and brute force), then the projection's own chain rule in float64:
``grad_h = Re(W^H gz)`` and ``grad_[Wr; Wi] = [Re gz; Im gz] h^T`` with
``gz`` the oracle's drive gradient.  Input widths 1 (raw waveform), 2, 3
and 16 (the one-pass input-gradient kernel, odd and even batch*time), 20
(MFCC features) and 64 (the MFMA GEMM), rows on and off the 256-step tile, and the
``needs_input_grad`` gating.  Bar: normwise relative error <= 1e-4 per
tensor, and per channel (floor 1e-2) for the coefficient gradients.  The
cotangent is zeroed where the fp64 state lies within 1e-4 of its maximum of a
split-ReLU kink: there the mask is decided by rounding, and with long-memory
poles one flipped element moves ``grad_h`` by ~1e-3.

Host-side argument checks run on the CPU (no launch).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from prospective_rqf_amd.fbt_scan_kernel import fbt_layer0_real_scan, fbt_recompute_scan
from tests.helpers import PARITY_RTOL, chanerr, cotangent_off_relu_kink, crandn, relerr


def _coeffs(rng, F):
    c1 = rng.uniform(0.8, 0.995, F) * np.exp(1j * rng.uniform(0, 2 * np.pi, F))
    c = [np.asarray(v, np.complex64).astype(np.complex128)
         for v in (c1, 0.1 * crandn(rng, F), 0.5 * crandn(rng, F))]
    return c


def _f32(a):
    return np.asarray(a, np.float32).astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize("F,D,B,T", [(16, 1, 2, 1000), (8, 20, 3, 4096), (5, 64, 2, 1023),
                                     (3, 2, 1, 1), (32, 1, 4, 16000), (6, 16, 2, 777),
                                     (4, 3, 3, 501),
                                     # one feature: 256-step-aligned rows (row-block
                                     # backward) and rows of odd length (element loads)
                                     (8, 1, 2, 1024), (5, 1, 3, 777)])
def test_layer0_matches_fp64_composition(F, D, B, T):
    from oracle import oracle

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print(f"case: layer0 F={F} D={D} B={B} T={T}", flush=True)
    rng = np.random.default_rng(F * 31 + D * 7 + T)
    c1, t0, t1 = _coeffs(rng, F)
    w = _f32(rng.standard_normal((2 * F, D)) / np.sqrt(D))
    h = _f32(rng.standard_normal((D, B * T)))
    gy = np.asarray(crandn(rng, F, B, T), np.complex64).astype(np.complex128)
    z = ((w[:F] + 1j * w[F:]) @ h).reshape(F, B, T)
    y_ref, act_ref = oracle.twotap_fwd(c1, t0, t1, z, layout=oracle.FBT, act=True)
    # Where the state is within rounding of a split-ReLU kink the fp32 replay
    # and the oracle may take different branches; keep the cotangent off them.
    gy, _ = cotangent_off_relu_kink(y_ref, gy)
    gy = gy.astype(np.complex64).astype(np.complex128)
    gz_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(c1, t0, t1, z, y_ref, gy,
                                                          layout=oracle.FBT, mask_act=True)
    gz2 = gz_ref.reshape(F, B * T)
    gw_ref = np.concatenate([gz2.real @ h.T, gz2.imag @ h.T])
    gh_ref = w[:F].T @ gz2.real + w[F:].T @ gz2.imag

    dev = lambda a, dt: torch.as_tensor(a.astype(dt), device="cuda").requires_grad_(True)  # noqa
    W, H = dev(w, np.float32), dev(h, np.float32)
    C1, T0, T1 = (dev(v, np.complex64) for v in (c1, t0, t1))
    act = fbt_layer0_real_scan(W, H, C1, T0, T1, B)
    assert act.shape == (F, B, T) and act.dtype == torch.complex64
    act.backward(torch.as_tensor(gy.astype(np.complex64), device="cuda"))
    for name, got, want in (("act", act, act_ref), ("grad_w_stacked", W.grad, gw_ref),
                            ("grad_h", H.grad, gh_ref), ("grad_C1", C1.grad, gc1_ref),
                            ("grad_tap0", T0.grad, gt0_ref), ("grad_tap1", T1.grad, gt1_ref)):
        err = relerr(got, want)
        assert err <= PARITY_RTOL, (name, err)
        if name.startswith(("grad_C", "grad_tap")):
            assert chanerr(got, want) <= PARITY_RTOL, (name + "/channel", chanerr(got, want))


@pytest.mark.gpu
def test_layer0_equals_complex_path_and_gates_gradients():
    """Same result as the complex projection into the recompute scan (the
    reference's stated equivalence), and grads only where asked."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("case: layer0 vs complex path", flush=True)
    g = torch.Generator().manual_seed(5)
    F, D, B, T = 12, 4, 2, 777
    w = torch.randn(2 * F, D, generator=g).cuda()
    h = torch.randn(D, B * T, generator=g).cuda()
    c1 = (0.95 * torch.exp(1j * torch.rand(F, generator=g, dtype=torch.float64) * 6.28)).to(
        torch.complex64).cuda()
    t0 = torch.randn(F, generator=g, dtype=torch.complex64).cuda()
    t1 = torch.randn(F, generator=g, dtype=torch.complex64).cuda()
    act = fbt_layer0_real_scan(w, h, c1, t0, t1, B)
    z = (torch.complex(w[:F], w[F:]) @ h.to(torch.complex64)).reshape(F, B, T)
    ref = fbt_recompute_scan(c1, t0, t1, z)
    assert relerr(act, ref) <= 1e-5
    # Only h asks for a gradient.
    hh = h.clone().requires_grad_(True)
    out = fbt_layer0_real_scan(w, hh, c1, t0, t1, B)
    out.real.sum().backward()
    assert hh.grad is not None and hh.grad.shape == h.shape and torch.isfinite(hh.grad).all()


@pytest.mark.parametrize("bad", ["odd_rows", "complex_w", "width", "batch"])
def test_layer0_rejects_bad_shapes_before_launch(bad):
    F, D, B, T = 4, 3, 2, 10
    w = torch.zeros(2 * F, D)
    h = torch.zeros(D, B * T)
    c = torch.zeros(F, dtype=torch.complex64)
    batch = B
    if bad == "odd_rows":
        w = torch.zeros(2 * F + 1, D)
    elif bad == "complex_w":
        w = torch.zeros(2 * F, D, dtype=torch.complex64)
    elif bad == "width":
        h = torch.zeros(D + 1, B * T)
    else:
        batch = 3
    with pytest.raises(ValueError):
        fbt_layer0_real_scan(w, h, c, c, c, batch)


@pytest.mark.gpu
@pytest.mark.parametrize("D,n", [(1, 2000), (2, 64000), (2, 4100)])
def test_layer0_grads_read_no_element_past_grad_z(D, n):
    """``rqf_layer0_grads`` with 16-byte loads (n % 4 == 0) and n not a
    multiple of a block's 1024 columns: grad_z is the front of a larger buffer
    whose tail is NaN, so any load past its end would turn grad_w / grad_h
    into NaN.  Both must match the fp64 chain rule."""
    from prospective_rqf_amd.fbt_scan_kernel import _layer0_grads

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print(f"case: layer0 grads NaN tail D={D} n={n}", flush=True)
    rng = np.random.default_rng(n + D)
    F = 3
    w = _f32(rng.standard_normal((2 * F, D)))
    h = _f32(rng.standard_normal((D, n)))
    gz = np.asarray(crandn(rng, F, n), np.complex64).astype(np.complex128)
    buf = torch.full((F * n + 4096,), complex(float("nan"), float("nan")),
                     dtype=torch.complex64, device="cuda")
    buf[:F * n] = torch.as_tensor(gz.astype(np.complex64).reshape(-1), device="cuda")
    gz_dev = buf[:F * n].view(F, n)
    W = torch.as_tensor(w.astype(np.float32), device="cuda")
    H = torch.as_tensor(h.astype(np.float32), device="cuda")
    grad_w, grad_h = _layer0_grads(W, gz_dev, H, True, True)
    torch.cuda.synchronize()
    gw_ref = np.concatenate([gz.real @ h.T, gz.imag @ h.T])
    gh_ref = w[:F].T @ gz.real + w[F:].T @ gz.imag
    assert torch.isfinite(grad_w).all() and torch.isfinite(grad_h).all()
    assert relerr(grad_w, gw_ref) <= PARITY_RTOL
    assert relerr(grad_h, gh_ref) <= PARITY_RTOL


@pytest.mark.gpu
def test_layer0_input_not_16_byte_aligned():
    """One input feature whose row starts 4 bytes past a 16-byte boundary:
    the scan kernels form the drive with element loads (the row-block
    backward on 256-step-aligned rows included)."""
    from oracle import oracle

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    F, D, B, T = 6, 1, 2, 512
    print(f"case: layer0 misaligned F={F} B={B} T={T}", flush=True)
    rng = np.random.default_rng(17)
    c1, t0, t1 = _coeffs(rng, F)
    w = _f32(rng.standard_normal((2 * F, D)))
    h = _f32(rng.standard_normal((D, B * T)))
    gy = np.asarray(crandn(rng, F, B, T), np.complex64).astype(np.complex128)
    z = ((w[:F] + 1j * w[F:]) @ h).reshape(F, B, T)
    y_ref, act_ref = oracle.twotap_fwd(c1, t0, t1, z, layout=oracle.FBT, act=True)
    gy, _ = cotangent_off_relu_kink(y_ref, gy)
    gy = gy.astype(np.complex64).astype(np.complex128)
    gz_ref, gc1_ref, _, _ = oracle.twotap_bwd(c1, t0, t1, z, y_ref, gy, layout=oracle.FBT,
                                              mask_act=True)
    gh_ref = w[:F].T @ gz_ref.reshape(F, B * T).real + w[F:].T @ gz_ref.reshape(F, B * T).imag
    buf = torch.zeros(B * T + 1, dtype=torch.float32, device="cuda")
    buf[1:] = torch.as_tensor(h.astype(np.float32).reshape(-1), device="cuda")
    H = buf[1:].view(D, B * T).detach().requires_grad_(True)
    assert H.data_ptr() % 16 == 4
    W = torch.as_tensor(w.astype(np.float32), device="cuda").requires_grad_(True)
    C1 = torch.as_tensor(c1.astype(np.complex64), device="cuda").requires_grad_(True)
    T0, T1 = (torch.as_tensor(v.astype(np.complex64), device="cuda") for v in (t0, t1))
    act = fbt_layer0_real_scan(W, H, C1, T0, T1, B)
    act.backward(torch.as_tensor(gy.astype(np.complex64), device="cuda"))
    for name, got, want in (("act", act, act_ref), ("grad_h", H.grad, gh_ref),
                            ("grad_C1", C1.grad, gc1_ref)):
        assert relerr(got, want) <= PARITY_RTOL, name


@pytest.mark.gpu
@pytest.mark.parametrize("D", [1, 2, 3, 5, 9])
@pytest.mark.parametrize("need", ["both", "weights", "input"])
@pytest.mark.parametrize("n", [2000, 2001])
def test_layer0_grads_every_variant(D, need, n):
    """``rqf_layer0_grads`` for each input width class (1, 2; 3-4, 5-8, 9-16
    for the input gradient alone), each gradient subset the one-pass kernel
    serves, and rows of 16-byte and element loads (n % 4 == 0 or not).
    Against the fp64 chain rule."""
    from prospective_rqf_amd.fbt_scan_kernel import _layer0_grads

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    need_w, need_h = need in ("both", "weights"), need in ("both", "input")
    print(f"case: layer0 grads D={D} need={need} n={n}", flush=True)
    rng = np.random.default_rng(D * 10 + n)
    F = 4
    w = _f32(rng.standard_normal((2 * F, D)))
    h = _f32(rng.standard_normal((D, n)))
    gz = np.asarray(crandn(rng, F, n), np.complex64).astype(np.complex128)
    W = torch.as_tensor(w.astype(np.float32), device="cuda")
    H = torch.as_tensor(h.astype(np.float32), device="cuda")
    GZ = torch.as_tensor(gz.astype(np.complex64), device="cuda")
    grad_w, grad_h = _layer0_grads(W, GZ, H, need_w, need_h)
    torch.cuda.synchronize()
    if need_w:
        assert relerr(grad_w, np.concatenate([gz.real @ h.T, gz.imag @ h.T])) <= PARITY_RTOL
    else:
        assert grad_w is None
    if need_h:
        assert relerr(grad_h, w[:F].T @ gz.real + w[F:].T @ gz.imag) <= PARITY_RTOL
    else:
        assert grad_h is None

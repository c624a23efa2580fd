"""GPU parity of the fused projection GEMM (csrc/proj.hip) and the split weight
gradient on the device.

The fused forward must equal ``weight @ x`` and ``heads @ cat(x.real, x.imag)``
(rqf_models/ops/selective_scan.py:117-118, rqf_models/backbones/rqf/
selective.py:205-217); the fused input gradient must equal
``weight.mH @ dz + complex(dv[:D], dv[D:])`` with ``dv = heads.T @ cat(grads)``
(selective_scan.py:144, selective.py:96).  Expected values are fp64 products on
the CPU of the same fp32/complex64 inputs.  Bar: normwise relative error
<= 1e-4 (the products are fp32 sums of up to 1032 terms).
"""

import numpy as np
import pytest
import torch

from prospective_rqf_amd.projection import fused_dx, fused_forward, weight_grad
from tests.helpers import PARITY_RTOL, relerr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _c(rng, *shape):
    return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(np.complex64)


# (F, D, ml, N): shapes of the bench layer, odd sizes, no selector heads, odd N,
# N below one tile, rows straddling the 128-row tiles.
SHAPES = [(256, 256, 520, 64 * 1000), (5, 3, 7, 1001), (48, 48, 0, 4096), (16, 40, 37, 130),
          (1, 1, 1, 1), (130, 70, 3, 2 * 129)]


@pytest.mark.parametrize("shape", SHAPES)
def test_fused_forward_matches_the_two_gemms(shape):
    F, D, ml, N = shape
    print(f"case: fused forward {shape}", flush=True)
    rng = np.random.default_rng(F + D + ml + N)
    x, W = _c(rng, D, N), _c(rng, F, D) / np.float32(np.sqrt(D))
    heads = rng.standard_normal((ml, 2 * D)).astype(np.float32) if ml else None
    dev = lambda a: None if a is None else torch.as_tensor(a, device="cuda")  # noqa: E731
    z, logits = fused_forward(dev(x), dev(W), dev(heads))
    x64 = x.astype(np.complex128)
    assert relerr(z, W.astype(np.complex128) @ x64) <= PARITY_RTOL
    if ml:
        v = np.concatenate([x64.real, x64.imag], 0)
        assert relerr(logits, heads.astype(np.float64) @ v) <= PARITY_RTOL
    else:
        assert logits is None


@pytest.mark.parametrize("blocks", [(256, 8, 256), (3, 0, 4), (7,), ()])
@pytest.mark.parametrize("N", [64 * 1000, 1001, 130])
def test_fused_dx_matches_the_two_gemms_and_the_add(blocks, N):
    F, D = (256, 256) if blocks and blocks[0] == 256 else (6, 9)
    print(f"case: fused dx F={F} D={D} blocks={blocks} N={N}", flush=True)
    rng = np.random.default_rng(F + N + len(blocks))
    dz, W = _c(rng, F, N), _c(rng, F, D)
    ml = sum(blocks)
    heads = rng.standard_normal((ml, 2 * D)).astype(np.float32) if blocks else None
    grads = [rng.standard_normal((r, N)).astype(np.float32) for r in blocks]
    dev = lambda a: torch.as_tensor(a, device="cuda")  # noqa: E731
    dx = fused_dx(dev(dz), [dev(g) for g in grads], dev(W), None if heads is None else dev(heads))
    want = W.astype(np.complex128).conj().T @ dz.astype(np.complex128)
    if blocks:
        dv = heads.astype(np.float64).T @ np.concatenate(grads, 0).astype(np.float64)
        want = want + dv[:D] + 1j * dv[D:]
    assert relerr(dx, want) <= PARITY_RTOL


def test_fused_forward_on_strided_and_conjugate_inputs():
    print("case: fused forward views", flush=True)
    rng = np.random.default_rng(3)
    x, W = _c(rng, 24, 300), _c(rng, 8, 12)
    xt = torch.as_tensor(x, device="cuda")[::2]  # every other input row: a strided view
    z, _ = fused_forward(xt.conj(), torch.as_tensor(W, device="cuda"))
    assert relerr(z, W.astype(np.complex128) @ x[::2].astype(np.complex128).conj()) <= PARITY_RTOL


@pytest.mark.parametrize("complex_", [True, False])
def test_weight_grad_on_device(complex_):
    print(f"case: weight_grad complex={complex_}", flush=True)
    rng = np.random.default_rng(7)
    M, K, N = 64, 48, 300007
    if complex_:
        g, x = _c(rng, M, N), _c(rng, K, N)
        want = g.astype(np.complex128) @ x.astype(np.complex128).conj().T
    else:
        g = rng.standard_normal((M, N)).astype(np.float32)
        x = rng.standard_normal((K, N)).astype(np.float32)
        want = g.astype(np.float64) @ x.astype(np.float64).T
    got = weight_grad(torch.as_tensor(g, device="cuda"), torch.as_tensor(x, device="cuda"))
    assert relerr(got, want) <= PARITY_RTOL

"""FBT scans on one row longer than 2^30 steps.

The row-block kernels move each full tile through LDS from the row pointer
advanced to the tile's first step.  That advance is a 64-bit scalar offset:
a 32-bit step offset counted in floats passes 2^31 at 2^30 steps.  Each case
is one row (F = B = 1) that is zero but for a seeded tail of L steps:

* ``fbt_recompute_scan`` at T = 2^30 + 2048 (a multiple of the 256-step tile:
  row-block forward and row-block backward, split-ReLU mask);
* ``fbt_prospective_scan`` at T = 2^30 + 1000 (row-block forward with a
  partial last tile, the per-row backward), raw output.

Before the tail the drive, the state and every coefficient-gradient term are
zero, so the fp64 oracle over the last W steps gives the outputs and grad_z
in that window and the whole coefficient gradients.  The first steps of the
row must stay zero.  Bar: the suite's parity bar.  A complex tensor of the
row is 8 GiB; a case holds about 40 GiB of device memory.
"""

import numpy as np
import pytest
import torch

from oracle import oracle
from prospective_rqf_amd.fbt_scan_kernel import fbt_prospective_scan, fbt_recompute_scan
from tests.helpers import PARITY_RTOL, crandn, relerr

pytestmark = pytest.mark.gpu

L = 3000  # nonzero tail
W = 4096  # window checked against the oracle (L plus zero steps before it)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    yield
    torch.cuda.empty_cache()


@pytest.mark.parametrize("variant,T", [("recompute", 2**30 + 2048), ("prospective", 2**30 + 1000)])
def test_fbt_row_past_2_30_steps(variant, T):
    print(f"case: fbt {variant} F=1 B=1 T={T}", flush=True)
    rng = np.random.default_rng(T % 1000 + 17)
    mag = rng.uniform(0.5, 0.9, 1)
    c1 = (mag * np.exp(1j * rng.uniform(0, 2 * np.pi, 1))).astype(np.complex64)
    t0 = crandn(rng, 1).astype(np.complex64)
    t1 = (0.5 * crandn(rng, 1)).astype(np.complex64)
    z_tail = crandn(rng, 1, 1, L).astype(np.complex64)
    gy_tail = crandn(rng, 1, 1, L).astype(np.complex64)

    z_w = np.zeros((1, 1, W), np.complex128)
    z_w[..., W - L:] = z_tail
    gy_w = np.zeros((1, 1, W), np.complex128)
    gy_w[..., W - L:] = gy_tail
    mask = variant == "recompute"
    d = lambda a: a.astype(np.complex128)
    y_ref, act_ref = oracle.twotap_fwd(d(c1), d(t0), d(t1), z_w, layout=oracle.FBT, act=True)
    gz_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(d(c1), d(t0), d(t1), z_w, y_ref, gy_w,
                                                          layout=oracle.FBT, mask_act=mask)

    dev = lambda a: torch.as_tensor(a, device="cuda").requires_grad_(True)
    C1, T0, T1 = dev(c1), dev(t0), dev(t1)
    Z = torch.zeros(1, 1, T, dtype=torch.complex64, device="cuda")
    Z[..., T - L:] = torch.as_tensor(z_tail, device="cuda")
    Z.requires_grad_(True)
    if variant == "recompute":
        y = fbt_recompute_scan(C1, T0, T1, Z)
    else:
        y = fbt_prospective_scan(C1, T0, T1, Z, fuse_act=False)
    gy = torch.zeros_like(Z, requires_grad=False)
    gy[..., T - L:] = torch.as_tensor(gy_tail, device="cuda")
    y.backward(gy)
    del gy
    torch.cuda.synchronize()
    head_y = y[..., :256].detach().abs().max().item()
    y_w = y[..., T - W:].detach().clone()
    del y
    gz_w = Z.grad[..., T - W:].clone()
    out_ref = act_ref if mask else y_ref
    for name, got, want in (("out", y_w, out_ref), ("grad_z", gz_w, gz_ref),
                            ("grad_C1", C1.grad, gc1_ref), ("grad_tap0", T0.grad, gt0_ref),
                            ("grad_tap1", T1.grad, gt1_ref)):
        err = relerr(got, want)
        assert err <= PARITY_RTOL, (name, err)
    assert head_y == 0.0, head_y

"""The no-allocation entry point ``rqf_fbt_recompute_bwd_noalloc``.

It runs the kernels of ``rqf_fbt_recompute_bwd`` with their per-row partial
sums in the library's static per-GPU scratch instead of a workspace, so its
results must equal that entry point's bit for bit.  Two calls in a row, the
second smaller, check that nothing of the first call's scratch contents leaks
into the second; the last one is on unaligned rows (the other backward
kernel).  Both are called through the C ABI.
"""

import ctypes

import pytest
import torch

from prospective_rqf_amd import _lib, workloads
from prospective_rqf_amd.fbt_scan_kernel import (
    fbt_recompute_backward_noalloc,
    fbt_recompute_forward_raw,
)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _cn(g, *shape):
    return torch.complex(torch.randn(*shape, generator=g, device="cuda"),
                         torch.randn(*shape, generator=g, device="cuda"))


def _with_workspace(c1, t0, t1, x, carry, gy):
    """The existing entry point, rqf_fbt_recompute_bwd, with a workspace."""
    F, B, T = x.shape
    lib = _lib.load()
    n = lib.rqf_fbt_workspace(F, B, T)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    gz = torch.empty_like(x)
    gc = [torch.empty(F, dtype=torch.complex64, device="cuda") for _ in range(3)]
    _lib.check(lib.rqf_fbt_recompute_bwd(
        _lib.ptr(c1), _lib.ptr(t0), _lib.ptr(t1), _lib.ptr(x), _lib.ptr(carry), _lib.ptr(gy),
        _lib.ptr(gz), *(_lib.ptr(v) for v in gc), F, B, T, _lib.ptr(ws), n,
        _lib.stream_of(x)), "rqf_fbt_recompute_bwd")
    return (*gc, gz)


def _noalloc_c_abi(c1, t0, t1, x, carry, gy, outs):
    F, B, T = x.shape
    gc1, gt0, gt1, gz = outs
    rc = _lib.load().rqf_fbt_recompute_bwd_noalloc(
        _lib.ptr(c1), _lib.ptr(t0), _lib.ptr(t1), _lib.ptr(x), _lib.ptr(carry), _lib.ptr(gy),
        _lib.ptr(gz), _lib.ptr(gc1), _lib.ptr(gt0), _lib.ptr(gt1), F, B, T, _lib.stream_of(x))
    return rc


def _problem(F, B, T, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    c = workloads.static_two_tap(F, device="cuda", seed=seed)
    x, gy = _cn(g, F, B, T), _cn(g, F, B, T)
    act, carry, (c1, t0, t1, xs) = fbt_recompute_forward_raw(*c, x)
    return c1, t0, t1, xs, carry, gy


@pytest.mark.parametrize("shapes", [((64, 16, 4096), (16, 4, 1280), (8, 2, 3001))])
def test_noalloc_equals_workspace_entry_point(shapes):
    for i, (F, B, T) in enumerate(shapes):
        print(f"case: no-alloc call {i} F={F} B={B} T={T}", flush=True)
        c1, t0, t1, x, carry, gy = _problem(F, B, T, seed=10 + i)
        want = _with_workspace(c1, t0, t1, x, carry, gy)
        # outputs pre-filled with garbage: every element must be overwritten
        outs = [torch.full((F,), complex(7.0, -7.0), dtype=torch.complex64, device="cuda")
                for _ in range(3)] + [torch.full_like(x, complex(9.0, 9.0))]
        assert _noalloc_c_abi(c1, t0, t1, x, carry, gy, outs) == 0
        torch.cuda.synchronize()
        for name, got, ref in zip(("grad_C1", "grad_tap0", "grad_tap1", "grad_z"), outs, want):
            assert torch.equal(got, ref), (i, name)


def test_noalloc_python_wrapper_and_size_limit():
    F, B, T = 32, 8, 2048
    print(f"case: no-alloc wrapper F={F} B={B} T={T}", flush=True)
    c1, t0, t1, x, carry, gy = _problem(F, B, T, seed=3)
    want = _with_workspace(c1, t0, t1, x, carry, gy)
    outs = [torch.empty(F, dtype=torch.complex64, device="cuda") for _ in range(3)]
    gz = torch.empty_like(x)
    got = fbt_recompute_backward_noalloc(c1, t0, t1, x, carry, gy, gz, *outs)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    # beyond the scratch: rejected on the host, nothing launched
    rows = _lib.NOALLOC_SCRATCH_BYTES // 48
    rc = _lib.load().rqf_fbt_recompute_bwd_noalloc(*([None] * 10), rows + 1, 1, 16,
                                                    ctypes.c_void_p(0))
    assert rc == _lib.ERR_SCRATCH
    with pytest.raises(ValueError):
        fbt_recompute_backward_noalloc(c1, t0, t1, x, carry, gy, gz[:, :, :-1], *outs)

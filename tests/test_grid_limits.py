"""Launch-size limits of the C ABI, on the host.

A dispatch counts its work-items in 32 bits; a grid past 2^32 - 1 of them
would run truncated with no launch error.  Each entry point therefore
refuses, with RQF_ERR_ARG and before launching anything, a shape whose scan
grid needs more (the bounds are in include/rqf_scan.h).  These calls use
shapes one step past each bound and stand-in device pointers (aligned,
non-null, never dereferenced on the host).  Without the check, the call
would reach a HIP launch, and on this GPU-less host that returns a HIP
error code, not RQF_ERR_ARG.  Stand-in pointers must never reach a device,
so the module is skipped where one is visible.  The GPU side (results at
each bound, refusal one step past it) is tests/test_gpu_grid_limits.py.
"""

import ctypes

import pytest
import torch

from prospective_rqf_amd import _lib
from prospective_rqf_amd.build import LIB_PATH

pytestmark = pytest.mark.skipif(torch.cuda.is_available(),
                                reason="stand-in device pointers: host-side checks only")

P = 0x10000  # stand-in device pointer: non-null and 16-byte aligned
WS = 1 << 62  # workspace size that passes every workspace check
ERR_ARG = -1

BTF_BLOCKS = (2**32 - 1) // 512  # (B,T,F) scans: blocks of 512 threads
ROWS = (2**32 - 1) // 512  # FBT and selective forwards: one 512-thread block per row


@pytest.fixture(scope="module")
def lib():
    import os

    if not os.path.exists(LIB_PATH):
        from prospective_rqf_amd.build import build

        build()
    return _lib.load()


def test_btf_scans(lib):
    F = (BTF_BLOCKS + 1) * 16  # one 16-filter block past the bound at B = 1
    assert lib.rqf_chunked_scan_fwd(P, P, P, P, 1, 2, F, None, 0, None) == ERR_ARG
    assert lib.rqf_chunked_prospective_fwd(P, P, P, P, P, 1, 2, F, None, 0, None) == ERR_ARG
    assert lib.rqf_chunked_scan_bwd(P, P, P, None, P, P, P, P, 1, 2, F, P, WS, None) == ERR_ARG
    assert lib.rqf_chunked_prospective_bwd(P, P, P, P, None, P, P, P, P, P, 1, 2, F, P, WS,
                                           None) == ERR_ARG
    # the same blocks through the batch: B * ceil(F / 16) counts
    assert lib.rqf_chunked_scan_fwd(P, P, P, P, BTF_BLOCKS + 1, 2, 16, None, 0, None) == ERR_ARG


def test_multi_osc(lib):
    blocks = (2**32 - 1) // 1024  # forward blocks of up to 16 wavefronts
    assert lib.rqf_multi_osc_workspace(1, 2, blocks * 16, 1, 1) > 0
    F = (blocks + 1) * 16
    assert lib.rqf_multi_osc_workspace(1, 2, F, 1, 1) == 0
    assert lib.rqf_multi_osc_fwd(P, P, P, P, 0, P, 0, 1, 2, F, 1, P, WS, None) == ERR_ARG
    assert lib.rqf_multi_osc_bwd(P, P, P, P, 0, P, P, P, P, P, 1, 2, F, 1, P, WS,
                                 None) == ERR_ARG


def test_fbt_scans(lib):
    F, B = ROWS + 1, 1
    assert lib.rqf_fbt_prospective_fwd(P, P, P, P, P, None, F, B, 2, None) == ERR_ARG
    assert lib.rqf_fbt_recompute_fwd(P, P, P, P, P, P, F, B, 2, None) == ERR_ARG
    assert lib.rqf_fbt_recompute_skip_fwd(P, P, P, P, P, P, P, F, B, 2, None) == ERR_ARG
    assert lib.rqf_fbt_layer0_fwd(P, P, P, P, P, P, P, F, B, 4, None) == ERR_ARG
    # backward: 4-wavefront row blocks (T a multiple of 256) take twice the rows
    F = (2**32 - 1) // 256 + 1
    assert lib.rqf_fbt_recompute_bwd(P, P, P, P, P, P, P, P, P, P, F, B, 256, P, WS,
                                     None) == ERR_ARG
    assert lib.rqf_fbt_prospective_bwd(P, P, P, P, P, P, 0, P, P, P, P, F, B, 256, P, WS,
                                       None) == ERR_ARG


def _selective(F, B, T, warp):
    s = _lib.SelectiveInputsStruct()
    s.F, s.B, s.T, s.G = F, B, T, 1
    for name in ("gamma_logits", "warp_logits", "write_logits", "bias", "theta", "minimum",
                 "span", "step", "horizon", "theta_minimum", "theta_maximum", "groups"):
        setattr(s, name, P)
    s.has_gamma, s.has_write, s.has_warp = 1, 1, warp
    s.write_sigmoid, s.prospective, s.bound_warp = 1, 1, 1
    s.gamma_scale, s.warp_scale, s.write_max = 1.0, 1.0, 1.0
    return s


def test_selective(lib, monkeypatch):
    # forward rows: 8 XCD chunks of ceil(B / 8) batch elements, times F
    s = _selective(ROWS // 8 + 1, 8, 2, 1)
    assert lib.rqf_selective_fwd(ctypes.byref(s), P, 256, P, P, P, None) == ERR_ARG
    assert lib.rqf_selective_skip_fwd(ctypes.byref(s), P, 256, P, P, P, P, None) == ERR_ARG
    # backward in the group form ((group, batch element) blocks of 12
    # wavefronts), and without a warp head in the split form (4-wavefront team
    # blocks: 8 XCD chunks x 2 team slots x ceil(B / 8))
    monkeypatch.setenv("RQF_BWD_FORM", "group")
    for warp, B in ((1, (2**32 - 1) // 768 + 1), (0, 8 * ((2**32 - 1) // 256 // 16 + 1))):
        s = _selective(1, B, 2, warp)
        rc = lib.rqf_selective_bwd(ctypes.byref(s), P, P, 256, P, P, 1, 0, P, P, P, P, P, P, P,
                                   P, WS, None)
        assert rc == ERR_ARG, (warp, rc)
    # an empty backward (T = 0) still reduces dbias / dtheta, one wavefront
    # per channel in 4-wavefront blocks
    s = _selective(4 * ((2**32 - 1) // 256 + 1), 1, 0, 1)
    rc = lib.rqf_selective_bwd(ctypes.byref(s), P, P, 256, P, P, 1, 0, P, P, P, P, P, P, P, P,
                               WS, None)
    assert rc == ERR_ARG, rc


def test_layer0_grads(lib):
    n = ((2**32 - 1) // 256 + 1) * 256 * 4  # 256-thread blocks of 4 columns each
    assert lib.rqf_layer0_grads(P, P, P, P, None, 4, 1, n, None, 0, None) == ERR_ARG


def test_proj_gemm(lib):
    a = _lib.ProjGemmArgs()
    a.weights, a.k_pad, a.m_pad = P, 16, 128
    a.b_cplx, a.b_cplx_rows = P, 8
    a.out_cplx, a.out_cplx_rows = P, 8
    a.n = ((2**32 - 1) // 256 + 1) * 256  # >= one 256-thread tile per 256 columns
    assert lib.rqf_proj_gemm(ctypes.byref(a), None) == ERR_ARG

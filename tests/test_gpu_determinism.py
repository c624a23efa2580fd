"""Run-to-run determinism of every backward, bit for bit.

The library reduces coefficient and warp-group gradients from per-row or
per-split partial sums in a fixed order, with no floating-point atomics, so a
repeated call on the same inputs must return identical bits (the reference's
selective path promises this too, docs/selective_rqf.md:114).  The shapes
are large enough to spread each reduction over many blocks: several splits per
warp group in the selective backward, many segments and tasks in the
single-pass (B,T,F) and multi-oscillator scans.
"""

import numpy as np
import pytest
import torch

from prospective_rqf_amd import multi_osc_scan as mo
from prospective_rqf_amd import workloads
from prospective_rqf_amd.chunked_scan_kernel import (
    _chunked_prospective_backward_raw,
    _chunked_prospective_forward_raw,
    _chunked_scan_backward_raw,
    _chunked_scan_forward_raw,
)
from prospective_rqf_amd.fbt_scan_kernel import (
    _FBTProspectiveScan,
    fbt_recompute_backward_raw,
    fbt_recompute_forward_raw,
)
from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _cn(g, *shape):
    return torch.complex(torch.randn(*shape, generator=g, device="cuda"),
                         torch.randn(*shape, generator=g, device="cuda"))


def _same(a, b, what):
    assert len(a) == len(b)
    for i, (x, y) in enumerate(zip(a, b)):
        if x is None:
            assert y is None, (what, i)
        else:
            assert torch.equal(x, y), (what, i)


@pytest.mark.parametrize("form", ["group", "split"])
@pytest.mark.parametrize("truncated", [False, True])
def test_selective_repeat_bitwise(monkeypatch, truncated, form):
    """16 channels per warp group = 4 teams: all four in one block (group
    form), or two teams per split = two split rows per group summed by the
    split reduction."""
    F, B, T, G, chunk = 64, 8, 4096, 4, 256
    print(f"case: selective repeat F={F} B={B} T={T} G={G} truncated={truncated} "
          f"form={form}", flush=True)
    if form == "group":
        monkeypatch.setenv("RQF_BWD_FORM", "group")
    else:
        monkeypatch.setenv("RQF_BWD_SPLIT_TEAMS", "2")
    g = torch.Generator(device="cuda").manual_seed(5)
    inp = workloads.selective_inputs(F, B, T, G=G, device="cuda", seed=3)
    z, gy, gx = _cn(g, F, B, T), _cn(g, F, B, T), _cn(g, F, B, T)
    f1 = selective_forward(z, inp, True, True, chunk)
    f2 = selective_forward(z, inp, True, True, chunk)
    _same(f1, f2, "forward")
    b1 = selective_backward(z, inp, f1[2], gy, gx, True, truncated, chunk)
    b2 = selective_backward(z, inp, f1[2], gy, gx, True, truncated, chunk)
    _same(b1, b2, "backward")


def test_fbt_recompute_and_prospective_repeat_bitwise():
    F, B, T = 16, 4, 16384
    print(f"case: fbt repeat F={F} B={B} T={T}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(6)
    c = workloads.static_two_tap(F, device="cuda", seed=4)
    x, gy = _cn(g, F, B, T), _cn(g, F, B, T)
    a1, k1, saved = fbt_recompute_forward_raw(*c, x)
    a2, k2, _ = fbt_recompute_forward_raw(*c, x)
    _same((a1, k1), (a2, k2), "recompute forward")
    _same(fbt_recompute_backward_raw(*saved, k1, gy), fbt_recompute_backward_raw(*saved, k1, gy),
          "recompute backward")
    # unaligned rows take the per-row backward
    xu, gu = x[:, :, :3001].contiguous(), gy[:, :, :3001].contiguous()
    outs = []
    for _ in range(2):
        leaves = [v.clone().requires_grad_(True) for v in (*c, xu)]
        y = _FBTProspectiveScan.apply(*leaves, True)
        y.backward(gu)
        outs.append((y.detach(), *(v.grad for v in leaves)))
    _same(outs[0], outs[1], "prospective")


def test_chunked_repeat_bitwise():
    B, T, F = 4, 4096, 64
    print(f"case: chunked repeat B={B} T={T} F={F}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7)
    c = workloads.static_two_tap(F, device="cuda", seed=5)
    u, gy = _cn(g, B, T, F), _cn(g, B, T, F)
    _same([_chunked_scan_forward_raw(c[0], c[1], u)], [_chunked_scan_forward_raw(c[0], c[1], u)],
          "chunked forward")
    _same(_chunked_scan_backward_raw(c[0], c[1], u, None, gy),
          _chunked_scan_backward_raw(c[0], c[1], u, None, gy), "chunked backward")
    _same([_chunked_prospective_forward_raw(*c, u)], [_chunked_prospective_forward_raw(*c, u)],
          "prospective forward")
    _same(_chunked_prospective_backward_raw(*c, u, None, gy),
          _chunked_prospective_backward_raw(*c, u, None, gy), "prospective backward")


def test_multi_osc_repeat_bitwise():
    B, T, F, N = 2, 4000, 32, 4
    print(f"case: multi-osc repeat B={B} T={T} F={F} N={N}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(8)
    rng = np.random.default_rng(8)
    c1 = torch.as_tensor(rng.uniform(0.9, 0.999, F * N) * np.exp(1j * rng.uniform(0, 3, F * N)),
                         dtype=torch.complex64, device="cuda")
    c2 = _cn(g, F * N)
    cw = torch.randn(F * N, 2, generator=g, device="cuda")
    u, gy = _cn(g, B, T, F), _cn(g, B, T, F)
    r1 = mo._sequential_scan_multi_osc_backward_raw(c1, c2, u, cw, gy, N)
    r2 = mo._sequential_scan_multi_osc_backward_raw(c1, c2, u, cw, gy, N)
    _same(r1, r2, "multi-osc backward")

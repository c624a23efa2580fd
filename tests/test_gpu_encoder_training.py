"""A small selective encoder trained for three AdamW steps through the HIP kernels
matches the same encoder trained through the PyTorch restatement.

Mirrors the reference's ``test_encoder_dispatch_and_optimizer``
(tests/test_selective_cuda.py:271-298): a selective Pure RQF stack with a
skip connection, full BPTT and TBPTT(1), selector source the layer input or
the layer output (``source = raw + h``, pure.py:486-496), three AdamW steps
of ``mean |h|^2`` with the filter projection (``clamp_parameters``) after each
step, then the trained models' outputs are compared.

Here the stack is assembled from this package's pieces: the restated
controller (``selective_controller``, pinned bit for bit against the
reference's) builds each layer's scan inputs from trainable heads and filter
leaves, and ``selective_layer_scan`` runs the drive GEMM and the kernels.  The
expected model runs the same stack in float64 on the CPU with the PyTorch
restatement of ``reference_layer_scan`` (oracle/torch_ref.py) in place of the
kernels.  The reference compares at rtol 3e-3 / atol 3e-4; this bar is
normwise relative error <= 1e-4 on the trained outputs and on every trained
parameter.
"""

from __future__ import annotations

import copy
import math

import pytest
import torch

from oracle import torch_ref
from prospective_rqf_amd import workloads
from prospective_rqf_amd.selective_controller import SelectiveController, SelectiveRQFConfig
from prospective_rqf_amd.selective_scan import selective_layer_scan
from tests.helpers import PARITY_RTOL, relerr

pytestmark = pytest.mark.gpu

F, B, T, G, LAYERS = 8, 2, 65, 2, 2


class Stack:
    """Per layer: complex drive weight W, a controller with trainable heads, and
    a filter state with trainable log_gamma / log_theta (the reference's
    selective Pure RQF layer, pure.py:115-147, without its unrelated parts)."""

    def __init__(self, seed, input_source):
        g = torch.Generator().manual_seed(seed)
        self.input_source = input_source
        cfg = SelectiveRQFConfig(write_control=True, frequency_warp="grouped", num_groups=G,
                                 max_log_scale=math.log(4.0))
        self.layers = []
        for _ in range(LAYERS):
            rqf = workloads.recipe_filter(F, samp=16000.0, tau=5.0 / 16000.0, seq_duration=1.0,
                                          generator=g)
            ctl = SelectiveController(F, rqf, cfg)
            for name in ("W_gamma", "W_write", "W_delta"):
                head = getattr(ctl, name)
                setattr(ctl, name, 0.3 * torch.randn(head.shape, generator=g))
            W = torch.complex(torch.randn(F, F, generator=g), torch.randn(F, F, generator=g))
            self.layers.append(dict(W=W / math.sqrt(2 * F), ctl=ctl, rqf=rqf))

    def to(self, device, dtype):
        """A copy with every trainable tensor a leaf of `dtype` on `device`."""
        out = copy.deepcopy(self)
        cdtype = torch.complex128 if dtype == torch.float64 else torch.complex64
        for layer in out.layers:
            layer["W"] = layer["W"].to(device, cdtype).requires_grad_(True)
            ctl, rqf = layer["ctl"], layer["rqf"]
            for name in ("W_gamma", "W_write", "W_delta"):
                setattr(ctl, name, getattr(ctl, name).to(device, dtype).requires_grad_(True))
            ctl.warp_groups = ctl.warp_groups.to(device)
            for name in ("log_tau", "min_gamma", "max_gamma", "min_freq", "max_freq"):
                setattr(rqf, name, getattr(rqf, name).to(device, dtype))
            for name in ("log_gamma", "log_theta"):
                setattr(rqf, name, getattr(rqf, name).to(device, dtype).requires_grad_(True))
        return out

    def parameters(self):
        for layer in self.layers:
            ctl, rqf = layer["ctl"], layer["rqf"]
            yield from (layer["W"], ctl.W_gamma, ctl.W_write, ctl.W_delta, rqf.log_gamma,
                        rqf.log_theta)

    def clamp_parameters(self):
        for layer in self.layers:
            layer["rqf"].clamp_parameters()

    def __call__(self, x, *, kernel, truncated):
        h = source = x
        for layer in self.layers:
            W, ctl, rqf = layer["W"], layer["ctl"], layer["rqf"]
            inputs = ctl(source, rqf, prospective=True, mode="tau", prospective_tau=None)
            if kernel:
                raw, act = selective_layer_scan(h, W, inputs, truncated=truncated)
            else:
                cols = h.shape[1] * h.shape[2]
                z = (W @ h.reshape(-1, cols)).reshape(-1, *h.shape[1:])
                lag = ((W @ h.detach().reshape(-1, cols)).reshape(-1, *h.shape[1:])
                       if truncated else z)
                raw = torch_ref.selective_scan(z, inputs, truncated=truncated, z_lag=lag)
                act = torch_ref.split_relu(raw)
            out = act + h
            source = raw + h if self.input_source == "layer_output" else h
            h = out
        return h


@pytest.mark.parametrize("input_source", ["layer_input", "layer_output"])
@pytest.mark.parametrize("truncated", [False, True])
def test_encoder_trains_like_the_reference_path(truncated, input_source):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print(f"case: encoder training truncated={truncated} source={input_source}", flush=True)
    base = Stack(seed=11, input_source=input_source)
    actual = base.to("cuda", torch.float32)
    expected = base.to("cpu", torch.float64)
    gx = torch.Generator().manual_seed(12)
    x = torch.complex(torch.randn(F, B, T, generator=gx), torch.randn(F, B, T, generator=gx))
    xs = {True: x.to("cuda", torch.complex64), False: x.to(torch.complex128)}
    models = {True: actual, False: expected}
    opts = {k: torch.optim.AdamW(list(m.parameters()), lr=1e-3) for k, m in models.items()}
    for _ in range(3):
        for kernel, model in models.items():
            opts[kernel].zero_grad()
            model(xs[kernel], kernel=kernel, truncated=truncated).abs().square().mean().backward()
            opts[kernel].step()
            model.clamp_parameters()
    with torch.no_grad():
        got = actual(xs[True], kernel=True, truncated=truncated)
        want = expected(xs[False], kernel=False, truncated=truncated)
    assert relerr(got, want) <= PARITY_RTOL, ("output", relerr(got, want))
    for i, (p, q) in enumerate(zip(actual.parameters(), expected.parameters())):
        err = relerr(p.detach(), q.detach())
        assert err <= PARITY_RTOL, (f"parameter {i}", err)
    # Training moved the parameters (the comparison is not of the initial state).
    moved = max(relerr(p.detach(), q.detach()) for p, q in
                zip(actual.parameters(), base.to("cuda", torch.float32).parameters()))
    assert moved > 1e-4

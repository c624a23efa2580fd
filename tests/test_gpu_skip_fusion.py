"""The encoder's residual connection fused into the scans' output stores.

`PureRQFEncoder._forward_fbt_stack` and `_forward_selective_stack`
(rqf_models/backbones/rqf/pure.py:480-536) add the layer input to each
block's output (`h = out + h`, and `source = raw + h` for the next selective
layer's selectors) in separate passes.  `fbt_recompute_scan(..., skip=h)`,
`selective_forward(..., skip=h)` and `selective_layer_scan(..., skip=True)`
add it in the kernels' stores.  The fused results must equal the unfused
composition bit for bit in the forward (the same fp32 additions) and match it
to rounding in the gradients, and the kernels' own outputs must still match
the fp64 oracle.
"""

import numpy as np
import pytest
import torch

from oracle import oracle
from prospective_rqf_amd.fbt_scan_kernel import fbt_recompute_scan
from prospective_rqf_amd.selective_scan import selective_layer_scan
from prospective_rqf_amd.selective_scan_kernel import selective_forward
from tests.helpers import PARITY_RTOL, crandn, relerr
from tests.selective_cases import make_inputs, rounded_to_f32, to_torch

pytestmark = pytest.mark.gpu

CASE_ALL = dict(gamma=True, write=True, warp="grouped", log_shift=False, write_sigmoid=True)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _dev(a, grad=False):
    return torch.as_tensor(np.asarray(a, np.complex64), device="cuda").requires_grad_(grad)


def _coeffs(rng, F):
    c1 = rng.uniform(0.8, 0.99, F) * np.exp(1j * rng.uniform(0, 2 * np.pi, F))
    return c1, 0.1 * crandn(rng, F), 0.5 * crandn(rng, F)


@pytest.mark.parametrize("shape", [(6, 3, 4096), (5, 2, 3001), (4, 2, 513), (3, 2, 1)])
def test_fbt_recompute_skip_equals_unfused(shape):
    F, B, T = shape
    print(f"case: fbt skip {shape}", flush=True)
    rng = np.random.default_rng(F + T)
    c1, t0, t1 = _coeffs(rng, F)
    z, h, gy = crandn(rng, F, B, T), crandn(rng, F, B, T), crandn(rng, F, B, T)
    grads = []
    outs = []
    for fused in (True, False):
        C1, T0, T1, Z, H = _dev(c1, True), _dev(t0, True), _dev(t1, True), _dev(z, True), _dev(h, True)
        y = fbt_recompute_scan(C1, T0, T1, Z, skip=H) if fused else fbt_recompute_scan(C1, T0, T1, Z) + H
        y.backward(_dev(gy))
        outs.append(y.detach())
        grads.append([t.grad for t in (C1, T0, T1, Z, H)])
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    _, act_ref = oracle.twotap_fwd(c1.astype(np.complex64), t0.astype(np.complex64),
                                   t1.astype(np.complex64), np.asarray(z, np.complex64),
                                   layout=oracle.FBT, act=True)
    assert relerr(outs[0], act_ref + np.asarray(h, np.complex64)) <= PARITY_RTOL


@pytest.mark.parametrize("T", [1, 300, 4096, 5000])
@pytest.mark.parametrize("outputs", [(True, True), (True, False), (False, True)])
def test_selective_forward_skip_equals_unfused(T, outputs):
    write_raw, activate = outputs
    F, B = 5, 3
    print(f"case: selective skip T={T} outputs={outputs}", flush=True)
    rng = np.random.default_rng(T + 7)
    inp = rounded_to_f32(make_inputs(F, B, T, CASE_ALL, rng, prospective=True, G=2))
    ti = to_torch(inp, device="cuda")
    z, h = _dev(crandn(rng, F, B, T)), _dev(crandn(rng, F, B, T))
    raw_f, act_f, ent_f = selective_forward(z, ti, activate, write_raw, 256, skip=h)
    raw_u, act_u, ent_u = selective_forward(z, ti, activate, write_raw, 256)
    assert torch.equal(ent_f, ent_u)
    if write_raw:
        assert torch.equal(raw_f, raw_u + h)
    if activate:
        assert torch.equal(act_f, act_u + h)
    raw_o, act_o = oracle.selective_fwd(np.asarray(z.cpu(), np.complex128), inp)
    hn = h.cpu().numpy().astype(np.complex128)
    if write_raw:
        assert relerr(raw_f, raw_o + hn) <= PARITY_RTOL
    if activate:
        assert relerr(act_f, act_o + hn) <= PARITY_RTOL


@pytest.mark.parametrize("truncated", [False, True])
def test_selective_layer_skip_matches_unfused_autograd(truncated):
    print(f"case: selective layer skip truncated={truncated}", flush=True)
    rng = np.random.default_rng(31)
    F, B, T = 6, 2, 700
    inp = rounded_to_f32(make_inputs(F, B, T, CASE_ALL, rng, prospective=True, G=2))
    x, W = crandn(rng, F, B, T), 0.4 * crandn(rng, F, F)
    cot_raw, cot_act = _dev(crandn(rng, F, B, T)), _dev(crandn(rng, F, B, T))
    results = []
    for fused in (True, False):
        ti = to_torch(inp, device="cuda")
        leaves = [ti.gamma_logits, ti.warp_logits, ti.write_logits, ti.bias, ti.theta]
        for v in leaves:
            v.requires_grad_(True)
        X, Wt = _dev(x, True), _dev(W, True)
        raw, act = selective_layer_scan(X, Wt, ti, truncated=truncated, skip=fused)
        if not fused:
            raw, act = raw + X, act + X
        loss = (cot_raw.conj() * raw).real.sum() + (cot_act.conj() * act).real.sum()
        loss.backward()
        results.append(([raw.detach(), act.detach()], [X.grad, Wt.grad] + [v.grad for v in leaves]))
    (out_f, g_f), (out_u, g_u) = results
    for a, b in zip(out_f, out_u):
        assert torch.equal(a, b)
    for a, b in zip(g_f, g_u):
        assert relerr(a, b) <= 1e-6


def test_fbt_encoder_stack_fused_equals_unfused():
    """Three shape-preserving layers h <- split-ReLU(scan(W h)) + h, as
    `_forward_fbt_stack` runs them (pure.py:526-534)."""
    rng = np.random.default_rng(41)
    F, B, T, L = 8, 4, 2048, 3
    layers = [(0.3 * crandn(rng, F, F), *_coeffs(rng, F)) for _ in range(L)]
    h0 = crandn(rng, F, B, T)
    outs, grads = [], []
    for fused in (True, False):
        params = [[_dev(a, True) for a in layer] for layer in layers]
        H0 = _dev(h0, True)
        h = H0
        for W, c1, t0, t1 in params:
            z = (W @ h.reshape(F, B * T)).reshape(F, B, T)
            h = fbt_recompute_scan(c1, t0, t1, z, skip=h) if fused else fbt_recompute_scan(c1, t0, t1, z) + h
        h.abs().sum().backward()
        outs.append(h.detach())
        grads.append([H0.grad] + [p.grad for layer in params for p in layer])
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(*grads):
        assert relerr(a, b) <= 1e-6

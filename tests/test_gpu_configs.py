"""GPU parity at the benchmark configurations' own contracts and regimes.

Each case runs the configuration's kernel contract on the parameter regime of
its experiment config, against the fp64 oracle, at a batch the oracle finishes
in seconds; the full-size shape is covered by size-independent properties.

* Config 4 (token copy, experiment/selective_copying.yaml:22-35): two stacked
  selective layers at T = 4096, G = 4, warp scale ln 4.  Layer 0 is the
  intermediate contract (raw + act, cotangents gy and gx); layer 1 is raw
  only with gy, and its drive is a complex map of layer 0's act, so layer
  0's gx is layer 1's input gradient.
* Config 5 (Path-X, experiment/pathx.yaml:17-21): the FBT recompute scan at
  T = 16384 on tile-aligned rows with the slow poles of that recipe
  (theta in [5/16384, pi/2], tau = 5/16384: memories up to ~16k steps), and
  a four-layer stack with the residual add fused into the scan
  (``skip=h``), forward and backward, against the oracle chain.
* Config 3 (north star): the full F = 256, G = 8 channel layout at
  T = 16000, with two teams per backward split as the full grid picks
  (the split rows and their reduction), at B = 2 against the oracle; and the
  full B = 64 shape through properties: every per-row output equals the
  same rows computed in a small batch bit for bit, and the per-channel
  gradients are the fp64 sums of the small batches'.

The reference's kernel suite covers the same contracts at small shapes
(tests/test_selective_cuda.py:193-269).
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle
from prospective_rqf_amd import workloads
from prospective_rqf_amd.fbt_scan_kernel import (
    fbt_recompute_backward_raw,
    fbt_recompute_forward_raw,
    fbt_recompute_scan,
)
from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward
from tests.helpers import (
    PARITY_RTOL,
    SELECTIVE_CHANNEL_RTOL,
    chanerr,
    cotangent_off_relu_kink,
    crandn,
    relerr,
)
from tests.selective_cases import from_torch

pytestmark = pytest.mark.gpu

NAMES = ("dz", "dzw", "dg", "dd", "dw", "dbias", "dtheta")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _c64(a):
    return np.asarray(a, dtype=np.complex64).astype(np.complex128)


def _dev(a):
    return torch.as_tensor(np.asarray(a, dtype=np.complex64), device="cuda")


def _assert_all(errs, case, channel_bar=PARITY_RTOL):
    """Normwise errors against PARITY_RTOL; per-channel ones ("/channel")
    against ``channel_bar``."""
    print(f"  {case}: " + " ".join(f"{k} {v:.1e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items()
           if not v <= (channel_bar if k.endswith("/channel") else PARITY_RTOL)}
    assert not bad, (case, bad)


def _grad_errs(tag, got, want, errs):
    for name, g, w in zip(NAMES, got, want):
        if w is None:
            assert g is None, (tag, name)
            continue
        errs[f"{tag}.{name}"] = relerr(g, w)
        if name in ("dbias", "dtheta"):
            errs[f"{tag}.{name}/channel"] = chanerr(g, w)


def _kink_mask(raw_ref, band=1e-4):
    """(re, im) masks of the state components within band*max of zero, where
    a split-ReLU mask decision is left to rounding (see cotangent_off_relu_kink)."""
    lim = band * float(np.max(np.abs(raw_ref)))
    return np.abs(raw_ref.real) <= lim, np.abs(raw_ref.imag) <= lim


def _zero_at(g, masks):
    """Zero the components of g (numpy or device tensor) flagged by masks."""
    mre, mim = masks
    if isinstance(g, torch.Tensor):
        re = g.real.masked_fill(torch.as_tensor(mre, device=g.device), 0.0)
        im = g.imag.masked_fill(torch.as_tensor(mim, device=g.device), 0.0)
        return torch.complex(re, im)
    return np.where(mre, 0.0, g.real) + 1j * np.where(mim, 0.0, g.imag)


# ---------------------------------------------------------------------------
# Config 4: two stacked selective layers, token-copy options
# ---------------------------------------------------------------------------

def _config4_inputs(F, B, T, layer):
    return workloads.selective_inputs(F, B, T, G=4, warp_scale=math.log(4.0), samp=1.0, tau=5.0,
                                      seq_duration=4096.0, device="cuda", seed=layer)


@pytest.mark.parametrize("F,B,form", [(16, 2, None), (256, 1, None), (256, 1, "group")])
def test_config4_two_layer_stack(monkeypatch, F, B, form):
    """Both layers against the fp64 oracle chain.  B = 1 takes the split form
    of the backward; forced into the group form, F = 256 in 4 groups of 64 at
    T = 4096 picks the 6 x 2 block shape (16 tiles in 8 full super-tiles, 11
    teams of 6), the shape the full config-4 grid runs for layer 0."""
    T, chunk = 4096, 256
    print(f"case: config 4 stack F={F} B={B} T={T} form={form}", flush=True)
    if form:
        monkeypatch.setenv("RQF_BWD_FORM", form)
    rng = np.random.default_rng(4000 + F + B)
    ins = [_config4_inputs(F, B, T, layer) for layer in range(2)]
    assert ins[0].options[1] and ins[0].warp_logits.shape[0] == 4
    oins = [from_torch(i) for i in ins]
    z0 = _c64(crandn(rng, F, B, T))
    w1 = _c64(crandn(rng, F, F) / math.sqrt(2 * F))  # layer 1 drive: complex map of act0
    gy0, gy1 = _c64(crandn(rng, F, B, T)), _c64(crandn(rng, F, B, T))

    # fp64 oracle chain
    raw0_o, act0_o = oracle.selective_fwd(z0, oins[0])
    z1_o = (w1 @ act0_o.reshape(F, B * T)).reshape(F, B, T)
    raw1_o, _ = oracle.selective_fwd(z1_o, oins[1])
    g1_o = oracle.selective_bwd(z1_o, oins[1], gy1, None)
    kinks = _kink_mask(raw0_o)
    gx0_o = _zero_at((w1.conj().T @ g1_o[0].reshape(F, B * T)).reshape(F, B, T), kinks)
    g0_o = oracle.selective_bwd(z0, oins[0], gy0, gx0_o)

    # the HIP chain
    w1d = _dev(w1)
    raw0, act0, ent0 = selective_forward(_dev(z0), ins[0], True, True, chunk)
    z1 = (w1d @ act0.reshape(F, B * T)).reshape(F, B, T)
    raw1, act1, ent1 = selective_forward(z1, ins[1], False, True, chunk)
    assert act1 is None
    g1 = selective_backward(z1, ins[1], ent1, _dev(gy1), None, False, False, chunk)
    gx0 = _zero_at((w1d.mH @ g1[0].reshape(F, B * T)).reshape(F, B, T), kinks)
    g0 = selective_backward(_dev(z0), ins[0], ent0, _dev(gy0), gx0, True, False, chunk)
    torch.cuda.synchronize()

    errs = {"L0.raw": relerr(raw0, raw0_o), "L0.act": relerr(act0, act0_o),
            "L1.raw": relerr(raw1, raw1_o)}
    _grad_errs("L1", g1, g1_o, errs)
    _grad_errs("L0", g0, g0_o, errs)
    _assert_all(errs, f"config 4 F={F} B={B} ({int(kinks[0].sum() + kinks[1].sum())} "
                      "cotangent components zeroed at the ReLU kink)", SELECTIVE_CHANNEL_RTOL)


# ---------------------------------------------------------------------------
# Config 5: slow poles at T = 16384, single layer and a fused-skip stack
# ---------------------------------------------------------------------------

def _config5_coefs(F, seed):
    return workloads.static_two_tap(F, samp=16384.0, tau=5.0 / 16384.0,
                                    seq_duration=2 * math.pi, max_freq_factor=0.25, seed=seed,
                                    device="cuda")


def _np(t):
    return t.detach().cpu().numpy().astype(np.complex128)


def test_config5_coefficients_are_the_slow_recipe():
    c1 = _np(_config5_coefs(64, 0)[0])
    # |C1| = exp(-gamma*eta) with eta = 0.2 and gamma = theta/(1+theta), theta >= 5/16384
    assert np.abs(c1).max() > 0.9995 and np.abs(c1).max() < 1.0
    assert np.abs(np.angle(c1)).max() < 0.2 * math.pi / 2


@pytest.mark.parametrize("F,B", [(8, 2), (64, 1)])
def test_config5_recompute_slow_poles(F, B):
    T = 16384
    print(f"case: config 5 recompute F={F} B={B} T={T}", flush=True)
    rng = np.random.default_rng(5000 + F)
    c = _config5_coefs(F, 1)
    cn = [_np(v) for v in c]
    z = _c64(crandn(rng, F, B, T))
    y_ref, act_ref = oracle.twotap_fwd(*cn, z, layout=oracle.FBT, act=True)
    g, n = cotangent_off_relu_kink(y_ref, _c64(crandn(rng, F, B, T)))
    gz_ref, gc1_ref, gt0_ref, gt1_ref = oracle.twotap_bwd(*cn, z, y_ref, g, layout=oracle.FBT,
                                                          mask_act=True)
    leaves = [v.clone().requires_grad_(True) for v in c]
    Z = _dev(z).requires_grad_(True)
    y = fbt_recompute_scan(*leaves, Z)
    y.backward(_dev(g))
    errs = {"act": relerr(y, act_ref), "grad_z": relerr(Z.grad, gz_ref)}
    for name, got, want in (("grad_C1", leaves[0].grad, gc1_ref),
                            ("grad_tap0", leaves[1].grad, gt0_ref),
                            ("grad_tap1", leaves[2].grad, gt1_ref)):
        errs[name] = relerr(got, want)
        errs[name + "/channel"] = chanerr(got, want)
    _assert_all(errs, f"config 5 F={F} B={B} ({n} cotangent components zeroed)")


def test_config5_fused_skip_stack_four_layers():
    """h[l+1] = split-ReLU(scan_l(W_l h[l])) + h[l], the skip added in the scan's
    store (pure.py:530-534), four layers forward and backward."""
    F, B, T, L = 8, 2, 16384, 4
    print(f"case: config 5 fused-skip stack F={F} B={B} T={T} L={L}", flush=True)
    rng = np.random.default_rng(5005)
    coefs = [_config5_coefs(F, 10 + layer) for layer in range(L)]
    cn = [[_np(v) for v in c] for c in coefs]
    ws = [_c64(crandn(rng, F, F) / math.sqrt(2 * F)) for _ in range(L)]
    h0 = _c64(crandn(rng, F, B, T))
    gout = _c64(crandn(rng, F, B, T))

    # fp64 oracle chain, forward
    hs, zs, ys = [h0], [], []
    for layer in range(L):
        z = (ws[layer] @ hs[-1].reshape(F, B * T)).reshape(F, B, T)
        y, act = oracle.twotap_fwd(*cn[layer], z, layout=oracle.FBT, act=True)
        zs.append(z)
        ys.append(y)
        hs.append(act + hs[-1])

    # HIP chain, forward (kernel-level entry points, as the stack drives them)
    hd = [_dev(h0)]
    saved = []
    for layer in range(L):
        wd = _dev(ws[layer])
        z = (wd @ hd[-1].reshape(F, B * T)).reshape(F, B, T)
        out, carry, keep = fbt_recompute_forward_raw(*coefs[layer], z, skip=hd[-1])
        saved.append((carry, keep))
        hd.append(out)
    errs = {f"h{layer + 1}": relerr(hd[layer + 1], hs[layer + 1]) for layer in range(L)}

    # backward: the cotangent of h[l+1] reaches the scan (masked) and the skip
    g_o, g_d = gout, _dev(gout)
    zeroed = 0
    for layer in reversed(range(L)):
        kinks = _kink_mask(ys[layer])
        zeroed += int(kinks[0].sum() + kinks[1].sum())
        g_o, g_d = _zero_at(g_o, kinks), _zero_at(g_d, kinks)
        gz_o, gc1_o, gt0_o, gt1_o = oracle.twotap_bwd(*cn[layer], zs[layer], ys[layer], g_o,
                                                      layout=oracle.FBT, mask_act=True)
        carry, (c1, t0, t1, z) = saved[layer]
        gc1, gt0, gt1, gz = fbt_recompute_backward_raw(c1, t0, t1, z, carry, g_d)
        for name, got, want in (("grad_C1", gc1, gc1_o), ("grad_tap0", gt0, gt0_o),
                                ("grad_tap1", gt1, gt1_o)):
            errs[f"L{layer}.{name}"] = relerr(got, want)
            errs[f"L{layer}.{name}/channel"] = chanerr(got, want)
        errs[f"L{layer}.grad_z"] = relerr(gz, gz_o)
        wd = _dev(ws[layer])
        g_o = g_o + (ws[layer].conj().T @ gz_o.reshape(F, B * T)).reshape(F, B, T)
        g_d = g_d + (wd.mH @ gz.reshape(F, B * T)).reshape(F, B, T)
        errs[f"grad_h{layer}"] = relerr(g_d, g_o)
    _assert_all(errs, f"config 5 stack ({zeroed} cotangent components zeroed)")


# ---------------------------------------------------------------------------
# Config 3: the full channel layout, and the full shape by properties
# ---------------------------------------------------------------------------

def _config3_inputs(B, T=16000, seed=0):
    return workloads.selective_inputs(256, B, T, G=8, device="cuda", seed=seed)


@pytest.mark.parametrize("form", ["group", "split"])
def test_config3_team_layout(monkeypatch, form):
    """F = 256 in 8 warp groups of 32 channels (8 teams of 4 per group), in
    both forms of the backward: one block running all 8 teams of a group (the
    form the full config-3 grid picks), and two teams per split with four
    split rows per group summed by the split reduction."""
    F, B, T, chunk = 256, 2, 16000, 256
    print(f"case: config 3 team layout F={F} B={B} T={T} form={form}", flush=True)
    if form == "group":
        monkeypatch.setenv("RQF_BWD_FORM", "group")
    else:
        monkeypatch.setenv("RQF_BWD_SPLIT_TEAMS", "2")
    rng = np.random.default_rng(3000)
    inp = _config3_inputs(B, T)
    counts = torch.bincount(inp.groups.cpu(), minlength=8)
    assert counts.tolist() == [32] * 8
    oin = from_torch(inp)
    z = _c64(crandn(rng, F, B, T))
    raw_o, act_o = oracle.selective_fwd(z, oin)
    # With memories of ~2500 steps, one split-ReLU mask decision left to
    # rounding moves the adjoint over thousands of steps: zero gx there.
    gy = _c64(crandn(rng, F, B, T))
    gx, n = cotangent_off_relu_kink(raw_o, _c64(crandn(rng, F, B, T)))
    raw, act, ent = selective_forward(_dev(z), inp, True, True, chunk)
    got = selective_backward(_dev(z), inp, ent, _dev(gy), _dev(gx), True, False, chunk)
    torch.cuda.synchronize()
    want = oracle.selective_bwd(z, oin, gy, gx)
    errs = {"raw": relerr(raw, raw_o), "act": relerr(act, act_o)}
    _grad_errs("bwd", got, want, errs)
    _assert_all(errs, f"config 3 team layout ({n} gx components zeroed at the ReLU kink)",
                SELECTIVE_CHANNEL_RTOL)


@pytest.mark.parametrize("cfg,form", [(3, "group"), (3, "split"), (4, "group"), (4, "split")])
def test_full_shape_properties(monkeypatch, cfg, form):
    """The full config-3 shape (B = 64), and config 4's layer 0 (T = 4096,
    4 groups), against small-batch calls on the same rows, both in the same
    form of the backward: per-row outputs bit for bit, warp-logit gradients to
    rounding (bit for bit in the group form; in the split form the grid's split
    layout changes the order of the channel sum), and dbias / dtheta as the
    fp64 sum over the small batches."""
    F, B, T, chunk, SB = 256, 64, (16000 if cfg == 3 else 4096), 256, 4
    print(f"case: config {cfg} full shape B={B} vs {B // SB} calls of B={SB} form={form}",
          flush=True)
    monkeypatch.setenv("RQF_BWD_FORM", form)
    g = torch.Generator(device="cuda").manual_seed(33)

    def cn(*shape):
        return torch.complex(torch.randn(*shape, generator=g, device="cuda"),
                             torch.randn(*shape, generator=g, device="cuda"))

    inp = _config3_inputs(B, T) if cfg == 3 else _config4_inputs(F, B, T, 0)
    z, gy, gx = cn(F, B, T), cn(F, B, T), cn(F, B, T)
    raw, act, ent = selective_forward(z, inp, True, True, chunk)
    full = selective_backward(z, inp, ent, gy, gx, True, False, chunk)
    nc = ent.shape[1]
    dbias_sum = torch.zeros(F, dtype=torch.float64, device="cuda")
    dtheta_sum = torch.zeros_like(dbias_sum)
    worst_dd = 0.0
    for b0 in range(0, B, SB):
        sl = slice(b0, b0 + SB)
        sub = inp._replace(gamma_logits=inp.gamma_logits[:, sl].contiguous(),
                           warp_logits=inp.warp_logits[:, sl].contiguous(),
                           write_logits=inp.write_logits[:, sl].contiguous())
        zs = z[:, sl].contiguous()
        r2, a2, e2 = selective_forward(zs, sub, True, True, chunk)
        part = selective_backward(zs, sub, e2, gy[:, sl].contiguous(), gx[:, sl].contiguous(),
                                  True, False, chunk)
        assert torch.equal(r2, raw[:, sl]) and torch.equal(a2, act[:, sl])
        assert torch.equal(e2.reshape(F, SB, nc), ent.reshape(F, B, nc)[:, sl])
        for name, p, f in zip(NAMES[:5], part[:5], full[:5]):
            if name == "dd":
                worst_dd = max(worst_dd, relerr(p, f[:, sl]))
            elif name != "dzw":
                assert torch.equal(p, f[:, sl]), (name, b0)
        dbias_sum += part[5].double()
        dtheta_sum += part[6].double()
    errs = {"dd (rounding of the channel-sum order)": worst_dd,
            "dbias": relerr(full[5], dbias_sum), "dtheta": relerr(full[6], dtheta_sum),
            "dbias/channel": chanerr(full[5], dbias_sum),
            "dtheta/channel": chanerr(full[6], dtheta_sum)}
    print("  " + " ".join(f"{k} {v:.1e}" for k, v in errs.items()), flush=True)
    assert worst_dd <= (0.0 if form == "group" else 1e-6)
    assert max(errs.values()) <= 1e-5, errs

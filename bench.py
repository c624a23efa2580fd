"""Benchmark of the complex-scan backends on one MI355X.

Default workload (the north-star metric): selective
fused scan, F=H=256 channels, B=64, T=16000, grouped warp (G=8), sigmoid gamma
and write heads, prospective tau-mode input, intermediate-layer contract
(raw + split-ReLU outputs, cotangents on both, full BPTT).  One step = one
forward + one backward of the scan kernels over the whole batch; inputs are
resident in HBM before timing starts.  The drive and logit GEMMs are outside
the metric.

``--config`` selects the other BASELINE.json configs (1-based) for manual runs:
  1  Pure RQF depth 2, (B,T,F) chunked scan, B=4 T=161 F=64 (latency-bound)
  2  non-selective two-tap FBT recompute scan, B=32 T=16000 F=128
  3  selective fused scan, B=64 T=16000 F=256 G=8 (default)
  4  selective token-copy shape, two layers, B=64 T=4096 F=256 G=4
  5  long-sequence Pure RQF, 4 FBT recompute layers, B=16 T=16384 F=256

Every entry point is bracketed by HIP events on the stream the kernels run on
(torch's current stream, which the C ABI receives).  ``roofline`` describes
the entry point with the largest share of the step; ``traffic`` is read from
the committed rocprofv3 FETCH_SIZE/WRITE_SIZE table (profiles/traffic.md)
when it has a row for the workload, else null.

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "scan Gelem/s (B·T·H complex) fwd+bwd at T=16000; % of HBM roofline"
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "traffic.md")


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5, 6, 7],
                    help="1-5: BASELINE.json configs; 6: multi-oscillator C-weighted scan; "
                         "7: fused |y| readout scan")
    ap.add_argument("--cpu-baseline", dest="cpu", action="store_true", default=True)
    ap.add_argument("--no-cpu-baseline", dest="cpu", action="store_false")
    ap.add_argument("--cpu-reps", type=int, default=3,
                    help="timed runs of the CPU baseline sample (median reported, after one "
                         "warm-up run)")
    ap.add_argument("--cpu-batch", type=int, default=0,
                    help="batch of the CPU baseline sample (0: the config's, capped at 64)")
    ap.add_argument("--cpu-steps", type=int, default=0,
                    help="time steps of the CPU baseline sample (0: the config's default)")
    ap.add_argument("--batch", type=int, default=0,
                    help="override the config's batch size (experiments only)")
    ap.add_argument("--seq-len", type=int, default=0,
                    help="override the config's sequence length (experiments only)")
    ap.add_argument("--stack", choices=["none", "fused", "unfused"], default="none",
                    help="configs 3 and 5: include the encoder's residual add (h = out + h) in "
                         "each layer's forward, fused into the scan's stores or as a separate "
                         "pass (the reference's pure.py:486-496, 530-534)")
    ap.add_argument("--layer", choices=["scan", "fused", "split", "single"], default="scan",
                    help="config 3: 'split'/'single' time the whole selective layer, adding the "
                         "selector projection (selective.py:205-217) and the drive GEMM "
                         "(selective_scan.py:117-118) forward, and their backward GEMMs "
                         "(selective_scan.py:144-146, selective.py:86-97) with the weight "
                         "gradients as split-K batched GEMMs ('split') or as the reference's "
                         "single GEMMs ('single'); 'fused' runs the forward and the input "
                         "gradient as one MFMA GEMM each (csrc/proj.hip) with split-K weight "
                         "gradients")
    ap.add_argument("--readout", choices=["none", "fused", "reference"], default="none",
                    help="configs 2 and 5: add the per-timestep [Re; Im] MLP readout "
                         "(train.py:74-136, hidden 256, 10 classes, per-step logits and their "
                         "backward) on the last layer's output: 'fused' runs "
                         "readout.complex_readout on the (F, B, T) features, 'reference' the "
                         "reference's permute + cat + Linear + ReLU + Linear")
    ap.add_argument("--layout", choices=["fbt", "btf"], default="fbt",
                    help="config 2: 'btf' runs the same workload on (batch, time, filters) "
                         "tensors through the chunked prospective scan (the layout RQF-S4 "
                         "and the non-FBT Pure RQF cells use, block.py:690-733)")
    ap.add_argument("--layer0", action="store_true",
                    help="config 2: time the whole real-input layer 0 through "
                         "fbt_layer0_real_scan (fbt_scan_kernel.py:899-1032): the stacked "
                         "[Wr; Wi] projection of the waveform on the MFMA projection GEMM, the "
                         "recompute scan, and in the backward grad_h and grad_[Wr; Wi] besides "
                         "the coefficient gradients")
    ap.add_argument("--chunk", type=int, default=0,
                    help="configs 3 and 4: the selective scans' chunk (default 256, the "
                         "reference's min(256, next_pow2(T)); a longer one makes the backward "
                         "rebuild its 256-step tile entries from the chunk entries)")
    ap.add_argument("--act-only", action="store_true",
                    help="config 3 with the act-only contract (no raw output, no gy)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 plain 1 GiB device copies (scale for FETCH/WRITE_SIZE)")
    return ap.parse_args()


def copy_calibration():
    """Five device-to-device copies of exactly 1 GiB each (read 1 GiB, write 1 GiB)."""
    import torch

    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "copies": 5}), flush=True)


# ---------------------------------------------------------------------------
# Plans: a step is a list of named entry-point calls
# ---------------------------------------------------------------------------


class Plan:
    """One benchmark step as a sequence of named entry-point calls.

    ``ops`` is a list of ``(name, fn)``; each fn takes the step's state dict.
    ``bytes`` maps an op name to its algorithmic HBM bytes per call."""

    def __init__(self, workload, config, elems, ops, nbytes, kernels, cpu=None, contract=""):
        self.workload = workload
        self.config = config
        self.elems = elems
        self.ops = ops
        self.bytes = nbytes
        self.kernels = kernels
        self.cpu = cpu
        self.contract = contract


def _cn(g, device, *shape):
    import torch

    return torch.complex(torch.randn(*shape, generator=g, device=device),
                         torch.randn(*shape, generator=g, device=device))


def selective_bytes(F, B, T, G, chunk, *, write_raw=True, activate=True, truncated=False):
    """Algorithmic HBM bytes (each boundary tensor once) of one selective fwd and bwd call.

    fwd: z, gamma/write logits, warp logits, raw and/or act, entries.
    bwd: z, logits, entries, gy/gx, dz (+dzw when truncated), logit gradients."""
    N = F * B * T
    nc = -(-T // chunk)
    ent = 8 * F * B * nc
    warp = 4 * G * B * T
    fwd = N * (8 + 4 + 4 + 8 * write_raw + 8 * activate) + warp + ent
    bwd = (N * (8 + 4 + 4 + 8 * write_raw + 8 * activate + 8 + 8 * truncated + 4 + 4)
           + 2 * warp + ent)
    return fwd, bwd


def fbt_recompute_bytes(F, B, T):
    """Algorithmic bytes of one FBT recompute fwd and bwd call (x, act, carries; x, gy, gx)."""
    from prospective_rqf_amd import _lib

    N = F * B * T
    carry = 8 * F * B * max(_lib.load().rqf_fbt_carry_chunks(T), 1)
    return N * 16 + carry, N * 24 + carry


def plan_selective(cfg, args, dev):
    import torch

    from prospective_rqf_amd import workloads
    from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward

    if cfg == 3:
        F, B, T, G, log_scale = 256, 64, 16000, 8, math.log(1.25)
        samp, tau, seq = 16000.0, 5.0 / 16000.0, 1.0
        layers = [(not args.act_only, True)]
        name = "selective fused scan B=64 T=16000 H=256 G=8 (config 3)"
        contract = ("act only, gx cotangent, full BPTT" if args.act_only
                    else "raw+act outputs, gy+gx cotangents, full BPTT")
    else:
        F, B, T, G, log_scale = 256, 64, 4096, 4, math.log(4.0)
        samp, tau, seq = 1.0, 5.0, 4096.0
        layers = [(True, True), (True, False)]
        name = "selective token-copy shape B=64 T=4096 H=256 G=4, depth 2 (config 4)"
        contract = "layer 0: raw+act, gy+gx; layer 1: raw only, gy; full BPTT"
    if args.batch:
        B = args.batch
        name += f" [batch overridden to {B}]"
    if args.seq_len:
        T = args.seq_len
        name += f" [sequence length overridden to {T}]"
    chunk = args.chunk or 256
    if args.chunk:
        name += f" [chunk {chunk}: the backward rebuilds its tile entries first]"
    g = torch.Generator(device=dev).manual_seed(1)
    state = {}
    layer_inputs = []
    for li, (write_raw, activate) in enumerate(layers):
        inputs = workloads.selective_inputs(
            F, B, T, G=G, gamma=True, write=True, warp="grouped", write_sigmoid=True,
            write_max=2.0, gamma_scale=math.log(1.25), warp_scale=log_scale, prospective=True,
            samp=samp, tau=tau, seq_duration=seq, device=dev, seed=li)
        layer_inputs.append((inputs, write_raw, activate))
    layer = args.layer if cfg == 3 else "scan"
    if layer != "scan":
        # Layer input x (D = F, square layer), drive weight W and the selector heads
        # Ws (gamma F, warp G, write F rows) over v = [Re x; Im x].  The heads' output
        # replaces the synthetic logits, at the same N(0, 1) scale.
        state["x"] = _cn(g, dev, F, B * T)
        state["W"] = _cn(g, dev, F, F) / math.sqrt(2 * F)
        state["Ws"] = torch.randn(2 * F + G, 2 * F, generator=g, device=dev) / math.sqrt(2 * F)
    elif cfg == 3:
        state["z0"] = _cn(g, dev, F, B, T)
    else:
        # Token-copy drive: one-hot tokens (16 markers in the first T-16 steps,
        # noise tokens elsewhere), a fixed random 16->64 embedding and a complex
        # 64->H input map.  Layer 1's drive maps [Re; Im] of layer 0's act.
        gc = torch.Generator().manual_seed(2)
        tok = torch.randint(1, 15, (B, T), generator=gc)
        for b in range(B):
            pos = torch.randperm(T - 16, generator=gc)[:16]
            tok[b, pos] = 15
        emb = torch.randn(16, 64, generator=gc)
        x = emb[tok].to(dev)  # (B, T, 64)
        w0 = _cn(g, dev, F, 64) / 8.0
        xt = x.reshape(B * T, 64).t().contiguous().to(w0.dtype)
        state["z0"] = (w0 @ xt).reshape(F, B, T).contiguous()
        raw0, act0, _ = selective_forward(state["z0"], layer_inputs[0][0], True, True, chunk)
        feat = torch.cat([act0.real, act0.imag], dim=0).reshape(2 * F, B * T)
        w1 = _cn(g, dev, F, 2 * F) / math.sqrt(2 * F)
        state["z1"] = (w1 @ feat.to(w1.dtype)).reshape(F, B, T).contiguous()
        del raw0, act0, feat
    for li, (_, write_raw, activate) in enumerate(layer_inputs):
        state[f"gy{li}"] = _cn(g, dev, F, B, T) if write_raw else None
        state[f"gx{li}"] = _cn(g, dev, F, B, T) if activate else None

    ops, nbytes = [], {}
    if layer != "scan":
        from prospective_rqf_amd.projection import fused_dx, fused_forward, stacked, weight_grad

        inputs0 = layer_inputs[0][0]

        def proj_fwd(st):
            x = st["x"]
            if layer == "fused":
                z, logits = fused_forward(x, st["W"], st["Ws"])
                lg, ld, lw = logits.split((F, G, F))
            else:
                v = torch.cat((x.real, x.imag), 0)  # the controller's source features
                lg, ld, lw = (st["Ws"] @ v).split((F, G, F))
                st["v"] = v
                z = st["W"] @ x
            st["inputs0"] = inputs0._replace(gamma_logits=lg.reshape(F, B, T),
                                             warp_logits=ld.reshape(G, B, T),
                                             write_logits=lw.reshape(F, B, T))
            st["z0"] = z.reshape(F, B, T)

        def proj_bwd(st):
            dz, dzw, dg, dd, dw = st["grads0"][:5]
            n = B * T
            x = st["x"]
            if layer == "fused":
                dx = fused_dx(dz.reshape(F, n), [dg, dd, dw], st["W"], st["Ws"])
                glog = stacked([dg, dd, dw])  # one buffer: no copy
                v = torch.cat((x.real, x.imag), 0)
                st["layer_grads"] = (dx, weight_grad(dzw.reshape(F, n), x), weight_grad(glog, v))
                return
            glog = stacked([dg, dd, dw])
            dv = st["Ws"].T @ glog
            v = st.pop("v")
            dx = st["W"].mH @ dz.reshape(F, B * T) + torch.complex(dv[:F], dv[F:])
            if layer == "split":
                dW = weight_grad(dzw.reshape(F, B * T), x)
                dWs = weight_grad(glog, v)
            else:
                dW = dzw.reshape(F, B * T) @ x.mH
                dWs = glog @ v.T
            st["layer_grads"] = (dx, dW, dWs)

        ops.append(("proj_fwd[L0]", proj_fwd))
        nbytes["proj_fwd[L0]"] = 0
    stack = args.stack if cfg == 3 else "none"
    if stack != "none":
        for li in range(len(layer_inputs)):
            state[f"h{li}"] = _cn(g, dev, F, B, T)  # the layer input the skip adds
    for li, (inputs, write_raw, activate) in enumerate(layer_inputs):
        def fwd(st, li=li, inputs=inputs, write_raw=write_raw, activate=activate):
            if stack == "fused":
                st[f"out{li}"] = selective_forward(st[f"z{li}"], inputs, activate, write_raw,
                                                   chunk, skip=st[f"h{li}"])
            else:
                inp = st.get(f"inputs{li}", inputs)
                out = selective_forward(st[f"z{li}"], inp, activate, write_raw, chunk)
                if stack == "unfused":  # source = raw + h; h = act + h
                    h = st[f"h{li}"]
                    out = (None if out[0] is None else out[0] + h,
                           None if out[1] is None else out[1] + h, out[2])
                st[f"out{li}"] = out

        ops.append((f"rqf_selective_fwd[L{li}]", fwd))
    for li in reversed(range(len(layer_inputs))):
        inputs, write_raw, activate = layer_inputs[li]

        def bwd(st, li=li, inputs=inputs, activate=activate):
            entries = st.pop(f"out{li}")[2]
            inp = st.get(f"inputs{li}", inputs)
            st[f"grads{li}"] = selective_backward(st[f"z{li}"], inp, entries, st[f"gy{li}"],
                                                  st[f"gx{li}"], activate, False, chunk)

        ops.append((f"rqf_selective_bwd[L{li}]", bwd))
    if layer != "scan":
        ops.append(("proj_bwd[L0]", proj_bwd))
        nbytes["proj_bwd[L0]"] = 0
    for li, (_, write_raw, activate) in enumerate(layer_inputs):
        fb, bb = selective_bytes(F, B, T, G, chunk, write_raw=write_raw, activate=activate)
        nbytes[f"rqf_selective_fwd[L{li}]"] = fb + (8 * F * B * T if stack != "none" else 0)
        nbytes[f"rqf_selective_bwd[L{li}]"] = bb
    kernels = {
        "rqf_selective_fwd": "selective_fwd_rb_kernel",
        "rqf_selective_bwd": ("selective_bwd_grp_kernel + bwd_finish_kernel (group form: "
                              "G*B >= 256, nearly full super-tiles, and a gx cotangent or the "
                              "6x2 block shape: configs 3 and 4), else team_build_kernel + "
                              "selective_bwd_team_kernel + bwd_finish_kernel (split form)"),
    }
    if stack != "none":
        contract += f"; encoder residual add (raw + h, act + h) {stack}"
    if layer != "scan":
        how = {"fused": "fused MFMA projections, split-K", "split": "split-K batched",
               "single": "single"}[layer]
        contract += (f"; whole layer: selector projection and drive GEMM (fp32), weight "
                     f"gradients as {how} GEMMs")
        name += f" [whole layer, {layer} weight gradients]"
    config = {"workload": name, "F": F, "B": B, "T": T, "G": G, "layers": len(layers),
              "chunk": chunk, "contract": contract}
    cpu_steps = args.cpu_steps or (500 if cfg == 3 else 100)

    def cpu():
        base = cpu_baseline_selective(F, args.cpu_batch or min(B, 64), G, cpu_steps, log_scale,
                                      samp, tau, seq, layers)
        if cfg == 3 and not (args.cpu_steps or args.cpu_batch):
            # The planned T = 2000 sample, at B = 16 (one run of ~40 s; the
            # reference's per-element cost grows with T, so this is the more
            # faithful rate), reported next to the T = 500 one.
            base["long_sample"] = cpu_baseline_selective(F, 16, G, 2000, log_scale, samp, tau,
                                                         seq, layers, reps=1, warmup=False)
        return base

    return Plan(name, config, F * B * T * len(layers), (state, ops), nbytes, kernels, cpu,
                contract)


def _plan_layer0(F, B, T, coefs, u, w, state, name, gy):
    """Config 2 as layer 0 of the raw-waveform encoder: one real input row (the
    waveform), the complex drive weight w as the stacked real [Re w; Im w]."""
    import torch

    from prospective_rqf_amd.fbt_scan_kernel import fbt_layer0_real_scan

    state.clear()
    state["gy"] = gy
    coefs = [c.detach().clone().requires_grad_(True) for c in coefs]
    w_stacked = torch.cat((w.real, w.imag))[:, None].contiguous().requires_grad_(True)
    h = u.reshape(1, B * T).contiguous().requires_grad_(True)

    def fwd(st):
        st["act"] = fbt_layer0_real_scan(w_stacked, h, *coefs, B)

    def bwd(st):
        st.pop("act").backward(st["gy"])
        st["grads"] = (w_stacked.grad, h.grad, *(c.grad for c in coefs))
        for t in (w_stacked, h, *coefs):
            t.grad = None

    ops = [("fbt_layer0_real_scan_fwd", fwd), ("fbt_layer0_real_scan_bwd", bwd)]
    elems = F * B * T
    # Bytes the layer must move: the waveform in and the activation out, then
    # the cotangent in and grad_h out.  grad_z, which the backward writes and
    # reads once more for the projection's gradients, is not counted.
    nbytes = {"fbt_layer0_real_scan_fwd": 8 * elems + 4 * B * T,
              "fbt_layer0_real_scan_bwd": 8 * elems + 8 * B * T}
    kernels = {"fbt_layer0_real_scan_fwd": "fbt_fwd_rb_kernel<layer-0 drive z = wz x>",
               "fbt_layer0_real_scan_bwd": ("fbt_bwd_rb_kernel / fbt_bwd_kernel <layer-0 drive> "
                                            "+ coef_reduce_kernel + layer0_grads_kernel + "
                                            "layer0_wpart_reduce_kernel")}
    contract = ("layer 0 on the raw waveform: stacked real projection + split-ReLU recompute "
                "scan; gy cotangent; grads of [Wr; Wi], the waveform and the coefficients")
    config = {"workload": name + " [whole layer 0: fbt_layer0_real_scan]", "F": F, "B": B, "T": T,
              "layers": 1, "contract": contract}
    return Plan(config["workload"], config, elems, (state, ops), nbytes, kernels, None, contract)


def plan_fbt(cfg, args, dev):
    import torch

    from prospective_rqf_amd import workloads
    from prospective_rqf_amd.fbt_scan_kernel import (
        fbt_recompute_backward_raw,
        fbt_recompute_forward_raw,
    )

    if cfg == 2:
        F, B, T, L = 128, 32, 16000, 1
        coef = dict(samp=16000.0, tau=5.0 / 16000.0, seq_duration=1.0)
        name = "non-selective two-tap FBT recompute scan B=32 T=16000 H=128 (config 2)"
    else:
        F, B, T, L = 256, 16, 16384, 4
        coef = dict(samp=16384.0, tau=5.0 / 16384.0, seq_duration=2 * math.pi,
                    max_freq_factor=0.25)
        name = "long-sequence Pure RQF B=16 T=16384 H=256, 4 FBT recompute layers (config 5)"
    if args.batch:
        B = args.batch
        name += f" [batch overridden to {B}]"
    if args.seq_len:
        T = args.seq_len
        name += f" [sequence length overridden to {T}]"
    g = torch.Generator(device=dev).manual_seed(1)
    gcpu = torch.Generator().manual_seed(3)
    state = {}
    coefs = [workloads.static_two_tap(F, seed=li, device=dev, **coef) for li in range(L)]
    if cfg == 2:
        u = workloads.raw_waveform(B, T, samp=16000.0, generator=gcpu).to(dev)  # (B, T)
        w = _cn(g, dev, F)
        state["x0"] = (w[:, None, None] * u[None].to(w.dtype)).contiguous()
    else:
        # Flattened 128x128 images of uniform 8-bit pixels; layer l > 0 is driven
        # by a residual-stream stand-in of the same shape.
        img = torch.randint(0, 256, (B, T), generator=gcpu).float().div_(255.0).to(dev)
        state["x0"] = (img[None].expand(F, B, T).to(torch.complex64) * _cn(g, dev, F)[:, None, None]
                       ).contiguous()
        for li in range(1, L):
            state[f"x{li}"] = _cn(g, dev, F, B, T)
    for li in range(L):
        state[f"gy{li}"] = _cn(g, dev, F, B, T)

    if cfg == 2 and args.layer0:
        return _plan_layer0(F, B, T, coefs[0], u, w, state, name, gy=state["gy0"])
    ops = []
    stack = args.stack if cfg == 5 else "none"
    if stack != "none":
        for li in range(L):
            state[f"h{li}"] = _cn(g, dev, F, B, T)  # the layer input the skip adds
    for li in range(L):
        def fwd(st, li=li):
            if stack == "fused":
                st[f"out{li}"] = fbt_recompute_forward_raw(*coefs[li], st[f"x{li}"],
                                                           skip=st[f"h{li}"])
            else:
                act, carry, saved = fbt_recompute_forward_raw(*coefs[li], st[f"x{li}"])
                if stack == "unfused":  # h = out + h
                    act = act + st[f"h{li}"]
                st[f"out{li}"] = (act, carry, saved)

        ops.append((f"rqf_fbt_recompute_fwd[L{li}]", fwd))
    for li in reversed(range(L)):
        def bwd(st, li=li):
            act, carry, (c1, t0, t1, x) = st.pop(f"out{li}")
            st[f"grads{li}"] = fbt_recompute_backward_raw(c1, t0, t1, x, carry, st[f"gy{li}"])

        ops.append((f"rqf_fbt_recompute_bwd[L{li}]", bwd))
    if args.readout != "none":
        from prospective_rqf_amd.readout import complex_readout

        H, C = 256, 10
        gw = torch.Generator(device=dev).manual_seed(7)
        w1 = (torch.randn(H, 2 * F, generator=gw, device=dev) / math.sqrt(2 * F)).requires_grad_(True)
        b1 = torch.zeros(H, device=dev, requires_grad=True)
        w2 = (torch.randn(C, H, generator=gw, device=dev) * 1e-3).requires_grad_(True)
        b2 = torch.zeros(C, device=dev, requires_grad=True)
        l1, l2 = torch.nn.Linear(2 * F, H).to(dev), torch.nn.Linear(H, C).to(dev)
        with torch.no_grad():
            l1.weight.copy_(w1), l1.bias.copy_(b1), l2.weight.copy_(w2), l2.bias.copy_(b2)
        state["readout_cot"] = torch.randn(B, T, C, generator=gw, device=dev)
        last = L - 1

        def ro_fwd(st):
            feats = st[f"out{last}"][0].detach().requires_grad_(True)
            if args.readout == "fused":
                logits = complex_readout(feats, w1, b1, w2, b2, pool=False)
            else:  # the FBT stack's exit copy (pure.py:536), then train.py:130-132
                f = feats.permute(1, 2, 0).contiguous()
                x = torch.cat([f.real, f.imag], dim=-1).reshape(B * T, 2 * F)
                logits = l2(torch.relu(l1(x))).reshape(B, T, C)
            st["readout"] = (feats, logits)

        def ro_bwd(st):
            feats, logits = st.pop("readout")
            logits.backward(st["readout_cot"])
            st["grads_readout"] = feats.grad

        ops.insert(L, ("readout_fwd", ro_fwd))
        ops.append(("readout_bwd", ro_bwd))
    fb, bb = fbt_recompute_bytes(F, B, T)
    if stack != "none":
        fb += 8 * F * B * T
    nbytes = {}
    for li in range(L):
        nbytes[f"rqf_fbt_recompute_fwd[L{li}]"] = fb
        nbytes[f"rqf_fbt_recompute_bwd[L{li}]"] = bb
    if args.readout != "none":
        nbytes["readout_fwd"] = nbytes["readout_bwd"] = 0
    kernels = {"rqf_fbt_recompute_fwd": "fbt_fwd_rb_kernel",
               "rqf_fbt_recompute_bwd": ("fbt_bwd_rb_kernel<replay> (T % 256 == 0) or "
                                         "fbt_bwd_kernel<replay>, + coef_reduce_kernel")}
    contract = "split-ReLU output, per-tile carries; gy cotangent, full BPTT"
    if stack != "none":
        contract += f"; encoder residual add (act + h) {stack}"
    if args.readout != "none":
        contract += f"; per-timestep [Re; Im] MLP readout (hidden 256, 10 classes), {args.readout}"
        name += f" [+ readout, {args.readout}]"
    config = {"workload": name, "F": F, "B": B, "T": T, "layers": L, "contract": contract}
    cpu_steps = args.cpu_steps or (1000 if cfg == 2 else 500)

    def cpu():
        return cpu_baseline_timeinv(F, B, cpu_steps, L, prospective=True, coef=coef)

    return Plan(name, config, F * B * T * L, (state, ops), nbytes, kernels, cpu, config["contract"])


def plan_chunked_raw(cfg, args, dev):
    """Config 2's workload on (B, T, F) tensors: the chunked two-tap prospective
    scan (rqf_chunked_prospective_fwd / _bwd), whose backward takes the
    forward's output as the reference's autograd context saves it."""
    import torch

    from prospective_rqf_amd import workloads
    from prospective_rqf_amd.chunked_scan_kernel import (
        _chunked_prospective_backward_raw,
        _chunked_prospective_forward_raw,
    )

    F, B, T = 128, 32, 16000
    coef = dict(samp=16000.0, tau=5.0 / 16000.0, seq_duration=1.0)
    name = ("non-selective two-tap scan B=32 T=16000 H=128 on (B,T,F) tensors: chunked "
            "prospective scan (config 2, --layout btf)")
    if args.batch:
        B = args.batch
        name += f" [batch overridden to {B}]"
    if args.seq_len:
        T = args.seq_len
        name += f" [sequence length overridden to {T}]"
    g = torch.Generator(device=dev).manual_seed(1)
    gcpu = torch.Generator().manual_seed(3)
    c1, t0, t1 = workloads.static_two_tap(F, seed=0, device=dev, **coef)
    u = workloads.raw_waveform(B, T, samp=16000.0, generator=gcpu).to(dev)  # (B, T)
    state = {"x": (u[:, :, None].to(torch.complex64) * _cn(g, dev, F)).contiguous(),
             "gy": _cn(g, dev, B, T, F)}

    def fwd(st):
        st["out"] = _chunked_prospective_forward_raw(c1, t0, t1, st["x"])

    def bwd(st):
        st["grads"] = _chunked_prospective_backward_raw(c1, t0, t1, st["x"], st.pop("out"),
                                                        st["gy"])

    ops = [("rqf_chunked_prospective_fwd", fwd), ("rqf_chunked_prospective_bwd", bwd)]
    N = B * T * F
    # The backward's contract reads x and gy and writes grad_x; the saved output
    # it is handed is not needed (grad_C1 comes from x, csrc/timeinv.hip).
    nbytes = {"rqf_chunked_prospective_fwd": 16 * N, "rqf_chunked_prospective_bwd": 24 * N}
    kernels = {"rqf_chunked_prospective_fwd": "btf_fwd_kernel<prospective> (single pass)",
               "rqf_chunked_prospective_bwd": ("btf_bwd_kernel<prospective> (single pass) + "
                                               "btf_coef_reduce_kernel")}
    config = {"workload": name, "F": F, "B": B, "T": T, "layers": 1,
              "contract": "(B,T,F) two-tap scan; x in, y out; backward reads x and gy, "
                          "writes grad_x; full BPTT"}

    def cpu():
        return cpu_baseline_timeinv(F, B, args.cpu_steps or 1000, 1, prospective=True, coef=coef)

    return Plan(name, config, N, (state, ops), nbytes, kernels, cpu, config["contract"])


def plan_chunked(cfg, args, dev):
    import torch

    from prospective_rqf_amd.chunked_scan_kernel import (
        _chunked_scan_backward_raw,
        _chunked_scan_forward_raw,
    )

    B, T, F, L = 4, 161, 64, 2
    if args.batch:
        B = args.batch
    name = "Pure RQF encoder depth 2, (B,T,F) chunked scan B=4 T=161 F=64 (config 1)"
    gcpu = torch.Generator().manual_seed(0)
    state, coefs = {}, []
    for li in range(L):
        r = 0.9 + 0.099 * torch.rand(F, generator=gcpu, dtype=torch.float64)
        ph = math.pi * torch.rand(F, generator=gcpu, dtype=torch.float64)
        c1 = torch.polar(r, ph)
        a = torch.log(c1)
        c2 = -a.real * (c1 - 1) / a  # ZOH gain with a = log C1
        coefs.append((c1.to(torch.complex64).to(dev), c2.to(torch.complex64).to(dev)))
        state[f"u{li}"] = torch.complex(torch.randn(B, T, F, generator=gcpu),
                                        torch.randn(B, T, F, generator=gcpu)).to(dev)
        state[f"gy{li}"] = torch.complex(torch.randn(B, T, F, generator=gcpu),
                                         torch.randn(B, T, F, generator=gcpu)).to(dev)
    ops = []
    for li in range(L):
        def fwd(st, li=li):
            st[f"out{li}"] = _chunked_scan_forward_raw(*coefs[li], st[f"u{li}"])

        ops.append((f"rqf_chunked_scan_fwd[L{li}]", fwd))
    for li in reversed(range(L)):
        def bwd(st, li=li):
            states = st.pop(f"out{li}")
            st[f"grads{li}"] = _chunked_scan_backward_raw(*coefs[li], st[f"u{li}"], states,
                                                          st[f"gy{li}"])

        ops.append((f"rqf_chunked_scan_bwd[L{li}]", bwd))
    N = B * T * F
    nbytes = {}
    for li in range(L):
        nbytes[f"rqf_chunked_scan_fwd[L{li}]"] = 16 * N
        nbytes[f"rqf_chunked_scan_bwd[L{li}]"] = 24 * N
    kernels = {"rqf_chunked_scan_fwd": "btf_fwd_kernel (single pass)",
               "rqf_chunked_scan_bwd": "btf_bwd_kernel (single pass) + btf_coef_reduce_kernel"}
    config = {"workload": name, "F": F, "B": B, "T": T, "layers": L,
              "contract": "(B,T,F) scan, full BPTT; latency-bound, cache-resident"}

    def cpu():
        return cpu_baseline_timeinv(F, B, T, L, prospective=False, coef=None, btf=(coefs, T))

    return Plan(name, config, N * L, (state, ops), nbytes, kernels, cpu, config["contract"])


def plan_multi_osc(cfg, args, dev):
    """Config 6: RQF-S4-style multi-oscillator scan (N = 4 oscillators per filter,
    complex C-weights), fwd + bwd.  Config 7: the fused |y| readout
    (``sequential_scan_abs``) of a single-oscillator scan on real input, forward
    only (an inference path).  Both on the raw-waveform shape of config 2."""
    import torch

    from prospective_rqf_amd import multi_osc_scan as mo
    from prospective_rqf_amd import workloads

    B, T, F = 32, 16000, 128
    N = 4 if cfg == 6 else 1
    if args.batch:
        B = args.batch
    if args.seq_len:
        T = args.seq_len
    g = torch.Generator().manual_seed(6)
    r = 0.9 + 0.0999 * torch.rand(F * N, generator=g, dtype=torch.float64)
    ph = math.pi * torch.rand(F * N, generator=g, dtype=torch.float64)
    c1 = torch.polar(r, ph)
    a = torch.log(c1)
    c2 = (-a.real * (c1 - 1) / a).to(torch.complex64).to(dev)  # ZOH gain with a = log C1
    c1 = c1.to(torch.complex64).to(dev)
    cw = torch.randn(F * N, 2, generator=g).to(dev)
    wave = workloads.raw_waveform(B, T, samp=16000.0, generator=g)  # (B, T)
    gain = torch.randn(F, generator=g)
    state = {}
    if cfg == 6:
        name = ("multi-oscillator C-weighted scan, N=4 oscillators x 128 filters, "
                "B=32 T=16000, complex input (config 6)")
        state["u"] = (wave[:, :, None] * gain).to(torch.complex64).to(dev)
        state["gy"] = workloads.randn_c64(B, T, F, generator=g).to(dev)

        def fwd(st):
            st["y"] = mo._sequential_scan_multi_osc_forward_raw(c1, c2, st["u"], cw[:, 0],
                                                                cw[:, 1], N)

        def bwd(st):
            st["grads"] = mo._sequential_scan_multi_osc_backward_raw(c1, c2, st["u"], cw,
                                                                     st["gy"], N)

        ops = [("rqf_multi_osc_fwd", fwd), ("rqf_multi_osc_bwd", bwd)]
        elems = B * T * F
        nbytes = {"rqf_multi_osc_fwd": 16 * elems, "rqf_multi_osc_bwd": 24 * elems}
        kernels = {"rqf_multi_osc_fwd": "mosc_fwd_kernel<4 oscillators> (single pass)",
                   "rqf_multi_osc_bwd": ("mosc_bwd_kernel<4 oscillators> (single pass) + "
                                         "mosc_coef_kernel")}
        contract = "complex u in, complex y out; grad_u + grad_C1/C2/c_weights"
    else:
        name = ("fused |y| readout: single-oscillator scan on real input, 128 filters, "
                "B=32 T=16000, forward only (config 7)")
        state["u"] = (wave[:, :, None] * gain).to(torch.float32).to(dev)

        def fwd(st):
            st["y"] = mo._sequential_scan_real_forward_abs_raw_block_f(c1, c2, st["u"])

        ops = [("rqf_multi_osc_fwd[abs]", fwd)]
        elems = B * T * F
        nbytes = {"rqf_multi_osc_fwd[abs]": 8 * elems}
        kernels = {"rqf_multi_osc_fwd": "mosc_fwd_kernel<1 oscillator, real, abs> (single pass)"}
        contract = "real u in, |y| real out, no autograd"
    config = {"workload": name, "F": F, "B": B, "T": T, "oscillators": N, "layers": 1,
              "contract": contract}

    def cpu():
        return cpu_baseline_multi_osc(F, N, B, args.cpu_steps or 500, c1.cpu(), c2.cpu(),
                                      cw.cpu(), absolute=cfg == 7)

    return Plan(name, config, elems, (state, ops), nbytes, kernels, cpu, contract)


# ---------------------------------------------------------------------------
# CPU baselines: fp32 PyTorch restatement of the reference CPU path
# ---------------------------------------------------------------------------


def _cpu_threads():
    import torch

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    return threads


CPU_REPS = 3


def _median_time(run, reps=None, warmup=True):
    """Median wall time of ``reps`` runs after one warm-up run (none without
    ``warmup``); each run's time goes to stderr as it ends (long samples would
    otherwise print nothing for minutes)."""
    reps = CPU_REPS if reps is None else reps
    times = []
    for i in range(0 if warmup else 1, reps + 1):
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        print(f"cpu baseline: {'warm-up' if i == 0 else f'run {i} of {reps}'} {dt:.1f} s",
              file=sys.stderr, flush=True)
        if i:
            times.append(dt)
    times.sort()
    return times[len(times) // 2]


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline_selective(F, B, G, steps, log_scale, samp, tau, seq, layers, reps=None,
                           warmup=True):
    import torch

    from oracle import torch_ref
    from prospective_rqf_amd import workloads

    threads = _cpu_threads()
    g = torch.Generator().manual_seed(1)
    per_layer = []
    for li, (write_raw, activate) in enumerate(layers):
        inp = workloads.selective_inputs(F, B, steps, G=G, warp_scale=log_scale, samp=samp,
                                         tau=tau, seq_duration=seq, device="cpu", seed=li)
        z = workloads.randn_c64(F, B, steps, generator=g)
        cot = workloads.randn_c64(F, B, steps, generator=g)
        per_layer.append((inp, z, cot, write_raw, activate))

    def run():
        for inp, z, cot, write_raw, activate in per_layer:
            leaves = [inp.gamma_logits, inp.warp_logits, inp.write_logits, inp.bias, inp.theta]
            for v in leaves:
                v.requires_grad_(True)
                v.grad = None
            zz = z.clone().requires_grad_(True)
            raw = torch_ref.selective_scan(zz, inp)
            loss = (cot.conj() * raw).real.sum() if write_raw else 0.0
            if activate:
                loss = loss + (cot.conj() * torch_ref.split_relu(raw)).real.sum()
            loss.backward()

    reps = CPU_REPS if reps is None else reps
    t = _median_time(run, reps, warmup)
    timing = (f"median of {reps} after 1 warm-up" if warmup
              else f"{'one run' if reps == 1 else f'median of {reps}'}, no warm-up")
    return {
        "value": F * B * steps * len(layers) / t / 1e9,
        "unit": "Gelem/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"fp32 PyTorch restatement of reference_layer_scan after the drive GEMM "
                   f"(oracle/torch_ref.py), fwd + autograd bwd, {len(layers)} layer(s), F={F} "
                   f"B={B} T={steps} (T reduced from the GPU shape: like the reference's loop, "
                   f"whose backward of each A[..., t] select materialises a full (F,B,T) "
                   f"gradient, the cost per element grows with T, about 8x from T=200 to "
                   f"T=1000), {timing}; torch threads={threads} (the GPU box's CPU share is "
                   f"16 threads), os.cpu_count()={os.cpu_count()}, cpu={_cpu_model()}"),
    }


def cpu_baseline_timeinv(F, B, steps, L, *, prospective, coef, btf=None):
    """_sequential_scan_cpu (+ _apply_prospective_taps) in (B,T,F), fwd + autograd bwd."""
    import torch

    from oracle import torch_ref
    from prospective_rqf_amd import workloads

    threads = _cpu_threads()
    g = torch.Generator().manual_seed(1)
    layers = []
    for li in range(L):
        if btf is not None:
            c1, c2 = (c.cpu() for c in btf[0][li])
            t0 = t1 = None
        else:
            c1, t0, t1 = workloads.static_two_tap(F, seed=li, **coef)
            c2 = torch.ones_like(c1)
        u = workloads.randn_c64(B, steps, F, generator=g)
        cot = workloads.randn_c64(B, steps, F, generator=g)
        layers.append((c1, c2, t0, t1, u, cot))

    def run():
        for c1, c2, t0, t1, u, cot in layers:
            uu = u.clone().requires_grad_(True)
            cc = c1.clone().requires_grad_(True)
            drive = torch_ref.prospective_drive(uu, t0, t1) if prospective else uu
            y = torch_ref.sequential_scan(cc, c2, drive)
            out = torch_ref.split_relu(y) if prospective else y
            (cot.conj() * out).real.sum().backward()

    t = _median_time(run)
    what = ("_sequential_scan_cpu + _apply_prospective_taps + split-ReLU" if prospective
            else "_sequential_scan_cpu")
    return {
        "value": F * B * steps * L / t / 1e9,
        "unit": "Gelem/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"fp32 PyTorch restatement of {what} (oracle/torch_ref.py), (B,T,F) layout, "
                   f"fwd + autograd bwd, {L} layer(s), F={F} B={B} T={steps}, median of {CPU_REPS} after "
                   f"1 warm-up; torch threads={threads}, os.cpu_count()={os.cpu_count()}, "
                   f"cpu={_cpu_model()}"),
    }


def cpu_baseline_multi_osc(F, N, B, steps, c1, c2, cw, *, absolute):
    """The reference's unfused CPU path for the multi-oscillator scan: expand the
    input over the oscillators, `_sequential_scan_cpu`, C-weighted sum
    (block.py:599-630, 766-785); fwd + autograd bwd, or |y| forward only."""
    import torch

    from oracle import torch_ref
    from prospective_rqf_amd import workloads

    threads = _cpu_threads()
    g = torch.Generator().manual_seed(2)
    u = workloads.randn_c64(B, steps, F, generator=g)
    cot = workloads.randn_c64(B, steps, F, generator=g)
    cwc = torch.view_as_complex(cw.contiguous())

    def run():
        uu = u.clone().requires_grad_(not absolute)
        cc = c1.clone().requires_grad_(not absolute)
        x = torch_ref.sequential_scan(cc, c2, uu.repeat_interleave(N, dim=-1))
        y = (x.view(B, steps, F, N) * cwc.view(F, N)).sum(-1) if N > 1 else x
        if absolute:
            y.abs()
        else:
            (cot.conj() * y).real.sum().backward()

    with torch.set_grad_enabled(not absolute):
        t = _median_time(run)
    what = ("expand + _sequential_scan_cpu + C-weighted sum, fwd + autograd bwd" if not absolute
            else "_sequential_scan_cpu(...).abs(), forward")
    return {
        "value": F * B * steps / t / 1e9,
        "unit": "Gelem/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"fp32 PyTorch restatement of {what} (oracle/torch_ref.py), (B,T,F) layout, "
                   f"N={N} oscillators, F={F} B={B} T={steps} (T reduced), median of {CPU_REPS} after 1 "
                   f"warm-up; torch threads={threads}, os.cpu_count()={os.cpu_count()}, "
                   f"cpu={_cpu_model()}"),
    }


# ---------------------------------------------------------------------------
# Traffic table (rocprofv3 FETCH_SIZE / WRITE_SIZE, committed under profiles/)
# ---------------------------------------------------------------------------


def traffic_from_table(workload_key, entry):
    """HBM bytes per call of ``entry`` for ``workload_key`` from profiles/traffic.md, or None.

    Rows look like ``| config3 | rqf_selective_bwd | <fetch bytes> | <write bytes> | ... |``
    with bytes already scaled by the copy-kernel calibration."""
    try:
        with open(TRAFFIC_TABLE) as fh:
            for line in fh:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 4 and cells[0] == workload_key and cells[1] == entry:
                    return int(float(cells[2]) + float(cells[3]))
    except (OSError, ValueError):
        return None
    return None


# ---------------------------------------------------------------------------
# Main
# ---------------------------------------------------------------------------


def main():
    global CPU_REPS
    args = _args()
    CPU_REPS = max(1, args.cpu_reps)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (single-GPU scan kernels; "
              "no collectives). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    import torch

    from prospective_rqf_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    cfg = args.config
    if cfg in (3, 4):
        plan = plan_selective(cfg, args, dev)
    elif cfg == 2 and args.layout == "btf":
        plan = plan_chunked_raw(cfg, args, dev)
    elif cfg in (2, 5):
        plan = plan_fbt(cfg, args, dev)
    elif cfg in (6, 7):
        plan = plan_multi_osc(cfg, args, dev)
    else:
        plan = plan_chunked(cfg, args, dev)
    state, ops = plan.ops
    torch.cuda.synchronize()

    def step(events=None):
        for i, (_, fn) in enumerate(ops):
            if events is not None:
                events[i].record()
            fn(state)
        if events is not None:
            events[len(ops)].record()
        for k in [k for k in state if k.startswith("grads")]:
            del state[k]

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(ops) + 1)]
              for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    per_op = {name: sum(ev[i].elapsed_time(ev[i + 1]) for ev in events) / args.steps
              for i, (name, _) in enumerate(ops)}
    scan_ms = sum(per_op.values())
    fwd_ms = sum(v for k, v in per_op.items() if "_fwd" in k)
    proj_ms = {k: v for k, v in per_op.items() if k.startswith(("proj_", "readout_"))}
    bwd_ms = scan_ms - fwd_ms
    value = plan.elems / (scan_ms * 1e-3) / 1e9
    scan_ops = {k: v for k, v in per_op.items() if not k.startswith(("proj_", "readout_"))}
    dom = max(scan_ops, key=scan_ops.get)
    entry = dom.split("[")[0]
    dom_bytes = plan.bytes[dom]
    achieved = dom_bytes / (per_op[dom] * 1e-3) / 1e9
    all_bytes = sum(plan.bytes.values())
    # a per-layer row ("rqf_selective_bwd[L0]") where the table has one, else
    # the entry point's; the table's rows are the default workloads and the
    # (B,T,F) layout of config 2, so other variants report none
    key = f"config{cfg}" + (" (B,T,F)" if cfg == 2 and args.layout == "btf" else "")
    variant = (args.batch or args.seq_len or args.stack != "none" or args.act_only or
               args.chunk or (cfg == 2 and args.layer0))
    traffic = (None if variant else
               traffic_from_table(key, dom) or traffic_from_table(key, entry))
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (complex64 state)",
        "data": "synthetic (seeded N(0,1) drive, logits and cotangents; recipe parameters)",
        "config": plan.config,
        "roofline": {
            "bound": "hbm",
            "kernel": f"{entry}: {plan.kernels[entry]}",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "alg_bytes": dom_bytes,
            "avg_ms": round(per_op[dom], 4),
        },
        "detail": {
            "scan_ms": round(scan_ms, 4),
            "fwd_ms": round(fwd_ms, 4),
            "bwd_ms": round(bwd_ms, 4),
            "per_entry_ms": {k: round(v, 4) for k, v in per_op.items()},
            "per_entry_GBs": {k: round(plan.bytes[k] / (v * 1e-3) / 1e9, 1)
                              for k, v in per_op.items()},
            "step_frac_of_hbm": round(all_bytes / (scan_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "alg_bytes_step": all_bytes,
            "alg_bytes_entries": plan.bytes,
        },
    }
    if proj_ms:
        result["detail"]["outside_scan_ms"] = {k: round(v, 4) for k, v in proj_ms.items()}
        result["detail"]["scan_only_ms"] = round(scan_ms - sum(proj_ms.values()), 4)
    if args.cpu and plan.cpu is not None:
        result["cpu_baseline"] = plan.cpu()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the complex-scan backends on one MI355X.

Default workload (the north-star metric): selective
fused scan, F=H=256 channels, B=64, T=16000, grouped warp (G=8), sigmoid gamma
and write heads, prospective tau-mode input, intermediate-layer contract
(raw + split-ReLU outputs, cotangents on both, full BPTT).  One step = one
forward + one backward of the scan kernels over the whole batch; inputs are
resident in HBM before timing starts.  The drive and logit GEMMs are outside
the metric.

Prints ONE JSON line (rank 0).  ``--config`` 2/4/5 select the other configs
for manual runs.
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


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, choices=[2, 3, 4, 5])
    ap.add_argument("--cpu-baseline", dest="cpu", action="store_true", default=True)
    ap.add_argument("--no-cpu-baseline", dest="cpu", action="store_false")
    ap.add_argument("--cpu-steps", type=int, default=0,
                    help="time steps of the CPU baseline sample (0: auto, ~10-30 s)")
    ap.add_argument("--batch", type=int, default=0,
                    help="override the config's batch size (experiments only)")
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
# Workloads
# ---------------------------------------------------------------------------


def selective_workload(F, B, T, G, device, *, log_scale, seq_duration=1.0, samp=16000.0,
                       tau=5.0 / 16000.0, write_raw=True, activate=True, seed=0):
    import torch

    from prospective_rqf_amd import workloads

    inputs = workloads.selective_inputs(
        F, B, T, G=G, gamma=True, write=True, warp="grouped", write_sigmoid=True, write_max=2.0,
        gamma_scale=math.log(1.25), warp_scale=log_scale, prospective=True, samp=samp, tau=tau,
        seq_duration=seq_duration, device=device, seed=seed)
    g = torch.Generator(device=device).manual_seed(seed + 1)

    def cn(*shape):
        return torch.complex(torch.randn(*shape, generator=g, device=device),
                             torch.randn(*shape, generator=g, device=device))

    z = cn(F, B, T)
    gy = cn(F, B, T) if write_raw else None
    gx = cn(F, B, T) if activate else None
    return inputs, z, gy, gx


def selective_bytes(F, B, T, G, chunk, *, write_raw=True, activate=True):
    """Algorithmic HBM bytes (each boundary tensor once) for fwd and bwd."""
    N = F * B * T
    nc = -(-T // chunk)
    ent = 8 * F * B * nc
    warp = 4 * G * B * T
    fwd = N * (8 + 4 + 4 + 8 * write_raw + 8 * activate) + warp + ent
    bwd = N * (8 + 4 + 4 + 8 * write_raw + 8 * activate + 8 + 4 + 4) + 2 * warp + ent
    return fwd, bwd


# ---------------------------------------------------------------------------
# CPU baseline: fp32 PyTorch restatement of the reference CPU path
# ---------------------------------------------------------------------------


def cpu_baseline_selective(F, B, G, steps, log_scale):
    import torch

    from oracle import torch_ref
    from prospective_rqf_amd import workloads

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    inp = workloads.selective_inputs(F, B, steps, G=G, warp_scale=log_scale, device="cpu",
                                     seed=0)
    leaves = [inp.gamma_logits, inp.warp_logits, inp.write_logits, inp.bias, inp.theta]
    g = torch.Generator().manual_seed(1)
    z = workloads.randn_c64(F, B, steps, generator=g)
    cot = workloads.randn_c64(F, B, steps, generator=g)

    def run():
        for v in leaves:
            v.requires_grad_(True)
            v.grad = None
        zz = z.clone().requires_grad_(True)
        raw = torch_ref.selective_scan(zz, inp)
        act = torch_ref.split_relu(raw)
        loss = (cot.conj() * raw).real.sum() + (cot.conj() * act).real.sum()
        loss.backward()

    run()  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[1]
    return {
        "value": F * B * steps / t / 1e9,
        "unit": "Gelem/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"fp32 PyTorch restatement of reference_layer_scan after the drive GEMM "
                   f"(oracle/torch_ref.py), fwd + autograd bwd, F={F} B={B} T={steps} "
                   f"(T reduced from 16000), median of 3 after 1 warm-up; "
                   f"torch threads={threads}, cpu={platform.processor() or platform.machine()}"),
    }


# ---------------------------------------------------------------------------
# Main
# ---------------------------------------------------------------------------


def main():
    args = _args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (single-GPU scan kernels; "
              "no collectives). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    import torch

    from prospective_rqf_amd import _lib
    from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward

    _lib.load()
    dev = torch.device("cuda:0")
    cfg = args.config
    if cfg == 3:
        F, B, T, G, layers = 256, 64, 16000, 8, 1
        log_scale = math.log(1.25)
        workload = "selective fused scan B=64 T=16000 H=256 G=8 (config 3)"
        seq_duration, samp, tau = 1.0, 16000.0, 5.0 / 16000.0
    elif cfg == 4:
        F, B, T, G, layers = 256, 64, 4096, 4, 1
        log_scale = math.log(4.0)
        workload = "selective fused scan B=64 T=4096 H=256 G=4 (config 4, one layer)"
        seq_duration, samp, tau = 4096.0, 1.0, 5.0
    else:
        raise SystemExit("configs 2 and 5 are measured by bench_fbt (not yet wired)")
    if args.batch:
        B = args.batch
        workload += f" [batch overridden to {B}]"
    chunk = 256
    inputs, z, gy, gx = selective_workload(F, B, T, G, dev, log_scale=log_scale,
                                           seq_duration=seq_duration, samp=samp, tau=tau)
    torch.cuda.synchronize()

    def step(ev=None):
        if ev:
            ev[0].record()
        raw, act, entries = selective_forward(z, inputs, True, True, chunk)
        if ev:
            ev[1].record()
        outs = selective_backward(z, inputs, entries, gy, gx, True, False, chunk)
        if ev:
            ev[2].record()
        return raw, act, outs

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        out = step(events[i])
        del out
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = [e[0].elapsed_time(e[1]) for e in events]
    bwd_ms = [e[1].elapsed_time(e[2]) for e in events]
    fwd = sum(fwd_ms) / len(fwd_ms)
    bwd = sum(bwd_ms) / len(bwd_ms)
    ms_per_step = wall * 1e3 / args.steps
    elems = F * B * T * layers
    fwd_bytes, bwd_bytes = selective_bytes(F, B, T, G, chunk)
    value = elems / ((fwd + bwd) * 1e-3) / 1e9
    achieved_bwd = bwd_bytes / (bwd * 1e-3) / 1e9
    achieved_fwd = fwd_bytes / (fwd * 1e-3) / 1e9
    result = {
        "metric": "scan Gelem/s (B·T·H complex) fwd+bwd at T=16000; % of HBM roofline",
        "value": round(value, 3),
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (complex64 state)",
        "data": "synthetic (seeded N(0,1) drive, logits and cotangents; recipe parameters)",
        "config": {"workload": workload, "F": F, "B": B, "T": T, "G": G, "chunk": chunk,
                   "contract": "raw+act outputs, gy+gx cotangents, full BPTT"},
        "roofline": {
            "bound": "hbm",
            "kernel": "rqf_selective_bwd (selective_bwd_kernel + group/partial reductions)",
            "achieved": round(achieved_bwd, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_bwd / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "detail": {
            "fwd_ms": round(fwd, 4),
            "bwd_ms": round(bwd, 4),
            "fwd_GBs": round(achieved_fwd, 1),
            "fwd_frac": round(achieved_fwd / HBM_PEAK_GBS, 4),
            "fwd_bwd_frac": round((fwd_bytes + bwd_bytes) / ((fwd + bwd) * 1e-3) / 1e9
                                  / HBM_PEAK_GBS, 4),
            "alg_bytes_fwd": fwd_bytes,
            "alg_bytes_bwd": bwd_bytes,
        },
    }
    if args.cpu:
        steps = args.cpu_steps or 200
        result["cpu_baseline"] = cpu_baseline_selective(F, B, G, steps, log_scale)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

"""Extract the RQF filter parameters of the reference's packaged checkpoints.

Writes, next to this script:

* ``checkpoint_params.npz`` - per-channel float32 leaves and bound buffers of every
  ``rqf_fwd`` module in the Pure RQF and RQF-S4 checkpoints of
  ``/root/reference/pretrained`` (``log_tau``, ``freq_param``, ``gamma_param``,
  ``_min/_max_gamma``, ``_min/_max_freq``), flattened over (checkpoint, block, channel);
* ``checkpoint_params.json`` - one record per checkpoint: name, model family, input
  variant, depth, prospective/skip flags from its ``hydra_overrides``, and the
  settings the filters were built with (``dt = 1/samp_frequency``, discretization,
  clamp_gamma, activation, prospective mode, sequence length), read from the
  reference's model and data YAML (configs/model/{pure_rqf,rqf_s4}.yaml,
  configs/data/speech_commands_{raw,mfcc}.yaml, train.py:443-448 for the MFCC
  override), plus each block's row range in the arrays;
* ``encoder_<name>.npz`` - input projection and complex ``W`` of every block of three
  Pure RQF checkpoints, for the end-to-end encoder parity test.

Checkpoints are read with ``torch.load(weights_only=True)``; YAML with
``yaml.safe_load``.  Nothing of the reference is imported or executed.  Run in a
container that has ``/root/reference``:  ``python tests/golden/make_checkpoint_params.py``.
The ORGaNICs checkpoints hold no RQF filter and are skipped.
"""

from __future__ import annotations

import json
import os
import re

import numpy as np
import torch
import yaml

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
LEAVES = ("log_tau", "freq_param", "gamma_param", "_min_gamma", "_max_gamma", "_min_freq",
          "_max_freq")
ENCODER_CHECKPOINTS = ("pure_rqf_raw_full_M_res_p_seed0", "pure_rqf_raw_full_M_nores_np_seed0",
                       "pure_rqf_mfcc_full_L_res_p_seed0")


def _overrides(lst):
    out = {}
    for item in lst:
        k, _, v = item.partition("=")
        out[k] = v
    return out


def _model_settings(family, variant):
    with open(f"{REF}/configs/model/{family}.yaml") as f:
        model = yaml.safe_load(f)
    with open(f"{REF}/configs/data/speech_commands_{variant}.yaml") as f:
        data = yaml.safe_load(f)
    kw = dict(model["encoder_kwargs"])
    if variant == "mfcc" and "mfcc_encoder_kwargs" in model:
        kw.update(model["mfcc_encoder_kwargs"])
    return model, kw, data


def main():
    names = sorted(n[:-3] for n in os.listdir(f"{REF}/pretrained")
                   if n.endswith(".pt") and re.match(r"(pure_rqf|rqf_s4)_", n))
    arrays = {k: [] for k in LEAVES}
    records = []
    row = 0
    for name in names:
        ck = torch.load(f"{REF}/pretrained/{name}.pt", map_location="cpu", weights_only=True)
        ov = _overrides(ck["hydra_overrides"])
        family = ov["model"]
        variant = ov["data"].rsplit("_", 1)[-1]
        model, kw, data = _model_settings(family, variant)
        sd = ck["state_dict"]
        depth = int(ov.get("model.depth", model["depth"]))
        blocks = []
        for b in range(depth):
            prefix = f"encoder.blocks.{b}.rqf_fwd."
            n = sd[prefix + "log_tau"].numel()
            for k in LEAVES:
                arrays[k].append(sd[prefix + k].detach().float().numpy().reshape(-1))
            blocks.append([row, n])
            row += n
        truthy = lambda v: str(v).lower() == "true"  # noqa: E731
        records.append(dict(
            name=name, family=family, variant=variant, depth=depth,
            prospective=truthy(ov.get("model.prospective_input", model["prospective_input"])),
            skip=truthy(ov.get("model.skip_connection", model["skip_connection"])),
            training=ov.get("training"), epoch=int(ck.get("epoch", -1)),
            dt=1.0 / float(kw["samp_frequency"]), samp_frequency=float(kw["samp_frequency"]),
            discretization=kw["discretization"], clamp_gamma=bool(kw["clamp_gamma"]),
            activation=kw["activation"], prospective_mode=model["prospective_mode"],
            prospective_tau=model["prospective_tau"], seq_len=int(data["sequence_length"]),
            input_dims=int(data["feature_dim"]), blocks=blocks,
        ))
        if name in ENCODER_CHECKPOINTS:
            enc = {"input_proj_weight": sd["encoder.input_proj.weight"].float().numpy(),
                   "input_proj_bias": sd["encoder.input_proj.bias"].float().numpy()}
            for b in range(depth):
                enc[f"W{b}"] = sd[f"encoder.blocks.{b}.W"].to(torch.complex64).numpy()
            np.savez_compressed(os.path.join(HERE, f"encoder_{name}.npz"), **enc)
    np.savez_compressed(os.path.join(HERE, "checkpoint_params.npz"),
                        **{k.lstrip("_"): np.concatenate(v) for k, v in arrays.items()})
    with open(os.path.join(HERE, "checkpoint_params.json"), "w") as f:
        f.write("[\n" + ",\n".join(json.dumps(r) for r in records) + "\n]\n")
    print(f"{len(records)} checkpoints, {row} filter channels")


if __name__ == "__main__":
    main()

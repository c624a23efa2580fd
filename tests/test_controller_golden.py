"""The restated selective controller against the reference's own.

``tests/golden/controller_golden.npz`` holds what the reference's
``SelectiveController`` (rqf_models/backbones/rqf/selective.py:100-278) built
on its own ``RQF`` filter module, written by
``tests/golden/make_controller_golden.py``: 64 cases over four filters
(resonant recipe, a band past Nyquist in float32 and float64, the stability
band), eight settings (interior / straight-through clamp, log-shift link,
modulus features, global / grouped warp, band / no band, affine / sigmoid
write) and five call forms (prospective or not, tau / gamma mode,
prospective_tau None / scalar / per filter).  The restatement
(``prospective_rqf_amd.selective_controller``) must reproduce the filter
projection done at construction and every field of the scan inputs exactly:
the same torch operations in the same order give the same bits.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from prospective_rqf_amd.selective_controller import (
    FilterState,
    SelectiveController,
    SelectiveRQFConfig,
)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "controller_golden.npz")
FIELDS = ("gamma_logits", "warp_logits", "write_logits", "bias", "theta", "minimum", "span",
          "step", "horizon", "theta_minimum", "theta_maximum")


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as z:
        data = {k: z[k] for k in z.files}
    return data, json.loads(str(data["meta"]))


def _filter(data, p, case):
    t = {k: torch.from_numpy(data[p + "pre_" + k].copy())
         for k in ("log_tau", "log_gamma", "log_theta", "min_gamma", "max_gamma", "min_freq",
                   "max_freq")}
    return FilterState(dt=case["dt"], clamp_gamma=case["clamp_gamma"], **t)


def _run(data, case):
    p = f"c{case['case']}/"
    rqf = _filter(data, p, case)
    ctl = SelectiveController(data_n_in(data), rqf, SelectiveRQFConfig(**case["config"]))
    for name in ("W_gamma", "W_write", "W_delta"):
        if p + name in data:
            assert getattr(ctl, name) is not None, name
            setattr(ctl, name, torch.from_numpy(data[p + name].copy()))
        else:
            assert getattr(ctl, name) is None, name
    source = torch.complex(torch.from_numpy(data[p + "source_re"].copy()),
                           torch.from_numpy(data[p + "source_im"].copy()))
    inp = ctl(source, rqf, prospective=case["prospective"], mode=case["mode"],
              prospective_tau=case["prospective_tau"])
    return p, rqf, inp


def data_n_in(data):
    return int(json.loads(str(data["meta"]))["n_in"])


def test_golden_covers_every_branch(golden):
    """The fixture exercises each setting the mapping branches on."""
    _, meta = golden
    cases = meta["cases"]
    assert len(cases) == 64
    seen = {(c["config"].get("gamma_link", "sigmoid"), c["config"].get("gamma_edge", "interior_clamp"),
             c["config"].get("gamma_control", True)) for c in cases}
    assert ("sigmoid", "st_clamp", True) in seen and ("log_shift", "interior_clamp", True) in seen
    assert any(not c["config"].get("gamma_control", True) for c in cases)
    assert {c["config"].get("frequency_warp", "none") for c in cases} == {"none", "global",
                                                                          "grouped"}
    assert {type(c["prospective_tau"]).__name__ for c in cases} == {"NoneType", "float", "list"}
    assert any(c["float64"] for c in cases) and any(c["clamp_gamma"] for c in cases)


def test_controller_matches_reference(golden):
    data, meta = golden
    moved = 0
    for case in meta["cases"]:
        p, rqf, inp = _run(data, case)
        tag = f"case {case['case']} ({case['filter']}, {case['config']}, {case['mode']})"
        # Construction-time projection of the filter's leaves.
        for leaf in ("log_gamma", "log_theta"):
            want = data[p + "post_" + leaf]
            got = getattr(rqf, leaf).numpy()
            assert got.dtype == want.dtype and np.array_equal(got, want), f"{tag}: {leaf}"
            moved += not np.array_equal(data[p + "pre_" + leaf], want)
        for name in FIELDS:
            want = data[p + "out_" + name]
            got = getattr(inp, name).detach().numpy()
            assert got.dtype == want.dtype, f"{tag}: {name} dtype {got.dtype} != {want.dtype}"
            assert got.shape == want.shape, f"{tag}: {name} shape"
            # NaN where the reference gives NaN: the stability-band projection
            # can push gamma below min_gamma, whose logit is then undefined.
            assert np.array_equal(got, want, equal_nan=True), (
                f"{tag}: {name} max diff {np.nanmax(np.abs(got.astype(np.float64) - want))}")
        if p + "out_groups" in data:
            assert inp.groups is not None and np.array_equal(inp.groups.numpy(),
                                                             data[p + "out_groups"]), tag
        else:
            assert inp.groups is None, tag
        assert np.array_equal(np.array([float(v) for v in inp.options]), data[p + "out_options"]), tag
        assert [type(v) for v in inp.options] == [bool] * 4 + [float] * 2 + [bool] * 3 + \
            [float] * 2 + [bool], tag
    # The projection is exercised, not just carried through.
    assert moved > 10


def test_controller_rejects_what_the_reference_rejects(golden):
    data, meta = golden
    for err in meta["errors"]:
        if err["where"] == "config":
            with pytest.raises((ValueError, TypeError)) as exc:
                SelectiveRQFConfig(**err["config"])
        else:
            case = next(c for c in meta["cases"] if c["filter"] == err["filter"])
            rqf = _filter(data, f"c{case['case']}/", case)
            with pytest.raises(ValueError) as exc:
                SelectiveController(data_n_in(data), rqf, SelectiveRQFConfig(**err["config"]))
        assert type(exc.value).__name__ == err["type"]
        assert str(exc.value) == err["message"]


def test_assemble_is_forward_after_the_head_gemm(golden):
    """``forward`` = ``assemble(project(source))`` (what the workloads rely on)."""
    data, meta = golden
    case = meta["cases"][5]
    p, rqf, inp = _run(data, case)
    ctl = SelectiveController(data_n_in(data), _filter(data, p, case),
                              SelectiveRQFConfig(**case["config"]))
    for name in ("W_gamma", "W_write", "W_delta"):
        if p + name in data:
            setattr(ctl, name, torch.from_numpy(data[p + name].copy()))
    logits = tuple(getattr(inp, n) for n in ("gamma_logits", "warp_logits", "write_logits"))
    again = ctl.assemble(*logits, rqf, prospective=case["prospective"], mode=case["mode"],
                         prospective_tau=case["prospective_tau"])
    for name in FIELDS:
        assert torch.equal(getattr(again, name), getattr(inp, name)), name

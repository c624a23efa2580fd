"""Every compiled kernel variant of the selective scan, against the fp64 oracle.

The library compiles the selective kernels per option set (the reference's
constexpr flags, selective_scan_kernel.py:35-46), per row layout (float4
rows when T % 4 == 0, element rows otherwise), per output set of the forward
(raw only: 4-wavefront blocks; act or act+raw: 8), and, in the backward, per
cotangent set (gy, gx, both; fixed under full BPTT with float4 rows and a
compiled option set) and per form (split teams, or the group form in its
three block shapes).  This matrix reaches each of them at a small shape, so
no compiled variant ships without a parity check:

* option sets: the selective-copying cell's (sigmoid gamma, grouped warp
  with band bound, sigmoid write, prospective), sigmoid gamma + prospective,
  sigmoid gamma alone (pure_rqf_selective.yaml), and a set with no compiled
  form (gamma-horizon mode) that runs the run-time-flag kernels;
* T = 256 (float4 rows, whole tiles) and T = 301 (element rows, a ragged
  tile);
* outputs raw only, act only, raw + act; full BPTT and TBPTT(1);
* backward forms split, group 3 x 4, 4 x 3 and 6 x 2 (the group form needs
  the warp head).

Bar: the same as every selective parity test (normwise 1e-4 per tensor,
per-channel dbias / dtheta).  The empty-time call (T = 0), which only
clears the partial sums, is checked for zero gradients.
"""

import numpy as np
import pytest
import torch

from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward
from tests.selective_cases import make_inputs, to_torch
from tests.test_gpu_selective import CASE_ALL, run_case

pytestmark = pytest.mark.gpu

GAMMA_ONLY = dict(gamma=True, write=False, warp="none", log_shift=False, write_sigmoid=True)
SETS = {
    "copy-cell": (CASE_ALL, dict(prospective=True, gamma_horizon=False)),
    "gamma-prospective": (GAMMA_ONLY, dict(prospective=True, gamma_horizon=False)),
    "gamma": (GAMMA_ONLY, dict(prospective=False)),
    "runtime": (CASE_ALL, dict(prospective=True, gamma_horizon=True)),
}
OUTPUTS = {"raw": (False, True), "act": (True, False), "raw+act": (True, True)}


def _cases():
    for name, (case, _) in SETS.items():
        forms = ["split"] + (["group3", "group4", "group6"] if case["warp"] != "none" else [])
        for form in forms:
            for T in (256, 301):
                for out in OUTPUTS:
                    for truncated in (False, True):
                        yield name, form, T, out, truncated


@pytest.mark.parametrize("name,form,T,out,truncated", list(_cases()))
def test_selective_kernel_variants(monkeypatch, name, form, T, out, truncated):
    print(f"case: variant {name} {form} T={T} outputs={out} truncated={truncated}", flush=True)
    case, opts = SETS[name]
    if form == "split":
        monkeypatch.setenv("RQF_BWD_FORM", "split")
    else:
        monkeypatch.setenv("RQF_BWD_FORM", "group")
        monkeypatch.setenv("RQF_BWD_GRP_TEAM", form[-1])
    activate, write_raw = OUTPUTS[out]
    run_case(7, 2, T, case, truncated=truncated, activate=activate, write_raw=write_raw,
             chunk=256, G=3, seed=T + len(name) + 3 * len(form), **opts)


@pytest.mark.parametrize("form", ["split", "group"])
def test_empty_time_clears_the_partials(monkeypatch, form):
    """T = 0: no scan runs; the per-row partial sums are cleared on the
    device (a fill kernel, not a memset node) and reduce to zero gradients."""
    monkeypatch.setenv("RQF_BWD_FORM", form)
    print(f"case: empty time {form}", flush=True)
    F, B = 6, 3
    rng = np.random.default_rng(5)
    inp = to_torch(make_inputs(F, B, 0, CASE_ALL, rng, G=2), device="cuda")
    z = torch.zeros(F, B, 0, dtype=torch.complex64, device="cuda")
    raw, act, entries = selective_forward(z, inp, True, True, 256)
    assert entries.shape == (F * B, 0)
    out = selective_backward(z, inp, entries, torch.zeros_like(z), torch.zeros_like(z), True,
                             False, 256)
    torch.cuda.synchronize()
    dbias, dtheta = out[5], out[6]
    assert dbias.shape == (F,) and dtheta.shape == (F,)
    assert torch.count_nonzero(dbias) == 0 and torch.count_nonzero(dtheta) == 0


@pytest.mark.parametrize("F,G", [(4100, 3), (1100, 1030)])
def test_team_table_without_lds_staging(F, G):
    """The split form's team table is built in LDS for F <= 4096 channels and
    G <= 1024 warp groups; past either it is built from global memory
    (team_build_global).  A short row keeps the oracle cheap."""
    print(f"case: team table F={F} G={G}", flush=True)
    case = dict(CASE_ALL, warp="grouped")
    run_case(F, 1, 12, case, chunk=256, G=G, seed=F + G, prospective=True, gamma_horizon=False)


@pytest.mark.parametrize("name", list(SETS))
@pytest.mark.parametrize("T,chunk", [(1024, 512), (1023, 512), (1024, 2048), (700, 1024)])
def test_tile_entry_rebuild_variants(monkeypatch, name, T, chunk):
    """A chunk longer than the backward's 256-step tile: the backward first
    rebuilds the state entering every tile from the forward's chunk entries
    (selective_rebuild_kernel, compiled per option set and row layout).
    float4 rows (T % 4 == 0) and element rows; several chunks, one chunk
    longer than the row, a ragged last chunk."""
    print(f"case: tile-entry rebuild {name} T={T} chunk={chunk}", flush=True)
    case, opts = SETS[name]
    monkeypatch.setenv("RQF_BWD_FORM", "split")
    run_case(7, 2, T, case, truncated=False, activate=True, write_raw=True, chunk=chunk, G=3,
             seed=T + chunk + len(name), **opts)

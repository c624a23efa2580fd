"""Backend-selection surface: the import-time flags of the reference's scan
module and the call-time FBT toggle of its cells.

Mirrors rqf_models/ops/scan.py:38-70 (``ORGANICS_DISABLE_TRITON`` and
``ORGANICS_SCAN_BACKEND``, read once at import), pure.py:34-40
(``_HAS_FBT_PROSPECTIVE``, independent of ``ORGANICS_DISABLE_TRITON``) and
pure.py:143-144, 500-508 (``ORGANICS_RQF_FBT``, read at every call), and the
routing checks of tests/test_scan_backends_parity.py:113-184.  Each
import-time case runs in a fresh interpreter, since the flags are read when
the module is first imported.
"""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROBE = r"""
import json, os, torch
from prospective_rqf_amd import scan
out = {k: getattr(scan, k) for k in ("_TRITON_DISABLED", "_SCAN_BACKEND", "_USE_CHUNKED",
                                     "_HAS_TRITON", "_HAS_FBT_PROSPECTIVE")}
out["fbt_enabled"] = scan.fbt_enabled()
out["use_kernel"] = scan.selective_use_kernel()
os.environ["ORGANICS_RQF_FBT"] = "0"
out["fbt_enabled_off"] = scan.fbt_enabled()
out["use_kernel_off"] = scan.selective_use_kernel()
os.environ["ORGANICS_RQF_FBT"] = "1"
out["fbt_enabled_on"] = scan.fbt_enabled()
out["fbt_enabled_cpu_x"] = scan.fbt_enabled(torch.zeros(1))
u = torch.zeros(1, 4, 2, dtype=torch.complex64)
c = torch.ones(2, dtype=torch.complex64)
for name in ("sequential_scan", "parallel_scan", "sequential_scan_abs"):
    try:
        getattr(scan, name)(c, c, u)
        out[name] = "ok"
    except RuntimeError as e:
        out[name] = str(e)
print("PROBE" + json.dumps(out))
"""


def _probe(**env):
    e = {k: v for k, v in os.environ.items() if not k.startswith("ORGANICS_")}
    e.update(env)
    e["PYTHONPATH"] = ROOT + os.pathsep + e.get("PYTHONPATH", "")
    res = subprocess.run([sys.executable, "-c", PROBE], cwd=ROOT, env=e, capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    line = [ln for ln in res.stdout.splitlines() if ln.startswith("PROBE")][-1]
    return json.loads(line[len("PROBE"):])


@pytest.fixture(scope="module")
def library_built():
    from prospective_rqf_amd.build import LIB_PATH

    if not os.path.exists(LIB_PATH):
        pytest.skip("librqf_hip.so not built")


DISABLED = "HIP scan backend disabled"
NEEDS_DEVICE = "HIP backend needs a device tensor"


def test_defaults(library_built):
    out = _probe()
    assert out["_SCAN_BACKEND"] == "chunked" and out["_USE_CHUNKED"] is True
    assert out["_TRITON_DISABLED"] is False
    assert out["_HAS_TRITON"] is True and out["_HAS_FBT_PROSPECTIVE"] is True
    assert out["fbt_enabled"] is True and out["use_kernel"] is True
    # the call-time toggle
    assert out["fbt_enabled_off"] is False and out["use_kernel_off"] is False
    assert out["fbt_enabled_on"] is True
    # a host tensor is never FBT-eligible (pure.py:504 requires x.is_cuda)
    assert out["fbt_enabled_cpu_x"] is False
    # served backend, host tensor: raises instead of running on the CPU
    for name in ("sequential_scan", "parallel_scan", "sequential_scan_abs"):
        assert NEEDS_DEVICE in out[name], out[name]


@pytest.mark.parametrize("value", ["sequential", "SEQUENTIAL", "Sequential"])
def test_sequential_backend(library_built, value):
    """ORGANICS_SCAN_BACKEND is lower-cased (scan.py:47); any backend but
    "chunked" turns the chunked kernels and the fused cell paths off."""
    out = _probe(ORGANICS_SCAN_BACKEND=value)
    assert out["_SCAN_BACKEND"] == "sequential" and out["_USE_CHUNKED"] is False
    assert out["_HAS_TRITON"] is True and out["_HAS_FBT_PROSPECTIVE"] is True
    assert out["fbt_enabled"] is False and out["use_kernel"] is False
    assert out["fbt_enabled_on"] is False
    for name in ("sequential_scan", "parallel_scan", "sequential_scan_abs"):
        assert DISABLED in out[name], out[name]


def test_disable_triton(library_built):
    """ORGANICS_DISABLE_TRITON=1 turns the dispatch kernels off (scan.py:39, 66)
    but, as in the reference, not the fused cell paths (pure.py:34-40, 503)."""
    out = _probe(ORGANICS_DISABLE_TRITON="1")
    assert out["_TRITON_DISABLED"] is True and out["_HAS_TRITON"] is False
    assert out["_USE_CHUNKED"] is True and out["_HAS_FBT_PROSPECTIVE"] is True
    assert out["fbt_enabled"] is True and out["use_kernel"] is True
    for name in ("sequential_scan", "parallel_scan", "sequential_scan_abs"):
        assert DISABLED in out[name], out[name]


def test_disable_triton_only_on_exact_one(library_built):
    """Only the string "1" disables (scan.py:39)."""
    out = _probe(ORGANICS_DISABLE_TRITON="true")
    assert out["_TRITON_DISABLED"] is False and out["_HAS_TRITON"] is True


def test_fbt_flag_at_import_is_not_sticky(library_built):
    """ORGANICS_RQF_FBT=0 in the environment at import time still only acts
    per call: setting it back to 1 re-enables the fused path."""
    out = _probe(ORGANICS_RQF_FBT="0")
    assert out["fbt_enabled"] is False and out["use_kernel"] is False
    assert out["fbt_enabled_on"] is True


def test_missing_library(tmp_path):
    """Without the built library nothing is served and nothing falls back."""
    out = _probe(RQF_HIP_LIB=str(tmp_path / "absent.so"))
    assert out["_HAS_TRITON"] is False and out["_HAS_FBT_PROSPECTIVE"] is False
    assert out["fbt_enabled"] is False
    for name in ("sequential_scan", "parallel_scan", "sequential_scan_abs"):
        assert DISABLED in out[name], out[name]

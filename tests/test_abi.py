"""The C-ABI library loads and exports every entry point the header declares
(CPU only: no compute call is made)."""

import ctypes
import os
import re
import subprocess

import pytest

from prospective_rqf_amd import _lib
from prospective_rqf_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rqf_scan.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rqf_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def built_lib():
    if not os.path.exists(LIB_PATH):
        from prospective_rqf_amd.build import build

        build()
    return LIB_PATH


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    assert "rqf_selective_fwd" in names and "rqf_selective_bwd" in names
    assert "rqf_fbt_recompute_fwd" in names and "rqf_chunked_scan_bwd" in names


def test_library_exports_every_declared_symbol(built_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", built_lib], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\b(rqf_[a-z0-9_]+)\b", out))
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, missing


def test_binding_covers_the_header_exactly():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_library_loads_and_reports_version(built_lib):
    lib = _lib.load()
    assert b"gfx950" in lib.rqf_version()
    assert lib.rqf_error_string(-2) == b"workspace missing or too small"
    assert b"no-allocation" in lib.rqf_error_string(_lib.ERR_SCRATCH)
    # Pure host-side queries (no device access).
    assert lib.rqf_fbt_carry_chunks(16000) == 63  # one entry state per 256-step tile
    assert lib.rqf_fbt_workspace(128, 32, 16000) >= 6 * 8 * 128 * 32
    assert lib.rqf_btf_scan_workspace(4, 161, 64) > 0
    s = _lib.SelectiveInputsStruct(F=256, B=64, T=16000, G=8, has_warp=1)
    assert lib.rqf_selective_bwd_workspace(ctypes.byref(s), 256) >= 2 * 8 * 256 * 64


def test_struct_layout_matches_header():
    # Offsets of the C struct: 4 int64, 12 pointers, then 4+2+3+2+1 scalars.
    s = _lib.SelectiveInputsStruct
    assert s.gamma_logits.offset == 32
    assert s.groups.offset == 32 + 11 * 8
    assert s.has_gamma.offset == 32 + 12 * 8
    assert s.bound_warp.offset == 32 + 12 * 8 + 44
    assert s.order.offset == 32 + 12 * 8 + 48
    assert ctypes.sizeof(s) == 32 + 12 * 8 + 56


@pytest.mark.parametrize("cname,image", [("rqf_selective_inputs", "SelectiveInputsStruct"),
                                         ("rqf_proj_gemm_args", "ProjGemmArgs")])
def test_struct_layout_matches_c_compiler(tmp_path, cname, image):
    """offsetof() of every field of the header's struct, as gcc lays it out,
    equals the ctypes image's offsets."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    s = getattr(_lib, image)
    fields = [name for name, _ in s._fields_]
    src = tmp_path / "offsets.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "rqf_scan.h"\nint main(void) {\n'
        + "".join(f'  printf("{f} %zu\\n", offsetof({cname}, {f}));\n' for f in fields)
        + f'  printf("sizeof %zu\\n", sizeof({cname}));\n  return 0;\n}}\n')
    exe = tmp_path / "offsets"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = dict(line.split() for line in subprocess.run(
        [str(exe)], check=True, capture_output=True, text=True).stdout.splitlines())
    for f in fields:
        assert int(got[f]) == getattr(s, f).offset, f
    assert int(got["sizeof"]) == ctypes.sizeof(s)


def test_product_refuses_cpu_tensors():
    import torch

    from prospective_rqf_amd.fbt_scan_kernel import fbt_prospective_scan

    z = torch.zeros(2, 1, 4, dtype=torch.complex64)
    c = torch.zeros(2, dtype=torch.complex64)
    with pytest.raises(_lib.RQFError):
        fbt_prospective_scan(c, c, c, z)


def test_header_constants_match_the_binding():
    text = open(HEADER).read()
    assert re.search(r"RQF_ERR_SCRATCH = (-\d+)", text).group(1) == str(_lib.ERR_SCRATCH)
    m = re.search(r"#define RQF_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    assert int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES


def test_noalloc_rejects_oversized_problems_before_any_device_call(built_lib):
    """Beyond the static scratch (6 fp64 partials per row) the entry point
    returns RQF_ERR_SCRATCH before looking at a pointer or calling HIP (here
    every pointer is NULL and there is no device)."""
    lib = _lib.load()
    rows = _lib.NOALLOC_SCRATCH_BYTES // 48
    args = [None] * 10
    assert lib.rqf_fbt_recompute_bwd_noalloc(*args, rows + 1, 1, 16, None) == _lib.ERR_SCRATCH
    assert lib.rqf_fbt_recompute_bwd_noalloc(*args, 1024, rows // 1024 + 1, 16,
                                             None) == _lib.ERR_SCRATCH
    assert lib.rqf_fbt_recompute_bwd_noalloc(*args, 2 ** 40, 2 ** 40, 16,
                                             None) == _lib.ERR_SCRATCH
    assert lib.rqf_fbt_recompute_bwd_noalloc(*args, -1, 1, 16, None) == -1


def test_multi_osc_rejects_oversized_grids(built_lib):
    """The multi-oscillator entry points take any number of filters whose
    grid fits one dispatch (past 65536 the forward addresses its passes with
    64-bit addresses).  Grids past 2^32 - 1 work-items (B * ceil(F / 16) past
    4194303 blocks of up to 1024 threads), and F * N past 2^31 - 1, are
    refused with RQF_ERR_ARG (-1; and the workspace query 0) before looking at
    a pointer or calling HIP.  The exact bound is in test_grid_limits.py."""
    lib = _lib.load()
    assert lib.rqf_multi_osc_workspace(2, 100, 65537, 4, 1) > 0
    assert lib.rqf_multi_osc_workspace(2, 100, 65536, 4, 1) > 0
    big_b = 2 ** 31 // 4 + 1  # B * ceil(F / 16) = 2^31 + 4 blocks with F = 64
    assert lib.rqf_multi_osc_workspace(big_b, 1, 64, 1, 1) == 0
    assert lib.rqf_multi_osc_fwd(None, None, None, None, 0, None, 0, big_b, 1, 64, 1, None, 0,
                                 None) == -1
    assert lib.rqf_multi_osc_bwd(None, None, None, None, 0, None, None, None, None, None, big_b,
                                 1, 64, 1, None, 0, None) == -1
    assert lib.rqf_multi_osc_fwd(None, None, None, None, 0, None, 0, 1, 1, 2 ** 20, 4096, None,
                                 0, None) == -1  # F * N coefficient reductions past 2^31 - 1


def test_shape_queries_take_edge_shapes_without_crashing(built_lib):
    """The host-side shape logic (workspace sizes, the backward's form and
    block shape) runs before any launch and must take empty and degenerate
    shapes: zero batch, time or filters, a warp head with no rows.  Run in a
    child process, so that a host crash (an integer division by zero, as an
    empty-time selective call with a warp head once caused) fails this test
    rather than the suite."""
    import subprocess
    import sys

    code = """
import ctypes, itertools
from prospective_rqf_amd import _lib
lib = _lib.load()
for F, B, T, G, warp, chunk in itertools.product((0, 1, 7, 256), (0, 1, 3), (0, 1, 255, 256, 257),
                                                 (0, 1, 3), (0, 1), (1, 256, 1024)):
    s = _lib.SelectiveInputsStruct()
    s.F, s.B, s.T, s.G = F, B, T, G
    s.has_warp, s.has_gamma, s.has_write = warp, 1, 1
    lib.rqf_selective_bwd_workspace(ctypes.byref(s), chunk)
for B, T, F, N in itertools.product((0, 1, 5), (0, 1, 300), (0, 1, 17), (1, 4, 5)):
    lib.rqf_btf_scan_workspace(B, T, F)
    lib.rqf_fbt_workspace(F, B, T)
    lib.rqf_fbt_carry_chunks(T)
    lib.rqf_multi_osc_workspace(B, T, F, N, 0)
    lib.rqf_multi_osc_workspace(B, T, F, N, 1)
    lib.rqf_layer0_grads_workspace(F, 1, T)
print("ok")
"""
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=120, cwd=os.path.dirname(os.path.dirname(__file__)))
    assert out.returncode == 0 and out.stdout.strip() == "ok", (out.returncode, out.stderr[-2000:])

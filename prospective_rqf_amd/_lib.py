"""ctypes binding of ``librqf_hip.so`` (declared in ``include/rqf_scan.h``).

The library is loaded lazily on first use and fails loudly: there is no
silent PyTorch substitute for any kernel in this package.  ``torch`` is
imported first so that the process uses a single HIP runtime (torch's).
"""

from __future__ import annotations

import ctypes
import os

import torch

from prospective_rqf_amd.build import LIB_PATH

_lib = None

# Every symbol the header declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_SZ = ctypes.c_size_t


class SelectiveInputsStruct(ctypes.Structure):
    """ctypes image of ``rqf_selective_inputs``."""

    _fields_ = [
        ("F", _I64), ("B", _I64), ("T", _I64), ("G", _I64),
        ("gamma_logits", _P), ("warp_logits", _P), ("write_logits", _P),
        ("bias", _P), ("theta", _P), ("minimum", _P), ("span", _P), ("step", _P),
        ("horizon", _P), ("theta_minimum", _P), ("theta_maximum", _P),
        ("groups", _P),
        ("has_gamma", _I32), ("has_warp", _I32), ("has_write", _I32), ("log_shift", _I32),
        ("gamma_scale", ctypes.c_float), ("warp_scale", ctypes.c_float),
        ("prospective", _I32), ("gamma_horizon", _I32), ("write_sigmoid", _I32),
        ("write_max", ctypes.c_float), ("write_bias", ctypes.c_float),
        ("bound_warp", _I32),
        ("order", _P),
    ]


class ProjGemmArgs(ctypes.Structure):
    """ctypes image of ``rqf_proj_gemm_args``."""

    _fields_ = [
        ("weights", _P), ("k_pad", _I64), ("m_pad", _I64),
        ("b_cplx", _P), ("b_cplx_rows", _I64),
        ("b_real", _P), ("b_real_rows", _I64),
        ("n", _I64),
        ("out_cplx", _P), ("out_cplx_rows", _I64),
        ("out_real", _P), ("out_real_rows", _I64),
        ("out_real_bias", _P), ("out_real_relu", _I64),
    ]


SIGNATURES = {
    "rqf_proj_gemm": (ctypes.c_int, [_P, _P]),
    "rqf_layer0_grads_workspace": (_SZ, [_I64, _I64, _I64]),
    "rqf_layer0_grads": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_version": (ctypes.c_char_p, []),
    "rqf_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "rqf_btf_scan_workspace": (_SZ, [_I64, _I64, _I64]),
    "rqf_chunked_scan_fwd": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_chunked_scan_bwd": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_chunked_prospective_fwd": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_chunked_prospective_bwd": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_multi_osc_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32]),
    "rqf_multi_osc_fwd": (
        ctypes.c_int, [_P, _P, _P, _P, _I32, _P, _I32, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_multi_osc_bwd": (
        ctypes.c_int,
        [_P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_fbt_carry_chunks": (_I64, [_I64]),
    "rqf_fbt_workspace": (_SZ, [_I64, _I64, _I64]),
    "rqf_fbt_prospective_fwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rqf_fbt_prospective_bwd": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_fbt_recompute_fwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rqf_fbt_recompute_skip_fwd": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rqf_fbt_recompute_bwd": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_fbt_layer0_fwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rqf_fbt_layer0_bwd": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "rqf_fbt_recompute_bwd_noalloc": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rqf_selective_fwd": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P]),
    "rqf_selective_skip_fwd": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P, _P]),
    "rqf_selective_bwd_workspace": (_SZ, [_P, _I64]),
    "rqf_selective_bwd": (
        ctypes.c_int,
        [_P, _P, _P, _I64, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "rqf_selftest_wave_scan": (ctypes.c_int, [_P, _P, _P, _P]),
}


class RQFError(RuntimeError):
    pass


# Return code of a no-allocation entry point whose static scratch is too
# small for the problem (RQF_ERR_SCRATCH), and that scratch's size
# (RQF_NOALLOC_SCRATCH_BYTES), as include/rqf_scan.h defines them.
ERR_SCRATCH = -4
NOALLOC_SCRATCH_BYTES = 4 << 20


def lib_path() -> str:
    return os.environ.get("RQF_HIP_LIB", LIB_PATH)


def load():
    """Load the library (idempotent).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RQFError(
            f"{path} is missing: build it with `python -m prospective_rqf_amd.build` "
            "(the HIP kernels have no CPU fallback)"
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def available() -> bool:
    """True when the library loads and a HIP device is visible."""
    try:
        load()
    except (OSError, RQFError):
        return False
    return torch.cuda.is_available()


def check(code: int, what: str) -> None:
    if code != 0:
        msg = load().rqf_error_string(code).decode()
        raise RQFError(f"{what} failed: {msg} (code {code})")


def ptr(t: torch.Tensor | None):
    """Device pointer of a tensor as an int (None -> NULL); the bound
    functions declare ``c_void_p`` arguments, which take either."""
    if t is None:
        return None
    return t.data_ptr()


def stream_of(t: torch.Tensor):
    """Handle of torch's current stream on the tensor's device (the launch
    stream), read without building a ``torch.cuda.Stream`` object: this is on
    every call's path, and small calls are bound by their host time."""
    return _raw_stream(t.get_device())


_raw_stream = torch._C._cuda_getCurrentRawStream


def require_device(*tensors: torch.Tensor | None) -> None:
    """Every kernel input must live on one HIP device, the current one (the
    library launches there, on torch's current stream of the inputs' device);
    raise otherwise, before any pointer reaches a kernel."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RQFError(
                "prospective_rqf_amd kernels run on HIP devices only; got a tensor on "
                f"{t.device}"
            )
        d = t.get_device()
        if dev is None:
            dev = d
        elif d != dev:
            raise RQFError(f"kernel inputs on different devices: cuda:{dev} and cuda:{d}")
    if dev is not None and dev != _current_device():
        raise RQFError(
            f"kernel inputs on cuda:{dev} while cuda:{_current_device()} is current; "
            f"call under torch.cuda.device({dev})"
        )


_current_device = torch._C._cuda_getDevice


def workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)

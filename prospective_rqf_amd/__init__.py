"""MI355X-native complex linear-recurrence scans for prospective RQF models.

Drop-in replacements for the Triton scan backends of rqf_models/ops:

* :mod:`.chunked_scan_kernel` -- time-invariant scans on (batch, time, filters)
* :mod:`.fbt_scan_kernel`     -- two-tap prospective scans on (filters, batch, time)
* :mod:`.selective_scan_kernel` / :mod:`.selective_scan` -- fused selective scan
* :mod:`.scan`                -- dispatch surface and backend flags

All compute runs in ``librqf_hip.so`` (hand-written gfx950 HIP, C ABI in
``include/rqf_scan.h``); build it with ``python -m prospective_rqf_amd.build``.
"""

from prospective_rqf_amd._lib import available
from prospective_rqf_amd.chunked_scan_kernel import (
    _triton_chunked_scan,
    _triton_chunked_scan_prospective,
)
from prospective_rqf_amd.fbt_scan_kernel import fbt_prospective_scan, fbt_recompute_scan
from prospective_rqf_amd.selective_scan import SelectiveScanInputs, selective_layer_scan
from prospective_rqf_amd.selective_scan_kernel import selective_backward, selective_forward

__all__ = [
    "available",
    "_triton_chunked_scan",
    "_triton_chunked_scan_prospective",
    "fbt_prospective_scan",
    "fbt_recompute_scan",
    "SelectiveScanInputs",
    "selective_layer_scan",
    "selective_forward",
    "selective_backward",
]

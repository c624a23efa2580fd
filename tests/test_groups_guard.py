"""Host-side validation of the warp-group indices (no device needed).

The kernels read ``warp_logits[groups[f]]``; the reference's controller builds
``groups = rank * G // F`` (rqf_models/backbones/rqf/selective.py:164-165), so
every entry lies in [0, G).  The host layer must reject anything else before a
launch, for every tensor it is given: the validation is cached per tensor
object and version, never per address.
"""

import gc

import numpy as np
import pytest
import torch

from prospective_rqf_amd import selective_scan_kernel as ssk
from tests.selective_cases import CASES, make_inputs, to_torch

GROUPED = next(c for c in CASES if c["warp"] == "grouped" and c["gamma"] and c["write"])


def _inputs(groups):
    rng = np.random.default_rng(0)
    inp = to_torch(make_inputs(6, 2, 9, GROUPED, rng, G=3))
    return inp._replace(groups=groups)


def _z():
    return torch.zeros(6, 2, 9, dtype=torch.complex64)


def test_valid_groups_pass_and_order_is_group_sorted():
    g = torch.tensor([2, 0, 1, 0, 2, 1])
    s, keep = ssk.inputs_struct(_z(), _inputs(g))
    assert s.G == 3
    order = keep[4]
    assert order.tolist() == [1, 3, 2, 5, 0, 4]


@pytest.mark.parametrize("bad", [[0, 1, 2, 3, 0, 1], [0, -1, 2, 1, 0, 1], [9, 9, 9, 9, 9, 9]])
def test_out_of_range_groups_rejected(bad):
    with pytest.raises(ValueError, match="warp-logit rows"):
        ssk.inputs_struct(_z(), _inputs(torch.tensor(bad)))


def test_second_tensor_after_a_valid_one_is_checked():
    """A valid tensor is checked and cached; a different tensor with an
    out-of-range entry (here allocated after the first is freed, so it may
    reuse its id and storage) is still rejected."""
    good = torch.tensor([0, 1, 2, 0, 1, 2])
    ssk.inputs_struct(_z(), _inputs(good))
    del good
    gc.collect()
    for _ in range(8):
        bad = torch.tensor([0, 1, 2, 0, 1, 3])
        with pytest.raises(ValueError):
            ssk.inputs_struct(_z(), _inputs(bad))
        del bad


def test_in_place_edit_invalidates_cache():
    g = torch.tensor([0, 1, 2, 0, 1, 2])
    ssk.inputs_struct(_z(), _inputs(g))
    ssk.inputs_struct(_z(), _inputs(g))  # cached
    g[3] = 7
    with pytest.raises(ValueError):
        ssk.inputs_struct(_z(), _inputs(g))
    g[3] = 0
    ssk.inputs_struct(_z(), _inputs(g))
    # an edit through a view shares the version counter
    v = g[2:]
    v[0] = -3
    with pytest.raises(ValueError):
        ssk.inputs_struct(_z(), _inputs(g))


def test_non_int64_and_reused_storage_tensors_are_checked():
    """int32 groups are converted per call; the conversion's temporary never
    lets a later invalid tensor through."""
    ok32 = torch.tensor([0, 1, 2, 0, 1, 2], dtype=torch.int32)
    for _ in range(3):
        ssk.inputs_struct(_z(), _inputs(ok32))
    storage = torch.tensor([0, 1, 2, 0, 1, 2])
    ssk.inputs_struct(_z(), _inputs(storage))
    alias = torch.empty(0, dtype=torch.int64).set_(storage.untyped_storage(), 0, (6,))
    alias[5] = 4  # the same memory, another tensor object
    with pytest.raises(ValueError):
        ssk.inputs_struct(_z(), _inputs(alias))
    # `storage` itself saw no in-place op of its own (its version counter is
    # unchanged), so its cached validation stands; the device code clamps
    # every group index into [0, G), so even such an entry stays in bounds.


def test_shape_and_dtype_errors():
    with pytest.raises(ValueError, match=r"\(F,\)"):
        ssk.inputs_struct(_z(), _inputs(torch.tensor([0, 1, 2])))
    with pytest.raises(ValueError, match=r"\(F,\)"):
        ssk.inputs_struct(_z(), _inputs(None))
    with pytest.raises(ValueError, match="integer"):
        ssk.inputs_struct(_z(), _inputs(torch.zeros(6)))

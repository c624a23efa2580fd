"""Lane-layout check of the DPP / ds_bpermute wave scans on the device."""

import numpy as np
import pytest
import torch

from prospective_rqf_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def test_wave_scan_forward_and_reverse():
    rng = np.random.default_rng(0)
    P = rng.uniform(0.7, 1.1, 64) * np.exp(1j * rng.uniform(-1, 1, 64))
    s = rng.standard_normal(64) + 1j * rng.standard_normal(64)
    packed = np.stack([P.real, P.imag, s.real, s.imag], axis=1).astype(np.float32)
    dev_in = torch.as_tensor(packed, device="cuda").contiguous()
    out_f = torch.empty_like(dev_in)
    out_r = torch.empty_like(dev_in)
    print("case: wave_scan selftest", flush=True)
    _lib.check(_lib.load().rqf_selftest_wave_scan(_lib.ptr(dev_in), _lib.ptr(out_f),
                                                  _lib.ptr(out_r), _lib.stream_of(dev_in)),
               "rqf_selftest_wave_scan")
    torch.cuda.synchronize()
    of = out_f.cpu().numpy().astype(np.float64)
    orv = out_r.cpu().numpy().astype(np.float64)
    Pf = of[:, 0] + 1j * of[:, 1]
    sf = of[:, 2] + 1j * of[:, 3]
    Pr = orv[:, 0] + 1j * orv[:, 1]
    sr = orv[:, 2] + 1j * orv[:, 3]
    # prefix: x -> P x + s composed lanes 0..i (lane 0 first)
    accP, accs = 1.0 + 0j, 0j
    for i in range(64):
        accs = accs * P[i] + s[i]
        accP = accP * P[i]
        assert abs(Pf[i] - accP) <= 1e-5 * abs(accP), i
        assert abs(sf[i] - accs) <= 1e-5 * (1 + abs(accs)), i
    # suffix: d -> Q d + r composed lanes i..63 (lane 63 applied first)
    accQ, accr = 1.0 + 0j, 0j
    for i in range(63, -1, -1):
        accr = P[i] * accr + s[i]
        accQ = P[i] * accQ
        assert abs(Pr[i] - accQ) <= 1e-5 * abs(accQ), i
        assert abs(sr[i] - accr) <= 1e-5 * (1 + abs(accr)), i

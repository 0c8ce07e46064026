"""Per-call scratch comes from the library's own memory pool.

The chunked Mamba-3 scan allocates its gate records and the four-direction 2D scan
its column-major copies and planes on the caller's stream. Both come from a pool the
library creates per device; the device's default pool, which torch or the caller may
use, keeps its release threshold across such calls.
"""

import ctypes

import numpy as np
import pytest

from armhackathon_amd import workloads
from util import case, dev, host, rel_err

pytestmark = pytest.mark.gpu

RELEASE_THRESHOLD = 0x4  # hipMemPoolAttrReleaseThreshold
SISO_KEYS = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias")


def _threshold(hip, device):
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), device) == 0
    value = ctypes.c_uint64()
    assert hip.hipMemPoolGetAttribute(pool, RELEASE_THRESHOLD, ctypes.byref(value)) == 0
    return value.value


def test_default_pool_keeps_its_release_threshold():
    import torch

    import armhackathon_amd as arm_scan
    import oracle

    case("default pool release threshold across scratch-allocating calls")
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch and the library share
    device = torch.cuda.current_device()
    before = _threshold(hip, device)
    x = workloads.m3_siso(batch=1, length=80, heads=2, dv=16, dqk=32, seed=21)
    t = dev(x)
    for _ in range(3):
        out = arm_scan.mamba3_scan(*[t[k] for k in SISO_KEYS], cos=t["cos"], sin=t["sin"])
    ref = oracle.mamba3_scan(*[x[k] for k in SISO_KEYS], x["cos"], x["sin"], dtype=np.float64)
    assert rel_err(host(out), ref.transpose(0, 2, 1, 3)) < 1e-4
    g = workloads.ss2d(batch=1, dim=16, height=8, width=12, state=8, seed=22)
    tg = dev(g)
    for _ in range(3):
        arm_scan.ss2d_scan(tg["u"], tg["delta"], tg["A"], tg["B4"], tg["C4"], D=tg["D"],
                           z=tg["z"], merge="sum", per_direction=True)
    torch.cuda.synchronize()
    assert _threshold(hip, device) == before

"""Four-direction 2D cross-scan on the GPU.

Pinned by the reference's 2D goldens (tests/golden/2d, per-direction planes,
gate 1e-4: verify_golden_2d.py:36) and, for the per-direction B/C + z
extension the benchmark configuration needs, by composing four oracle scans
over the row-/column-major orderings (oracle.ss2d).
"""

import json

import numpy as np
import pytest

import oracle
from armhackathon_amd import workloads
from util import case, dev, host, rel_err

pytestmark = pytest.mark.gpu

PLANES = ("out_row_fwd", "out_row_bwd", "out_col_fwd", "out_col_bwd")


def test_ss2d_goldens(golden_dir):
    import armhackathon_amd as arm_scan

    files = sorted((golden_dir / "2d").glob("*.npz"))
    assert len(files) == 6
    for f in files:
        case(f"ss2d golden {f.name}")
        z = {k: np.asarray(v, np.float32) for k, v in np.load(f).items()}
        t = dev(z)
        planes = arm_scan.ss2d_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"],
                                    delta_bias=t["delta_bias"], delta_softplus=True,
                                    merge="none")
        for got, name in zip(planes, PLANES):
            assert np.abs(host(got) - z[name]).max() < 1e-4, (f.name, name)
        # the reference's view-based composition over the bidirectional seam
        planes2 = arm_scan.ss2d_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"],
                                     delta_bias=t["delta_bias"], delta_softplus=True,
                                     merge="none", scan_pair=arm_scan.ss2d.scan_pair_arm)
        for got, name in zip(planes2, PLANES):
            assert np.abs(host(got) - z[name]).max() < 1e-4, (f.name, name, "views")
        s = arm_scan.ss2d_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"],
                               delta_bias=t["delta_bias"], delta_softplus=True, merge="sum")
        assert np.abs(host(s) - sum(z[p] for p in PLANES)).max() < 4e-4, f.name


@pytest.mark.parametrize("shape", [(2, 16, 12, 20, 16), (1, 8, 7, 5, 13), (3, 32, 64, 64, 16),
                                   (1, 16, 1, 33, 8), (2, 16, 32, 16, 16), (1, 32, 16, 48, 5)],
                         ids=lambda s: "x".join(map(str, s)))
def test_ss2d_per_direction_vs_oracle(shape):
    import armhackathon_amd as arm_scan

    b, d, h, w, n = shape
    case(f"ss2d per-direction {shape}")
    x = workloads.ss2d(batch=b, dim=d, height=h, width=w, state=n, seed=h * w)
    rng = np.random.default_rng(1)
    bias = rng.uniform(-1, 1, d).astype(np.float32)
    t = dev(x)
    tb = dev(bias)
    for merge in ("none", "sum", "mean"):
        out, last = arm_scan.ss2d_scan(t["u"], t["delta"], t["A"], t["B4"], t["C4"], D=t["D"],
                                       z=t["z"], delta_bias=tb, delta_softplus=True,
                                       merge=merge, per_direction=True,
                                       return_last_state=True)
        ref, rlast = oracle.ss2d(x["u"], x["delta"], x["A"], x["B4"], x["C4"], D=x["D"],
                                 z=x["z"], delta_bias=bias, delta_softplus=True,
                                 dtype=np.float64, want_state=True)
        if merge == "none":
            for k in range(4):
                assert rel_err(host(out[k]), ref[k]) < 1e-4, (merge, k)
        else:
            want = ref.sum(0) * (0.25 if merge == "mean" else 1.0)
            assert rel_err(host(out), want) < 1e-4, merge
        assert rel_err(host(last), rlast) < 1e-4, merge


@pytest.mark.parametrize("shape", [(2, 16, 7, 7, 16), (1, 32, 45, 45, 16)],
                         ids=lambda s: "x".join(map(str, s)))
def test_ss2d_unaligned_rows(shape):
    """Grids whose rows are not 16-byte multiples (7x7, 45x45) and inputs placed one
    float past an aligned base: the one-launch route with single-float moves."""
    import torch
    import armhackathon_amd as arm_scan

    b, d, h, w, n = shape
    case(f"ss2d unaligned rows {shape}")
    x = workloads.ss2d(batch=b, dim=d, height=h, width=w, state=n, seed=h * w + 1)

    def shifted(a):  # the same values one float past a 256-byte aligned allocation
        t = torch.empty(a.size + 1, dtype=torch.float32, device="cuda")
        t[1:] = torch.from_numpy(np.ascontiguousarray(a)).reshape(-1).cuda()
        return t[1:].view(a.shape)

    t = {k: shifted(v) if k in ("u", "delta", "B4", "C4", "z") else dev(v) for k, v in x.items()}
    out, last = arm_scan.ss2d_scan(t["u"], t["delta"], t["A"], t["B4"], t["C4"], D=t["D"],
                                   z=t["z"], delta_softplus=False, merge="sum",
                                   per_direction=True, return_last_state=True)
    ref, rlast = oracle.ss2d(x["u"], x["delta"], x["A"], x["B4"], x["C4"], D=x["D"], z=x["z"],
                             dtype=np.float64, want_state=True)
    assert rel_err(host(out), ref.sum(0)) < 1e-4
    assert rel_err(host(last), rlast) < 1e-4


def test_ss2d_benchmark_shape():
    """64x64 grid, batch 16, d_inner 192, d_state 16,
    per-direction B/C, D skip and z gate, summed onto the grid."""
    import armhackathon_amd as arm_scan

    case("ss2d config 5")
    x = workloads.ss2d(batch=16, dim=192, height=64, width=64, state=16, seed=5)
    t = dev(x)
    out, last = arm_scan.ss2d_scan(t["u"], t["delta"], t["A"], t["B4"], t["C4"], D=t["D"],
                                   z=t["z"], delta_softplus=False, merge="sum",
                                   per_direction=True, return_last_state=True)
    ref, rlast = oracle.ss2d(x["u"], x["delta"], x["A"], x["B4"], x["C4"], D=x["D"], z=x["z"],
                             dtype=np.float64, want_state=True)
    assert rel_err(host(out), ref.sum(0)) < 1e-4
    assert rel_err(host(last), rlast) < 1e-4


@pytest.mark.parametrize("merge", ["sum", "mean", "none"])
def test_ss2d_out_off_aligned_base(merge):
    """An 8x8 grid (rows of 16-byte multiples, so the merge may move float4 pieces) with
    the caller's out one float past an aligned base: the merge checks out's alignment,
    not only the grid's, and moves single floats there. Through the C ABI, against the
    oracle, and equal to the same call into an aligned out."""
    import torch

    from armhackathon_amd import _ffi

    b, d, h, w, n = 2, 16, 8, 8, 16
    case(f"ss2d 8x8, out one float off an aligned base, merge={merge}")
    x = workloads.ss2d(batch=b, dim=d, height=h, width=w, state=n, seed=88)
    t = dev(x)
    planes = 4 if merge == "none" else 1
    size = planes * b * d * h * w
    buf = torch.full((size + 1,), float("nan"), device="cuda")
    aligned = torch.full((size,), float("nan"), device="cuda")
    dims = _ffi.ArmSS2DDims(b, d, h, w, n)
    st = torch.cuda.current_stream().cuda_stream
    for out in (buf[1:], aligned):
        _ffi.ss2d_raw(dims, t["u"].data_ptr(), t["delta"].data_ptr(), t["A"].data_ptr(),
                      t["B4"].data_ptr(), t["C4"].data_ptr(), t["D"].data_ptr(),
                      t["z"].data_ptr(), 0, False, merge, out.data_ptr(), stream=st)
    torch.cuda.synchronize()
    assert np.isnan(host(buf[:1])).all()  # nothing written before out
    ref = oracle.ss2d(x["u"], x["delta"], x["A"], x["B4"], x["C4"], D=x["D"], z=x["z"],
                      dtype=np.float64)
    want = ref if merge == "none" else ref.sum(0) * (0.25 if merge == "mean" else 1.0)
    got = host(buf[1:]).reshape(want.shape)
    assert rel_err(got, want) < 1e-4
    assert np.array_equal(got, host(aligned).reshape(want.shape))

"""Size-independent properties at the benchmark shapes.

For fixed gates every scan here is linear in its input sequence: Mamba-1 in u
(h_t = e^{dt A} h_{t-1} + dt u_t B_t, y = C h + D u, the z gate a per-step factor),
Mamba-3 in v (the state and the output are sums of decayed v k^T terms, gated per
step), and the 2D cross-scan in u. So y(a u1 + b u2) = a y(u1) + b y(u2), outputs and
final states, to fp32 rounding. The parity tests pin these kernels against the oracle
at the same shapes; these check the kernels' structure over every chunk, segment and
traversal of the full-size launches, the tail chunks included.
"""

import numpy as np
import pytest

from armhackathon_amd import workloads
from util import case, dev, host

pytestmark = pytest.mark.gpu

TOL = 2e-5  # tensor-scale relative error of the combination, fp32 rounding only
ALPHA, BETA = 0.75, -1.5


def _lin_err(f, x1, x2):
    """max |f(a x1 + b x2) - (a f(x1) + b f(x2))| / max |a f(x1) + b f(x2)|, per output."""
    y1, y2, y12 = f(x1), f(x2), f(ALPHA * x1 + BETA * x2)
    errs = []
    for a, b, c in zip(y1, y2, y12):
        want = ALPHA * host(a).astype(np.float64) + BETA * host(b).astype(np.float64)
        errs.append(float(np.abs(host(c) - want).max() / np.abs(want).max()))
    return errs


@pytest.mark.parametrize("length", [2048, 2048 + 77])
def test_m1_linear_in_u(length):
    import armhackathon_amd as arm_scan

    case(f"m1 linearity in u, B8 D1536 L{length} (bias, softplus, D, z, final state)")
    x = dev(workloads.m1_layer(batch=8, dim=1536, length=length, seed=31))
    u2 = dev(np.random.default_rng(32).standard_normal((8, 1536, length), dtype=np.float32))

    def f(u):
        return arm_scan.selective_scan(u, x["delta"], x["A"], x["B"], x["C"], D=x["D"],
                                       z=x["z"], delta_bias=x["delta_bias"],
                                       delta_softplus=True, return_last_state=True)

    errs = _lin_err(f, x["u"], u2)
    assert max(errs) < TOL, errs


def test_m1_linear_in_u_few_rows():
    """Config 1's shape, which takes the segmented scan (fold, then replay)."""
    import armhackathon_amd as arm_scan

    case("m1 linearity in u, B1 D1536 L2048 (segmented)")
    x = dev(workloads.m1_op(batch=1, dim=1536, length=2048, state=16, seed=33))
    u2 = dev(np.random.default_rng(34).standard_normal((1, 1536, 2048), dtype=np.float32))

    def f(u):
        return arm_scan.selective_scan(u, x["delta"], x["A"], x["B"], x["C"], D=x["D"],
                                       z=x["z"], return_last_state=True)

    errs = _lin_err(f, x["u"], u2)
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("mimo", [False, True], ids=["siso", "mimo"])
def test_m3_linear_in_v(mimo):
    import armhackathon_amd as arm_scan

    case(f"m3 linearity in v, config {'4' if mimo else '3'} shape")
    x = workloads.m3_mimo(seed=35) if mimo else workloads.m3_siso(seed=35)
    t = dev(x)
    v2 = dev(np.random.default_rng(36).standard_normal(x["v"].shape, dtype=np.float32))
    keys = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias")

    def f(v):
        args = [v if k == "v" else t[k] for k in keys]
        if mimo:
            out = arm_scan.mamba3_mimo_scan(*args, t["psi"], t["zeta"], t["phi"],
                                            cos=t["cos"], sin=t["sin"], return_last_state=True)
        else:
            out = arm_scan.mamba3_scan(*args, cos=t["cos"], sin=t["sin"],
                                       return_last_state=True)
        return out[:2]  # output and final state (last_bx, scale k, does not involve v)

    errs = _lin_err(f, t["v"], v2)
    assert max(errs) < TOL, errs


def test_ss2d_linear_in_u():
    import armhackathon_amd as arm_scan

    case("ss2d linearity in u, config 5 shape (merge sum, final states)")
    x = dev(workloads.ss2d(batch=16, dim=192, height=64, width=64, state=16, seed=37))
    u2 = dev(np.random.default_rng(38).standard_normal((16, 192, 64, 64), dtype=np.float32))

    def f(u):
        return arm_scan.ss2d_scan(u, x["delta"], x["A"], x["B4"], x["C4"], D=x["D"], z=x["z"],
                                  merge="sum", per_direction=True, return_last_state=True,
                                  delta_softplus=False)

    errs = _lin_err(f, x["u"], u2)
    assert max(errs) < TOL, errs

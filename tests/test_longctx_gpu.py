"""Long-context Mamba-1 through the C ABI against the float64 oracle.

The reference streams the Mamba-1 scan at B1 D768 N16 up to L 131072
(bench/bench_longctx.py:30-33, README.md:336-337). Those shapes have 768 rows, far
too few to fill the chip, so the kernels run the few-rows plan: each row cut into up
to 16 segments of whole 256-step chunks, a fold pass for the segments' affine maps,
then every segment replayed from its entry state. Both entry points that take that
plan are checked, the allocating one (maps in stream-ordered scratch) and the
allocation-free one (maps in the library's static scratch), forward and reverse,
seeded from h0 and writing the final state, at L 32768 and 131072: the tensor-scale
relative error of outputs and final states stays within 1e-4.
"""

import ctypes

import numpy as np
import pytest

import oracle
from armhackathon_amd import _ffi, workloads
from util import case, dev, host, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4
LENGTHS = [32768, 131072]
_inputs = {}


def _x(length):
    if length not in _inputs:
        _inputs.clear()  # one length at a time: 131072 steps x 768 rows are 400 MB a tensor
        x = workloads.m1_layer(batch=1, dim=768, length=length, state=16, seed=length % 997)
        x["h0"] = np.random.default_rng(length).standard_normal((1, 768, 16)).astype(np.float32)
        _inputs[length] = x
    return _inputs[length]


def _call(fn_name, t, shape, reverse):
    import torch

    b, d, L, n = shape
    out = torch.full((b, d, L), float("nan"), device="cuda")
    last = torch.full((b, d, n), float("nan"), device="cuda")
    rc = getattr(_ffi.load(), fn_name)(
        ctypes.byref(_ffi.ArmScanDims(b, d, L, n, 1)), t["u"].data_ptr(),
        t["delta"].data_ptr(), t["A"].data_ptr(), t["B"].data_ptr(), t["C"].data_ptr(),
        t["D"].data_ptr(), t["z"].data_ptr(), t["delta_bias"].data_ptr(), 1, int(reverse), 0,
        0, out.data_ptr(), last.data_ptr(), t["h0"].data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _ffi.load().arm_scan_last_error()
    torch.cuda.synchronize()
    return host(out), host(last)


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("length", LENGTHS)
def test_m1_long_context(length, reverse):
    import torch

    x = _x(length)
    ref, ref_last = oracle.selective_scan(
        x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
        delta_bias=x["delta_bias"], delta_softplus=True, reverse=reverse, h0=x["h0"],
        dtype=np.float64)
    t = dev(x)
    shape = (1, 768, length, 16)
    outs = {}
    for fn in ("arm_scan_selective_scan_f32", "arm_scan_selective_scan_noalloc_f32"):
        case(f"long context B1 D768 L{length} N16 reverse={reverse} via {fn}")
        out, last = _call(fn, t, shape, reverse)
        assert rel_err(out, ref) < TOL, fn
        assert rel_err(last, ref_last) < TOL, fn
        outs[fn] = (out, last)
    del t
    torch.cuda.empty_cache()
    # the two entries plan the same segments here (the maps, 1.5 MB, fit the scratch),
    # so they run the same kernels on the same inputs
    a, b = outs.values()
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])

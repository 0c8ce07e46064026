"""arm_scan_selective_scan_noalloc_f32 (the allocation-free variant of
arm_scan_selective_scan_f32) through the C ABI, against the allocating entry point.

Two calls in a row share the library's static scratch, the second on a smaller
input: config 1's shape (its plan cuts 1536 rows into 8 segments whose maps live in
the scratch), then B1 D256 L1024 (4 segments). Same plan, same kernels: the outputs
and final states must be bit-identical. A third call whose maps would not fit
(N 64 at L 4096) takes a plan cut to fewer segments, so only the tolerance of the
float64 oracle applies there, and the allocating call is checked the same way.
"""

import ctypes

import numpy as np
import pytest

import oracle
from armhackathon_amd import _ffi, workloads
from util import case, dev, host, rel_err

pytestmark = pytest.mark.gpu


def _call(fn_name, x, softplus=False, reverse=False):
    import torch

    b, d, L = x["u"].shape
    n = x["A"].shape[1]
    t = dev(x)
    out = torch.full((b, d, L), float("nan"), device="cuda")
    last = torch.full((b, d, n), float("nan"), device="cuda")
    p = lambda k: None if t.get(k) is None else t[k].data_ptr()  # noqa: E731
    rc = getattr(_ffi.load(), fn_name)(
        ctypes.byref(_ffi.ArmScanDims(b, d, L, n, 1)), p("u"), p("delta"), p("A"), p("B"),
        p("C"), p("D"), p("z"), p("delta_bias"), int(softplus), int(reverse), 0, 0,
        out.data_ptr(), last.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _ffi.load().arm_scan_last_error()
    torch.cuda.synchronize()
    return host(out), host(last)


@pytest.mark.parametrize("reverse", [False, True])
def test_noalloc_matches_allocating_entry(reverse):
    for (b, d, L, n, seed) in ((1, 1536, 2048, 16, 40), (1, 256, 1024, 16, 41)):
        case(f"noalloc vs selective_scan_f32 {b}x{d}x{L} N{n} reverse={reverse}")
        x = workloads.m1_layer(batch=b, dim=d, length=L, state=n, seed=seed)
        got, got_last = _call("arm_scan_selective_scan_noalloc_f32", x, True, reverse)
        ref, ref_last = _call("arm_scan_selective_scan_f32", x, True, reverse)
        assert np.array_equal(got, ref) and np.array_equal(got_last, ref_last)


def test_noalloc_plan_cut_to_the_scratch():
    case("noalloc B1 D1536 L4096 N64 (maps above the scratch: fewer segments)")
    x = workloads.m1_op(batch=1, dim=1536, length=4096, state=64, seed=42)
    got, got_last = _call("arm_scan_selective_scan_noalloc_f32", x)
    ref, ref_last = _call("arm_scan_selective_scan_f32", x)
    o64, l64 = oracle.selective_scan(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"],
                                     z=x["z"], dtype=np.float64)
    for out, last in ((got, got_last), (ref, ref_last)):
        assert rel_err(out, o64) < 1e-4 and rel_err(last, l64) < 1e-4
    assert rel_err(got, ref) < 1e-4


@pytest.mark.parametrize("reverse", [False, True])
def test_noalloc_unaligned_rows(reverse):
    """Rows that are not 16-byte multiples (L % 4 != 0): the allocating entry copies B
    and C to a padded pitch and fills the tiles by 16-byte DMA, the allocation-free one
    moves them as single floats into the same tiles; the results are bit-identical."""
    for (b, d, L, n, seed) in ((1, 1536, 2050, 16, 43), (2, 256, 1030, 13, 44)):
        case(f"noalloc unaligned {b}x{d}x{L} N{n} reverse={reverse}")
        x = workloads.m1_layer(batch=b, dim=d, length=L, state=n, seed=seed)
        got, got_last = _call("arm_scan_selective_scan_noalloc_f32", x, True, reverse)
        ref, ref_last = _call("arm_scan_selective_scan_f32", x, True, reverse)
        assert np.array_equal(got, ref) and np.array_equal(got_last, ref_last)


def _hip():
    """The HIP runtime already in the process (torch's and the library's, one soname)."""
    import torch  # noqa: F401  (loads the runtime)

    hip = ctypes.CDLL("libamdhip64.so.7")
    vp = ctypes.c_void_p
    hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    hip.hipGraphGetNodes.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_size_t)]
    hip.hipGraphNodeGetType.argtypes = [vp, ctypes.POINTER(ctypes.c_int)]
    hip.hipGraphDestroy.argtypes = [vp]
    return hip


KERNEL, MEMSET, MEM_ALLOC, MEM_FREE = 0, 2, 10, 11  # hipGraphNodeType


def _captured_node_types(fn_name, x, reverse):
    """Record one call into a HIP graph on a capturing stream (nothing runs: the graph is
    inspected and destroyed, never launched) and return the types of its nodes."""
    import torch

    hip = _hip()
    b, d, L = x["u"].shape
    n = x["A"].shape[1]
    t = dev(x)
    out = torch.empty((b, d, L), device="cuda")
    last = torch.empty((b, d, n), device="cuda")
    p = lambda k: None if t.get(k) is None else t[k].data_ptr()  # noqa: E731
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(s.cuda_stream, 2) == 0  # hipStreamCaptureModeRelaxed
    rc = getattr(_ffi.load(), fn_name)(
        ctypes.byref(_ffi.ArmScanDims(b, d, L, n, 1)), p("u"), p("delta"), p("A"), p("B"),
        p("C"), p("D"), p("z"), p("delta_bias"), 1, int(reverse), 0, 0, out.data_ptr(),
        last.data_ptr(), None, s.cuda_stream)
    end = hip.hipStreamEndCapture(s.cuda_stream, ctypes.byref(graph))
    if rc != 0 or end != 0:
        return None  # the capture refused a call (the control below allows that)
    count = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(graph, None, ctypes.byref(count)) == 0
    nodes = (ctypes.c_void_p * max(count.value, 1))()
    assert hip.hipGraphGetNodes(graph, nodes, ctypes.byref(count)) == 0
    types = []
    for i in range(count.value):
        ty = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(nodes[i], ctypes.byref(ty)) == 0
        types.append(ty.value)
    assert hip.hipGraphDestroy(graph) == 0
    return types


@pytest.mark.parametrize("shape", [(1, 1536, 2048, 16), (1, 1536, 2050, 16), (8, 64, 300, 16)],
                         ids=["segmented", "unaligned", "whole_rows"])
def test_noalloc_records_no_allocation(shape):
    """The defining property: a call of the allocation-free entry, recorded into a HIP
    graph by stream capture, holds kernel nodes only (no allocation, free or memset
    node), on the few-rows plan (segment maps in the static scratch), on rows that are
    not 16-byte multiples (B/C read in place, where the allocating entry makes a padded
    copy) and on whole rows. The allocating entry on the segmented shape records an
    allocation and a free (or the capture refuses it), so the check tells them apart."""
    b, d, L, n = shape
    x = workloads.m1_layer(batch=b, dim=d, length=L, state=n, seed=45)
    _call("arm_scan_selective_scan_noalloc_f32", x, True)  # set-up (scratch lookup) first
    for reverse in (False, True):
        case(f"noalloc capture {shape} reverse={reverse}")
        types = _captured_node_types("arm_scan_selective_scan_noalloc_f32", x, reverse)
        assert types and all(t == KERNEL for t in types), types
    if shape[2] == 2048 and shape[0] == 1:
        # the allocating entry either records its stream-ordered allocation and free, or
        # the capture refuses the pool allocation: either way it is not allocation-free
        case("allocating entry capture (control)")
        types = _captured_node_types("arm_scan_selective_scan_f32", x, False)
        assert types is None or (MEM_ALLOC in types and MEM_FREE in types), types


def test_noalloc_calls_on_two_streams():
    """Calls on two streams share the device's scratch: the library makes each call's
    stream wait for the previous call's kernels when it was made on the other stream,
    so the two run one after the other. Long rows on the few-rows plan (maps in the
    scratch), alternating streams with nothing synchronised in between: every output
    equals the allocating entry's, bit for bit."""
    import torch

    shape = (1, 768, 32768, 16)
    b, d, L, n = shape
    xs = [workloads.m1_layer(batch=b, dim=d, length=L, state=n, seed=60 + i) for i in range(2)]
    refs = [_call("arm_scan_selective_scan_f32", x, True) for x in xs]
    ts = [dev(x) for x in xs]
    outs = [[torch.empty((b, d, L), device="cuda") for _ in range(3)] for _ in range(2)]
    lasts = [[torch.empty((b, d, n), device="cuda") for _ in range(3)] for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    lib = _ffi.load()
    for rnd in range(3):
        for i in range(2):
            case(f"noalloc two streams: round {rnd} input {i} on stream {i}")
            t = ts[i]
            p = lambda k: None if t.get(k) is None else t[k].data_ptr()  # noqa: E731
            rc = lib.arm_scan_selective_scan_noalloc_f32(
                ctypes.byref(_ffi.ArmScanDims(b, d, L, n, 1)), p("u"), p("delta"), p("A"),
                p("B"), p("C"), p("D"), p("z"), p("delta_bias"), 1, 0, 0, 0,
                outs[i][rnd].data_ptr(), lasts[i][rnd].data_ptr(), None,
                streams[i].cuda_stream)
            assert rc == 0, lib.arm_scan_last_error()
    torch.cuda.synchronize()
    for i in range(2):
        for rnd in range(3):
            assert np.array_equal(host(outs[i][rnd]), refs[i][0]), (i, rnd)
            assert np.array_equal(host(lasts[i][rnd]), refs[i][1]), (i, rnd)

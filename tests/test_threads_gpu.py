"""Host threads calling the library at once, each on a stream of its own (default
priority): the reference's call is reentrant across threads (arm-scan-ffi/src/lib.rs;
ctypes releases the GIL). Every thread's results must equal, bit for bit, what one
thread computes alone: the kernels share no state, and the stream-ordered scratch each
call takes (segment maps, gate records, SS2D planes) comes from the library's pool."""

import threading

import pytest

from util import case

pytestmark = pytest.mark.gpu


def test_concurrent_calls_on_separate_streams():
    import torch
    import torch.nn.functional as F

    import armhackathon_amd as arm_scan
    from armhackathon_amd import workloads

    case("4 host threads, 4 streams")
    m1 = {k: torch.from_numpy(v).cuda() for k, v in
          workloads.m1_op(batch=2, dim=64, length=1000, state=16, seed=3).items()
          if v is not None}
    m3 = {k: torch.from_numpy(v).cuda() for k, v in
          workloads.m3_siso(batch=1, length=300, heads=4, dv=32, dqk=64, seed=4).items()}
    keys = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias")
    g = {k: torch.from_numpy(v).cuda() for k, v in
         workloads.ss2d(batch=1, dim=16, height=12, width=20, state=8, seed=5).items()}

    def work():
        y1 = arm_scan.selective_scan(m1["u"], F.softplus(m1["delta"]), m1["A"], m1["B"],
                                     m1["C"], D=m1["D"], z=m1["z"])
        y3 = arm_scan.mamba3_scan(*[m3[k] for k in keys], cos=m3["cos"], sin=m3["sin"])
        nc = arm_scan.noncausal_scan(*[m3[k] for k in keys], cos=m3["cos"], sin=m3["sin"])
        y2 = arm_scan.ss2d_scan(g["u"], g["delta"], g["A"], g["B4"], g["C4"], D=g["D"],
                                z=g["z"], merge="sum", per_direction=True)
        return y1, y3, nc, y2

    want = work()
    torch.cuda.synchronize()
    results, errors = [None] * 4, []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                outs = [work() for _ in range(5)]
            s.synchronize()
            results[i] = outs
        except Exception as e:  # noqa: BLE001 (reported below)
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for outs in results:
        for got in outs:
            for g, w in zip(got, want):
                assert torch.equal(g, w)

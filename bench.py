"""Benchmark of the MI355X selective-scan engine (one GPU).

A step is one pass of the hot path over one batch: the Mamba-1 selective scan
of one Mamba-130M layer at prefill, batch 8 x length 2048 (d_inner 1536,
d_state 16, with delta_bias + softplus, D skip and the silu(z) gate -- exactly
what BASELINE config 2 hands the scan 24 times per forward). Inputs are
synthetic, seeded, already resident in HBM; two input sets alternate so that
no step reads data the previous step left in the 256 MB MALL.

The JSON line carries:
  value         scan throughput, algorithmic GB/s (every input read once, every
                output written once, fp32) over the timed steps;
  roofline      that kernel's achieved GB/s against MI355X's 8 TB/s, timed with
                HIP events on the stream the kernel runs on;
  prefill       BASELINE config 2 end to end: Hugging Face Mamba-130M
                architecture, random init, fp32, batch 8 x 2048 tokens, scan in
                the HIP kernel (patched), everything else in PyTorch-ROCm;
  other_configs BASELINE configs 3-5 (Mamba-3 SISO, MIMO, SS2D) through the
                public API, algorithmic GB/s of one call, each with the CPU
                oracle timed on a bounded sample of it;
  cpu_baseline  the CPU oracle (a C++ restatement of the reference's x86
                scalar scan path) on a bounded sample of the same workload.

`--workload m3_siso|m3_mimo|ss2d` times one of configs 3-5 alone, and
`--workload m1_seam` the config-2 scan in the Hugging Face mixer's layouts (the
commands behind their rocprofv3 summaries in profiles/).
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "selective-scan GB/s (% of ~8 TB/s HBM) + Mamba-1 130m prefill tokens/s"
HBM_PEAK_GBS = 8000.0
SHAPE = dict(batch=8, dim=1536, length=2048, state=16)
# The GPU's clocks ramp up from idle over tens of milliseconds: every timed region
# follows at least this much wall time of the same calls.
WARM_S = 0.5


def warm_up(fn, n):
    """`n` untimed calls fn(i), continued until the GPU has run them for WARM_S seconds
    (synchronising every 8 calls, so that the wall time is the GPU's)."""
    import torch

    t0 = time.perf_counter()
    i = 0
    while i < n or time.perf_counter() - t0 < WARM_S:
        fn(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=3)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-only", choices=("scan", "scan_conv"), default=None,
                    help="time only this patched prefill (no unpatched forward, no parity "
                         "check): the command behind the prefill kernel trace")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--workload", choices=("m1", "m1_b1", "m1_seam", "m3_siso", "m3_mimo",
                                           "ss2d", "m1_longctx", "m1_bidir_few",
                                           "m3_siso_angles", "m3_mimo_angles",
                                           "m3_noncausal", "m3_block"),
                    default="m1",
                    help="m1 (default): the headline line below; the others time one of the "
                         "configs 3-5, or the config-2 scan in the HF mixer's layouts "
                         "(m1_seam), alone (for profiling) and print its own line")
    ap.add_argument("--decode", action="store_true",
                    help="also time greedy generation (config-2 architecture, batch 1) "
                         "with and without the patched decode step")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip timing configs 3-5 in the headline line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device-to-device copy of 1 GiB (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    return ap.parse_args()


def scan_inputs(seed, dev):
    import torch

    from armhackathon_amd import workloads

    # the HF layer passes the raw dt_proj output with its bias and asks for softplus
    x = workloads.m1_layer(seed=seed, **SHAPE)
    return {k: torch.from_numpy(v).to(dev) for k, v in x.items()}


def bench_scan(args, dev):
    import torch

    from armhackathon_amd import _ffi, workloads

    sets = [scan_inputs(s, dev) for s in (0, 1)]
    b, d, L, n = SHAPE["batch"], SHAPE["dim"], SHAPE["length"], SHAPE["state"]
    outs = [torch.empty((b, d, L), device=dev) for _ in sets]
    lasts = [torch.empty((b, d, n), device=dev) for _ in sets]
    dims = _ffi.ArmScanDims(b, d, L, n, 1)
    stream = torch.cuda.current_stream(dev)

    def step(i):
        x, o, l = sets[i & 1], outs[i & 1], lasts[i & 1]
        _ffi.scan_raw(dims, x["u"].data_ptr(), x["delta"].data_ptr(), x["A"].data_ptr(),
                      x["B"].data_ptr(), x["C"].data_ptr(), x["D"].data_ptr(),
                      x["z"].data_ptr(), x["delta_bias"].data_ptr(), True, "auto", "auto",
                      o.data_ptr(), l.data_ptr(), 0, reverse=False, stream=stream.cuda_stream)

    warm_up(step, args.warmup)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        step(i)
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop) / args.steps
    nbytes = workloads.m1_bytes(b, d, L, n, z=True, D=True, bias=True, last_state=True)
    return dict(ms_per_step=ms, wall_ms_per_step=1e3 * wall / args.steps, bytes=nbytes,
                gbs=nbytes / (ms * 1e-3) / 1e9)


def config_inputs(name, dev):
    """Seeded inputs of BASELINE config 3 (m3_siso), 4 (m3_mimo) or 5 (ss2d) on dev,
    and the config's algorithmic bytes per call."""
    import torch

    from armhackathon_amd import workloads

    if name == "m1_b1":
        sets = []
        for sd in range(8):
            x = workloads.m1_op(batch=1, dim=1536, length=2048, state=16, seed=100 + sd)
            sets.append({k: torch.from_numpy(v).to(dev) for k, v in x.items() if v is not None})
        return sets, workloads.m1_bytes(1, 1536, 2048, 16, z=True, D=True, last_state=True)
    if name == "m1_longctx":
        # the reference's long-context shape (bench/bench_longctx.py:30-33): 768 rows,
        # the few-rows plan cuts each into 16 segments; one set is 1.2 GB of inputs
        x = workloads.m1_layer(batch=1, dim=768, length=131072, state=16, seed=9)
        return ({k: torch.from_numpy(v).to(dev) for k, v in x.items()},
                workloads.m1_bytes(1, 768, 131072, 16, z=True, D=True, bias=True,
                                   last_state=True))
    if name == "ss2d":
        # two sets (236 MB each) alternate: one alone would fit in the 256 MB MALL
        xs = [workloads.ss2d(seed=sd) for sd in (5, 6)]
        nbytes = workloads.ss2d_bytes(xs[0], merge="sum")
        return [{k: torch.from_numpy(v).to(dev) for k, v in x.items()} for x in xs], nbytes
    if name == "m1_seam":
        t = scan_inputs(0, dev)
        b, d, L, n = SHAPE["batch"], SHAPE["dim"], SHAPE["length"], SHAPE["state"]
        proj = torch.empty((b, L, 2 * d), device=dev)  # the mixer's in_proj output
        proj[..., d:] = t["z"].transpose(1, 2)
        t["z"] = proj.transpose(1, 2)[:, d:]
        # u: the causal convolution's output, stored (b, L, D) for the mixer's x_proj
        t["u"] = t["u"].transpose(1, 2).contiguous().transpose(1, 2)
        return t, workloads.m1_bytes(b, d, L, n, z=True, D=True, bias=True, last_state=True)
    if name in ("m3_siso_angles", "m3_mimo_angles"):
        base = workloads.m3_siso(seed=3) if name == "m3_siso_angles" else \
            workloads.m3_mimo(seed=4)
        x = workloads.m3_with_angles(base, seed=6)
        return {k: torch.from_numpy(v).to(dev) for k, v in x.items()}, workloads.m3_bytes(x)
    if name == "m3_block":
        from armhackathon_amd.mamba3_block import Mamba3Mixer

        torch.manual_seed(7)
        m = Mamba3Mixer().to(dev)  # the published SISO mixer's dimensions
        with torch.no_grad():
            for pname, prm in m.named_parameters():
                if pname.endswith("proj.weight"):
                    prm.normal_(0.0, prm.shape[1] ** -0.5)
                elif pname == "dt_bias":
                    prm.uniform_(-4.0, -2.0)
        u = torch.randn((4, 4096, m.d_model), device=dev)
        # what the mixer's scan core reads and writes once: the projection, the
        # parameters, the output (b, l, h, p)
        nbytes = 4 * (u.shape[0] * u.shape[1] * (sum(m.split_sizes) + m.d_inner))
        return {"mixer": m, "u": u}, nbytes
    if name == "m3_noncausal":
        x = workloads.m3_siso(seed=3)
        nbytes = workloads.m3_bytes(x, want_state=False)
    elif name == "m3_siso":
        x = workloads.m3_siso(seed=3)
        nbytes = workloads.m3_bytes(x)
    elif name == "m3_mimo":
        x = workloads.m3_mimo(seed=4)
        nbytes = workloads.m3_bytes(x)
    else:
        x = workloads.ss2d(seed=5)
        nbytes = workloads.ss2d_bytes(x, merge="sum")
    return {k: torch.from_numpy(v).to(dev) for k, v in x.items()}, nbytes


CONFIG_NAMES = {
    "m1_b1": "config 1: Mamba-1 selective_scan B1 D1536 L2048 N16, z and D, final state "
             "(8 input sets rotated: one set fits in the 256 MB MALL)",
    "m1_seam": "config 2 scan at the Hugging Face seam: B8 D1536 L2048 N16, bias+softplus, "
               "D, z read in place from the mixer's (b, L, 2D) projection, u from the "
               "convolution's (b, L, D) output, out written time-major",
    "m3_siso": "config 3: Mamba-3 SISO B4 L4096 24 heads x 64, dqk 128 (final states too)",
    "m3_siso_angles": "config 3 from raw angles (b, l, h, 32): the angle pre-pass fused",
    "m3_mimo_angles": "config 4 from raw angles (b, l, h, 32): the angle pre-pass fused",
    "m3_block": "Mamba-3 SISO mixer forward at the published dimensions (d_model 768, "
                "d_state 128, 24 heads x 64, 32 angles), B4 L4096: in_proj, front-end, "
                "scan, out_proj (random-init weights)",
    "m3_noncausal": "config 3 shapes aggregated non-causally (every position over every "
                    "other): forward traversal, then the backward one accumulated without "
                    "the same-step term",
    "m3_mimo": "config 4: Mamba-3 MIMO rank 4, B4 L4096 24 heads x 64, dqk 128 (final state)",
    "ss2d": "config 5: SS2D 4 directions, B16 D192 64x64 N16, D, z, merge sum (final states; "
            "2 input sets rotated: one set fits in the 256 MB MALL)",
    "m1_longctx": "long context: Mamba-1 selective_scan B1 D768 L131072 N16, bias+softplus, "
                  "D, z, final state (the reference's bench_longctx shape)",
}


def bench_config(name, dev, steps, warmup):
    """One config through the public Python API (what a model calls), timed with
    HIP events on the current stream: the whole call, pre-passes included."""
    import torch

    import armhackathon_amd as arm_scan

    t, nbytes = config_inputs(name, dev)
    K = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias")
    if name == "m1_b1":
        from armhackathon_amd import _ffi
        outs = [torch.empty_like(x["u"]) for x in t]
        lasts = [x["u"].new_empty((1, 1536, 16)) for x in t]
        dims = _ffi.ArmScanDims(1, 1536, 2048, 16, 1)
        it = {"i": 0}

        def call():
            i = it["i"] = (it["i"] + 1) % len(t)
            x = t[i]
            _ffi.scan_raw(dims, x["u"].data_ptr(), x["delta"].data_ptr(), x["A"].data_ptr(),
                          x["B"].data_ptr(), x["C"].data_ptr(), x["D"].data_ptr(),
                          x["z"].data_ptr(), 0, False, "auto", "auto", outs[i].data_ptr(),
                          lasts[i].data_ptr(), 0, reverse=False,
                          stream=torch.cuda.current_stream(dev).cuda_stream)
    elif name == "m1_longctx":
        def call():
            return arm_scan.selective_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"],
                                           z=t["z"], delta_bias=t["delta_bias"],
                                           delta_softplus=True, return_last_state=True)
    elif name == "m1_seam":
        def call():
            return arm_scan.selective_scan_time_major(
                t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"], z=t["z"],
                delta_bias=t["delta_bias"], delta_softplus=True, return_last_state=True)
    elif name == "m3_siso_angles":
        def call():
            return arm_scan.mamba3_scan(*[t[k] for k in K], angles=t["angles"],
                                        return_last_state=True)
    elif name == "m3_mimo_angles":
        def call():
            return arm_scan.mamba3_mimo_scan(*[t[k] for k in K], t["psi"], t["zeta"],
                                             t["phi"], angles=t["angles"],
                                             return_last_state=True)
    elif name == "m3_block":
        mixer, u = t["mixer"], t["u"]

        def call():
            with torch.no_grad():
                return mixer(u)
    elif name == "m3_noncausal":
        def call():
            return arm_scan.noncausal_scan(*[t[k] for k in K], cos=t["cos"], sin=t["sin"])
    elif name == "m3_siso":
        def call():
            return arm_scan.mamba3_scan(*[t[k] for k in K], cos=t["cos"], sin=t["sin"],
                                        return_last_state=True)
    elif name == "m3_mimo":
        def call():
            return arm_scan.mamba3_mimo_scan(*[t[k] for k in K], t["psi"], t["zeta"], t["phi"],
                                             cos=t["cos"], sin=t["sin"], return_last_state=True)
    else:
        it = {"i": 0}

        def call():
            x = t[it["i"] & 1]
            it["i"] += 1
            return arm_scan.ss2d_scan(x["u"], x["delta"], x["A"], x["B4"], x["C4"], D=x["D"],
                                      z=x["z"], delta_softplus=False, merge="sum",
                                      per_direction=True, return_last_state=True)
    warm_up(lambda i: call(), warmup)
    stream = torch.cuda.current_stream(dev)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        call()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    gbs = nbytes / (ms * 1e-3) / 1e9
    extra = {}
    if name.endswith("_angles"):
        # the same call through the unfused route: the pre-pass in torch ops, then
        # the scan on cos/sin (what the reference's Python layer does)
        from armhackathon_amd.mamba3 import angles_to_cos_sin

        def unfused():
            cos, sin = angles_to_cos_sin(t["angles"], t["dt"], t["q"].shape[-1] // 2)
            if name == "m3_siso_angles":
                return arm_scan.mamba3_scan(*[t[k] for k in K], cos=cos, sin=sin,
                                            return_last_state=True)
            return arm_scan.mamba3_mimo_scan(*[t[k] for k in K], t["psi"], t["zeta"],
                                             t["phi"], cos=cos, sin=sin,
                                             return_last_state=True)
        warm_up(lambda i: unfused(), warmup)
        start.record(stream)
        for _ in range(steps):
            unfused()
        stop.record(stream)
        torch.cuda.synchronize()
        extra["unfused_ms_per_call"] = round(start.elapsed_time(stop) / steps, 4)
    if name == "m3_block":
        # the reference's block on the same scan kernel: the front-end in torch ops and
        # the contiguous copies of x, z and the head-broadcast angles the scan's Python
        # layer makes (apps/mamba3_lm/block.py:146-199, python/arm_scan/mamba3.py)
        import torch.nn.functional as F

        m = mixer

        def torch_route():
            with torch.no_grad():
                b, L, _ = u.shape
                h, p, n = m.nheads, m.headdim, m.d_state
                zz, xx, B, C, ddt, dda, tr, ang = torch.split(m.in_proj(u), m.split_sizes,
                                                              dim=-1)
                zz, xx = zz.reshape(b, L, h, p), xx.reshape(b, L, h, p)
                B = m.B_norm(B.reshape(b, L, 1, 1, n))
                C = m.C_norm(C.reshape(b, L, 1, 1, n))
                A = torch.clamp(-(dda.clamp_min(0) + torch.reciprocal(1 - dda.clamp_max(0))),
                                max=-m.A_floor)
                DT = F.softplus(ddt + m.dt_bias)
                ADT = (A * DT).permute(0, 2, 1)
                DT = DT.permute(0, 2, 1)
                ang = ang.unsqueeze(-2).expand(-1, -1, h, -1)
                y = arm_scan.mamba3_scan(C[:, :, 0], B[:, :, 0], xx, ADT, DT,
                                         tr.permute(0, 2, 1), m.C_bias[:, 0], m.B_bias[:, 0],
                                         angles=ang, D=m.D, z=zz)
                return m.out_proj(y.reshape(b, L, h * p))

        def gemms():
            with torch.no_grad():
                proj = m.in_proj(u)
                return m.out_proj(proj[..., :m.d_inner])
        for key, fn in (("torch_front_end_ms_per_call", torch_route),
                        ("gemms_only_ms_per_call", gemms)):
            warm_up(lambda i: fn(), warmup)
            start.record(stream)
            for _ in range(steps):
                fn()
            stop.record(stream)
            torch.cuda.synchronize()
            extra[key] = round(start.elapsed_time(stop) / steps, 4)
    if name == "m3_noncausal":
        # the reference's composition on the same kernels: both traversals into two
        # outputs, then forward + backward - the same-step term in torch ops
        # (python/arm_scan/mamba3_noncausal.py:47-98)
        def pair_route():
            fwd, bwd = arm_scan.mamba3_scan_pair(*[t[k] for k in K], cos=t["cos"],
                                                 sin=t["sin"])
            qk = ((t["q"] + t["q_bias"]) * (t["k"] + t["k_bias"])).sum(-1)  # (b, l, h)
            gamma = (t["dt"] * torch.sigmoid(t["trap"])).permute(0, 2, 1)
            return fwd + bwd - (gamma * qk).unsqueeze(-1) * t["v"]

        def causal():
            return arm_scan.mamba3_scan(*[t[k] for k in K], cos=t["cos"], sin=t["sin"])
        for key, fn in (("pair_route_ms_per_call", pair_route),
                        ("causal_ms_per_call", causal)):
            warm_up(lambda i: fn(), warmup)
            start.record(stream)
            for _ in range(steps):
                fn()
            stop.record(stream)
            torch.cuda.synchronize()
            extra[key] = round(start.elapsed_time(stop) / steps, 4)
    del t
    torch.cuda.empty_cache()
    return dict(workload=CONFIG_NAMES[name], ms_per_call=round(ms, 4), bytes_per_call=nbytes,
                gbs=round(gbs, 2), frac_of_8tbs=round(gbs / HBM_PEAK_GBS, 4), steps=steps,
                **extra)


def bench_bidir_few(dev, steps):
    """Bidirectional Mamba-1 on few rows: the entry point's route (the exp-sharing
    kernel where a row fits it, else two launches that cut rows into segments) against
    two single-direction calls and, for reference, the two-job whole-row launch that
    wide shapes take. ms per call, HIP events, after the warm-up."""
    import torch

    import armhackathon_amd as arm_scan
    from armhackathon_amd import workloads

    out = {}
    for (b, d, L) in ((1, 16, 65536), (1, 768, 32768), (1, 1536, 2048), (16, 192, 4096)):
        x = workloads.m1_op(batch=b, dim=d, length=L, state=16, seed=11)
        t = {k: torch.from_numpy(v).to(dev) for k, v in x.items() if v is not None}
        a = (t["u"], t["delta"], t["A"], t["B"], t["C"])
        kw = dict(D=t["D"], z=t["z"])

        def pair():
            return arm_scan.selective_scan_bidirectional(*a, **kw)

        def singles():
            return (arm_scan.selective_scan(*a, **kw),
                    arm_scan.selective_scan(*a, reverse=True, **kw))
        r = {}
        stream = torch.cuda.current_stream(dev)
        for key, fn in (("bidirectional_ms", pair), ("two_calls_ms", singles)):
            warm_up(lambda i: fn(), 5)
            st, sp = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            st.record(stream)
            for _ in range(steps):
                fn()
            sp.record(stream)
            torch.cuda.synchronize()
            r[key] = round(st.elapsed_time(sp) / steps, 4)
        out[f"B{b} D{d} L{L}"] = r
        del t, a, kw
        torch.cuda.empty_cache()
    return out


def bench_config_cpu(name, seconds):
    """The C++ restatement of the reference's x86 path on host cores for one of
    configs 1 and 3-5, over a bounded sample of the config (config 1 whole, batch 1 of
    4 for Mamba-3, 2 of 16 for SS2D), repeated until `seconds` of wall time have
    passed."""
    import oracle
    from armhackathon_amd import workloads

    host_oracle()
    K = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias")
    if name == "m1_b1":
        x = workloads.m1_op(batch=1, dim=1536, length=2048, state=16, seed=100)
        nbytes = workloads.m1_bytes(1, 1536, 2048, 16, z=True, D=True, last_state=True)
        sample = "config 1"

        def call():
            oracle.selective_scan(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"],
                                  z=x["z"])
    elif name == "m3_siso":
        x = workloads.m3_siso(batch=1, seed=3)
        nbytes, sample = workloads.m3_bytes(x), "batch 1 of config 3"

        def call():
            oracle.mamba3_scan(*[x[k] for k in K], x["cos"], x["sin"], want_state=True)
    elif name == "m3_noncausal":
        from oracle import naive
        x = workloads.m3_siso(batch=1, seed=3)
        nbytes = workloads.m3_bytes(x, want_state=False)
        sample = "batch 1 of config 3, both traversals and the same-step term"

        def call():
            args = [x[k] for k in K] + [x["cos"], x["sin"]]
            fwd = oracle.mamba3_scan(*args)
            bwd = oracle.mamba3_scan(*args, reverse=True)
            return fwd + bwd - naive.m3_same_step(x["q"], x["k"], x["v"], x["dt"], x["trap"],
                                                  x["q_bias"], x["k_bias"]).transpose(0, 2, 1, 3)
    elif name == "m1_longctx":
        x = workloads.m1_layer(batch=1, dim=48, length=131072, state=16, seed=9)
        nbytes = workloads.m1_bytes(1, 48, 131072, 16, z=True, D=True, bias=True)
        sample = "48 of the 768 channels of the long-context shape"

        def call():
            oracle.selective_scan(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"],
                                  z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    elif name == "m3_mimo":
        x = workloads.m3_mimo(batch=1, seed=4)
        nbytes, sample = workloads.m3_bytes(x), "batch 1 of config 4"

        def call():
            oracle.mamba3_scan(*[x[k] for k in K], x["cos"], x["sin"], psi=x["psi"],
                               zeta=x["zeta"], phi=x["phi"], want_state=True)
    else:
        x = workloads.ss2d(batch=2, seed=5)
        nbytes, sample = workloads.ss2d_bytes(x, merge="sum"), "batch 2 of config 5"

        def call():
            planes, _ = oracle.ss2d(x["u"], x["delta"], x["A"], x["B4"], x["C4"], D=x["D"],
                                    z=x["z"], want_state=True)
            planes.sum(axis=0)
    return cpu_rates(call, nbytes, sample, seconds, 50)


def host_oracle():
    """Build the C++ restatement of the reference's x86 path on this host (g++, the
    committed oracle/Makefile: -O3 -march=x86-64, no fast-math or contraction, as
    cargo's portable release build) into a temporary directory, and load it. Once per
    process; returns the build record."""
    import tempfile

    import oracle

    if "build" in _HOST:
        return _HOST["build"]
    out = Path(tempfile.mkdtemp(prefix="arm_scan_oracle_")) / "libarm_scan_cpu.so"
    t0 = time.perf_counter()
    oracle.build(out=out)
    oracle.use(out)
    oracle.lib()
    model = "unknown"
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    _HOST["build"] = dict(built_on_host=True, build_s=round(time.perf_counter() - t0, 1),
                          compiler="g++ -O3 -march=x86-64 -ffp-contract=off (oracle/Makefile)",
                          nproc=os.cpu_count(), cpu_model=model)
    return _HOST["build"]


_HOST = {}
# the box's CPU share for one GPU: all-thread figures use this many (nproc may show more)
CPU_SHARE = 16


def cpu_rates(call, nbytes, sample, seconds, max_reps):
    """Time `call` (one pass over `nbytes` algorithmic bytes) on all of the host share's
    threads and on one thread, each until `seconds` of wall time or `max_reps` passes."""
    import oracle

    def rate(threads, budget):
        oracle.set_threads(threads)
        reps, t0 = 0, time.perf_counter()
        while True:
            call()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget or reps >= max_reps:
                return nbytes * reps / el / 1e9, reps, el

    threads = min(CPU_SHARE, os.cpu_count() or 1)
    v, reps, el = rate(threads, seconds)
    v1, reps1, el1 = rate(1, seconds / 2)
    oracle.set_threads(threads)
    return dict(value=round(v, 3), unit="GB/s", cores=threads, kind="port",
                sample=f"{reps} passes of {sample} in {el:.1f} s, {threads} threads",
                one_thread=dict(value=round(v1, 3), unit="GB/s", cores=1,
                                sample=f"{reps1} passes of {sample} in {el1:.1f} s, 1 thread"),
                **host_oracle())


def bench_prefill(args, dev):
    """random-init Mamba-130M architecture, batch 8 x 2048, fp32.
    Timed three ways in one process, as the reference reports its patch
    (bench/results/RESULTS.md:54-58, unpatched vs patched):
      unpatched   upstream's torch recurrence;
      patched     patch(): only the scan in the HIP kernel (config 2 as defined);
      scan_conv   patch(conv=True): the mixer's causal conv in its kernel as well
                  (an extra outside config 2, labelled as such)."""
    import torch
    from transformers import MambaConfig, MambaForCausalLM

    import armhackathon_amd as arm_scan

    cfg = MambaConfig(vocab_size=50280, hidden_size=768, state_size=16, num_hidden_layers=24,
                      expand=2, conv_kernel=4, time_step_rank=48, use_cache=False)
    torch.manual_seed(0)
    model = MambaForCausalLM(cfg).to(dev).float().eval()
    ids = torch.randint(0, 50280, (8, 2048), device=dev,
                        generator=torch.Generator(device=dev).manual_seed(0))
    tokens = ids.numel()

    def timed(steps):
        with torch.no_grad():
            logits = model(ids, use_cache=False, logits_to_keep=1).logits
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                model(ids, use_cache=False, logits_to_keep=1)
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, logits

    if args.prefill_only:
        arm_scan.patch(conv=args.prefill_only == "scan_conv")
        try:
            t, _ = timed(args.prefill_steps)
        finally:
            arm_scan.unpatch()
        return dict(batch=8, seq_len=2048, mode=args.prefill_only, tokens_per_s=tokens / t,
                    ms_per_forward=t * 1e3)
    t_ref, ref = timed(1)
    scale = max(1.0, ref.abs().max().item())
    out = dict(batch=8, seq_len=2048, logits="last position only (logits_to_keep=1)",
               unpatched_tokens_per_s=tokens / t_ref, unpatched_ms_per_forward=t_ref * 1e3)
    for conv in (False, True):
        s0 = arm_scan.stats()
        arm_scan.patch(conv=conv)
        try:
            t, got = timed(args.prefill_steps)
        finally:
            arm_scan.unpatch()
        s1 = arm_scan.stats()
        n = 1 + args.prefill_steps
        r = dict(tokens_per_s=tokens / t, ms_per_forward=t * 1e3,
                 scan_calls_per_forward=(s1["fast_calls"] - s0["fast_calls"]) / n,
                 conv_calls_per_forward=(s1["conv_calls"] - s0["conv_calls"]) / n,
                 fallback_calls=(s1["fallback_calls"] - s0["fallback_calls"]
                                 + s1["conv_fallback_calls"] - s0["conv_fallback_calls"]),
                 logits_max_abs_diff_over_scale=(got - ref).abs().max().item() / scale)
        if conv:
            out["scan_conv"] = dict(r, note="extra, outside config 2: patch(conv=True) also "
                                            "runs the mixer's causal conv in its HIP kernel")
        else:
            out.update(r)
            out["speedup_vs_unpatched"] = t_ref / t
    return out


def bench_decode(dev, new_tokens=64, prompt=128):
    """Greedy generation with the cache (Mamba-130M architecture, random init, batch 1):
    ms per new token unpatched; patched but with upstream's two decode-step functions
    (mamba_selective_state_update, causal_conv1d_update); and fully patched."""
    import torch
    from transformers import MambaConfig, MambaForCausalLM
    from transformers.models.mamba import modeling_mamba

    import armhackathon_amd as arm_scan
    from armhackathon_amd import hf_patch

    cfg = MambaConfig(vocab_size=50280, hidden_size=768, state_size=16, num_hidden_layers=24,
                      expand=2, conv_kernel=4, time_step_rank=48)
    torch.manual_seed(0)
    model = MambaForCausalLM(cfg).to(dev).float().eval()
    ids = torch.randint(0, 50280, (1, prompt), device=dev,
                        generator=torch.Generator(device=dev).manual_seed(1))

    def gen(n):
        return model.generate(ids, max_new_tokens=n, min_new_tokens=n, do_sample=False)

    def ms_per_token():
        with torch.no_grad():
            gen(4)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            gen(1)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            out = gen(new_tokens + 1)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
        # the prefill and first token cost (t1 - t0); the rest are decode steps
        return ((t2 - t1) - (t1 - t0)) / new_tokens * 1e3, out

    r = {"batch": 1, "prompt": prompt, "new_tokens": new_tokens}
    r["unpatched_ms_per_token"], ref = ms_per_token()
    arm_scan.patch(conv=True)
    try:
        step = modeling_mamba.mamba_selective_state_update
        conv_step = modeling_mamba.causal_conv1d_update
        modeling_mamba.mamba_selective_state_update = hf_patch._STATE["orig_step"]
        modeling_mamba.causal_conv1d_update = hf_patch._STATE["orig_conv_step"]
        r["upstream_decode_steps_ms_per_token"], _ = ms_per_token()
        modeling_mamba.mamba_selective_state_update = step
        modeling_mamba.causal_conv1d_update = conv_step
        r["ms_per_token"], got = ms_per_token()
    finally:
        arm_scan.unpatch()
    r["tokens_identical"] = bool(torch.equal(ref, got))
    return {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}


def bench_cpu(seconds):
    """The C++ restatement of the reference's x86 scalar path on host cores,
    over a bounded sample: the same layer scan restricted to a slice of
    channels, repeated until `seconds` of CPU time have passed."""
    import oracle
    from armhackathon_amd import workloads

    host_oracle()
    dim = 1536
    x = workloads.m1_layer(batch=1, dim=dim, length=SHAPE["length"], state=SHAPE["state"],
                           seed=0)

    def call():
        oracle.selective_scan(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
                              delta_bias=x["delta_bias"], delta_softplus=True, threading=2)

    nbytes = workloads.m1_bytes(1, dim, SHAPE["length"], SHAPE["state"], z=True, D=True,
                                bias=True)
    return cpu_rates(call, nbytes, f"B1 D{dim} L{SHAPE['length']} N{SHAPE['state']} (one "
                     "batch row of the step; softplus+bias, D, z)", seconds, 1000)


def issue_floor(ms_per_step):
    """The step's fp32 issue floor: one v_exp_f32 (two VALU slots, 8 cycles per wave64)
    and five VALU ops (4 cycles each) per (step, state), spread over MI355X's 1024 SIMDs
    at 2.4 GHz. The kernel is bound by this issue, not by HBM; `frac` is floor / step."""
    b, d, L, n = SHAPE["batch"], SHAPE["dim"], SHAPE["length"], SHAPE["state"]
    cycles = b * d * L * n / 64 * (8 + 5 * 4) / 1024
    floor_ms = cycles / 2.4e9 * 1e3
    return {"unit": "ms", "value": round(floor_ms, 4), "frac": round(floor_ms / ms_per_step, 4),
            "model": "(v_exp_f32 8 + 5 VALU x 4) cycles per (step, state) wave-element, "
                     "1024 SIMDs, 2.4 GHz"}


def traffic_from_profiles():
    """HBM bytes per launch measured by rocprofv3 counters (profiles/), or None."""
    p = ROOT / "profiles" / "m1_scan_ns_traffic.json"
    if not p.is_file():
        return None
    try:
        return json.loads(p.read_text()).get("bytes_per_launch")
    except (ValueError, OSError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the scan shards "
              "over batch and channel rows with no communication across them, so each GPU "
              "runs this kernel on its share", file=sys.stderr)
        sys.exit(2)
    import torch

    from armhackathon_amd import _ffi

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.ones(1 << 28, device=dev)  # 1 GiB of fp32
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel() * 4}), flush=True)
        return
    _ffi.load()
    if args.workload == "m1_bidir_few":
        print(json.dumps({"metric": "ms per call", "unit": "ms", "n_gpus": 1, "dtype": "f32",
                          "data": "synthetic", "detail": bench_bidir_few(dev, args.steps)}),
              flush=True)
        return
    if args.workload != "m1":
        r = bench_config(args.workload, dev, args.steps, args.warmup)
        print(json.dumps({"metric": "algorithmic GB/s of one call", "value": r["gbs"],
                          "unit": "GB/s", "n_gpus": 1, "dtype": "f32", "data": "synthetic",
                          "config": {"workload": r["workload"]}, "detail": r}), flush=True)
        return
    r = bench_scan(args, dev)
    prefill = None if args.no_prefill else bench_prefill(args, dev)
    decode = bench_decode(dev) if args.decode else None
    configs = None if args.no_configs else {
        name: bench_config(name, dev, steps, 10)
        for name, steps in (("m1_b1", 400), ("m3_siso", 100), ("m3_mimo", 40), ("ss2d", 100),
                            ("m3_noncausal", 50), ("m1_longctx", 40))}
    cpu = None if args.no_cpu else bench_cpu(args.cpu_seconds)
    if configs is not None and not args.no_cpu:
        for name in configs:
            configs[name]["cpu_baseline"] = bench_config_cpu(name, args.cpu_seconds / 4)
    achieved = r["gbs"]
    line = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded PCG64; random-init weights for the prefill)",
        "config": {"workload": "Mamba-1 selective_scan of one Mamba-130M prefill layer "
                               "(BASELINE config 2 scan): B8 D1536 L2048 N16, "
                               "delta_bias+softplus, D, z; groups 1",
                   "bytes_per_step": r["bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(),
                     "issue_floor": issue_floor(r["ms_per_step"])},
        "prefill": prefill,
        **({"decode": decode} if decode is not None else {}),
        "other_configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Mamba-1 selective scan on the GPU vs the CPU oracle and the reference goldens.

Gates (fp32): tensor-scale relative error <= 1e-4 on outputs and final states
plus the reference's own golden gates
(check_ffi.py:153-154,205-206: max_abs < 1e-4 vs out_f64, last_state rel < 1e-4).
Cases follow the reference's test strategy: every golden, reverse, h0 streaming,
grouped B/C, missing optional inputs, ragged lengths (L not a multiple of the
kernel's chunking, L = 1), D = 1, N = 8 and 13, and the full benchmark shapes.
"""

import json

import numpy as np
import pytest

import oracle
from armhackathon_amd import workloads
from util import case, dev, host, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _scan(x, **kw):
    import armhackathon_amd as arm_scan

    t = dev(x)
    return arm_scan.selective_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t.get("D"),
                                   z=t.get("z"), delta_bias=t.get("delta_bias"),
                                   return_last_state=True,
                                   initial_state=t.get("h0"), **kw)


def _ref(x, dtype=np.float64, **kw):
    return oracle.selective_scan(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x.get("D"),
                                 z=x.get("z"), delta_bias=x.get("delta_bias"),
                                 h0=x.get("h0"), dtype=dtype, **kw)


def test_m1_goldens(golden_dir):
    """Every reference Mamba-1 golden under the reference's gates."""
    man = json.loads((golden_dir / "1d" / "manifest.json").read_text())
    for m in man:
        case(f"golden {m['name']}")
        z = np.load(golden_dir / "1d" / f"{m['name']}.npz")
        meta = json.loads(bytes(z["meta_json"]).decode())
        x = {k: z[k].astype(np.float32) for k in ("u", "delta", "A", "B", "C")}
        for k, name in (("D", "D_skip"), ("z", "z"), ("delta_bias", "delta_bias")):
            if name in z.files:
                x[k] = z[name].astype(np.float32)
        out, last = _scan(x, delta_softplus=meta["delta_softplus"])
        out, last = host(out), host(last)
        err = np.abs(out - z["out_f64"]).max()
        floor = float(m.get("f32_max_abs_err") or 0.0)
        assert err < 1e-4, (m["name"], err)
        if floor > 0:
            assert err < 50 * max(floor, 1e-7), (m["name"], err, floor)
        assert rel_err(last, z["last_state_f64"]) < 1e-4, m["name"]


SHAPES = [
    # (batch, dim, len, state, groups)
    (1, 4, 1, 16, 1),
    (2, 8, 7, 16, 1),
    (1, 3, 129, 5, 1),
    (2, 16, 1000, 16, 4),
    (1, 12, 2049, 13, 3),
    (3, 10, 4096, 16, 2),
    (1, 8, 9000, 8, 1),
    (2, 64, 333, 16, 64),
    # 16-row blocks inside one batch/group (the LDS-tiled kernel), with row tails
    (2, 32, 1000, 16, 1),
    (1, 16, 300, 16, 1),
    (1, 32, 600, 13, 2),
    (2, 48, 512, 8, 3),
    (1, 16, 4096, 16, 1),
    # the tiled kernel's tail chunk in its tile loop (L % 256 != 0), and rows that are
    # not 16-byte multiples (L % 4 != 0: single-float DMA and loads)
    (1, 16, 260, 16, 1),
    (2, 32, 1001, 16, 1),
    (1, 16, 3, 16, 1),
    (1, 32, 258, 16, 2),
    (1, 48, 2050, 13, 3),
    (2, 16, 256, 16, 1),
    # few rows: the segmented scan (fold + replay) with a tail, aligned and not
    (1, 1536, 2052, 16, 1),
    (1, 1536, 2050, 16, 1),
    (1, 1536, 777, 13, 1),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("reverse", [False, True])
def test_m1_random_vs_oracle(shape, reverse):
    b, d, L, n, g = shape
    case(f"m1 random {shape} reverse={reverse}")
    rng = np.random.default_rng(hash((shape, reverse)) & 0xFFFF)
    f = np.float32
    x = dict(u=rng.standard_normal((b, d, L)).astype(f),
             delta=(rng.standard_normal((b, d, L)) * 0.5).astype(f),
             A=(-np.exp(rng.uniform(-0.7, 2.7, (d, n)))).astype(f),
             B=rng.standard_normal((b, g, n, L)).astype(f),
             C=rng.standard_normal((b, g, n, L)).astype(f),
             D=rng.standard_normal(d).astype(f), z=rng.standard_normal((b, d, L)).astype(f),
             delta_bias=rng.uniform(-6, -3, d).astype(f),
             h0=rng.standard_normal((b, d, n)).astype(f))
    out, last = _scan(x, delta_softplus=True, reverse=reverse)
    ref, ref_last = _ref(x, delta_softplus=True, reverse=reverse)
    assert rel_err(host(out), ref) < TOL
    assert rel_err(host(last), ref_last) < TOL


@pytest.mark.parametrize("dim", [24, 32])
def test_m1_optional_inputs_absent(dim):
    """dim 24: the global-load kernel; dim 32: the tiled one, with unaligned rows and
    a tail chunk (L 777)."""
    x = workloads.m1_op(batch=2, dim=dim, length=777, state=16, seed=3, z=False, D=False)
    case(f"m1 without D/z/bias, softplus off, dim {dim}")
    out, last = _scan(x)
    ref, ref_last = _ref(x)
    assert rel_err(host(out), ref) < TOL and rel_err(host(last), ref_last) < TOL


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("shifted", ["u_delta_z", "all"])
def test_m1_unaligned_bases(shifted, reverse):
    """L % 4 == 0 but inputs placed one float past an aligned base: u, delta and z (B/C
    aligned: read in place by 16-byte DMA) or every tensor (B/C copied to an aligned
    pitch). The tiled kernel with single-float row moves, against the oracle."""
    import torch
    import armhackathon_amd as arm_scan

    case(f"m1 unaligned bases {shifted} reverse={reverse}")
    x = workloads.m1_layer(batch=2, dim=32, length=1000, state=16, seed=7)
    names = ("u", "delta", "z") if shifted == "u_delta_z" else ("u", "delta", "z", "B", "C")

    def place(k, a):
        if k not in names:
            return torch.from_numpy(np.ascontiguousarray(a)).cuda()
        t = torch.empty(a.size + 1, dtype=torch.float32, device="cuda")
        t[1:] = torch.from_numpy(np.ascontiguousarray(a)).reshape(-1).cuda()
        return t[1:].view(a.shape)

    t = {k: place(k, v) for k, v in x.items()}
    out, last = arm_scan.selective_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"],
                                        z=t["z"], delta_bias=t["delta_bias"],
                                        delta_softplus=True, return_last_state=True,
                                        reverse=reverse)
    ref, ref_last = _ref(x, delta_softplus=True, reverse=reverse)
    assert rel_err(host(out), ref) < TOL and rel_err(host(last), ref_last) < TOL


def test_m1_reverse_is_flip_forward_flip():
    """property.rs:138: reverse == flip -> forward -> flip."""
    x = workloads.m1_op(batch=2, dim=32, length=3000, state=16, seed=4)
    case("m1 reverse == flip-forward-flip")
    rev, lr = _scan(x, reverse=True)
    fl = {k: (np.ascontiguousarray(v[..., ::-1]) if k in ("u", "delta", "B", "C", "z") else v)
          for k, v in x.items()}
    fwd, lf = _scan(fl)
    assert rel_err(host(rev), host(fwd)[..., ::-1]) < 1e-6
    assert rel_err(host(lr), host(lf)) < 1e-6
    assert rel_err(host(rev), host(_scan(x)[0])) > 1e-2


def test_m1_streaming_equals_one_shot():
    """property.rs:500 / check_ffi.py:174-194: prefix then suffix with h0."""
    x = workloads.m1_op(batch=2, dim=16, length=2500, state=16, seed=5)
    case("m1 h0 streaming")
    full, lfull = _scan(x)
    cut = 1111
    a = {k: (np.ascontiguousarray(v[..., :cut]) if k in ("u", "delta", "B", "C", "z") else v)
         for k, v in x.items()}
    b = {k: (np.ascontiguousarray(v[..., cut:]) if k in ("u", "delta", "B", "C", "z") else v)
         for k, v in x.items()}
    o1, l1 = _scan(a)
    b["h0"] = host(l1)
    o2, l2 = _scan(b)
    assert rel_err(np.concatenate([host(o1), host(o2)], -1), host(full)) < 1e-5
    assert rel_err(host(l2), host(lfull)) < 1e-5


def test_m1_deterministic():
    """Two launches on the same inputs are bit-identical (property.rs:453-497)."""
    x = workloads.m1_op(batch=1, dim=64, length=4096, state=16, seed=6)
    case("m1 determinism")
    o1, _ = _scan(x)
    o2, _ = _scan(x)
    assert np.array_equal(host(o1), host(o2))


def test_m1_bidirectional_fused():
    """Fused pair == forward scan + reverse scan (property.rs:240). Every route of
    the entry point: the two-traversal launch (dim % 16 == 0: 16x1024 and 32x4096 whole
    chunks, 16x700 with a tail chunk, 16x1001 with unaligned rows), the single-pass
    kernel (dim 8, L 2048) and two launches (dim 4, L 6000)."""
    import armhackathon_amd as arm_scan
    from armhackathon_amd.op import selective_scan_bidirectional_with_state

    for (b, d, L) in ((2, 16, 700), (1, 8, 2048), (1, 4, 6000), (1, 16, 1024), (2, 32, 4096),
                      (2, 16, 1001)):
        case(f"m1 bidirectional {b}x{d}x{L}")
        x = workloads.m1_op(batch=b, dim=d, length=L, state=16, seed=L)
        x["delta_bias"] = np.full(d, -0.5, np.float32)
        t = dev(x)
        of, ob, lf, lb = selective_scan_bidirectional_with_state(
            t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"], z=t["z"],
            delta_bias=t["delta_bias"], delta_softplus=True)
        rf, rb, rlf, rlb = oracle.selective_scan_bidirectional(
            x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
            delta_bias=x["delta_bias"], delta_softplus=True, dtype=np.float64)
        assert rel_err(host(of), rf) < TOL and rel_err(host(ob), rb) < TOL
        assert rel_err(host(lf), rlf) < TOL and rel_err(host(lb), rlb) < TOL
        s = arm_scan.bidirectional_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"],
                                        z=t["z"], delta_bias=t["delta_bias"],
                                        delta_softplus=True, merge="sum")
        assert rel_err(host(s), rf + rb) < TOL


@pytest.mark.parametrize("batch", [1, 8])
def test_m1_benchmark_shape(batch):
    """BASELINE config 1 (batch 1) and the north-star shape (batch 8): D 1536,
    L 2048, N 16, against the float64 oracle, outputs and final states."""
    case(f"m1 benchmark shape batch={batch}")
    x = workloads.m1_op(batch=batch, dim=1536, length=2048, state=16, seed=0)
    out, last = _scan(x)
    ref, ref_last = _ref(x)
    assert rel_err(host(out), ref) < TOL
    assert rel_err(host(last), ref_last) < TOL


def test_m1_bench_step_inputs():
    """The headline bench step exactly as bench.py times it: B8 D1536 L2048 N16 with
    the raw delta, delta_bias and softplus, D and z (workloads.m1_layer, both input
    sets), against the float64 oracle, outputs and final states."""
    for seed in (0, 1):
        case(f"m1 bench step inputs seed={seed}")
        x = workloads.m1_layer(seed=seed)
        out, last = _scan(x, delta_softplus=True)
        ref, ref_last = _ref(x, delta_softplus=True)
        assert rel_err(host(out), ref) < TOL
        assert rel_err(host(last), ref_last) < TOL


def _time_major_inputs(x):
    """Device tensors laid out as the Hugging Face mixer hands them over: the gate
    z a (b, D, L) view of (b, L, 2D) storage (modeling_mamba.py: projected_states
    = in_proj(h).transpose(1, 2); gate = chunk(2, dim=1)[1])."""
    import torch

    t = dev(x)
    b, d, L = x["u"].shape
    proj = torch.empty((b, L, 2 * d), device="cuda")
    proj[..., d:] = t["z"].transpose(1, 2)
    proj[..., :d] = -7.0  # the other half of the storage is never read
    t["z"] = proj.transpose(1, 2)[:, d:]
    assert t["z"].stride() == (L * 2 * d, 1, 2 * d)
    return t


TM_SHAPES = [
    # (batch, dim, len, state, groups): tiled shapes with and without row tails
    # (z staged through LDS when state > 8, read with buffer loads at state 8),
    # and (dim % 16 != 0) one the strided kernel does not serve
    (2, 32, 1000, 16, 1),
    (2, 32, 1000, 8, 1),
    (1, 16, 256, 16, 1),
    (3, 48, 2052, 13, 3),
    (2, 64, 4096, 16, 2),
    (1, 12, 700, 16, 1),
]


@pytest.mark.parametrize("shape", TM_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("reverse", [False, True])
def test_m1_time_major_seam(shape, reverse):
    """selective_scan_time_major (z read in place from time-major storage, out
    written time-major) equals selective_scan bit for bit, and the oracle."""
    import armhackathon_amd as arm_scan

    b, d, L, n, g = shape
    case(f"m1 time-major seam {shape} reverse={reverse}")
    rng = np.random.default_rng(hash((shape, reverse, "tm")) & 0xFFFF)
    f = np.float32
    x = dict(u=rng.standard_normal((b, d, L)).astype(f),
             delta=(rng.standard_normal((b, d, L)) * 0.5).astype(f),
             A=(-np.exp(rng.uniform(-0.7, 2.7, (d, n)))).astype(f),
             B=rng.standard_normal((b, g, n, L)).astype(f),
             C=rng.standard_normal((b, g, n, L)).astype(f),
             D=rng.standard_normal(d).astype(f), z=rng.standard_normal((b, d, L)).astype(f),
             delta_bias=rng.uniform(-6, -3, d).astype(f),
             h0=rng.standard_normal((b, d, n)).astype(f))
    t = _time_major_inputs(x)
    out, last = arm_scan.selective_scan_time_major(
        t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"], z=t["z"],
        delta_bias=t["delta_bias"], delta_softplus=True, return_last_state=True,
        initial_state=t["h0"], reverse=reverse)
    assert out.shape == (b, d, L) and out.stride() == (L * d, 1, d)
    ref_out, ref_last = _scan(x, delta_softplus=True, reverse=reverse)
    assert np.array_equal(host(out), host(ref_out))
    assert np.array_equal(host(last), host(ref_last))
    o64, l64 = _ref(x, delta_softplus=True, reverse=reverse)
    assert rel_err(host(out), o64) < TOL and rel_err(host(last), l64) < TOL


def test_m1_time_major_without_gate():
    """No z: only the output is strided."""
    import armhackathon_amd as arm_scan

    case("m1 time-major seam, z absent")
    x = workloads.m1_op(batch=2, dim=32, length=1500, state=16, seed=9, z=False)
    t = dev(x)
    out = arm_scan.selective_scan_time_major(t["u"], t["delta"], t["A"], t["B"], t["C"],
                                             D=t["D"])
    assert out.stride() == (1500 * 32, 1, 32)
    assert np.array_equal(host(out), host(_scan(x)[0]))


@pytest.mark.parametrize("reverse", [False, True])
def test_m1_strided_gate_channel_stride(reverse):
    """z with a channel stride of 2 (every other channel of a wider tensor, so no
    16-byte channel runs): the buffer-load path of the strided kernel."""
    import torch

    import armhackathon_amd as arm_scan

    case(f"m1 strided gate, channel stride 2, reverse={reverse}")
    x = workloads.m1_op(batch=2, dim=32, length=1024, state=16, seed=11)
    t = dev(x)
    wide = torch.empty((2, 64, 1024), device="cuda")
    wide[:, ::2] = t["z"]
    wide[:, 1::2] = 5.0
    zv = wide[:, ::2]
    assert zv.stride() == (64 * 1024, 2 * 1024, 1)
    out, last = arm_scan.selective_scan_time_major(
        t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"], z=zv, return_last_state=True,
        reverse=reverse)
    ref, ref_last = _scan(x, reverse=reverse)
    assert np.array_equal(host(out), host(ref)) and np.array_equal(host(last), host(ref_last))


STEP_SHAPES = [(1, 1536, 16), (8, 1536, 16), (3, 40, 5), (2, 7, 1)]


@pytest.mark.parametrize("shape", STEP_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_m1_decode_step(shape):
    """One decode step (the state updated in place) against the oracle's one-step
    scan from h0 = the state: x, dt and z as strided (b, D) views and B, C as
    strided (b, N) views, the way a decoder hands them over."""
    import torch

    import armhackathon_amd as arm_scan

    b, d, n = shape
    case(f"m1 decode step {shape}")
    rng = np.random.default_rng(b * d + n)
    f = np.float32
    x = rng.standard_normal((b, d)).astype(f)
    dt = (rng.standard_normal((b, d)) * 0.5).astype(f)
    z = rng.standard_normal((b, d)).astype(f)
    A = (-np.exp(rng.uniform(-0.7, 2.7, (d, n)))).astype(f)
    B = rng.standard_normal((b, n)).astype(f)
    C = rng.standard_normal((b, n)).astype(f)
    D = rng.standard_normal(d).astype(f)
    bias = rng.uniform(-6, -3, d).astype(f)
    h = rng.standard_normal((b, d, n)).astype(f)
    ref, ref_h = oracle.selective_scan(x[..., None], dt[..., None], A, B[..., None],
                                       C[..., None], D=D, z=z[..., None], delta_bias=bias,
                                       delta_softplus=True, h0=h, dtype=np.float64)

    def strided(a2, extra):  # a (rows, cols) view inside a wider tensor
        wide = torch.zeros((a2.shape[0], a2.shape[1] + extra), device="cuda")
        wide[:, extra:] = torch.from_numpy(a2).cuda()
        return wide[:, extra:]

    t = dev(dict(A=A, D=D, bias=bias, h=h))
    out = arm_scan.selective_state_update(
        t["h"], strided(x, 3), strided(dt, 5).t().contiguous().t(), t["A"], strided(B, 2),
        strided(C, 1), D=t["D"], z=strided(z, 7), dt_bias=t["bias"], dt_softplus=True)
    assert rel_err(host(out), ref[..., 0]) < TOL
    assert rel_err(host(t["h"]), ref_h) < TOL


def test_m1_decode_step_optional_absent():
    import armhackathon_amd as arm_scan

    case("m1 decode step without D, z, bias")
    rng = np.random.default_rng(3)
    f = np.float32
    b, d, n = 2, 64, 16
    x, dt = rng.standard_normal((b, d)).astype(f), np.abs(rng.standard_normal((b, d))).astype(f)
    A = (-np.exp(rng.uniform(-0.7, 2.7, (d, n)))).astype(f)
    B, C = rng.standard_normal((b, n)).astype(f), rng.standard_normal((b, n)).astype(f)
    h = rng.standard_normal((b, d, n)).astype(f)
    ref, ref_h = oracle.selective_scan(x[..., None], dt[..., None], A, B[..., None],
                                       C[..., None], h0=h, dtype=np.float64)
    t = dev(dict(x=x, dt=dt, A=A, B=B, C=C, h=h))
    out = arm_scan.selective_state_update(t["h"], t["x"], t["dt"], t["A"], t["B"], t["C"])
    assert rel_err(host(out), ref[..., 0]) < TOL
    assert rel_err(host(t["h"]), ref_h) < TOL


def test_numpy_api_and_scan_fn():
    """selective_scan_numpy (numpy in and out, python/arm_scan/numpy_api.py:16-70) and
    the SS2D single-direction seam scan_fn_arm against the oracle; the reference's CPU
    backends are refused with code 3."""
    import torch

    import armhackathon_amd as arm_scan
    from armhackathon_amd import _ffi
    from armhackathon_amd.ss2d import scan_fn_arm

    case("numpy API and scan_fn_arm")
    rng = np.random.default_rng(41)
    b, d, L, n = 2, 32, 300, 16
    u = rng.standard_normal((b, d, L)).astype(np.float32)
    dl = (rng.standard_normal((b, d, L)) * 0.5 - 3.0).astype(np.float32)
    A = -np.exp(rng.normal(0, 0.5, (d, n))).astype(np.float32)
    B = rng.standard_normal((b, n, L)).astype(np.float32)
    C = rng.standard_normal((b, n, L)).astype(np.float32)
    D = rng.standard_normal(d).astype(np.float32)
    z = rng.standard_normal((b, d, L)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, d).astype(np.float32)
    ref, ref_last = oracle.selective_scan(u, dl, A, B, C, D=D, z=z, delta_bias=bias,
                                          delta_softplus=True, dtype=np.float64)
    out, last = arm_scan.selective_scan_numpy(u, dl, A, B, C, D=D, z=z, delta_bias=bias,
                                              delta_softplus=True, return_last_state=True)
    assert isinstance(out, np.ndarray) and out.dtype == np.float32
    assert rel_err(out, ref) <= 1e-4 and rel_err(last, ref_last) <= 1e-4
    with pytest.raises(_ffi.ArmScanError) as e:
        arm_scan.selective_scan_numpy(u, dl, A, B, C, backend="scalar")
    assert e.value.code == 3
    t = {k: torch.from_numpy(v).cuda() for k, v in
         dict(u=u, dl=dl, A=A, B=B, C=C, D=D, bias=bias).items()}
    got = scan_fn_arm(t["u"], t["dl"], t["A"], t["B"], t["C"], D=t["D"], delta_bias=t["bias"])
    ref2, _ = oracle.selective_scan(u, dl, A, B, C, D=D, delta_bias=bias, delta_softplus=True,
                                    dtype=np.float64)
    assert rel_err(host(got), ref2) <= 1e-4


CONV = [  # (batch, dim, len, width, bias, silu, time-major view)
    (2, 64, 300, 4, True, True, True),
    (1, 100, 70, 4, False, True, True),
    (3, 37, 5, 4, True, False, False),
    (1, 16, 1, 2, True, True, True),
    (2, 130, 257, 8, True, True, False),
    (1, 64, 64, 1, False, False, True),
]


@pytest.mark.parametrize("shape", CONV, ids=lambda s: "x".join(map(str, s)))
def test_causal_conv1d(shape):
    """The mixer's causal convolution against numpy's full convolution per row, on the
    HF mixer's layout (a (b, D, L) view of (b, L, 2D) storage) and on contiguous
    input; widths 1 .. 8, lengths shorter than the filter, ragged tiles."""
    import torch

    import armhackathon_amd as arm_scan
    from oracle import naive

    b, d, L, K, with_bias, act, tm = shape
    case(f"causal conv1d {shape}")
    rng = np.random.default_rng(43)
    x = rng.standard_normal((b, d, L)).astype(np.float32)
    w = rng.standard_normal((d, K)).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32) if with_bias else None
    ref = naive.causal_conv1d(x, w, bias, silu_act=act)
    if tm:
        store = torch.zeros((b, L, 2 * d), device="cuda")
        store[..., :d] = torch.from_numpy(x).cuda().transpose(1, 2)
        xt = store[..., :d].transpose(1, 2)
        assert not xt.is_contiguous() or L == 1  # one step: torch counts it contiguous
    else:
        xt = torch.from_numpy(x).cuda()
    out = arm_scan.causal_conv1d(xt, torch.from_numpy(w).cuda(),
                                 None if bias is None else torch.from_numpy(bias).cuda(),
                                 activation="silu" if act else None)
    assert out.is_contiguous() and out.shape == (b, d, L)
    assert rel_err(host(out), ref) <= 1e-5


@pytest.mark.parametrize("width", [4, 2, 1])
def test_causal_conv1d_update_token_by_token(width):
    """The decode step, run token by token from a zero state, gives the full causal
    convolution of the sequence (the oracle's), and leaves the last `width` inputs in
    the state; x read from a strided (b, D) view as the mixer passes it."""
    import torch

    import armhackathon_amd as arm_scan
    from oracle import naive

    b, d, L = 2, 40, 9
    case(f"causal conv1d update width {width}")
    rng = np.random.default_rng(47)
    x = rng.standard_normal((b, d, L)).astype(np.float32)
    w = rng.standard_normal((d, width)).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32)
    ref = naive.causal_conv1d(x, w, bias, silu_act=True)
    store = torch.zeros((b, L, 2 * d), device="cuda")
    store[..., d:] = torch.from_numpy(x).cuda().transpose(1, 2)
    state = torch.zeros((b, d, width), device="cuda")
    wt, bt = torch.from_numpy(w).cuda(), torch.from_numpy(bias).cuda()
    outs = []
    for t in range(L):
        xt = store[:, t, d:]  # (b, D) view, channels contiguous
        outs.append(host(arm_scan.causal_conv1d_update(xt, state, wt, bt, activation="silu")))
    got = np.stack(outs, axis=-1)
    assert rel_err(got, ref) <= 1e-5
    np.testing.assert_array_equal(host(state), x[:, :, L - width:])


@pytest.mark.parametrize("shape", [(2, 64, 512, False), (1, 32, 300, False), (2, 64, 512, True),
                                   (8, 1024, 512, True), (8, 1536, 2048, False),
                                   (1, 32, 300, True), (2, 48, 100, False), (2, 64, 1500, True),
                                   (8, 1024, 700, False), (8, 1024, 700, True)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("gate", [True, False], ids=["z", "noz"])
@pytest.mark.parametrize("utm", [True, False], ids=["utm", "ucont"])
def test_time_major_u(shape, gate, utm):
    """z and out views of time-major storage, and u one too (the HF mixer's convolution
    output laid out for its x_proj) or contiguous: bit-identical to the contiguous
    call. Time-major u goes through the block's LDS stage, with z or without it. Few
    rows take the segmented scan (its fold reads u by strides too); L 300, 1500 and 700
    end in a tail chunk, and L 100 is one, whose stage reads zeros past the row's end
    and stores only the steps inside it, forward and reverse."""
    import torch

    import armhackathon_amd as arm_scan

    b, d, L, rev = shape
    case(f"time-major inputs {shape} gate={gate} u tm={utm}")
    g = torch.Generator(device="cuda").manual_seed(5)
    f = dict(device="cuda", generator=g)
    u_tm = torch.randn(b, L, d, **f).transpose(1, 2)
    z_tm = torch.randn(b, L, 2 * d, **f)[..., d:].transpose(1, 2)
    dl = torch.randn(b, d, L, **f) * 0.5 - 3.0
    A = -torch.exp(torch.randn(d, 16, **f) * 0.5)
    B, C = torch.randn(b, 16, L, **f), torch.randn(b, 16, L, **f)
    D, bias = torch.randn(d, **f), torch.rand(d, **f) - 0.5
    kw = dict(D=D, delta_bias=bias, delta_softplus=True, return_last_state=True, reverse=rev)
    if not gate:
        z_tm = None
    u_in = u_tm if utm else u_tm.contiguous()
    got, last = arm_scan.selective_scan_time_major(u_in, dl, A, B, C, z=z_tm, **kw)
    want, wlast = arm_scan.selective_scan(u_tm.contiguous(), dl, A, B, C,
                                          z=None if z_tm is None else z_tm.contiguous(), **kw)
    assert torch.equal(got, want) and torch.equal(last, wlast)


@pytest.mark.parametrize("width,dim,length", [(4, 96, 300), (1, 30, 5), (8, 64, 3),
                                              (3, 130, 129), (2, 1536, 2048)])
def test_causal_conv1d_time_major_out(width, dim, length):
    """The convolution written as (b, L, D) storage, returned as a (b, D, L) view, has
    the bits of the contiguous output (itself checked against numpy above): a partial
    channel tile (96, 130), channels not in 16-byte pieces (30, 130), lengths shorter
    than the filter and than one tile."""
    import torch

    import armhackathon_amd as arm_scan

    case(f"causal conv1d time-major out K{width} D{dim} L{length}")
    g = torch.Generator(device="cuda").manual_seed(6 + width)
    store = torch.randn(2, length, 2 * dim, device="cuda", generator=g)
    x = store[..., :dim].transpose(1, 2)
    w = torch.randn(dim, width, device="cuda", generator=g)
    bias = torch.randn(dim, device="cuda", generator=g)
    for act in ("silu", None):
        a = arm_scan.causal_conv1d(x, w, bias, activation=act)
        t = arm_scan.causal_conv1d(x, w, bias, activation=act, time_major=True)
        assert t.stride() == (length * dim, 1, dim) and a.is_contiguous()
        assert torch.equal(a, t)


@pytest.mark.parametrize("reverse", [False, True])
def test_m1_broadcast_views(reverse):
    """Broadcast views of the gate (stride 0): through the op they are rerouted to the
    contiguous path; through the strided C entry point their zero strides are read as
    given (a broadcast), never as 'contiguous'. Both against the float64 oracle with
    the gate materialised."""
    import torch

    import armhackathon_amd as arm_scan
    from armhackathon_amd import _ffi

    b, d, L, n = 2, 32, 1024, 16
    x = workloads.m1_op(batch=b, dim=d, length=L, state=n, seed=21)
    t = dev(x)
    rng = np.random.default_rng(22)
    zc = rng.standard_normal((1, d, 1)).astype(np.float32)
    z_scalar = np.full((1, 1, 1), 0.7, np.float32)
    for name, small in (("per-channel", zc), ("scalar", z_scalar)):
        case(f"m1 broadcast gate {name} reverse={reverse}")
        zt = torch.from_numpy(small).cuda().expand(b, d, L)
        xm = dict(x, z=np.ascontiguousarray(np.broadcast_to(small, (b, d, L))))
        ref, ref_last = _ref(xm, reverse=reverse)
        out, last = arm_scan.selective_scan_time_major(
            t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"], z=zt,
            return_last_state=True, reverse=reverse)
        assert rel_err(host(out), ref) < TOL and rel_err(host(last), ref_last) < TOL
        out2 = torch.empty((b, d, L), device="cuda")
        last2 = torch.empty((b, d, n), device="cuda")
        _ffi.scan_strided_raw(_ffi.ArmScanDims(b, d, L, n, 1), t["u"].data_ptr(),
                              t["delta"].data_ptr(), t["A"].data_ptr(), t["B"].data_ptr(),
                              t["C"].data_ptr(), t["D"].data_ptr(), zt.data_ptr(), zt.stride(),
                              0, False, out2.data_ptr(), None, last2.data_ptr(), 0,
                              reverse=reverse,
                              stream=torch.cuda.current_stream().cuda_stream)
        assert rel_err(host(out2), ref) < TOL and rel_err(host(last2), ref_last) < TOL

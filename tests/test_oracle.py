"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so a plausible transcription mistake in oracle/cpu_ref.cpp
fails at least one of them:
  * the reference's own golden vectors, under the reference's own gates
    (golden.rs:15-19 / check_ffi.py:153-154,205-206 for Mamba-1,
    verify_golden_2d.py:36 for SS2D, verify_golden_mamba3.py:47-65 and
    check_mamba3_mimo_op.py:66 for Mamba-3);
  * hand-computed closed forms (scalar.rs:210-294, arm-scan-ffi/src/lib.rs:585-729);
  * independent float64 restatements (oracle/naive.py), including the O(L^2)
    dual form of Mamba-3 SISO, which has no state matrix at all;
  * the reference's invariants: reverse == flip->forward->flip (property.rs:138),
    fused bidirectional == two scans (property.rs:240), h0 streaming == one
    shot (property.rs:500), threads bit-identical (property.rs:453), rank-1 MIMO
    with no rotation == SISO (check_mamba3_mimo_op.py:89-122);
  * the ABI's rejection codes (arm-scan-ffi/src/lib.rs:53-58, :117-158, :461-487).
"""

import ctypes
import json

import numpy as np
import pytest

import oracle
from oracle import naive

BF16_EPS = 2.0 ** -8


def _npz(path):
    z = np.load(path)
    return {k: z[k] for k in z.files}


def _m1_cases(golden_dir):
    man = json.loads((golden_dir / "1d" / "manifest.json").read_text())
    return man


def _bf16(x):
    x = np.asarray(x, np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    # round to nearest even at bit 16
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    return rounded.astype(np.uint32).view(np.float32)


# ------------------------------------------------------------------ Mamba-1
def test_m1_goldens(golden_dir):
    """Every Mamba-1 golden: f64 oracle vs out_f64, f32 oracle under the gates."""
    man = _m1_cases(golden_dir)
    assert len(man) >= 15
    for m in man:
        z = _npz(golden_dir / "1d" / f"{m['name']}.npz")
        meta = json.loads(bytes(z["meta_json"]).decode())
        kw = dict(D=z.get("D_skip"), z=z.get("z"), delta_bias=z.get("delta_bias"),
                  delta_softplus=meta["delta_softplus"])
        o64, l64 = oracle.selective_scan(z["u"], z["delta"], z["A"], z["B"], z["C"],
                                         dtype=np.float64, **kw)
        np.testing.assert_allclose(o64, z["out_f64"], rtol=1e-9, atol=1e-12,
                                   err_msg=m["name"])
        np.testing.assert_allclose(l64, z["last_state_f64"], rtol=1e-9, atol=1e-12,
                                   err_msg=m["name"])
        o32, l32 = oracle.selective_scan(z["u"], z["delta"], z["A"], z["B"], z["C"], **kw)
        err = np.abs(o32 - z["out_f64"]).max()
        floor = float(m.get("f32_max_abs_err") or 0.0)
        assert err < 1e-4, (m["name"], err)
        if floor > 0:
            assert err < 50 * max(floor, 1e-7), (m["name"], err, floor)
        lrel = np.abs(l32 - z["last_state_f64"]).max() / max(
            np.abs(z["last_state_f64"]).max(), 1e-30)
        assert lrel < 1e-4, (m["name"], lrel)


def test_m1_naive_agrees(golden_dir):
    """C++ f64 oracle vs the independent numpy loop, incl. reverse, h0, groups."""
    rng = np.random.default_rng(0)
    b, d, L, n, g = 2, 6, 37, 5, 3
    u = rng.standard_normal((b, d, L))
    delta = rng.standard_normal((b, d, L)) * 0.5 - 3
    A = -np.exp(rng.uniform(-0.7, 2.7, (d, n)))
    B = rng.standard_normal((b, g, n, L))
    C = rng.standard_normal((b, g, n, L))
    D = rng.standard_normal(d)
    z = rng.standard_normal((b, d, L))
    bias = rng.uniform(-1, 1, d)
    h0 = rng.standard_normal((b, d, n))
    for rev in (False, True):
        for hh in (None, h0):
            o, l = oracle.selective_scan(u, delta, A, B, C, D=D, z=z, delta_bias=bias,
                                         delta_softplus=True, reverse=rev, h0=hh,
                                         dtype=np.float64)
            on, ln = naive.m1_scan(u, delta, A, B, C, D=D, z=z, delta_bias=bias,
                                   delta_softplus=True, reverse=rev, h0=hh)
            np.testing.assert_allclose(o, on, rtol=1e-11, atol=1e-12)
            np.testing.assert_allclose(l, ln, rtol=1e-11, atol=1e-12)


def test_m1_closed_forms():
    """scalar.rs:210-294 and arm-scan-ffi/src/lib.rs:585-729, hand-computed."""
    # single step with softplus, bias, D and z (f64, 1e-15)
    u, dt_raw, a, bb, c, ds, zz, bias = 0.7, -1.2, [-1.5, -4.0], [0.3, -0.8], [1.1, 0.4], \
        0.9, 0.25, 0.5
    out, last = oracle.selective_scan(
        [[[u]]], [[[dt_raw]]], [a], [[[bb[0]], [bb[1]]]], [[[c[0]], [c[1]]]], D=[ds],
        z=[[[zz]]], delta_bias=[bias], delta_softplus=True, dtype=np.float64)
    dt = np.log1p(np.exp(dt_raw + bias))
    h = [dt * u * bb[0], dt * u * bb[1]]
    expect = (c[0] * h[0] + c[1] * h[1] + ds * u) * (zz / (1 + np.exp(-zz)))
    assert abs(out[0, 0, 0] - expect) < 1e-15
    assert np.abs(last[0, 0] - h).max() < 1e-15
    # two steps: decay carries over
    u2, dt2, A2, B2, C2 = [1.0, 2.0], [0.1, 0.2], [[-2.0]], [[[1.0, 3.0]]], [[[1.0, 1.0]]]
    out, _ = oracle.selective_scan([[u2]], [[dt2]], A2, B2, C2, dtype=np.float64)
    h1 = 0.1 * 1.0 * 1.0
    h2 = np.exp(0.2 * -2.0) * h1 + 0.2 * 2.0 * 3.0
    assert abs(out[0, 0, 0] - h1) < 1e-15 and abs(out[0, 0, 1] - h2) < 1e-15
    # reverse: state starts at the END; output still lands at index t
    out, last = oracle.selective_scan([[u2]], [[dt2]], A2, B2, C2, reverse=True)
    b1 = np.float32(0.2) * np.float32(2.0) * np.float32(3.0)
    b0 = np.exp(np.float32(0.1) * np.float32(-2.0)) * b1 + np.float32(0.1)
    assert abs(out[0, 0, 1] - b1) < 1e-6 and abs(out[0, 0, 0] - b0) < 1e-6
    assert abs(last[0, 0, 0] - b0) < 1e-6
    # bidirectional = forward + that reverse
    of, ob, _, _ = oracle.selective_scan_bidirectional([[u2]], [[dt2]], A2, B2, C2)
    f0 = 0.1
    f1 = np.exp(0.2 * -2.0) * f0 + 0.2 * 2.0 * 3.0
    assert abs(of[0, 0, 0] - f0) < 1e-6 and abs(of[0, 0, 1] - f1) < 1e-6
    assert abs(ob[0, 0, 1] - b1) < 1e-6 and abs(ob[0, 0, 0] - b0) < 1e-6


def _m1_rand(seed, b=2, d=8, L=64, n=16, g=None):
    rng = np.random.default_rng(seed)
    f = np.float32
    bc = (b, g, n, L) if g else (b, n, L)
    return dict(
        u=rng.standard_normal((b, d, L)).astype(f),
        delta=(rng.standard_normal((b, d, L)) * 0.5).astype(f),
        A=(-np.exp(rng.uniform(-0.7, 2.7, (d, n)))).astype(f),
        B=rng.standard_normal(bc).astype(f), C=rng.standard_normal(bc).astype(f),
        D=rng.standard_normal(d).astype(f), z=rng.standard_normal((b, d, L)).astype(f),
        delta_bias=rng.uniform(-6, -3, d).astype(f))


def test_m1_invariants():
    x = _m1_rand(1)
    kw = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    args = (x["u"], x["delta"], x["A"], x["B"], x["C"])
    fwd, lf = oracle.selective_scan(*args, **kw)
    rev, lr = oracle.selective_scan(*args, reverse=True, **kw)
    fl = lambda t: np.ascontiguousarray(t[..., ::-1])  # noqa: E731
    frev, lfr = oracle.selective_scan(fl(x["u"]), fl(x["delta"]), x["A"], fl(x["B"]),
                                      fl(x["C"]), D=x["D"], z=fl(x["z"]),
                                      delta_bias=x["delta_bias"], delta_softplus=True)
    # reverse == flip -> forward -> flip, bit-exact on the scalar path
    assert np.array_equal(rev, fl(frev)) and np.array_equal(lr, lfr)
    assert not np.allclose(rev, fwd)
    # fused bidirectional == the two scans, bit-exact
    of, ob, lbf, lbb = oracle.selective_scan_bidirectional(*args, **kw)
    assert np.array_equal(of, fwd) and np.array_equal(ob, rev)
    assert np.array_equal(lbf, lf) and np.array_equal(lbb, lr)
    # streaming: prefix then suffix with h0 == one shot
    cut = 23
    p = lambda t, s: np.ascontiguousarray(t[..., s])  # noqa: E731
    o1, l1 = oracle.selective_scan(p(x["u"], slice(0, cut)), p(x["delta"], slice(0, cut)),
                                   x["A"], p(x["B"], slice(0, cut)), p(x["C"], slice(0, cut)),
                                   D=x["D"], z=p(x["z"], slice(0, cut)),
                                   delta_bias=x["delta_bias"], delta_softplus=True)
    o2, l2 = oracle.selective_scan(p(x["u"], slice(cut, None)), p(x["delta"], slice(cut, None)),
                                   x["A"], p(x["B"], slice(cut, None)),
                                   p(x["C"], slice(cut, None)), D=x["D"],
                                   z=p(x["z"], slice(cut, None)), delta_bias=x["delta_bias"],
                                   delta_softplus=True, h0=l1)
    assert np.array_equal(np.concatenate([o1, o2], -1), fwd) and np.array_equal(l2, lf)
    # threads: sequential == parallel, bit-identical
    seq, _ = oracle.selective_scan(*args, threading=1, **kw)
    par, _ = oracle.selective_scan(*args, threading=2, **kw)
    assert np.array_equal(seq, par)


def test_m1_error_codes():
    L = oracle.lib()
    assert L.arm_scan_abi_version() == 7
    x = np.zeros(64, np.float32)
    p = x.ctypes.data
    out = np.zeros(64, np.float32)
    f = L.arm_scan_selective_scan_f32

    def call(dims, u=p, backend=0, threading=0, last=None):
        return f(ctypes.byref(dims), u, p, p, p, p, None, None, None, 0, 0, backend,
                 threading, out.ctypes.data, last, None)

    ok = oracle.ArmScanDims(1, 2, 2, 2, 1)
    assert call(ok) == 0
    assert call(ok, u=None) == 1
    assert call(ok, backend=7) == 4 and call(ok, threading=-1) == 4
    assert call(oracle.ArmScanDims(0, 2, 2, 2, 1)) == 2
    assert call(oracle.ArmScanDims(1, 3, 2, 2, 2)) == 2  # groups does not divide dim
    assert call(oracle.ArmScanDims(2**40, 2**40, 2, 2, 1)) == 2  # overflow
    assert call(ok, backend=2) == 3  # neon is aarch64-only
    fb = L.arm_scan_selective_scan_bidirectional_f32
    rc = fb(ctypes.byref(ok), p, p, p, p, p, None, None, None, 0, 0, 0, out.ctypes.data,
            out.ctypes.data, out.ctypes.data, None)
    assert rc == 2  # half of the last-state pair


# ------------------------------------------------------------------ SS2D
def test_ss2d_goldens(golden_dir):
    """Four direction planes vs the reference's 2D goldens at its 1e-4 gate."""
    files = sorted((golden_dir / "2d").glob("*.npz"))
    assert len(files) == 6
    for f in files:
        z = _npz(f)
        B4 = np.stack([z["B"]] * 4)
        C4 = np.stack([z["C"]] * 4)
        names = ("out_row_fwd", "out_row_bwd", "out_col_fwd", "out_col_bwd")
        p64 = oracle.ss2d(z["u"], z["delta"], z["A"], B4, C4, D=z["D"],
                          delta_bias=z["delta_bias"], delta_softplus=True, dtype=np.float64)
        p32 = oracle.ss2d(z["u"], z["delta"], z["A"], B4, C4, D=z["D"],
                          delta_bias=z["delta_bias"], delta_softplus=True)
        for k, name in enumerate(names):
            np.testing.assert_allclose(p64[k], z[name], rtol=1e-9, atol=1e-12,
                                       err_msg=f"{f.name}:{name}")
            assert np.abs(p32[k] - z[name]).max() < 1e-4, (f.name, name)


# ------------------------------------------------------------------ Mamba-3
def _m3_load(path):
    z = _npz(path)
    kw = {k[3:]: v for k, v in z.items() if k.startswith("kw_")}
    return kw, z["out"]


def _ulps(got, gold):
    gold = np.asarray(gold, np.float64)
    scale = max(np.abs(gold).max(), 1e-30)
    return np.abs(_bf16(got).astype(np.float64) - gold).max() / (scale * BF16_EPS)


def _siso_args(kw, dtype=np.float64):
    half = kw["Q"].shape[-1] // 2
    cos, sin = oracle.angles_to_cos_sin(kw["Angles"], kw["DT"], half)
    return (kw["Q"], kw["K"], kw["V"], kw["ADT"], kw["DT"], kw["Trap"], kw["Q_bias"],
            kw["K_bias"], cos.astype(dtype), sin.astype(dtype))


def test_m3_siso_goldens(golden_dir):
    """Official Triton kernel captures, <= 8 bf16 ULP at tensor scale."""
    files = sorted((golden_dir / "mamba3").glob("*.npz"))
    assert len(files) == 9  # every capture the reference holds (_09 is missing upstream)
    for f in files:
        kw, gold = _m3_load(f)
        args = _siso_args(kw)
        for backend in (0, 1):  # tiled (x86 Auto) and naive (Scalar)
            out = oracle.mamba3_scan(*args, D=kw.get("D"), z=kw.get("Z"), backend=backend,
                                     dtype=np.float64)
            tm = out.transpose(0, 2, 1, 3)
            assert _ulps(tm, gold) <= 8.0, (f.name, backend, _ulps(tm, gold))


def _m3_rand(seed, b=2, L=19, h=4, dv=8, dqk=12, g=1, r=None):
    rng = np.random.default_rng(seed)
    qshape = (b, L, g, dqk) if r is None else (b, L, r, g, dqk)
    bshape = (h, dqk) if r is None else (h, r, dqk)
    dt = np.log1p(np.exp(rng.standard_normal((b, h, L)) - 2))
    A = -np.exp(rng.normal(0, 0.5, h))
    ang = rng.uniform(-np.pi, np.pi, (b, L, h, dqk // 2)) * dt.transpose(0, 2, 1)[..., None]
    theta = np.cumsum(ang, axis=1)
    x = dict(q=rng.standard_normal(qshape) / np.sqrt(dqk),
             k=rng.standard_normal(qshape) / np.sqrt(dqk),
             v=rng.standard_normal((b, L, h, dv)), adt=A[None, :, None] * dt, dt=dt,
             trap=rng.standard_normal((b, h, L)),
             q_bias=rng.standard_normal(bshape) * 0.1,
             k_bias=rng.standard_normal(bshape) * 0.1,
             cos=np.cos(theta), sin=np.sin(theta), D=rng.standard_normal(h),
             z=rng.standard_normal((b, L, h, dv)))
    if r is not None:
        x.update(psi=rng.standard_normal((h, r, dv)), zeta=rng.standard_normal((h, r, dv)),
                 phi=rng.standard_normal((h, r, dv)) * 0.5)
    return x


def test_m3_siso_independent_forms():
    """f64 oracle == sequential numpy (fwd + rev) == O(L^2) dual form, per-head groups."""
    for g in (1, 2, 4):
        x = _m3_rand(3, g=g)
        args = [x[k] for k in ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias",
                               "cos", "sin")]
        for rev in (False, True):
            out, S, bx = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], reverse=rev,
                                            dtype=np.float64, want_state=True)
            nv, Sn = naive.m3_siso_scan(*args, D=x["D"], z=x["z"], reverse=rev)
            np.testing.assert_allclose(out.transpose(0, 2, 1, 3), nv, rtol=1e-10, atol=1e-12)
            np.testing.assert_allclose(S, Sn, rtol=1e-10, atol=1e-12)
        dense = naive.m3_siso_dense(*args, D=x["D"], z=x["z"])
        out = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], dtype=np.float64)
        np.testing.assert_allclose(out.transpose(0, 2, 1, 3), dense, rtol=1e-9, atol=1e-11)


def test_m3_noncausal_forms():
    """Non-causal Mamba-3 (python/arm_scan/mamba3_noncausal.py:89-98, 101-178), pinned
    the way tests/check_mamba3_noncausal.py pins it, in float64:
    * the mask form restricted to its causal half == the forward scan;
    * the full mask form == forward + backward - same-step (the recurrent route,
      with the same-step term from unrotated q/k);
    * it differs from the causal scan once L > 1 and equals it at L = 1."""
    keys = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias", "cos", "sin")
    for seed, (b, L, h, dv, dqk, g) in enumerate(
            [(1, 8, 2, 4, 8, 1), (2, 19, 4, 8, 12, 2), (1, 33, 3, 6, 16, 1)]):
        x = _m3_rand(20 + seed, b=b, L=L, h=h, dv=dv, dqk=dqk, g=g)
        args = [x[k] for k in keys]
        fwd = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], dtype=np.float64)
        bwd = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], reverse=True, dtype=np.float64)
        fwd, bwd = fwd.transpose(0, 2, 1, 3), bwd.transpose(0, 2, 1, 3)
        causal = naive.m3_noncausal_dense(*args, D=x["D"], z=x["z"], causal=True)
        np.testing.assert_allclose(causal, fwd, rtol=1e-10, atol=1e-12)
        full = naive.m3_noncausal_dense(*args, D=x["D"], z=x["z"])
        diag = naive.m3_same_step(x["q"], x["k"], x["v"], x["dt"], x["trap"], x["q_bias"],
                                  x["k_bias"], D=x["D"], z=x["z"])
        np.testing.assert_allclose(full, fwd + bwd - diag, rtol=1e-10, atol=1e-12)
        assert np.abs(full - fwd).max() > 1e-3 * np.abs(fwd).max()
    x = _m3_rand(30, L=1)
    args = [x[k] for k in keys]
    np.testing.assert_allclose(naive.m3_noncausal_dense(*args, D=x["D"], z=x["z"]),
                               naive.m3_noncausal_dense(*args, D=x["D"], z=x["z"],
                                                        causal=True), rtol=0, atol=0)


def test_m3_groups_equal_per_head_slices():
    """groups=heads (extension) == running each head alone with the v7 layout."""
    x = _m3_rand(5, g=4, h=4)
    args = [x[k] for k in ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias",
                           "cos", "sin")]
    full = oracle.mamba3_scan(*args, D=x["D"], z=x["z"])
    for h in range(4):
        sl = oracle.mamba3_scan(
            x["q"][:, :, h:h + 1], x["k"][:, :, h:h + 1], x["v"][:, :, h:h + 1],
            x["adt"][:, h:h + 1], x["dt"][:, h:h + 1], x["trap"][:, h:h + 1],
            x["q_bias"][h:h + 1], x["k_bias"][h:h + 1], x["cos"][:, :, h:h + 1],
            x["sin"][:, :, h:h + 1], D=x["D"][h:h + 1], z=x["z"][:, :, h:h + 1])
        assert np.array_equal(full[:, h:h + 1], sl)


def test_m3_siso_reverse_is_flip():
    x = _m3_rand(7)
    args = [x[k] for k in ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias",
                           "cos", "sin")]
    rev = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], reverse=True, dtype=np.float64)
    f1 = lambda t: np.ascontiguousarray(t[:, ::-1])  # noqa: E731
    f2 = lambda t: np.ascontiguousarray(t[..., ::-1])  # noqa: E731
    fwd = oracle.mamba3_scan(f1(x["q"]), f1(x["k"]), f1(x["v"]), f2(x["adt"]), f2(x["dt"]),
                             f2(x["trap"]), x["q_bias"], x["k_bias"], f1(x["cos"]),
                             f1(x["sin"]), D=x["D"], z=f1(x["z"]), dtype=np.float64)
    np.testing.assert_allclose(rev, fwd[:, :, ::-1], rtol=1e-12, atol=1e-14)
    assert not np.allclose(rev, oracle.mamba3_scan(*args, D=x["D"], z=x["z"],
                                                   dtype=np.float64))


def test_m3_tiled_matches_naive_f32():
    x = _m3_rand(9, dqk=70, L=40)  # dqk not a multiple of TILE=32
    args = [x[k].astype(np.float32) for k in ("q", "k", "v", "adt", "dt", "trap", "q_bias",
                                               "k_bias", "cos", "sin")]
    a = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], backend=0)
    b = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], backend=1)
    assert np.abs(a - b).max() / np.abs(b).max() < 1e-5


def _mimo_args(kw):
    q = kw["Q"]
    half = q.shape[-1] // 2
    cos, sin = oracle.angles_to_cos_sin(kw["Angles"], kw["DT"], half)
    return (q, kw["K"], kw["V"], kw["ADT"], kw["DT"], kw["Trap"], kw["Q_bias"], kw["K_bias"],
            cos, sin)


def test_m3_mimo_goldens(golden_dir):
    """Official TileLang MIMO captures, <= 12 bf16 ULP (check_mamba3_mimo_op.py:66)."""
    files = sorted((golden_dir / "mamba3_mimo").glob("*.npz"))
    assert len(files) == 10
    for f in files:
        kw, gold = _m3_load(f)
        out = oracle.mamba3_scan(*_mimo_args(kw), D=kw.get("D"), z=kw.get("Z"),
                                 psi=kw["MIMO_V"], zeta=kw["MIMO_Z"], phi=kw["MIMO_Out"],
                                 dtype=np.float64)
        u = _ulps(out.transpose(0, 2, 1, 3), gold)
        assert u <= 12.0, (f.name, u)


def test_m3_mimo_independent_and_collapse():
    """f64 oracle == numpy MIMO loop (fwd, rev, final state); rank-1 unrotated == SISO."""
    x = _m3_rand(11, r=3, g=2)
    args = [x[k] for k in ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias",
                           "cos", "sin")]
    for rev in (False, True):
        out, S, bx = oracle.mamba3_scan(*args, D=x["D"], z=x["z"], psi=x["psi"],
                                        zeta=x["zeta"], phi=x["phi"], reverse=rev,
                                        dtype=np.float64, want_state=True)
        assert bx is None
        nv, Sn = naive.m3_mimo_scan(*args[:8], x["psi"], x["zeta"], x["phi"], x["cos"],
                                    x["sin"], D=x["D"], z=x["z"], reverse=rev)
        np.testing.assert_allclose(out.transpose(0, 2, 1, 3), nv, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(S, Sn, rtol=1e-10, atol=1e-12)
    # rank-1 with identity rotation == SISO, output and final state
    y = _m3_rand(13, r=1)
    ones = np.ones_like(y["psi"])
    cos1, sin0 = np.ones_like(y["cos"]), np.zeros_like(y["sin"])
    m_out, m_S, _ = oracle.mamba3_scan(y["q"], y["k"], y["v"], y["adt"], y["dt"], y["trap"],
                                       y["q_bias"], y["k_bias"], cos1, sin0, D=y["D"],
                                       z=y["z"], psi=ones, zeta=ones, phi=ones,
                                       dtype=np.float64, want_state=True)
    s_out, s_S, _ = oracle.mamba3_scan(y["q"][:, :, 0], y["k"][:, :, 0], y["v"], y["adt"],
                                       y["dt"], y["trap"], y["q_bias"][:, 0],
                                       y["k_bias"][:, 0], cos1, sin0, D=y["D"], z=y["z"],
                                       dtype=np.float64, want_state=True)
    assert np.abs(m_out - s_out).max() / np.abs(s_out).max() < 1e-12
    assert np.abs(m_S - s_S).max() / np.abs(s_S).max() < 1e-12


def test_m3_error_codes():
    L = oracle.lib()
    x = np.zeros(4096, np.float32)
    p = x.ctypes.data
    out_buf = np.zeros(4096, np.float32)  # keep the array alive while its pointer is used
    out = out_buf.ctypes.data
    f = L.arm_scan_mamba3_scan_f32

    def call(dims, psi=None, zeta=None, phi=None, ls=None, lb=None, backend=0, q=p):
        return f(ctypes.byref(dims), q, p, p, p, p, p, p, p, p, p, None, None,
                 psi, zeta, phi, 0, backend, 0, out, ls, lb)

    ok = oracle.ArmMamba3Dims(1, 2, 4, 4, 3, 1)
    assert call(ok) == 0
    assert call(ok, q=None) == 1
    assert call(ok, ls=out) == 1  # half a carry
    assert call(ok, psi=p) == 1  # partial projections
    assert call(ok, backend=9) == 4
    assert call(oracle.ArmMamba3Dims(1, 2, 4, 5, 3, 1)) == 2  # odd dqk
    assert call(oracle.ArmMamba3Dims(1, 2, 4, 4, 3, 0)) == 2  # rank 0
    assert call(oracle.ArmMamba3Dims(1, 2, 4, 4, 3, 2)) == 2  # rank>1 without MIMO
    assert call(oracle.ArmMamba3Dims(1, 2, 4, 4, 3, 2), psi=p, zeta=p, phi=p) == 0
    assert call(ok, psi=p, zeta=p, phi=p, ls=out, lb=out) == 2  # MIMO with a carry
    assert call(ok, backend=2) == 3
    # widened entry: MIMO final state allowed, groups must divide heads
    g = L.oracle_mamba3_scan_f32
    d = oracle.OracleMamba3Dims(1, 2, 4, 4, 3, 2, 2)
    assert g(ctypes.byref(d), p, p, p, p, p, p, p, p, p, p, None, None, p, p, p, 0, 0, 0,
             out, out, None) == 0
    d = oracle.OracleMamba3Dims(1, 3, 4, 4, 3, 1, 2)
    assert g(ctypes.byref(d), p, p, p, p, p, p, p, p, p, p, None, None, None, None, None,
             0, 0, 0, out, None, None) == 2

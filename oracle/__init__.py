"""TEST INFRASTRUCTURE — the CPU oracle for the selective-scan path.

This package is the checker, never the product: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` import it.
The HIP library under `armhackathon_amd/` never calls into it.

Two independent restatements of the reference (AdityaP9116/ARMHackathon)
live here:

* `libarm_scan_cpu.so` (built from `cpu_ref.cpp` by `Makefile`): a C++
  restatement of the reference's x86 Rust path — `scalar.rs`, `mamba3/tiled.rs`,
  `mamba3/scalar.rs`, `mamba3/mimo.rs`, the `arm-scan-ffi` validation and
  return codes — in f32 (the reference's own arithmetic) and f64. It exports
  the reference's four v7 C symbols, so the same ctypes signatures drive it.
  This module wraps it for numpy arrays.
* `naive.py`: pure-numpy float64 loops written from the mathematics, sharing
  no code with the C++ file, used to pin it.

Every function here is pinned by tests/test_oracle.py: the reference's golden
vectors (tests/golden/), closed forms and invariants, and `naive.py`.
"""

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libarm_scan_cpu.so"

ERROR_NAMES = {
    0: "ok",
    1: "null pointer",
    2: "invalid dims/shapes",
    3: "backend unavailable on this platform",
    4: "bad backend/threading enum",
    5: "panic inside kernel",
}


class ArmScanDims(ctypes.Structure):
    # arm-scan-ffi/src/lib.rs:43-50
    _fields_ = [(n, ctypes.c_size_t) for n in ("batch", "dim", "len", "state", "groups")]


class ArmMamba3Dims(ctypes.Structure):
    # arm-scan-ffi/src/lib.rs:362-373 (ABI 7)
    _fields_ = [(n, ctypes.c_size_t) for n in ("batch", "heads", "dv", "dqk", "len", "rank")]


class OracleMamba3Dims(ctypes.Structure):
    # ABI 7 struct + the `groups` extension
    _fields_ = [(n, ctypes.c_size_t)
                for n in ("batch", "heads", "dv", "dqk", "len", "rank", "groups")]


class OracleError(RuntimeError):
    def __init__(self, code):
        super().__init__(f"oracle error {code}: {ERROR_NAMES.get(code, 'unknown')}")
        self.code = code


_lib = None


def build(out=None):
    """Compile libarm_scan_cpu.so with the committed Makefile; with `out`, a fresh
    build (on this host's compiler) into that path instead of the package's copy."""
    cmd = ["make", "-s", "-C", str(HERE)]
    if out is not None:
        cmd += ["-B", f"LIB={out}"]
    subprocess.run(cmd, check=True)


def use(path):
    """Load the oracle from `path` (a build(out=path) library) from now on."""
    global LIB_PATH
    if _lib is not None and Path(path) != LIB_PATH:
        raise RuntimeError(f"the oracle is already loaded from {LIB_PATH}")
    LIB_PATH = Path(path)


def lib():
    """Load (once) the oracle library, building it first if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.is_file():
        build()
    L = ctypes.CDLL(str(LIB_PATH))
    vp, ci = ctypes.c_void_p, ctypes.c_int
    for suffix in ("f32", "f64"):
        f = getattr(L, f"arm_scan_selective_scan_{suffix}")
        f.restype = ci
        f.argtypes = [ctypes.POINTER(ArmScanDims)] + [vp] * 8 + [ci] * 4 + [vp] * 3
        f = getattr(L, f"arm_scan_selective_scan_bidirectional_{suffix}")
        f.restype = ci
        f.argtypes = [ctypes.POINTER(ArmScanDims)] + [vp] * 8 + [ci] * 3 + [vp] * 4
        f = getattr(L, f"arm_scan_mamba3_scan_{suffix}")
        f.restype = ci
        f.argtypes = [ctypes.POINTER(ArmMamba3Dims)] + [vp] * 15 + [ci] * 3 + [vp] * 3
        f = getattr(L, f"oracle_mamba3_scan_{suffix}")
        f.restype = ci
        f.argtypes = [ctypes.POINTER(OracleMamba3Dims)] + [vp] * 15 + [ci] * 3 + [vp] * 3
    L.arm_scan_abi_version.restype = ctypes.c_uint32
    L.oracle_set_threads.restype = ci
    L.oracle_set_threads.argtypes = [ci]
    _lib = L
    return L


def set_threads(n):
    """Set the OpenMP thread count (0 = leave as is). Returns the count in use."""
    return lib().oracle_set_threads(int(n))


def _arr(x, dtype):
    return None if x is None else np.ascontiguousarray(x, dtype=dtype)


def _p(a):
    return None if a is None else a.ctypes.data


def _sfx(dtype):
    return "f64" if np.dtype(dtype) == np.float64 else "f32"


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                   delta_softplus=False, reverse=False, h0=None,
                   dtype=np.float32, backend=0, threading=0):
    """Mamba-1 scan (scalar.rs:11-89). B/C (b,n,l) or (b,g,n,l).

    Returns (out, last_state) as arrays of `dtype`.
    """
    u = _arr(u, dtype)
    b, d, L = u.shape
    A = _arr(A, dtype)
    n = A.shape[1]
    B, C = _arr(B, dtype), _arr(C, dtype)
    g = B.shape[1] if B.ndim == 4 else 1
    out = np.empty((b, d, L), dtype)
    last = np.empty((b, d, n), dtype)
    arrs = [_arr(x, dtype) for x in (delta, D, z, delta_bias, h0)]
    dims = ArmScanDims(b, d, L, n, g)
    rc = getattr(lib(), f"arm_scan_selective_scan_{_sfx(dtype)}")(
        ctypes.byref(dims), _p(u), _p(arrs[0]), _p(A), _p(B), _p(C), _p(arrs[1]),
        _p(arrs[2]), _p(arrs[3]), int(bool(delta_softplus)), int(bool(reverse)),
        backend, threading, _p(out), _p(last), _p(arrs[4]))
    if rc:
        raise OracleError(rc)
    return out, last


def selective_scan_bidirectional(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                                 delta_softplus=False, dtype=np.float32,
                                 backend=0, threading=0):
    """Fused bidirectional scan (scalar.rs:114-201).

    Returns (out_fwd, out_bwd, last_fwd, last_bwd).
    """
    u = _arr(u, dtype)
    b, d, L = u.shape
    A = _arr(A, dtype)
    n = A.shape[1]
    B, C = _arr(B, dtype), _arr(C, dtype)
    g = B.shape[1] if B.ndim == 4 else 1
    of, ob = np.empty((b, d, L), dtype), np.empty((b, d, L), dtype)
    lf, lb = np.empty((b, d, n), dtype), np.empty((b, d, n), dtype)
    arrs = [_arr(x, dtype) for x in (delta, D, z, delta_bias)]
    dims = ArmScanDims(b, d, L, n, g)
    rc = getattr(lib(), f"arm_scan_selective_scan_bidirectional_{_sfx(dtype)}")(
        ctypes.byref(dims), _p(u), _p(arrs[0]), _p(A), _p(B), _p(C), _p(arrs[1]),
        _p(arrs[2]), _p(arrs[3]), int(bool(delta_softplus)), backend, threading,
        _p(of), _p(ob), _p(lf), _p(lb))
    if rc:
        raise OracleError(rc)
    return of, ob, lf, lb


def mamba3_scan(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D=None, z=None,
                psi=None, zeta=None, phi=None, reverse=False, dtype=np.float32,
                backend=0, threading=0, want_state=False):
    """Mamba-3 SISO/MIMO scan through the widened oracle entry point.

    q, k : (b, l, g, dqk) for SISO or (b, l, r, g, dqk) for MIMO, with g the
           groups axis (g = 1 is the reference layout, g = heads is per-head).
    v, z : (b, l, h, dv); adt, dt, trap : (b, h, l); cos, sin : (b, l, h, dqk/2)
    q_bias, k_bias : (h, dqk) SISO or (h, r, dqk) MIMO; psi/zeta/phi (h, r, dv)
    Returns out head-major (b, h, l, dv) [, last_state (b,h,dv,dqk),
    last_bx (b,h,dqk) (SISO only, else None)].
    """
    q, k, v = _arr(q, dtype), _arr(k, dtype), _arr(v, dtype)
    mimo = psi is not None
    if mimo:
        b, L, r, g, dqk = q.shape
    else:
        b, L, g, dqk = q.shape
        r = 1
    h, dv = v.shape[2], v.shape[3]
    out = np.empty((b, h, L, dv), dtype)
    ls = np.empty((b, h, dv, dqk), dtype) if want_state else None
    lbx = np.empty((b, h, dqk), dtype) if (want_state and not mimo) else None
    a = [_arr(x, dtype) for x in (adt, dt, trap, q_bias, k_bias, cos, sin, D, z,
                                   psi, zeta, phi)]
    dims = OracleMamba3Dims(b, h, dv, dqk, L, r, g)
    rc = getattr(lib(), f"oracle_mamba3_scan_{_sfx(dtype)}")(
        ctypes.byref(dims), _p(q), _p(k), _p(v), *[_p(x) for x in a],
        int(bool(reverse)), backend, threading, _p(out), _p(ls), _p(lbx))
    if rc:
        raise OracleError(rc)
    if want_state:
        return out, ls, lbx
    return out


def angles_to_cos_sin(angles, dt, half):
    """RoPE angle pre-pass in float64 (python/arm_scan/mamba3.py:41-89).

    angles (b, l, h, r), dt (b, h, l) -> cos, sin (b, l, h, half); pairs past r
    get the identity rotation (cos 1, sin 0).
    """
    angles = np.asarray(angles, np.float64)
    dt = np.asarray(dt, np.float64)
    r = angles.shape[-1]
    theta = np.cumsum(np.tanh(angles) * np.pi * dt.transpose(0, 2, 1)[..., None], axis=1)
    cos, sin = np.cos(theta), np.sin(theta)
    if r < half:
        pad = theta.shape[:-1] + (half - r,)
        cos = np.concatenate([cos, np.ones(pad)], axis=-1)
        sin = np.concatenate([sin, np.zeros(pad)], axis=-1)
    return cos, sin


def ss2d(u, delta, A, B4, C4, D=None, z=None, delta_bias=None, delta_softplus=False,
         dtype=np.float32, want_state=False):
    """Four-direction cross-scan with per-direction B/C, composed from 1D oracle scans.

    u, delta, z : (b, d, H, W); B4, C4 : (4, b, n, H, W) in grid layout, one
    per direction in the order (row_fwd, row_bwd, col_fwd, col_bwd). Row
    directions walk the row-major flattening, column directions the
    column-major one; the backward ones are the reverse index mode, exactly
    as python/arm_scan/ss2d.py:53-71 builds its views and bidirectional.py
    reverses them. Returns the four planes (4, b, d, H, W) and, with
    `want_state`, the four final states (4, b, d, n).
    """
    u = np.asarray(u)
    b, d, H, W = u.shape
    n = np.asarray(A).shape[1]

    def rows(t):
        return np.ascontiguousarray(t.reshape(t.shape[0], t.shape[1], H * W))

    def cols(t):
        return np.ascontiguousarray(
            np.swapaxes(t, 2, 3).reshape(t.shape[0], t.shape[1], W * H))

    planes = np.empty((4, b, d, H, W), dtype)
    lasts = np.empty((4, b, d, n), dtype)
    for k, (view, rev) in enumerate(((rows, False), (rows, True), (cols, False), (cols, True))):
        o, last = selective_scan(
            view(u), view(delta), A, view(np.asarray(B4[k])), view(np.asarray(C4[k])),
            D=D, z=None if z is None else view(z), delta_bias=delta_bias,
            delta_softplus=delta_softplus, reverse=rev, dtype=dtype)
        if view is rows:
            planes[k] = o.reshape(b, d, H, W)
        else:
            planes[k] = np.swapaxes(o.reshape(b, d, W, H), 2, 3)
        lasts[k] = last
    return (planes, lasts) if want_state else planes


__all__ = [
    "ArmScanDims", "ArmMamba3Dims", "OracleMamba3Dims", "OracleError", "lib", "build",
    "set_threads", "selective_scan", "selective_scan_bidirectional", "mamba3_scan",
    "angles_to_cos_sin", "ss2d", "LIB_PATH",
]

if os.environ.get("ORACLE_THREADS"):
    set_threads(int(os.environ["ORACLE_THREADS"]))

"""ctypes bindings to libarm_scan_hip.so, the MI355X scan engine's C ABI.

Mirrors the reference loader (python/arm_scan/_ffi.py:1-224): the same search
order idea, the same ABI-version check, the same argtypes and the same
error-code -> exception mapping. What differs is what ABI 9 differs in
(include/arm_scan_hip.h): every tensor pointer is a device pointer, every entry
point takes a trailing hipStream_t, ArmMamba3Dims carries `groups`, and there are
new entry points (the fused 2D scan, the time-major, strided, raw-angle and
non-causal Mamba-3 scans, the Mamba-3 mixer front-end, the strided Mamba-1 scan,
its decode step and the mixer's causal convolution); the header lists them.

Library search order:
  1. the ARM_SCAN_LIB environment variable (full path to the library);
  2. next to this package (where `make -C armhackathon_amd/csrc` writes it).

There is no other implementation to fall back to: if the library is absent,
`load()` raises OSError naming the paths it tried.
"""

import ctypes
import os
from pathlib import Path

ABI_VERSION = 9

LIB_NAME = "libarm_scan_hip.so"

# arm-scan-ffi/src/lib.rs:53-58, plus code 6 (HIP launch / device error).
ERROR_NAMES = {
    0: "ok",
    1: "null pointer",
    2: "invalid dims/shapes",
    3: "backend unavailable on this platform",
    4: "bad backend/threading enum",
    5: "panic inside kernel",
    6: "HIP launch/device error",
}

BACKENDS = {"auto": 0, "scalar": 1, "neon": 2}
THREADING = {"auto": 0, "sequential": 1, "seq": 1, "rayon": 2}
SS2D_MERGES = {"none": 0, "sum": 1, "mean": 2}


class ArmScanDims(ctypes.Structure):
    # arm-scan-ffi/src/lib.rs:43-50 (unchanged in ABI 9)
    _fields_ = [(n, ctypes.c_size_t) for n in ("batch", "dim", "len", "state", "groups")]


class ArmMamba3Dims(ctypes.Structure):
    # arm-scan-ffi/src/lib.rs:362-373 plus `groups` (ABI 9)
    _fields_ = [(n, ctypes.c_size_t)
                for n in ("batch", "heads", "dv", "dqk", "len", "rank", "groups")]


class ArmSS2DDims(ctypes.Structure):
    # ABI 9: the fused four-direction 2D scan
    _fields_ = [(n, ctypes.c_size_t) for n in ("batch", "dim", "height", "width", "state")]


class ArmScanError(RuntimeError):
    """A nonzero return code from the C ABI; `.code` holds it."""

    def __init__(self, fn, code, detail=""):
        msg = f"{fn} failed with code {code}: {ERROR_NAMES.get(code, 'unknown')}"
        if detail:
            msg += f" ({detail})"
        super().__init__(msg)
        self.code = code


def _candidate_paths():
    env = os.environ.get("ARM_SCAN_LIB")
    if env:
        yield Path(env)
    yield Path(__file__).resolve().parent / LIB_NAME


_lib = None
_lib_path = None

_vp, _ci = ctypes.c_void_p, ctypes.c_int


def _declare(lib):
    lib.arm_scan_abi_version.restype = ctypes.c_uint32
    lib.arm_scan_abi_version.argtypes = []
    lib.arm_scan_last_error.restype = ctypes.c_char_p
    lib.arm_scan_last_error.argtypes = []
    for f in (lib.arm_scan_selective_scan_f32, lib.arm_scan_selective_scan_noalloc_f32):
        f.restype = _ci
        f.argtypes = [ctypes.POINTER(ArmScanDims),
                      *([_vp] * 8),          # u delta a b c d_skip z delta_bias
                      _ci, _ci, _ci, _ci,    # delta_softplus reverse backend threading
                      _vp, _vp, _vp,         # out last_state h0
                      _vp]                   # stream
    f = lib.arm_scan_selective_scan_strided_f32
    f.restype = _ci
    f.argtypes = [ctypes.POINTER(ArmScanDims),
                  _vp, _vp,              # u u_strides
                  *([_vp] * 6),          # delta a b c d_skip z
                  _vp, _vp,              # z_strides delta_bias
                  _ci, _ci,              # delta_softplus reverse
                  _vp, _vp,              # out out_strides
                  _vp, _vp,              # last_state h0
                  _vp]                   # stream
    f = lib.arm_scan_selective_state_update_f32
    f.restype = _ci
    f.argtypes = [*([ctypes.c_size_t] * 3),      # batch dim state_dim
                  _vp, _vp, _vp, _vp, _vp,       # state x x_strides dt dt_strides
                  _vp, _vp, _vp, _vp, _vp,       # a b b_strides c c_strides
                  _vp, _vp, _vp, _vp,            # d_skip z z_strides dt_bias
                  _ci, _vp, _vp]                 # dt_softplus out stream
    f = lib.arm_scan_selective_scan_bidirectional_f32
    f.restype = _ci
    f.argtypes = [ctypes.POINTER(ArmScanDims),
                  *([_vp] * 8),          # u delta a b c d_skip z delta_bias
                  _ci, _ci, _ci,         # delta_softplus backend threading
                  _vp, _vp, _vp, _vp,    # out_fwd out_bwd last_fwd last_bwd
                  _vp]                   # stream
    for f in (lib.arm_scan_mamba3_scan_f32, lib.arm_scan_mamba3_scan_time_major_f32):
        f.restype = _ci
        f.argtypes = [ctypes.POINTER(ArmMamba3Dims),
                      *([_vp] * 15),     # q k v adt dt trap q_bias k_bias cos sin d_skip z
                                         # psi zeta phi
                      _ci, _ci, _ci,     # reverse backend threading
                      _vp, _vp, _vp,     # out last_state last_bx
                      _vp]               # stream
    f = lib.arm_scan_mamba3_scan_angles_f32
    f.restype = _ci
    f.argtypes = [ctypes.POINTER(ArmMamba3Dims),
                  *([_vp] * 9),          # q k v adt dt trap q_bias k_bias angles
                  ctypes.c_size_t,       # n_angles
                  *([_vp] * 5),          # d_skip z psi zeta phi
                  _ci, _ci,              # backend threading
                  _vp, _vp, _vp,         # out last_state last_bx
                  _vp]                   # stream
    f = lib.arm_scan_causal_conv1d_f32
    f.restype = _ci
    f.argtypes = [*([ctypes.c_size_t] * 4),   # batch dim len width
                  _vp, _vp, _vp, _vp,         # x x_strides weight bias
                  _ci, _ci, _vp, _vp]         # silu out_time_major out stream
    f = lib.arm_scan_causal_conv1d_update_f32
    f.restype = _ci
    f.argtypes = [*([ctypes.c_size_t] * 3),   # batch dim width
                  _vp, _vp, _vp, _vp, _vp,    # x x_strides conv_state weight bias
                  _ci, _vp, _vp]              # silu out stream
    f = lib.arm_scan_mamba3_scan_strided_f32
    f.restype = _ci
    f.argtypes = [ctypes.POINTER(ArmMamba3Dims),
                  _vp, _vp, _vp, _vp,    # q k v v_strides
                  *([_vp] * 5),          # adt dt trap q_bias k_bias
                  _vp, ctypes.c_size_t, _vp,   # angles n_angles angle_strides
                  _vp, _vp, _vp,         # d_skip z z_strides
                  _vp, _vp, _vp,         # psi zeta phi
                  _ci, _ci,              # backend threading
                  _vp, _vp]              # out stream
    f = lib.arm_scan_mamba3_block_frontend_f32
    f.restype = _ci
    f.argtypes = [_vp, *([ctypes.c_size_t] * 9),   # proj batch len row_stride heads
                                                   # headdim d_state rank groups n_angles
                  _vp, ctypes.c_float, _vp, _vp,   # dt_bias a_floor b_norm c_norm
                  ctypes.c_float,                  # norm_eps
                  *([_vp] * 5),                    # q k adt dt trap
                  _vp]                             # stream
    f = lib.arm_scan_mamba3_noncausal_f32
    f.restype = _ci
    f.argtypes = [ctypes.POINTER(ArmMamba3Dims),
                  *([_vp] * 12),         # q k v adt dt trap q_bias k_bias cos sin d_skip z
                  _ci, _ci,              # backend threading
                  _vp, _vp]              # out stream
    f = lib.arm_scan_mamba3_angles_f32
    f.restype = _ci
    f.argtypes = [_vp, _vp,                      # angles dt
                  *([ctypes.c_size_t] * 5),      # batch len heads n_angles half
                  _vp, _vp, _vp]                 # cos sin stream
    f = lib.arm_scan_ss2d_f32
    f.restype = _ci
    f.argtypes = [ctypes.POINTER(ArmSS2DDims),
                  *([_vp] * 8),          # u delta a b4 c4 d_skip z delta_bias
                  _ci, _ci,              # delta_softplus merge
                  _vp, _vp,              # out last_states
                  _vp]                   # stream


def load():
    """Load (once) and return the ctypes handle of libarm_scan_hip.so."""
    global _lib, _lib_path
    if _lib is not None:
        return _lib
    tried = []
    for path in _candidate_paths():
        tried.append(str(path))
        if path.is_file():
            lib = ctypes.CDLL(str(path))
            version = lib.arm_scan_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(
                    f"{path} has ABI version {version}, this package needs {ABI_VERSION}; "
                    "rebuild with `make -C armhackathon_amd/csrc`")
            _declare(lib)
            _lib, _lib_path = lib, path
            return lib
    raise OSError("libarm_scan_hip.so not found; build it with "
                  "`make -C armhackathon_amd/csrc` (searched: " + ", ".join(tried) + ")")


def lib_path():
    load()
    return _lib_path


def _check(fn, code):
    if code != 0:
        detail = load().arm_scan_last_error()
        raise ArmScanError(fn, code, detail.decode() if detail else "")


def _p(x):
    return x or None


def scan_raw(dims, ptr_u, ptr_delta, ptr_a, ptr_b, ptr_c, ptr_d_skip, ptr_z,
             ptr_delta_bias, delta_softplus, backend, threading, ptr_out, ptr_last,
             ptr_h0=0, *, reverse=False, stream=0):
    """Call arm_scan_selective_scan_f32. Pointers are integer device addresses
    (0 = null); `stream` is a hipStream_t handle (0 = the null stream).

    `reverse` is keyword-only for the reason the reference gives
    (python/arm_scan/_ffi.py:150-163): in C it sits mid-signature, so a
    positional slot would let a caller shift `backend` into it.
    """
    code = load().arm_scan_selective_scan_f32(
        ctypes.byref(dims), ptr_u, ptr_delta, ptr_a, ptr_b, ptr_c, _p(ptr_d_skip), _p(ptr_z),
        _p(ptr_delta_bias), int(bool(delta_softplus)), int(bool(reverse)),
        BACKENDS[backend], THREADING[threading], ptr_out, _p(ptr_last), _p(ptr_h0),
        _p(stream))
    _check("arm_scan_selective_scan_f32", code)


def scan_strided_raw(dims, ptr_u, ptr_delta, ptr_a, ptr_b, ptr_c, ptr_d_skip, ptr_z,
                     z_strides, ptr_delta_bias, delta_softplus, ptr_out, out_strides,
                     ptr_last=0, ptr_h0=0, *, reverse=False, stream=0, u_strides=None):
    """Call arm_scan_selective_scan_strided_f32: u, z and out given by element
    strides (batch, dim, step); None = contiguous (batch, dim, len)."""
    def arr(s):
        return None if s is None else (ctypes.c_longlong * 3)(*[int(x) for x in s])
    zs, os_, us = arr(z_strides), arr(out_strides), arr(u_strides)
    code = load().arm_scan_selective_scan_strided_f32(
        ctypes.byref(dims), ptr_u, us, ptr_delta, ptr_a, ptr_b, ptr_c, _p(ptr_d_skip), _p(ptr_z),
        zs, _p(ptr_delta_bias), int(bool(delta_softplus)), int(bool(reverse)), ptr_out, os_,
        _p(ptr_last), _p(ptr_h0), _p(stream))
    _check("arm_scan_selective_scan_strided_f32", code)


def state_update_raw(batch, dim, state_dim, ptr_state, ptr_x, x_strides, ptr_dt, dt_strides,
                     ptr_a, ptr_b, b_strides, ptr_c, c_strides, ptr_d_skip, ptr_z, z_strides,
                     ptr_dt_bias, dt_softplus, ptr_out, *, stream=0):
    """Call arm_scan_selective_state_update_f32 (one decode step, state in place);
    strides are pairs of element strides or None (contiguous)."""
    def arr(s):
        return None if s is None else (ctypes.c_longlong * 2)(*[int(v) for v in s])
    code = load().arm_scan_selective_state_update_f32(
        batch, dim, state_dim, ptr_state, ptr_x, arr(x_strides), ptr_dt, arr(dt_strides),
        ptr_a, ptr_b, arr(b_strides), ptr_c, arr(c_strides), _p(ptr_d_skip), _p(ptr_z),
        arr(z_strides), _p(ptr_dt_bias), int(bool(dt_softplus)), ptr_out, _p(stream))
    _check("arm_scan_selective_state_update_f32", code)


def scan_bidir_raw(dims, ptr_u, ptr_delta, ptr_a, ptr_b, ptr_c, ptr_d_skip, ptr_z,
                   ptr_delta_bias, delta_softplus, backend, threading, ptr_out_fwd,
                   ptr_out_bwd, ptr_last_fwd=0, ptr_last_bwd=0, *, stream=0):
    """Call arm_scan_selective_scan_bidirectional_f32 (both or neither last_*)."""
    code = load().arm_scan_selective_scan_bidirectional_f32(
        ctypes.byref(dims), ptr_u, ptr_delta, ptr_a, ptr_b, ptr_c, _p(ptr_d_skip), _p(ptr_z),
        _p(ptr_delta_bias), int(bool(delta_softplus)), BACKENDS[backend],
        THREADING[threading], ptr_out_fwd, ptr_out_bwd, _p(ptr_last_fwd), _p(ptr_last_bwd),
        _p(stream))
    _check("arm_scan_selective_scan_bidirectional_f32", code)


def mamba3_raw(dims, ptrs, reverse, backend, threading, ptr_out, ptr_last_state,
               ptr_last_bx, *, stream=0, time_major=False):
    """Call arm_scan_mamba3_scan_f32 (out head-major (b, h, l, dv)), or with
    time_major its (b, l, h, dv) twin, with the 15 input pointers in signature
    order: q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z, psi,
    zeta, phi (d_skip, z and the MIMO triple are nullable)."""
    if len(ptrs) != 15:
        raise ValueError(f"expected 15 input pointers, got {len(ptrs)}")
    name = "arm_scan_mamba3_scan_time_major_f32" if time_major else "arm_scan_mamba3_scan_f32"
    code = getattr(load(), name)(
        ctypes.byref(dims), *[_p(x) for x in ptrs], int(reverse), int(backend),
        int(threading), ptr_out, _p(ptr_last_state), _p(ptr_last_bx), _p(stream))
    _check(name, code)


def mamba3_angles_raw(dims, ptrs, n_angles, backend, threading, ptr_out, ptr_last_state,
                      ptr_last_bx, *, stream=0):
    """Call arm_scan_mamba3_scan_angles_f32 (forward, out (b, l, h, dv)) with the 14
    input pointers in signature order: q, k, v, adt, dt, trap, q_bias, k_bias,
    angles, d_skip, z, psi, zeta, phi (the last five nullable)."""
    if len(ptrs) != 14:
        raise ValueError(f"expected 14 input pointers, got {len(ptrs)}")
    name = "arm_scan_mamba3_scan_angles_f32"
    code = getattr(load(), name)(
        ctypes.byref(dims), *[_p(x) for x in ptrs[:9]], int(n_angles),
        *[_p(x) for x in ptrs[9:]], int(backend), int(threading), ptr_out,
        _p(ptr_last_state), _p(ptr_last_bx), _p(stream))
    _check(name, code)


def mamba3_noncausal_raw(dims, ptrs, backend, threading, ptr_out, *, stream=0):
    """Call arm_scan_mamba3_noncausal_f32 (SISO, out (b, l, h, dv)) with the 12 input
    pointers in signature order: q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin,
    d_skip, z (the last two nullable)."""
    if len(ptrs) != 12:
        raise ValueError(f"expected 12 input pointers, got {len(ptrs)}")
    name = "arm_scan_mamba3_noncausal_f32"
    code = getattr(load(), name)(ctypes.byref(dims), *[_p(x) for x in ptrs], int(backend),
                                 int(threading), ptr_out, _p(stream))
    _check(name, code)


def _i64x(vals):
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def mamba3_strided_raw(dims, ptrs, strides, n_angles, backend, threading, ptr_out, *,
                       stream=0):
    """Call arm_scan_mamba3_scan_strided_f32 (forward, from raw angles, out (b, l, h, dv)).
    ptrs: q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi, zeta, phi (the
    last five nullable); strides: dict with "v" (batch, step), "angles" (batch, step,
    head) and, with z, "z" (batch, step), in elements."""
    if len(ptrs) != 14:
        raise ValueError(f"expected 14 input pointers, got {len(ptrs)}")
    q, k, v, adt, dt, trap, qb, kb, ang, d_skip, z, psi, zeta, phi = ptrs
    vs, angs = _i64x(strides["v"]), _i64x(strides["angles"])
    zs = _i64x(strides["z"]) if z else None
    name = "arm_scan_mamba3_scan_strided_f32"
    code = getattr(load(), name)(
        ctypes.byref(dims), _p(q), _p(k), _p(v), vs, _p(adt), _p(dt), _p(trap), _p(qb), _p(kb),
        _p(ang), int(n_angles), angs, _p(d_skip), _p(z), zs, _p(psi), _p(zeta), _p(phi),
        int(backend), int(threading), ptr_out, _p(stream))
    _check(name, code)


def causal_conv1d_raw(batch, dim, length, width, ptr_x, x_strides, ptr_w, ptr_bias, silu,
                      ptr_out, *, stream=0, time_major=False):
    """Call arm_scan_causal_conv1d_f32 (x strides in elements: batch, dim, step; out
    (batch, dim, len) contiguous, or (batch, len, dim) storage with time_major)."""
    code = load().arm_scan_causal_conv1d_f32(batch, dim, length, width, ptr_x,
                                             _i64x(x_strides), ptr_w, _p(ptr_bias),
                                             int(bool(silu)), int(bool(time_major)), ptr_out,
                                             _p(stream))
    _check("arm_scan_causal_conv1d_f32", code)


def causal_conv1d_update_raw(batch, dim, width, ptr_x, x_strides, ptr_state, ptr_w, ptr_bias,
                             silu, ptr_out, *, stream=0):
    """Call arm_scan_causal_conv1d_update_f32 (x strides in elements: batch, dim)."""
    code = load().arm_scan_causal_conv1d_update_f32(batch, dim, width, ptr_x, _i64x(x_strides),
                                                    ptr_state, ptr_w, _p(ptr_bias),
                                                    int(bool(silu)), ptr_out, _p(stream))
    _check("arm_scan_causal_conv1d_update_f32", code)


def block_frontend_raw(ptr_proj, batch, length, row_stride, heads, headdim, d_state, rank,
                       groups, n_angles, ptr_dt_bias, a_floor, ptr_b_norm, ptr_c_norm,
                       norm_eps, ptr_q, ptr_k, ptr_adt, ptr_dt, ptr_trap, *, stream=0):
    """Call arm_scan_mamba3_block_frontend_f32 (the Mamba-3 mixer's front-end)."""
    code = load().arm_scan_mamba3_block_frontend_f32(
        ptr_proj, batch, length, row_stride, heads, headdim, d_state, rank, groups, n_angles,
        ptr_dt_bias, float(a_floor), ptr_b_norm, ptr_c_norm, float(norm_eps), ptr_q, ptr_k,
        ptr_adt, ptr_dt, ptr_trap, _p(stream))
    _check("arm_scan_mamba3_block_frontend_f32", code)


def angles_raw(ptr_angles, ptr_dt, batch, length, heads, n_angles, half, ptr_cos, ptr_sin,
               *, stream=0):
    """Call arm_scan_mamba3_angles_f32 (the RoPE angle pre-pass)."""
    code = load().arm_scan_mamba3_angles_f32(ptr_angles, ptr_dt, batch, length, heads,
                                             n_angles, half, ptr_cos, ptr_sin, _p(stream))
    _check("arm_scan_mamba3_angles_f32", code)


def ss2d_raw(dims, ptr_u, ptr_delta, ptr_a, ptr_b4, ptr_c4, ptr_d_skip, ptr_z,
             ptr_delta_bias, delta_softplus, merge, ptr_out, ptr_last_states=0, *, stream=0):
    """Call arm_scan_ss2d_f32 (merge: "none" | "sum" | "mean")."""
    code = load().arm_scan_ss2d_f32(
        ctypes.byref(dims), ptr_u, ptr_delta, ptr_a, ptr_b4, ptr_c4, _p(ptr_d_skip), _p(ptr_z),
        _p(ptr_delta_bias), int(bool(delta_softplus)), SS2D_MERGES[merge], ptr_out,
        _p(ptr_last_states), _p(stream))
    _check("arm_scan_ss2d_f32", code)

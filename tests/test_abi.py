"""The C ABI of libarm_scan_hip.so, host side only (no GPU needed).

* every function declared in include/arm_scan_hip.h is exported by the library;
* the ABI version is 9 and the loader checks it;
* the reference's rejection codes (arm-scan-ffi/src/lib.rs:53-58, :117-158,
  :461-487) come back before any launch: null pointers -> 1, bad dims -> 2,
  CPU backends -> 3, bad enums -> 4. These calls never touch the device, so
  the pointers they carry are never dereferenced.
"""

import ctypes
import re
from pathlib import Path

import pytest

from armhackathon_amd import _ffi

ROOT = Path(__file__).resolve().parents[1]
FAKE = 0x1000  # never dereferenced: every call below is rejected on the host


def _declared():
    text = (ROOT / "include" / "arm_scan_hip.h").read_text()
    return sorted(set(re.findall(r"^\S.*?\b(arm_scan_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported():
    lib = _ffi.load()
    names = _declared()
    assert "arm_scan_selective_scan_f32" in names and len(names) >= 6
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version():
    assert _ffi.load().arm_scan_abi_version() == 9 == _ffi.ABI_VERSION


def _m1(dims, u=FAKE, backend=0, threading=0, last=None, h0=None):
    L = _ffi.load()
    return L.arm_scan_selective_scan_f32(ctypes.byref(dims), u, FAKE, FAKE, FAKE, FAKE, None,
                                         None, None, 0, 0, backend, threading, FAKE, last, h0,
                                         None)


def test_m1_rejections():
    ok = _ffi.ArmScanDims(1, 2, 2, 2, 1)
    assert _m1(ok, u=None) == 1
    assert _m1(ok, backend=7) == 4 and _m1(ok, threading=-1) == 4
    assert _m1(ok, backend=1) == 3 and _m1(ok, backend=2) == 3
    assert _m1(_ffi.ArmScanDims(0, 2, 2, 2, 1)) == 2
    assert _m1(_ffi.ArmScanDims(1, 3, 2, 2, 2)) == 2
    assert _m1(_ffi.ArmScanDims(2 ** 40, 2 ** 40, 2, 2, 1)) == 2
    msg = _ffi.load().arm_scan_last_error().decode()
    assert "overflow" in msg
    L = _ffi.load()
    rc = L.arm_scan_selective_scan_bidirectional_f32(
        ctypes.byref(ok), FAKE, FAKE, FAKE, FAKE, FAKE, None, None, None, 0, 0, 0, FAKE, FAKE,
        FAKE, None, None)
    assert rc == 2  # half of the last-state pair
    rc = L.arm_scan_selective_scan_bidirectional_f32(
        ctypes.byref(ok), FAKE, FAKE, FAKE, FAKE, FAKE, None, None, None, 0, 0, 0, FAKE, None,
        None, None, None)
    assert rc == 1


def _m3(dims, psi=None, zeta=None, phi=None, ls=None, lb=None, backend=0, q=FAKE):
    L = _ffi.load()
    return L.arm_scan_mamba3_scan_f32(ctypes.byref(dims), q, FAKE, FAKE, FAKE, FAKE, FAKE,
                                      FAKE, FAKE, FAKE, FAKE, None, None, psi, zeta, phi, 0,
                                      backend, 0, FAKE, ls, lb, None)


def test_m3_rejections():
    D = _ffi.ArmMamba3Dims
    ok = D(1, 2, 4, 4, 3, 1, 1)
    assert _m3(ok, q=None) == 1
    assert _m3(ok, ls=FAKE) == 1           # half a carry
    assert _m3(ok, psi=FAKE) == 1          # partial projections
    assert _m3(ok, backend=9) == 4
    assert _m3(ok, backend=1) == 3
    assert _m3(D(1, 2, 4, 5, 3, 1, 1)) == 2            # odd dqk
    assert _m3(D(1, 2, 4, 4, 3, 0, 1)) == 2            # rank 0
    assert _m3(D(1, 2, 4, 4, 3, 2, 1)) == 2            # rank > 1 without MIMO
    assert _m3(D(1, 3, 4, 4, 3, 1, 2)) == 2            # groups must divide heads
    assert _m3(ok, psi=FAKE, zeta=FAKE, phi=FAKE, ls=FAKE, lb=FAKE) == 2  # MIMO last_bx


def test_m3_noncausal_rejections():
    L = _ffi.load()
    D = _ffi.ArmMamba3Dims

    def call(dims, q=FAKE):
        return L.arm_scan_mamba3_noncausal_f32(ctypes.byref(dims), q, FAKE, FAKE, FAKE, FAKE,
                                               FAKE, FAKE, FAKE, FAKE, FAKE, None, None, 0,
                                               0, FAKE, None)

    assert call(D(1, 2, 4, 4, 3, 2, 1)) == 2   # the non-causal sum is rank 1
    assert call(D(1, 2, 4, 4, 3, 1, 1), q=None) == 1
    assert call(D(1, 2, 4, 5, 3, 1, 1)) == 2   # odd dqk


def test_m3_strided_rejections():
    L = _ffi.load()
    D = _ffi.ArmMamba3Dims

    def call(vs=(64, 16), zs=(64, 16), ang=(64, 16, 4), z=None, angles=FAKE):
        arr = lambda t: (ctypes.c_int64 * len(t))(*t)  # noqa: E731
        return L.arm_scan_mamba3_scan_strided_f32(
            ctypes.byref(D(1, 2, 8, 8, 4, 1, 1)), FAKE, FAKE, FAKE, arr(vs), FAKE, FAKE, FAKE,
            FAKE, FAKE, angles, 4, arr(ang), None, z, arr(zs) if zs else None, None, None,
            None, 0, 0, FAKE, None)

    assert call(angles=None) == 1                   # raw angles are required
    assert call(z=FAKE, zs=None) == 1               # z without its strides
    assert call(vs=(-64, 16)) == 2                  # negative strides
    assert call(ang=(64, 16, -4)) == 2


def test_ss2d_rejections():
    L = _ffi.load()
    d = _ffi.ArmSS2DDims(1, 2, 3, 3, 4)

    def call(dims, u=FAKE, merge=1):
        return L.arm_scan_ss2d_f32(ctypes.byref(dims), u, FAKE, FAKE, FAKE, FAKE, None, None,
                                   None, 0, merge, FAKE, None, None)

    assert call(d, u=None) == 1
    assert call(d, merge=5) == 4
    assert call(_ffi.ArmSS2DDims(1, 2, 0, 3, 4)) == 2


def test_python_errors_carry_code():
    with pytest.raises(_ffi.ArmScanError) as e:
        _ffi.scan_raw(_ffi.ArmScanDims(1, 2, 2, 2, 1), FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0,
                      False, "scalar", "auto", FAKE, 0)
    assert e.value.code == 3 and "backend" in str(e.value)


def test_host_tensor_is_an_error():
    torch = pytest.importorskip("torch")
    import armhackathon_amd as arm_scan

    u = torch.zeros(1, 2, 8)
    with pytest.raises(ValueError, match="device tensors"):
        arm_scan.selective_scan(u, u, torch.zeros(2, 4), torch.zeros(1, 4, 8),
                                torch.zeros(1, 4, 8))


def test_last_error_is_per_thread():
    """arm_scan_last_error() explains the calling thread's most recent failure
    (the reference's call is reentrant across threads, arm-scan-ffi/src/lib.rs)."""
    import threading

    L = _ffi.load()
    seen = {}
    barrier = threading.Barrier(2)

    def worker(name, dims):
        rc = _m1(dims)
        barrier.wait()  # both threads have failed before either reads its message
        seen[name] = (rc, L.arm_scan_last_error().decode())

    t1 = threading.Thread(target=worker, args=("zero", _ffi.ArmScanDims(0, 2, 2, 2, 1)))
    t2 = threading.Thread(target=worker, args=("groups", _ffi.ArmScanDims(1, 3, 2, 2, 2)))
    t1.start(); t2.start(); t1.join(); t2.join()
    assert seen["zero"][0] == 2 and seen["groups"][0] == 2
    assert seen["zero"][1] != seen["groups"][1]
    assert "zero" in seen["zero"][1] and "groups" in seen["groups"][1]


def test_m1_strided_out_overlap_rejected():
    """A strided out whose (batch, dim, step) elements would share addresses is rejected
    before any launch (blocks writing one element would race): a zero stride on any
    dimension of more than one element, or a batch stride inside one batch's extent."""
    L = _ffi.load()
    b, d, n_len = 2, 16, 8

    def call(os):
        arr = (ctypes.c_longlong * 3)(*os)
        return L.arm_scan_selective_scan_strided_f32(
            ctypes.byref(_ffi.ArmScanDims(b, d, n_len, 4, 1)), FAKE, None, FAKE, FAKE, FAKE,
            FAKE, None, None, None, None, 0, 0, FAKE, arr, None, None, None)

    for os in ((0, n_len, 1), (d * n_len, 0, 1), (d * n_len, n_len, 0), (64, n_len, 1),
               (d * n_len, 4, 1), (d, 1, 8)):
        assert call(os) == 2, os
        assert "overlap" in L.arm_scan_last_error().decode()

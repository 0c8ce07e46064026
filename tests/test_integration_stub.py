"""The reference-side binding printed in the repository's integration notes, executed
(no GPU needed).

The python block under "The binding a maintainer would add to the reference" is what a
maintainer pastes into the reference's python/arm_scan/_ffi.py (:13-22, :41-63,
:83-141, :150-224). This test runs that block as a module against
libarm_scan_hip.so, so the document cannot drift from the library:

* the loader accepts the library's ABI version;
* each argtypes list has exactly the parameters include/arm_scan_hip.h declares;
* the struct mirrors have the header's fields, in order;
* host-rejected calls through scan_raw, scan_bidir_raw and mamba3_raw come back as
  the reference's codes (arm-scan-ffi/src/lib.rs:53-58). They are rejected before any
  launch, so the fake pointers they carry are never dereferenced.
"""

import ctypes
import re
import types
from pathlib import Path

import pytest

from armhackathon_amd import _ffi

ROOT = Path(__file__).resolve().parents[1]
FAKE = 0x1000


def _stub_source():
    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text.split("## The binding a maintainer would add to the reference", 1)[1]
    m = re.search(r"```python\n(.*?)```", sec, re.S)
    assert m, "no python block in the binding section"
    return m.group(1)


@pytest.fixture(scope="module")
def stub(monkeypatch_module):
    monkeypatch_module.setenv("ARM_SCAN_LIB", str(_ffi.lib_path()))
    mod = types.ModuleType("arm_scan_ffi_stub")
    mod.__file__ = str(ROOT / "INTEGRATION.md")
    exec(compile(_stub_source(), "INTEGRATION.md", "exec"), mod.__dict__)
    mod.load()
    return mod


@pytest.fixture(scope="module")
def monkeypatch_module():
    mp = pytest.MonkeyPatch()
    yield mp
    mp.undo()


def _header_params():
    """name -> number of parameters, from the declarations in the header."""
    text = (ROOT / "include" / "arm_scan_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(arm_scan_\w+)\s*\(([^)]*)\)\s*;", text, re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _header_struct(name):
    text = (ROOT / "include" / "arm_scan_hip.h").read_text()
    m = re.search(r"typedef struct %s \{(.*?)\}" % name, text, re.S)
    body = m.group(1).replace("size_t", "").replace(";", "")
    return [f.strip() for f in body.split(",")]


def test_stub_abi_matches_library(stub):
    assert stub.ABI_VERSION == stub.load().arm_scan_abi_version() == _ffi.ABI_VERSION


def test_stub_argtypes_match_header(stub):
    lib, decl = stub.load(), _header_params()
    for name in ("arm_scan_selective_scan_f32", "arm_scan_selective_scan_bidirectional_f32",
                 "arm_scan_mamba3_scan_f32"):
        assert len(getattr(lib, name).argtypes) == decl[name], name


def test_stub_structs_match_header(stub):
    for cls, name in ((stub.ArmScanDims, "ArmScanDims"), (stub.ArmMamba3Dims, "ArmMamba3Dims")):
        assert [f for f, _ in cls._fields_] == _header_struct(name)
        assert ctypes.sizeof(cls) == 8 * len(cls._fields_)


def _codes(fn):
    try:
        fn()
    except RuntimeError as e:
        return int(re.search(r"error (\d+)", str(e)).group(1)), str(e)
    raise AssertionError("the call was not rejected")


def test_stub_scan_raw_rejections(stub):
    zero = stub.ArmScanDims(0, 16, 8, 4, 1)
    ok = stub.ArmScanDims(1, 16, 8, 4, 1)
    call = lambda dims, backend="auto": stub.scan_raw(
        dims, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0, True, backend, "auto", FAKE, 0)
    code, msg = _codes(lambda: call(zero))
    assert code == 2 and "zero" in msg
    assert _codes(lambda: call(ok, backend="neon"))[0] == 3
    assert _codes(lambda: call(stub.ArmScanDims(1, 3, 8, 4, 2)))[0] == 2  # groups


def test_stub_bidir_raw_rejections(stub):
    ok = stub.ArmScanDims(1, 16, 8, 4, 1)
    code, msg = _codes(lambda: stub.scan_bidir_raw(
        ok, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0, False, "auto", "auto", FAKE, FAKE,
        FAKE, 0))
    assert code == 2 and "last_fwd" in msg
    assert _codes(lambda: stub.scan_bidir_raw(
        ok, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0, False, "scalar", "auto", FAKE, FAKE))[0] == 3


def test_stub_mamba3_raw_rejections(stub):
    odd = stub.ArmMamba3Dims(1, 2, 16, 15, 8, 1, 1)
    ptrs = [FAKE] * 10 + [None] * 5
    assert _codes(lambda: stub.mamba3_raw(odd, ptrs, 0, 0, 0, FAKE, None, None))[0] == 2
    ok = stub.ArmMamba3Dims(1, 2, 16, 16, 8, 1, 1)
    half_mimo = [FAKE] * 10 + [None, None, FAKE, None, None]
    assert _codes(lambda: stub.mamba3_raw(ok, half_mimo, 0, 0, 0, FAKE, None, None))[0] == 1
    assert _codes(lambda: stub.mamba3_raw(ok, ptrs, 0, 0, 5, FAKE, None, None))[0] == 4
    with pytest.raises(ValueError):
        stub.mamba3_raw(ok, ptrs[:14], 0, 0, 0, FAKE, None, None)

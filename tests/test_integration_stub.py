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
  launch. Where a GPU is present their pointers are real (small) device buffers, so a
  loosened check shows as a failed assertion, not as a kernel reading an unmapped
  address; without a GPU nothing can launch and a placeholder address stands in;
* on the GPU, successful calls through the same three functions on device tensors,
  against the float64 oracle, and the reference's 1d goldens replayed through
  scan_raw under its own gates, as the reference replays them through its ABI
  (tests/check_ffi.py:157-233).
"""

import ctypes
import re
import types
from pathlib import Path

import numpy as np
import pytest

import oracle
from armhackathon_amd import _ffi, workloads
from util import case, dev, host, rel_err

ROOT = Path(__file__).resolve().parents[1]


def _gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


_bufs = []


def _buf():
    """A pointer for a call the host must reject: a real 4 KiB device buffer when a GPU
    is present (nothing out of bounds happens even if a check were loosened), else a
    placeholder address (no GPU: nothing can launch)."""
    if not _gpu():
        return 0x1000
    import torch
    t = torch.zeros(1024, device="cuda")
    _bufs.append(t)
    return t.data_ptr()


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
    FAKE = _buf()
    zero = stub.ArmScanDims(0, 16, 8, 4, 1)
    ok = stub.ArmScanDims(1, 16, 8, 4, 1)
    call = lambda dims, backend="auto": stub.scan_raw(
        dims, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0, True, backend, "auto", FAKE, 0)
    code, msg = _codes(lambda: call(zero))
    assert code == 2 and "zero" in msg
    assert _codes(lambda: call(ok, backend="neon"))[0] == 3
    assert _codes(lambda: call(stub.ArmScanDims(1, 3, 8, 4, 2)))[0] == 2  # groups


def test_stub_bidir_raw_rejections(stub):
    FAKE = _buf()
    ok = stub.ArmScanDims(1, 16, 8, 4, 1)
    code, msg = _codes(lambda: stub.scan_bidir_raw(
        ok, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0, False, "auto", "auto", FAKE, FAKE,
        FAKE, 0))
    assert code == 2 and "last_fwd" in msg
    assert _codes(lambda: stub.scan_bidir_raw(
        ok, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 0, False, "scalar", "auto", FAKE, FAKE))[0] == 3


def test_stub_mamba3_raw_rejections(stub):
    FAKE = _buf()
    odd = stub.ArmMamba3Dims(1, 2, 16, 15, 8, 1, 1)
    ptrs = [FAKE] * 10 + [None] * 5
    assert _codes(lambda: stub.mamba3_raw(odd, ptrs, 0, 0, 0, FAKE, None, None))[0] == 2
    ok = stub.ArmMamba3Dims(1, 2, 16, 16, 8, 1, 1)
    half_mimo = [FAKE] * 10 + [None, None, FAKE, None, None]
    assert _codes(lambda: stub.mamba3_raw(ok, half_mimo, 0, 0, 0, FAKE, None, None))[0] == 1
    assert _codes(lambda: stub.mamba3_raw(ok, ptrs, 0, 0, 5, FAKE, None, None))[0] == 4
    with pytest.raises(ValueError):
        stub.mamba3_raw(ok, ptrs[:14], 0, 0, 0, FAKE, None, None)


# ---- successful calls on device tensors (GPU) ------------------------------------

def _p(t, k):
    return 0 if t.get(k) is None else t[k].data_ptr()


@pytest.mark.gpu
@pytest.mark.parametrize("reverse", [False, True])
def test_stub_scan_raw_on_device(stub, reverse):
    """scan_raw as the reference's op.py calls it (device pointers in place of host
    ones), with D, z, delta_bias, softplus and h0, against the float64 oracle."""
    import torch

    case(f"stub scan_raw 2x48x777 reverse={reverse}")
    x = workloads.m1_layer(batch=2, dim=48, length=777, state=16, seed=70)
    x["h0"] = np.random.default_rng(71).standard_normal((2, 48, 16)).astype(np.float32)
    t = dev(x)
    out = torch.full((2, 48, 777), float("nan"), device="cuda")
    last = torch.full((2, 48, 16), float("nan"), device="cuda")
    stub.scan_raw(stub.ArmScanDims(2, 48, 777, 16, 1), _p(t, "u"), _p(t, "delta"),
                  _p(t, "A"), _p(t, "B"), _p(t, "C"), _p(t, "D"), _p(t, "z"),
                  _p(t, "delta_bias"), True, "auto", "auto", out.data_ptr(),
                  last.data_ptr(), _p(t, "h0"), reverse=reverse)
    torch.cuda.synchronize()
    ref, ref_last = oracle.selective_scan(
        x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
        delta_bias=x["delta_bias"], delta_softplus=True, reverse=reverse, h0=x["h0"],
        dtype=np.float64)
    assert rel_err(host(out), ref) < 1e-4
    assert rel_err(host(last), ref_last) < 1e-4


@pytest.mark.gpu
def test_stub_scan_bidir_raw_on_device(stub):
    import torch

    case("stub scan_bidir_raw 1x32x1000")
    x = workloads.m1_op(batch=1, dim=32, length=1000, state=16, seed=72)
    t = dev(x)
    o = [torch.full((1, 32, 1000), float("nan"), device="cuda") for _ in range(2)]
    la = [torch.full((1, 32, 16), float("nan"), device="cuda") for _ in range(2)]
    stub.scan_bidir_raw(stub.ArmScanDims(1, 32, 1000, 16, 1), _p(t, "u"), _p(t, "delta"),
                        _p(t, "A"), _p(t, "B"), _p(t, "C"), _p(t, "D"), _p(t, "z"), 0,
                        False, "auto", "auto", o[0].data_ptr(), o[1].data_ptr(),
                        la[0].data_ptr(), la[1].data_ptr())
    torch.cuda.synchronize()
    ref = oracle.selective_scan_bidirectional(x["u"], x["delta"], x["A"], x["B"], x["C"],
                                              D=x["D"], z=x["z"], dtype=np.float64)
    for got, want in zip((*o, *la), ref):
        assert rel_err(host(got), want) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("reverse", [False, True])
def test_stub_mamba3_raw_on_device(stub, reverse):
    """mamba3_raw with the fifteen input pointers of the reference's order (q k v adt dt
    trap q_bias k_bias cos sin D z psi zeta phi), out head-major, last_state and
    last_bx, against the float64 oracle."""
    import torch

    case(f"stub mamba3_raw 2x100x3 dv16 dqk32 reverse={reverse}")
    x = workloads.m3_siso(batch=2, length=100, heads=3, dv=16, dqk=32, seed=73)
    rng = np.random.default_rng(74)
    x["D"] = rng.standard_normal(3).astype(np.float32)
    x["z"] = rng.standard_normal(x["v"].shape).astype(np.float32)
    t = dev(x)
    keys = ("q", "k", "v", "adt", "dt", "trap", "q_bias", "k_bias", "cos", "sin", "D", "z")
    ptrs = [_p(t, k) for k in keys] + [None, None, None]
    out = torch.full((2, 3, 100, 16), float("nan"), device="cuda")
    ls = torch.full((2, 3, 16, 32), float("nan"), device="cuda")
    lbx = torch.full((2, 3, 32), float("nan"), device="cuda")
    stub.mamba3_raw(stub.ArmMamba3Dims(2, 3, 16, 32, 100, 1, 3), ptrs, int(reverse), 0, 0,
                    out.data_ptr(), ls.data_ptr(), lbx.data_ptr())
    torch.cuda.synchronize()
    ref, rls, rlbx = oracle.mamba3_scan(*[x[k] for k in keys[:10]], D=x["D"], z=x["z"],
                                        reverse=reverse, dtype=np.float64, want_state=True)
    assert rel_err(host(out), ref) < 1e-4
    assert rel_err(host(ls), rls) < 1e-4
    assert rel_err(host(lbx), rlbx) < 1e-4


@pytest.mark.gpu
def test_stub_replays_reference_goldens(stub, golden_dir):
    """Every 1d golden through scan_raw under the reference's gates (check_ffi.py:
    153-154, 205-206): max |out - out_f64| < 1e-4, last_state relative < 1e-4."""
    import json

    import torch

    man = json.loads((golden_dir / "1d" / "manifest.json").read_text())
    for m in man:
        case(f"stub golden {m['name']}")
        z = np.load(golden_dir / "1d" / f"{m['name']}.npz")
        meta = json.loads(bytes(z["meta_json"]).decode())
        x = {k: z[k].astype(np.float32) for k in ("u", "delta", "A", "B", "C")}
        for k, name in (("D", "D_skip"), ("z", "z"), ("delta_bias", "delta_bias")):
            if name in z.files:
                x[k] = z[name].astype(np.float32)
        b, d, L = x["u"].shape
        n = x["A"].shape[1]
        g = x["B"].shape[1] if x["B"].ndim == 4 else 1
        t = dev(x)
        out = torch.full((b, d, L), float("nan"), device="cuda")
        last = torch.full((b, d, n), float("nan"), device="cuda")
        stub.scan_raw(stub.ArmScanDims(b, d, L, n, g), _p(t, "u"), _p(t, "delta"),
                      _p(t, "A"), _p(t, "B"), _p(t, "C"), _p(t, "D"), _p(t, "z"),
                      _p(t, "delta_bias"), meta["delta_softplus"], "auto", "auto",
                      out.data_ptr(), last.data_ptr())
        torch.cuda.synchronize()
        assert np.abs(host(out) - z["out_f64"]).max() < 1e-4, m["name"]
        assert rel_err(host(last), z["last_state_f64"]) < 1e-4, m["name"]

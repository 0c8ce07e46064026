"""NumPy front-end (python/arm_scan/numpy_api.py:16-70): numpy arrays in and
out, the scan itself on the GPU.

The arrays are copied host -> HBM, scanned by the HIP kernels, and the result
copied back, so this entry point pays PCIe both ways; device-resident callers
use `selective_scan` on torch tensors instead.
"""

import numpy as np


def _prep(x, name, shape=None):
    arr = np.ascontiguousarray(x, dtype=np.float32)
    if shape is not None and arr.shape != shape:
        raise ValueError(f"{name}: expected shape {shape}, got {arr.shape}")
    return arr


def selective_scan_numpy(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                         delta_softplus=False, return_last_state=False,
                         backend="auto", threading="auto", initial_state=None,
                         reverse=False, device="cuda"):
    """Selective scan on numpy arrays; same layouts as `selective_scan`.

    `backend`/`threading` keep the reference's signature: "auto" is the HIP
    kernel; the reference's CPU backends ("scalar", "neon") are rejected by the
    library with code 3 (backend unavailable).
    """
    import torch

    from . import _ffi
    from .op import _CALLS, _check_m1

    u = _prep(u, "u")
    if u.ndim != 3:
        raise ValueError(f"u must be (batch, dim, len), got {u.shape}")
    batch, dim, length = u.shape
    delta = _prep(delta, "delta", (batch, dim, length))
    A = _prep(A, "A")
    if A.ndim != 2 or A.shape[0] != dim:
        raise ValueError(f"A must be ({dim}, state), got {A.shape}")
    state = A.shape[1]
    B, C = _prep(B, "B"), _prep(C, "C")
    if B.ndim == 3:
        B = B.reshape(batch, 1, state, length)
    if C.ndim == 3:
        C = C.reshape(batch, 1, state, length)
    D = None if D is None else _prep(D, "D", (dim,))
    z = None if z is None else _prep(z, "z", (batch, dim, length))
    delta_bias = None if delta_bias is None else _prep(delta_bias, "delta_bias", (dim,))
    h0 = None if initial_state is None else _prep(initial_state, "initial_state",
                                                  (batch, dim, state))
    dev = torch.device(device)
    t = {k: None if v is None else torch.from_numpy(v).to(dev)
         for k, v in dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, bias=delta_bias,
                          h0=h0).items()}
    _, _, _, _, groups = _check_m1(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"],
                                   t["z"], t["bias"], t["h0"])
    out = torch.empty_like(t["u"])
    last = t["u"].new_empty((batch, dim, state))
    p = {k: 0 if v is None else v.data_ptr() for k, v in t.items()}
    dims = _ffi.ArmScanDims(batch, dim, length, state, groups)
    with torch.cuda.device(dev):
        _ffi.scan_raw(dims, p["u"], p["delta"], p["A"], p["B"], p["C"], p["D"], p["z"],
                      p["bias"], delta_softplus, backend, threading, out.data_ptr(),
                      last.data_ptr(), ptr_h0=p["h0"], reverse=reverse,
                      stream=torch.cuda.current_stream(dev).cuda_stream)
    _CALLS["n"] += 1
    out_np, last_np = out.cpu().numpy(), last.cpu().numpy()
    return (out_np, last_np) if return_last_state else out_np

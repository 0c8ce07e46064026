"""NumPy front-end (python/arm_scan/numpy_api.py:16-70): numpy arrays in and
out, the scan itself on the GPU.

The arrays are copied host -> HBM, scanned by the HIP kernels, and the result
copied back, so this entry point pays PCIe both ways; device-resident callers
use `selective_scan` on torch tensors instead.
"""

import numpy as np


def selective_scan_numpy(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                         delta_softplus=False, return_last_state=False,
                         backend="auto", threading="auto", initial_state=None,
                         reverse=False, device="cuda"):
    """Selective scan on numpy arrays; same layouts as `selective_scan`.

    B and C may be 3-D (batch, state, len), one group. Shapes are checked once,
    by the torch ops' own `_check_m1`, after the float32 copies reach the device.
    `backend`/`threading` keep the reference's signature: "auto" is the HIP
    kernel; the reference's CPU backends ("scalar", "neon") are rejected by the
    library with code 3 (backend unavailable).
    """
    import torch

    from . import _ffi
    from .op import _CALLS, _check_m1

    dev = torch.device(device)
    arrays = dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, bias=delta_bias,
                  h0=initial_state)
    t = {name: None if x is None
         else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)
         for name, x in arrays.items()}
    for name in ("B", "C"):
        if t[name].dim() == 3:
            t[name] = t[name].unsqueeze(1)
    batch, dim, length, state, groups = _check_m1(
        t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["z"], t["bias"], t["h0"])
    out = torch.empty_like(t["u"])
    last = t["u"].new_empty((batch, dim, state))
    ptr = {name: 0 if x is None else x.data_ptr() for name, x in t.items()}
    with torch.cuda.device(dev):
        _ffi.scan_raw(_ffi.ArmScanDims(batch, dim, length, state, groups), ptr["u"],
                      ptr["delta"], ptr["A"], ptr["B"], ptr["C"], ptr["D"], ptr["z"],
                      ptr["bias"], delta_softplus, backend, threading, out.data_ptr(),
                      last.data_ptr(), ptr_h0=ptr["h0"], reverse=reverse,
                      stream=torch.cuda.current_stream(dev).cuda_stream)
    _CALLS["n"] += 1
    out_np, last_np = out.cpu().numpy(), last.cpu().numpy()
    return (out_np, last_np) if return_last_state else out_np

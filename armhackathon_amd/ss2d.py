"""SS2D -- the four-direction 2D cross-scan on the HIP engine
(python/arm_scan/ss2d.py:1-202 is the reference front end).

Directions, in the reference's order: row_fwd, row_bwd (the row-major
flattening t = i*W + j walked forward / backward) and col_fwd, col_bwd (the
column-major flattening t = j*H + i). Backward is the kernel's reverse index
mode, never a flip. D and z apply inside every direction, so a "sum" merge
carries 4*D*u, exactly as the reference (ss2d.py:125-129).

`ss2d_scan` goes through the fused entry point arm_scan_ss2d_f32, which takes
one B and one C per direction in grid layout; the reference's shared B/C is
the special case where the four are the same tensor. Grouped B/C
((b, g, n, h, w), g > 1) and the `scan_pair=` seam run the reference's
view-based composition over the bidirectional scan instead.
"""

import torch

from . import _ffi
from .op import _CALLS, _c, _device_of, _ptr, _stream

_MERGES = ("sum", "mean", "none")


def grid_to_views(t):
    """(b, c, h, w) -> (2b, c, h*w): row-major stacked over column-major
    (python/arm_scan/ss2d.py:53-63)."""
    b, c, h, w = t.shape
    rows = t.reshape(b, c, h * w)
    cols = t.transpose(2, 3).reshape(b, c, w * h)
    return torch.cat((rows, cols), dim=0)


def views_to_grid(row_seq, col_seq, h, w):
    """Inverse of the grid_to_views halves, back to (b, c, h, w)."""
    b, c, _ = row_seq.shape
    rows = row_seq.reshape(b, c, h, w)
    cols = col_seq.reshape(b, c, w, h).transpose(2, 3)
    return rows, cols


def scan_pair_arm(u, delta, A, B, C, D=None, delta_bias=None, delta_softplus=True):
    """(fwd, bwd) of one ordering from the fused bidirectional scan."""
    from .bidirectional import bidirectional_scan
    return bidirectional_scan(u, delta, A, B, C, D=D, delta_bias=delta_bias,
                              delta_softplus=delta_softplus, merge="none")


def scan_fn_arm(u, delta, A, B, C, D=None, delta_bias=None, delta_softplus=True):
    """Single-direction 1D scan (the reference's legacy seam)."""
    from .op import selective_scan
    return selective_scan(u, delta, A, B, C, D=D, delta_bias=delta_bias,
                          delta_softplus=delta_softplus)


def _ss2d_views(u, delta, A, B, C, D, delta_bias, delta_softplus, merge, scan_pair):
    b, _, h, w = u.shape

    def views(t):
        if t.dim() == 5:
            bb, g, n, hh, ww = t.shape
            v = grid_to_views(t.reshape(bb, g * n, hh, ww))
            return v.reshape(2 * bb, g, n, hh * ww)
        return grid_to_views(t)

    fwd, bwd = scan_pair(grid_to_views(u), grid_to_views(delta), A, views(B), views(C), D=D,
                         delta_bias=delta_bias, delta_softplus=delta_softplus)
    row_f, col_f = views_to_grid(fwd[:b], fwd[b:], h, w)
    row_b, col_b = views_to_grid(bwd[:b], bwd[b:], h, w)
    if merge == "none":
        return row_f, row_b, col_f, col_b
    out = row_f + row_b + col_f + col_b
    return out if merge == "sum" else out * 0.25


def ss2d_scan(u, delta, A, B, C, D=None, delta_bias=None, delta_softplus=True,
              merge="sum", scan_pair=None, z=None, return_last_state=False,
              per_direction=False):
    """Four-direction 2D cross-scan over a token grid.

    u, delta, z : (b, d, h, w);  A : (d, n);  D, delta_bias : (d,)
    B, C        : (b, n, h, w) shared by the four directions (the reference's
                  layout) or (b, g, n, h, w) grouped; with per_direction=True,
                  (4, b, n, h, w) -- one per direction, in the order
                  (row_fwd, row_bwd, col_fwd, col_bwd).
    merge       : "sum" | "mean" | "none" (the four planes, each (b, d, h, w)).
    z           : optional gate, applied as out * silu(z) inside every direction.
    return_last_state : also return the four final states (4, b, d, n).
    """
    if merge not in _MERGES:
        raise ValueError(f"merge must be one of {_MERGES}, got {merge!r}")
    if u.dim() != 4:
        raise ValueError(f"u must be (b, d, h, w), got {tuple(u.shape)}")
    if delta.shape != u.shape:
        raise ValueError(f"delta {tuple(delta.shape)} must match u {tuple(u.shape)}")
    b, d, h, w = u.shape
    per_dir = bool(per_direction)
    if per_dir and (B.dim() != 5 or B.shape[0] != 4 or C.shape != B.shape):
        raise ValueError(f"per_direction B/C must be (4, b, n, h, w), got {tuple(B.shape)}")
    grouped = B.dim() == 5 and not per_dir
    if scan_pair is not None or (grouped and B.shape[1] != 1):
        if z is not None or return_last_state or per_dir:
            raise ValueError("z, return_last_state and per-direction B/C need the fused "
                             "kernel (no scan_pair, ungrouped B/C)")
        return _ss2d_views(u, delta, A, B, C, D, delta_bias, delta_softplus, merge,
                           scan_pair or scan_pair_arm)
    if grouped:  # (b, 1, n, h, w)
        B, C = B[:, 0], C[:, 0]
    for name, t in (("B", B), ("C", C)):
        grid = t.shape[-2:]
        if tuple(grid) != (h, w) or t.shape[-4 if per_dir else 0] != b:
            raise ValueError(f"{name} must be (b={b}, n, {h}, {w}) or (4, b, n, {h}, {w}), "
                             f"got {tuple(t.shape)}")
    n = A.shape[1]
    if A.dim() != 2 or A.shape[0] != d:
        raise ValueError(f"A must be ({d}, n), got {tuple(A.shape)}")
    if not per_dir:
        B = B.unsqueeze(0).expand(4, b, n, h, w)
        C = C.unsqueeze(0).expand(4, b, n, h, w)
    for name, t, want in (("B4", B, (4, b, n, h, w)), ("C4", C, (4, b, n, h, w)),
                          ("D", D, (d,)), ("delta_bias", delta_bias, (d,)),
                          ("z", z, (b, d, h, w))):
        if t is not None and tuple(t.shape) != want:
            raise ValueError(f"{name} must be {want}, got {tuple(t.shape)}")
    dev = _device_of(u, delta, A, B, C, D, z, delta_bias)
    u, delta, A, B, C = _c(u), _c(delta), _c(A), _c(B), _c(C)
    D = None if D is None else _c(D)
    z = None if z is None else _c(z)
    delta_bias = None if delta_bias is None else _c(delta_bias)
    out = torch.empty((4, b, d, h, w) if merge == "none" else (b, d, h, w),
                      dtype=torch.float32, device=dev)
    last = torch.empty((4, b, d, n), dtype=torch.float32, device=dev) \
        if return_last_state else None
    dims = _ffi.ArmSS2DDims(b, d, h, w, n)
    with torch.cuda.device(dev):
        _ffi.ss2d_raw(dims, u.data_ptr(), delta.data_ptr(), A.data_ptr(), B.data_ptr(),
                      C.data_ptr(), _ptr(D), _ptr(z), _ptr(delta_bias), delta_softplus, merge,
                      out.data_ptr(), _ptr(last), stream=_stream(dev))
    _CALLS["n"] += 1
    res = tuple(out.unbind(0)) if merge == "none" else out
    return (res, last) if return_last_state else res


def use_arm_scan(module, enable=True):
    """Swap the scan implementation on every SS2D block in `module`
    (python/arm_scan/ss2d.py:170-202): blocks exposing `scan_pair_fn` get
    `scan_pair_arm`, blocks exposing `scan_fn` get `scan_fn_arm`. The previous
    functions are remembered on the module and put back by enable=False.
    Returns the number of blocks switched."""
    n = 0
    for m in module.modules():
        touched = False
        for attr, fn in (("scan_pair_fn", scan_pair_arm), ("scan_fn", scan_fn_arm)):
            if not hasattr(m, attr):
                continue
            saved = f"_arm_scan_saved_{attr}"
            if enable:
                if not hasattr(m, saved):
                    setattr(m, saved, getattr(m, attr))
                setattr(m, attr, fn)
            elif hasattr(m, saved):
                setattr(m, attr, getattr(m, saved))
                delattr(m, saved)
            touched = True
        n += int(touched)
    return n

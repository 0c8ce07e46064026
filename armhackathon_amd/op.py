"""PyTorch front-end: `torch.library` custom ops over the HIP scan engine.

Registered under the reference's names (python/arm_scan/op.py:23,103):
`arm_scan::selective_scan` and `arm_scan::selective_scan_bidirectional`, each
with a fake (meta) kernel so they trace under `torch.compile`.

What changes from the reference is where the tensors live: inputs are
PyTorch-ROCm device tensors, the kernels are enqueued on the current stream of
the tensors' device, and the call returns without synchronising. A host tensor
is an error, not a cue to fall back: this package has no CPU implementation.

Inference-only, like the reference: no autograd formula is registered.
"""

from typing import Optional, Tuple

import torch

from . import _ffi

_CALLS = {"n": 0}


def _c(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().float()


def _ptr(t):
    return 0 if t is None else t.data_ptr()


def _device_of(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                "arm_scan on MI355X takes device tensors (got a tensor on "
                f"{t.device}); move inputs with .to('cuda') first")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _check_m1(u, delta, a, b, c, d_skip, z, delta_bias, h0):
    """Shape checks for the Mamba-1 ops: the C side trusts element counts
    (arm-scan-ffi/src/lib.rs:92-96), so shape safety is owned here."""
    if u.dim() != 3:
        raise ValueError(f"u must be (batch, dim, len), got {tuple(u.shape)}")
    batch, dim, length = u.shape
    if tuple(delta.shape) != (batch, dim, length):
        raise ValueError(f"delta must be {(batch, dim, length)}, got {tuple(delta.shape)}")
    if a.dim() != 2 or a.shape[0] != dim:
        raise ValueError(f"A must be ({dim}, state), got {tuple(a.shape)}")
    state = a.shape[1]
    if b.dim() != 4 or c.dim() != 4:
        raise ValueError("B/C must be (batch, groups, state, len)")
    groups = b.shape[1]
    for name, t in (("B", b), ("C", c)):
        if tuple(t.shape) != (batch, groups, state, length):
            raise ValueError(
                f"{name} must be {(batch, groups, state, length)}, got {tuple(t.shape)}")
    for name, t, want in (("D", d_skip, (dim,)), ("delta_bias", delta_bias, (dim,)),
                          ("z", z, (batch, dim, length)),
                          ("initial_state", h0, (batch, dim, state))):
        if t is not None and tuple(t.shape) != want:
            raise ValueError(f"{name} must be {want}, got {tuple(t.shape)}")
    return batch, dim, length, state, groups


@torch.library.custom_op("arm_scan::selective_scan", mutates_args=())
def _selective_scan_op(
    u: torch.Tensor,
    delta: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    c: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    h0: Optional[torch.Tensor],
    delta_softplus: bool,
    reverse: bool,
) -> Tuple[torch.Tensor, torch.Tensor]:
    dev = _device_of(u, delta, a, b, c, d_skip, z, delta_bias, h0)
    batch, dim, length, state, groups = _check_m1(u, delta, a, b, c, d_skip, z, delta_bias, h0)
    out = torch.empty_like(u)
    last_state = u.new_empty((batch, dim, state))
    dims = _ffi.ArmScanDims(batch, dim, length, state, groups)
    with torch.cuda.device(dev):
        _ffi.scan_raw(dims, u.data_ptr(), delta.data_ptr(), a.data_ptr(), b.data_ptr(),
                      c.data_ptr(), _ptr(d_skip), _ptr(z), _ptr(delta_bias), delta_softplus,
                      "auto", "auto", out.data_ptr(), last_state.data_ptr(), ptr_h0=_ptr(h0),
                      reverse=reverse, stream=_stream(dev))
    _CALLS["n"] += 1
    return out, last_state


@_selective_scan_op.register_fake
def _(u, delta, a, b, c, d_skip, z, delta_bias, h0, delta_softplus, reverse):
    return torch.empty_like(u), u.new_empty((u.shape[0], u.shape[1], a.shape[1]))


def _bc4(t, batch, state, length):
    return t.reshape(batch, 1, state, length) if t.dim() == 3 else t


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                   delta_softplus=False, return_last_state=False,
                   initial_state=None, reverse=False):
    """Mamba-1 selective scan on device float32 tensors
    (the reference's `arm_scan.selective_scan`, python/arm_scan/op.py:63-100).

    u, delta, z: (batch, dim, len); A: (dim, state);
    B, C: (batch, state, len) or (batch, groups, state, len);
    D, delta_bias: (dim,); initial_state: (batch, dim, state) to resume from.
    Returns out (batch, dim, len) [, last_state (batch, dim, state)].

    reverse walks the sequence backward in time with the output layout
    unchanged (timestep t still lands at index t); under reverse, last_state
    is the state after consuming t = 0.
    """
    batch, dim, length = u.shape
    state = A.shape[1]
    B = _bc4(B, batch, state, length)
    C = _bc4(C, batch, state, length)
    out, last_state = _selective_scan_op(
        _c(u), _c(delta), _c(A), _c(B), _c(C),
        None if D is None else _c(D),
        None if z is None else _c(z),
        None if delta_bias is None else _c(delta_bias),
        None if initial_state is None else _c(initial_state),
        bool(delta_softplus), bool(reverse))
    return (out, last_state) if return_last_state else out


def _strided_ok(u, delta, b, c, z, dim, length, groups):
    """Whether arm_scan_selective_scan_strided_f32 serves these tensors (the
    conditions its declaration states)."""
    if length % 4 or dim % 16 or (dim // groups) % 16:
        return False
    if any(t.data_ptr() % 16 for t in (delta, b, c)):
        return False
    if u.is_contiguous() and u.data_ptr() % 16:
        return False
    for t in (z, None, u):
        st = (length * dim, 1, dim) if t is None else t.stride()
        if min(st) < 0 or 4 * ((dim - 1) * st[1] + (length - 1) * st[2] + 1) >= 1 << 32:
            return False
        # a broadcast view (stride 0 over an axis longer than 1) takes the contiguous
        # route, which materialises it
        if t is not None and any(s == 0 and n > 1 for s, n in zip(st, t.shape)):
            return False
    return True


@torch.library.custom_op("arm_scan::selective_scan_time_major", mutates_args=())
def _selective_scan_tm_op(
    u: torch.Tensor,
    delta: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    c: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    h0: Optional[torch.Tensor],
    delta_softplus: bool,
    reverse: bool,
) -> Tuple[torch.Tensor, torch.Tensor]:
    dev = _device_of(u, delta, a, b, c, d_skip, z, delta_bias, h0)
    batch, dim, length, state, groups = _check_m1(u, delta, a, b, c, d_skip, z, delta_bias, h0)
    out = u.new_empty((batch, length, dim)).transpose(1, 2)
    last_state = u.new_empty((batch, dim, state))
    dims = _ffi.ArmScanDims(batch, dim, length, state, groups)
    with torch.cuda.device(dev):
        if _strided_ok(u, delta, b, c, z, dim, length, groups):
            _ffi.scan_strided_raw(dims, u.data_ptr(), delta.data_ptr(), a.data_ptr(),
                                  b.data_ptr(), c.data_ptr(), _ptr(d_skip), _ptr(z),
                                  None if z is None else z.stride(), _ptr(delta_bias),
                                  delta_softplus, out.data_ptr(), out.stride(),
                                  last_state.data_ptr(), _ptr(h0), reverse=reverse,
                                  stream=_stream(dev),
                                  u_strides=None if u.is_contiguous() else u.stride())
        else:
            # a shape the strided kernel does not serve: the contiguous scan, then
            # the output laid out time-major
            zc = None if z is None else z.contiguous()
            u = u.contiguous()
            tmp = torch.empty_like(u)
            _ffi.scan_raw(dims, u.data_ptr(), delta.data_ptr(), a.data_ptr(), b.data_ptr(),
                          c.data_ptr(), _ptr(d_skip), _ptr(zc), _ptr(delta_bias),
                          delta_softplus, "auto", "auto", tmp.data_ptr(),
                          last_state.data_ptr(), ptr_h0=_ptr(h0), reverse=reverse,
                          stream=_stream(dev))
            out.copy_(tmp)
    _CALLS["n"] += 1
    return out, last_state


@_selective_scan_tm_op.register_fake
def _(u, delta, a, b, c, d_skip, z, delta_bias, h0, delta_softplus, reverse):
    batch, dim, length = u.shape
    return (u.new_empty((batch, length, dim)).transpose(1, 2),
            u.new_empty((batch, dim, a.shape[1])))


def selective_scan_time_major(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                              delta_softplus=False, return_last_state=False,
                              initial_state=None, reverse=False):
    """`selective_scan` for callers whose tensors are time-major underneath, as in
    Hugging Face's Mamba mixer (modeling_mamba.py MambaMixer.forward): z may be any
    strided (batch, dim, len) view (the mixer's gate is one of (batch, len, 2*dim)
    storage) and is read in place, and out is returned as a (batch, dim, len) view
    of (batch, len, dim) storage, so `out.transpose(1, 2)` is contiguous for the
    mixer's out_proj. Same arguments, values and final state as `selective_scan`.
    The reference copies z here (python/arm_scan/op.py:19-20); this has no
    counterpart there."""
    batch, dim, length = u.shape
    state = A.shape[1]
    B = _bc4(B, batch, state, length)
    C = _bc4(C, batch, state, length)
    if z is not None and z.dtype != torch.float32:
        z = z.float()
    # u, like z, may be a view of time-major storage (the mixer's convolution output
    # laid out for its x_proj): read in place
    u = u.float() if u.dtype != torch.float32 else u
    out, last_state = _selective_scan_tm_op(
        u, _c(delta), _c(A), _c(B), _c(C),
        None if D is None else _c(D),
        z,
        None if delta_bias is None else _c(delta_bias),
        None if initial_state is None else _c(initial_state),
        bool(delta_softplus), bool(reverse))
    return (out, last_state) if return_last_state else out


@torch.library.custom_op("arm_scan::selective_state_update", mutates_args=("state",))
def _state_update_op(
    state: torch.Tensor,
    x: torch.Tensor,
    dt: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    c: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    dt_bias: Optional[torch.Tensor],
    dt_softplus: bool,
) -> torch.Tensor:
    dev = _device_of(state, x, dt, a, b, c, d_skip, z, dt_bias)
    batch, dim, n = state.shape
    for name, t, want in (("x", x, (batch, dim)), ("dt", dt, (batch, dim)),
                          ("A", a, (dim, n)), ("B", b, (batch, n)), ("C", c, (batch, n)),
                          ("D", d_skip, (dim,)), ("z", z, (batch, dim)),
                          ("dt_bias", dt_bias, (dim,))):
        if t is not None and tuple(t.shape) != want:
            raise ValueError(f"{name} must be {want}, got {tuple(t.shape)}")
    if not state.is_contiguous():
        raise ValueError("state must be contiguous (it is updated in place)")
    out = x.new_empty((batch, dim))
    with torch.cuda.device(dev):
        _ffi.state_update_raw(batch, dim, n, state.data_ptr(), x.data_ptr(), x.stride(),
                              dt.data_ptr(), dt.stride(), a.data_ptr(), b.data_ptr(), b.stride(),
                              c.data_ptr(), c.stride(), _ptr(d_skip), _ptr(z),
                              None if z is None else z.stride(), _ptr(dt_bias), dt_softplus,
                              out.data_ptr(), stream=_stream(dev))
    _CALLS["n"] += 1
    return out


@_state_update_op.register_fake
def _(state, x, dt, a, b, c, d_skip, z, dt_bias, dt_softplus):
    return x.new_empty((state.shape[0], state.shape[1]))


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False):
    """One decode step of the Mamba-1 scan with `state` (batch, dim, N) updated in
    place; returns y (batch, dim). x, dt, z (batch, dim) and B, C (batch, N) may be
    strided views (they are read in place); A (dim, N); D, dt_bias (dim,). The
    semantics of transformers' mamba_selective_state_update, in one kernel; the
    reference has no counterpart (it leaves decoding to upstream, README.md:320-322)."""
    f = lambda t: None if t is None else (t if t.dtype == torch.float32 else t.float())
    return _state_update_op(state, f(x), f(dt), _c(A), f(B), f(C),
                            None if D is None else _c(D), f(z),
                            None if dt_bias is None else _c(dt_bias), bool(dt_softplus))


@torch.library.custom_op("arm_scan::selective_scan_bidirectional", mutates_args=())
def _selective_scan_bidir_op(
    u: torch.Tensor,
    delta: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    c: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    delta_softplus: bool,
) -> Tuple[torch.Tensor, torch.Tensor]:
    dev = _device_of(u, delta, a, b, c, d_skip, z, delta_bias)
    batch, dim, length, state, groups = _check_m1(u, delta, a, b, c, d_skip, z, delta_bias,
                                                  None)
    out_fwd = torch.empty_like(u)
    out_bwd = torch.empty_like(u)
    dims = _ffi.ArmScanDims(batch, dim, length, state, groups)
    with torch.cuda.device(dev):
        _ffi.scan_bidir_raw(dims, u.data_ptr(), delta.data_ptr(), a.data_ptr(), b.data_ptr(),
                            c.data_ptr(), _ptr(d_skip), _ptr(z), _ptr(delta_bias),
                            delta_softplus, "auto", "auto", out_fwd.data_ptr(),
                            out_bwd.data_ptr(), stream=_stream(dev))
    _CALLS["n"] += 1
    return out_fwd, out_bwd


@_selective_scan_bidir_op.register_fake
def _(u, delta, a, b, c, d_skip, z, delta_bias, delta_softplus):
    return torch.empty_like(u), torch.empty_like(u)


def selective_scan_bidirectional(u, delta, A, B, C, D=None, z=None,
                                 delta_bias=None, delta_softplus=False):
    """Forward and reverse scans of the same inputs in one call
    (python/arm_scan/op.py:138-160) -> (out_fwd, out_bwd), through
    arm_scan_selective_scan_bidirectional_f32 (its routes: include/arm_scan_hip.h)."""
    batch, dim, length = u.shape
    state = A.shape[1]
    B = _bc4(B, batch, state, length)
    C = _bc4(C, batch, state, length)
    return _selective_scan_bidir_op(
        _c(u), _c(delta), _c(A), _c(B), _c(C),
        None if D is None else _c(D),
        None if z is None else _c(z),
        None if delta_bias is None else _c(delta_bias),
        bool(delta_softplus))


def selective_scan_bidirectional_with_state(u, delta, A, B, C, D=None, z=None,
                                            delta_bias=None, delta_softplus=False):
    """As `selective_scan_bidirectional`, also returning both final states:
    (out_fwd, out_bwd, last_fwd, last_bwd). The reference's C ABI has these
    outputs (arm-scan-ffi/src/lib.rs:235-252) but its torch op drops them."""
    dev = _device_of(u, delta, A, B, C, D, z, delta_bias)
    batch, dim, length = u.shape
    state = A.shape[1]
    u, delta, A = _c(u), _c(delta), _c(A)
    B = _c(_bc4(B, batch, state, length))
    C = _c(_bc4(C, batch, state, length))
    D = None if D is None else _c(D)
    z = None if z is None else _c(z)
    delta_bias = None if delta_bias is None else _c(delta_bias)
    _, _, _, _, groups = _check_m1(u, delta, A, B, C, D, z, delta_bias, None)
    of, ob = torch.empty_like(u), torch.empty_like(u)
    lf, lb = u.new_empty((batch, dim, state)), u.new_empty((batch, dim, state))
    dims = _ffi.ArmScanDims(batch, dim, length, state, groups)
    with torch.cuda.device(dev):
        _ffi.scan_bidir_raw(dims, u.data_ptr(), delta.data_ptr(), A.data_ptr(), B.data_ptr(),
                            C.data_ptr(), _ptr(D), _ptr(z), _ptr(delta_bias), delta_softplus,
                            "auto", "auto", of.data_ptr(), ob.data_ptr(), lf.data_ptr(),
                            lb.data_ptr(), stream=_stream(dev))
    _CALLS["n"] += 1
    return of, ob, lf, lb


@torch.library.custom_op("arm_scan::causal_conv1d", mutates_args=())
def _causal_conv1d_op(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                      silu: bool, time_major: bool) -> torch.Tensor:
    dev = _device_of(x, weight, bias)
    batch, dim, length = x.shape
    if time_major:
        out = torch.empty((batch, length, dim), dtype=torch.float32,
                          device=dev).transpose(1, 2)
    else:
        out = torch.empty((batch, dim, length), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _ffi.causal_conv1d_raw(batch, dim, length, weight.shape[1], x.data_ptr(), x.stride(),
                               weight.data_ptr(), _ptr(bias), silu, out.data_ptr(),
                               stream=_stream(dev), time_major=time_major)
    _CALLS["n"] += 1
    return out


@_causal_conv1d_op.register_fake
def _(x, weight, bias, silu, time_major):
    b, d, length = x.shape
    if time_major:
        return x.new_empty((b, length, d), dtype=torch.float32).transpose(1, 2)
    return x.new_empty((b, d, length), dtype=torch.float32)


def causal_conv1d(x, weight, bias=None, activation=None, time_major=False):
    """The Mamba-1 mixer's depthwise causal convolution (transformers modeling_mamba.py
    causal_conv1d_fn; the reference leaves it upstream): x (batch, dim, len), any
    strides (read in place), weight (dim, width <= 8), bias (dim,) or None, activation
    None or "silu" -> (batch, dim, len) float32, contiguous; or, with time_major, a view
    of (batch, len, dim) storage, the layout the mixer's x_proj reads after its
    transpose (and the scan reads in place)."""
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"activation must be None or 'silu', got {activation!r}")
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError(f"x (batch, dim, len) and weight (dim, width) expected, got "
                         f"{tuple(x.shape)} and {tuple(weight.shape)}")
    if bias is not None and tuple(bias.shape) != (x.shape[1],):
        raise ValueError(f"bias must be ({x.shape[1]},), got {tuple(bias.shape)}")
    if x.dtype != torch.float32:
        x = x.float()
    return _causal_conv1d_op(x, _c(weight), None if bias is None else _c(bias),
                             activation is not None, bool(time_major))


@torch.library.custom_op("arm_scan::causal_conv1d_update", mutates_args=("conv_state",))
def _causal_conv1d_update_op(x: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor,
                             bias: Optional[torch.Tensor], silu: bool) -> torch.Tensor:
    dev = _device_of(x, conv_state, weight, bias)
    batch, dim = x.shape
    out = torch.empty((batch, dim), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _ffi.causal_conv1d_update_raw(batch, dim, weight.shape[1], x.data_ptr(), x.stride(),
                                      conv_state.data_ptr(), weight.data_ptr(), _ptr(bias),
                                      silu, out.data_ptr(), stream=_stream(dev))
    _CALLS["n"] += 1
    return out


@_causal_conv1d_update_op.register_fake
def _(x, conv_state, weight, bias, silu):
    return x.new_empty(x.shape, dtype=torch.float32)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None):
    """One decode step of `causal_conv1d` (transformers modeling_mamba.py
    causal_conv1d_update): conv_state (batch, dim, width), contiguous float32, holds the
    last width inputs and is shifted in place with x (batch, dim) appended (any strides,
    read in place); returns (batch, dim) = act(bias + weight . window)."""
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"activation must be None or 'silu', got {activation!r}")
    if x.dim() != 2 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError(f"x (batch, dim) and weight (dim, width) expected, got "
                         f"{tuple(x.shape)} and {tuple(weight.shape)}")
    if (tuple(conv_state.shape) != (x.shape[0], x.shape[1], weight.shape[1])
            or not conv_state.is_contiguous() or conv_state.dtype != torch.float32):
        raise ValueError("conv_state must be a contiguous float32 (batch, dim, width) tensor")
    if x.dtype != torch.float32:
        x = x.float()
    return _causal_conv1d_update_op(x, conv_state, _c(weight),
                                    None if bias is None else _c(bias), activation is not None)


def kernel_calls() -> int:
    """How many times the native library has been invoked (engagement check,
    python/arm_scan/op.py:163-166)."""
    return _CALLS["n"]

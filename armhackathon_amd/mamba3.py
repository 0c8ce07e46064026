"""PyTorch front-end for the Mamba-3 SISO and rank-r MIMO scans on MI355X.

Mirrors python/arm_scan/mamba3.py:1-334: `angles_to_cos_sin` (the RoPE angle
pre-pass), the `arm_scan::mamba3_scan` custom op with a fake kernel,
`mamba3_scan`, `mamba3_scan_pair` and `mamba3_mimo_scan`, with the same
contracts: trap is PRE-sigmoid, angles come in raw (or cos/sin precomputed),
shapes are checked here because the C side trusts element counts.

Two extensions over the reference, both exact supersets (with their default
values the behaviour is the reference's):
  * q/k may carry a groups axis of any size g dividing the head count
    ((b, l, g, dqk) for SISO, (b, l, r, g, dqk) for MIMO); head h reads group
    h // (heads // g). g = 1 is the reference layout.
  * `return_last_state=True` also returns the final state (b, h, dv, dqk)
    (and, for SISO, last_bx (b, h, dqk)); the reference rejects a MIMO carry.

Forward calls from raw angles whose v, z or angles are views (slices of a mixer's
projection, angles expanded over heads, as apps/mamba3_lm/block.py:150-174 passes
them) are read in place through arm_scan_mamba3_scan_strided_f32 instead of being
copied contiguous.

Tensors are device tensors; the scan runs in the HIP kernels of
libarm_scan_hip.so on the current stream.
"""

import math
from typing import Optional, Tuple

import torch

from . import _ffi
from .op import _CALLS, _c, _device_of, _ptr, _stream


def angles_to_cos_sin(angles: torch.Tensor, dt: torch.Tensor,
                      half: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """theta = cumsum_L(tanh(angle) * pi * dt) -> (cos, sin), each (b, l, h, half)
    (python/arm_scan/mamba3.py:41-89). angles (b, l, h, r) raw, dt (b, h, l)
    post-softplus; pairs past r get the identity rotation (cos 1, sin 0).
    float32 device tensors go through the HIP pre-pass (arm_scan_mamba3_angles_f32);
    other dtypes are computed in torch at the caller's precision, floored at float32,
    as the reference does for float64 analysis."""
    if angles.dim() != 4:
        raise ValueError(f"angles must be (b, l, h, r), got {tuple(angles.shape)}")
    r = angles.shape[-1]
    if r > half:
        raise ValueError(f"angles has {r} rotation pairs but the head dim allows {half}")
    if (angles.device.type == "cuda" and angles.dtype == torch.float32
            and dt.dtype == torch.float32 and dt.device == angles.device):
        # the HIP pre-pass: one kernel, angles and dt read once, cos/sin written once
        b, length, h, _ = angles.shape
        if tuple(dt.shape) != (b, h, length):
            raise ValueError(f"dt must be {(b, h, length)}, got {tuple(dt.shape)}")
        a, d = angles.contiguous(), dt.contiguous()
        cos = torch.empty((b, length, h, half), dtype=torch.float32, device=a.device)
        sin = torch.empty_like(cos)
        with torch.cuda.device(a.device):
            _ffi.angles_raw(a.data_ptr(), d.data_ptr(), b, length, h, r, half, cos.data_ptr(),
                            sin.data_ptr(), stream=_stream(a.device))
        return cos, sin
    dtype = torch.promote_types(angles.dtype, torch.float32)
    dt_blh = dt.permute(0, 2, 1).unsqueeze(-1).to(dtype)
    theta = torch.cumsum(torch.tanh(angles.to(dtype)) * math.pi * dt_blh, dim=1)
    cos, sin = torch.cos(theta), torch.sin(theta)
    if r < half:
        pad = (*theta.shape[:-1], half - r)
        cos = torch.cat([cos, torch.ones(pad, dtype=cos.dtype, device=cos.device)], dim=-1)
        sin = torch.cat([sin, torch.zeros(pad, dtype=sin.dtype, device=sin.device)], dim=-1)
    return cos, sin


def _run(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z, reverse, psi, zeta,
         phi, want_state):
    dev = _device_of(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z, psi, zeta,
                     phi)
    mimo = psi is not None
    if mimo:
        b, length, rank, groups, dqk = q.shape
    else:
        b, length, groups, dqk = q.shape
        rank = 1
    h, dv = v.shape[2], v.shape[3]
    dims = _ffi.ArmMamba3Dims(b, h, dv, dqk, length, rank, groups)
    # written time-major by the kernel (python/arm_scan/mamba3.py:142 permutes the
    # head-major result into this layout)
    out = torch.empty((b, length, h, dv), dtype=torch.float32, device=dev)
    last_state = torch.empty((b, h, dv, dqk), dtype=torch.float32, device=dev) \
        if want_state else None
    last_bx = torch.empty((b, h, dqk), dtype=torch.float32, device=dev) \
        if (want_state and not mimo) else None
    with torch.cuda.device(dev):
        _ffi.mamba3_raw(
            dims,
            [q.data_ptr(), k.data_ptr(), v.data_ptr(), adt.data_ptr(), dt.data_ptr(),
             trap.data_ptr(), q_bias.data_ptr(), k_bias.data_ptr(), cos.data_ptr(),
             sin.data_ptr(), _ptr(d_skip), _ptr(z), _ptr(psi), _ptr(zeta), _ptr(phi)],
            1 if reverse else 0, _ffi.BACKENDS["auto"], _ffi.THREADING["auto"],
            out.data_ptr(), _ptr(last_state), _ptr(last_bx), stream=_stream(dev),
            time_major=True)
    _CALLS["n"] += 1
    return out, last_state, last_bx


def _run_angles(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi, zeta, phi,
                want_state):
    """Forward scan with the angle pre-pass fused into the kernel
    (arm_scan_mamba3_scan_angles_f32): raw angles instead of cos/sin. Tensors that are
    not 16-byte aligned (views at odd offsets) take the pre-pass kernels and the scan
    on cos/sin instead: the same result, unfused."""
    if not _aligned16(q, k, v, q_bias, k_bias, angles, z):
        cos, sin = angles_to_cos_sin(angles, dt, q.shape[-1] // 2)
        return _run(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z, False, psi,
                    zeta, phi, want_state)
    dev = _device_of(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi, zeta,
                     phi)
    mimo = psi is not None
    if mimo:
        b, length, rank, groups, dqk = q.shape
    else:
        b, length, groups, dqk = q.shape
        rank = 1
    h, dv = v.shape[2], v.shape[3]
    dims = _ffi.ArmMamba3Dims(b, h, dv, dqk, length, rank, groups)
    out = torch.empty((b, length, h, dv), dtype=torch.float32, device=dev)
    last_state = torch.empty((b, h, dv, dqk), dtype=torch.float32, device=dev) \
        if want_state else None
    last_bx = torch.empty((b, h, dqk), dtype=torch.float32, device=dev) \
        if (want_state and not mimo) else None
    with torch.cuda.device(dev):
        _ffi.mamba3_angles_raw(
            dims,
            [q.data_ptr(), k.data_ptr(), v.data_ptr(), adt.data_ptr(), dt.data_ptr(),
             trap.data_ptr(), q_bias.data_ptr(), k_bias.data_ptr(), angles.data_ptr(),
             _ptr(d_skip), _ptr(z), _ptr(psi), _ptr(zeta), _ptr(phi)],
            angles.shape[-1], _ffi.BACKENDS["auto"], _ffi.THREADING["auto"],
            out.data_ptr(), _ptr(last_state), _ptr(last_bx), stream=_stream(dev))
    _CALLS["n"] += 1
    return out, last_state, last_bx


def _angles_fusable(angles, cos, sin, reverse, q, k, v, q_bias, k_bias, z, rank):
    """Whether the fused pre-pass serves this call by its shapes: the conditions
    arm_scan_mamba3_scan_angles_f32 declares (forward; angle pairs a positive
    multiple of 4 up to dqk/2; dv, dqk multiples of 16, dqk <= 128; rank 1, 2 or 4).
    Its last condition, 16-byte aligned tensors, is checked inside the op
    (`_run_angles`), where the tensors have storage: under torch.compile this runs
    on fake tensors, which have no data pointer."""
    if angles is None or cos is not None or sin is not None or reverse or angles.dim() != 4:
        return False
    dqk, dv, r = q.shape[-1], v.shape[-1], angles.shape[-1]
    if r == 0 or r % 4 or r > dqk // 2 or dv % 16 or dqk % 16 or dqk > 128:
        return False
    return rank in (1, 2, 4)


def _aligned16(*tensors):
    return all(t is None or t.data_ptr() % 16 == 0 for t in tensors)


def _inplace_strides(v, z, angles):
    """Element strides under which arm_scan_mamba3_scan_strided_f32 reads v and z
    ((batch, step), heads dv apart, unit channel stride) and the angles ((batch, step,
    head), unit pair stride) where they lie, or None when a layout does not fit. The
    reference's Mamba-3 block hands the scan exactly such views: x and z are slices of
    its in_proj output and the angles an `expand` over heads
    (apps/mamba3_lm/block.py:150-174)."""
    def broadcast(t, axes):
        return any(t.stride(a) == 0 and t.shape[a] > 1 for a in axes)

    def vz(t):
        b, length, h, dv = t.shape
        if (dv > 1 and t.stride(3) != 1) or (h > 1 and t.stride(2) != dv):
            return None
        if broadcast(t, (0, 1)):
            return None  # broadcast over batch or steps: the contiguous route
        return (t.stride(0), t.stride(1))

    sv = vz(v)
    sz = None if z is None else vz(z)
    if sv is None or (z is not None and sz is None):
        return None
    if (angles.shape[3] > 1 and angles.stride(3) != 1) or broadcast(angles, (0, 1)):
        return None  # the head stride alone may be 0 (one set of angles per step)
    return {"v": sv, "z": sz, "angles": (angles.stride(0), angles.stride(1), angles.stride(2))}


def _strided_route(angles, cos, sin, reverse, want_state, v, z):
    """Forward from raw angles, no carries, and v, z or the angles not contiguous."""
    if angles is None or cos is not None or sin is not None or reverse or want_state:
        return None
    if angles.dim() != 4 or all(t is None or t.is_contiguous() for t in (v, z, angles)):
        return None
    if any(t is not None and t.dtype != torch.float32 for t in (v, z, angles)):
        return None  # read as they lie, so they must already be float32
    return _inplace_strides(v, z, angles)


def _run_strided(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi, zeta, phi):
    dev = _device_of(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi, zeta,
                     phi)
    strides = _inplace_strides(v, z, angles)
    if strides is None:
        raise ValueError("v, z or angles have a layout the strided scan cannot read")
    mimo = psi is not None
    if mimo:
        b, length, rank, groups, dqk = q.shape
    else:
        b, length, groups, dqk = q.shape
        rank = 1
    h, dv = v.shape[2], v.shape[3]
    dims = _ffi.ArmMamba3Dims(b, h, dv, dqk, length, rank, groups)
    out = torch.empty((b, length, h, dv), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _ffi.mamba3_strided_raw(
            dims,
            [q.data_ptr(), k.data_ptr(), v.data_ptr(), adt.data_ptr(), dt.data_ptr(),
             trap.data_ptr(), q_bias.data_ptr(), k_bias.data_ptr(), angles.data_ptr(),
             _ptr(d_skip), _ptr(z), _ptr(psi), _ptr(zeta), _ptr(phi)],
            strides, angles.shape[-1], _ffi.BACKENDS["auto"], _ffi.THREADING["auto"],
            out.data_ptr(), stream=_stream(dev))
    _CALLS["n"] += 1
    return out


@torch.library.custom_op("arm_scan::mamba3_scan_strided", mutates_args=())
def _mamba3_scan_strided_op(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    adt: torch.Tensor,
    dt: torch.Tensor,
    trap: torch.Tensor,
    q_bias: torch.Tensor,
    k_bias: torch.Tensor,
    angles: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    psi: Optional[torch.Tensor] = None,
    zeta: Optional[torch.Tensor] = None,
    phi: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    return _run_strided(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi, zeta,
                        phi)


@_mamba3_scan_strided_op.register_fake
def _(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi=None, zeta=None,
      phi=None):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2], v.shape[3]))


@torch.library.custom_op("arm_scan::mamba3_scan_angles", mutates_args=())
def _mamba3_scan_angles_op(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    adt: torch.Tensor,
    dt: torch.Tensor,
    trap: torch.Tensor,
    q_bias: torch.Tensor,
    k_bias: torch.Tensor,
    angles: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    psi: Optional[torch.Tensor] = None,
    zeta: Optional[torch.Tensor] = None,
    phi: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    out, _, _ = _run_angles(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi,
                            zeta, phi, False)
    return out


@_mamba3_scan_angles_op.register_fake
def _(q, k, v, adt, dt, trap, q_bias, k_bias, angles, d_skip, z, psi=None, zeta=None,
      phi=None):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2], v.shape[3]))


@torch.library.custom_op("arm_scan::mamba3_scan", mutates_args=())
def _mamba3_scan_op(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    adt: torch.Tensor,
    dt: torch.Tensor,
    trap: torch.Tensor,
    q_bias: torch.Tensor,
    k_bias: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    d_skip: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    reverse: bool,
    psi: Optional[torch.Tensor] = None,
    zeta: Optional[torch.Tensor] = None,
    phi: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    out, _, _ = _run(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z, reverse,
                     psi, zeta, phi, False)
    return out


@_mamba3_scan_op.register_fake
def _(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z, reverse,
      psi=None, zeta=None, phi=None):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2], v.shape[3]))


def _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D, z,
                  rank=None, psi=None, zeta=None, phi=None, angles=None):
    """Every tensor against the layout contract (python/arm_scan/mamba3.py:153-195):
    a short buffer would be an out-of-bounds read on the device."""
    if v.dim() != 4:
        raise ValueError(f"v must be (b, l, h, dv), got {tuple(v.shape)}")
    b, length, h, dv = v.shape
    if rank is None:
        if q.dim() != 4:
            raise ValueError(f"q must be (b, l, groups, dqk), got {tuple(q.shape)}")
        _, _, g, dqk = q.shape
        qshape, bshape = (b, length, g, dqk), (h, dqk)
    else:
        if q.dim() != 5:
            raise ValueError(f"q must be (b, l, rank, groups, dqk), got {tuple(q.shape)}")
        _, _, _, g, dqk = q.shape
        qshape, bshape = (b, length, rank, g, dqk), (h, rank, dqk)
    if dqk % 2:
        raise ValueError(f"dqk must be even (RoPE lane pairs), got {dqk}")
    if g < 1 or h % g:
        raise ValueError(f"q/k groups ({g}) must divide the head count ({h})")
    half = dqk // 2
    want = {"q": qshape, "k": qshape, "adt": (b, h, length), "dt": (b, h, length),
            "trap": (b, h, length), "q_bias": bshape, "k_bias": bshape}
    got = dict(q=q, k=k, adt=adt, dt=dt, trap=trap, q_bias=q_bias, k_bias=k_bias)
    if cos is not None:
        want["cos"], got["cos"] = (b, length, h, half), cos
        want["sin"], got["sin"] = (b, length, h, half), sin
    if angles is not None:
        want["angles"], got["angles"] = (b, length, h, angles.shape[-1]), angles
    if D is not None:
        want["D"], got["D"] = (h,), D
    if z is not None:
        want["z"], got["z"] = (b, length, h, dv), z
    if rank is not None:
        for name, t in (("psi", psi), ("zeta", zeta), ("phi", phi)):
            want[name], got[name] = (h, rank, dv), t
    for name, shape in want.items():
        actual = tuple(got[name].shape)
        if actual != shape:
            raise ValueError(
                f"{name} must be {shape}, got {actual}. A short buffer would be an "
                "out-of-bounds read in the kernel, so shapes are checked here.")


def _cos_sin(angles, cos, sin, dt, half):
    if (cos is None) != (sin is None):
        raise ValueError("pass cos and sin together, or neither")
    if cos is None:
        if angles is None:
            raise ValueError("pass either `angles` or both `cos` and `sin`")
        cos, sin = angles_to_cos_sin(angles, dt, half)
    return cos, sin


def mamba3_scan(q, k, v, adt, dt, trap, q_bias, k_bias, angles=None,
                D=None, z=None, reverse=False, cos=None, sin=None,
                return_last_state=False):
    """Mamba-3 SISO selective scan.

    q, k    : (b, l, g, dqk) or (b, l, dqk); g divides h (g = 1: shared by heads)
    v, z    : (b, l, h, dv)
    adt, dt : (b, h, l)        adt = A*dt (<= 0); dt post-softplus
    trap    : (b, h, l)        PRE-sigmoid
    angles  : (b, l, h, r)     raw; the pre-pass runs here (or pass cos/sin)
    q_bias, k_bias : (h, dqk); D : (h,)
    returns : (b, l, h, dv) [, last_state (b, h, dv, dqk), last_bx (b, h, dqk)]
    """
    if q.dim() == 3:
        q = q.unsqueeze(2)
    if k.dim() == 3:
        k = k.unsqueeze(2)
    if (angles is not None and v.dim() == 4 and angles.dim() == 4
            and _strided_route(angles, cos, sin, reverse, return_last_state, v, z)):
        # v, z or the angles are views (e.g. of a mixer's projection): read in place
        _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, None, None, D, z, angles=angles)
        return _mamba3_scan_strided_op(
            _c(q), _c(k), v, _c(adt), _c(dt), _c(trap), _c(q_bias), _c(k_bias), angles,
            None if D is None else _c(D), z)
    q, k, v = _c(q), _c(k), _c(v)
    q_bias, k_bias = _c(q_bias), _c(k_bias)
    z = None if z is None else _c(z)
    angles = None if angles is None else _c(angles)
    if _angles_fusable(angles, cos, sin, reverse, q, k, v, q_bias, k_bias, z, 1):
        # the angle pre-pass runs inside the scan kernel
        _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, None, None, D, z,
                      angles=angles)
        args = (q, k, v, _c(adt), _c(dt), _c(trap), q_bias, k_bias, angles,
                None if D is None else _c(D), z)
        if not return_last_state:
            return _mamba3_scan_angles_op(*args)
        return _run_angles(*args, None, None, None, True)
    cos, sin = _cos_sin(angles, cos, sin, dt, q.shape[-1] // 2)
    _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D, z)
    args = (_c(q), _c(k), _c(v), _c(adt), _c(dt), _c(trap), _c(q_bias), _c(k_bias), _c(cos),
            _c(sin), None if D is None else _c(D), None if z is None else _c(z), bool(reverse))
    if not return_last_state:
        return _mamba3_scan_op(*args)
    return _run(*args, None, None, None, True)


def mamba3_scan_pair(q, k, v, adt, dt, trap, q_bias, k_bias, angles=None,
                     D=None, z=None, cos=None, sin=None):
    """Both traversal directions of the same inputs -> (fwd, bwd)
    (python/arm_scan/mamba3.py:235-258). The angle pre-pass runs once."""
    cos, sin = _cos_sin(angles, cos, sin, dt, q.shape[-1] // 2)
    common = dict(q_bias=q_bias, k_bias=k_bias, D=D, z=z, cos=cos, sin=sin)
    fwd = mamba3_scan(q, k, v, adt, dt, trap, reverse=False, **common)
    bwd = mamba3_scan(q, k, v, adt, dt, trap, reverse=True, **common)
    return fwd, bwd


def mamba3_mimo_scan(q, k, v, adt, dt, trap, q_bias, k_bias, psi, zeta, phi,
                     angles=None, D=None, z=None, reverse=False,
                     cos=None, sin=None, return_last_state=False):
    """Mamba-3 MIMO (rank-r) selective scan (python/arm_scan/mamba3.py:261-334).

    q, k    : (b, l, r, g, dqk) or (b, l, r, dqk); g divides h
    v, z    : (b, l, h, dv)
    q_bias, k_bias : (h, r, dqk); psi, zeta, phi : (h, r, dv); D : (h,)
    returns : (b, l, h, dv) [, last_state (b, h, dv, dqk)]

    MIMO rotates split-halves pairs (i, i + dqk/2), SISO interleaved pairs
    (2i, 2i+1): a rank-1 MIMO call equals a SISO call only without rotation.
    """
    if q.dim() == 4:
        q = q.unsqueeze(3)
    if k.dim() == 4:
        k = k.unsqueeze(3)
    rank = q.shape[2]
    if (angles is not None and v.dim() == 4 and angles.dim() == 4
            and _strided_route(angles, cos, sin, reverse, return_last_state, v, z)):
        # v, z or the angles are views: the pre-pass and the scan read them in place
        _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, None, None, D, z, rank=rank,
                      psi=psi, zeta=zeta, phi=phi, angles=angles)
        return _mamba3_scan_strided_op(
            _c(q), _c(k), v, _c(adt), _c(dt), _c(trap), _c(q_bias), _c(k_bias), angles,
            None if D is None else _c(D), z, _c(psi), _c(zeta), _c(phi))
    # From raw angles MIMO takes the HIP pre-pass and the scan on cos/sin: with
    # 16/rank-step chunks the fused pre-pass lengthens every iteration of a loop that
    # is latency-bound (arm_scan_mamba3_scan_angles_f32 still serves it).
    cos, sin = _cos_sin(angles, cos, sin, dt, q.shape[-1] // 2)
    _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D, z, rank=rank,
                  psi=psi, zeta=zeta, phi=phi)
    args = (_c(q), _c(k), _c(v), _c(adt), _c(dt), _c(trap), _c(q_bias), _c(k_bias), _c(cos),
            _c(sin), None if D is None else _c(D), None if z is None else _c(z),
            bool(reverse), _c(psi), _c(zeta), _c(phi))
    if not return_last_state:
        return _mamba3_scan_op(*args)
    out, ls, _ = _run(*args, True)
    return out, ls

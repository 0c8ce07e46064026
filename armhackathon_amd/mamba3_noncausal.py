"""Non-causal Mamba-3 aggregation on MI355X: every position sums over every other
position, 1D and 2D (python/arm_scan/mamba3_noncausal.py:1-46).

Unrolled, the SISO recurrence is y_t = sum_s M[t, s] (q_t . k_s) v_s + D v_t with a
decay e^{c_t - c_s} that factorises. The sum over all s is therefore the forward
traversal plus the backward one minus the same-step term, which both count
(mamba3_noncausal.py:89-98).

* `noncausal_scan` runs that as two launches of the SISO kernel through
  arm_scan_mamba3_noncausal_f32. The forward traversal writes the output; the
  backward one leaves the same-step term (gamma q.k + D) out of its outputs and
  adds them onto it. No second (b, l, h, dv) tensor, diagonal pass or sum pass is
  materialised.
* `noncausal_scan_dense` is the O(L^2) mask form (mamba3_noncausal.py:101-178):
  batched GEMMs on the device through torch.matmul, no scan. The reference keeps
  it as an algorithm independent of the scan (with `causal=True` it is the dual
  form of the causal scan) and as the other side of its scan-vs-dense comparison.
* `ss2d_noncausal_mamba3` is the 2D form: each of the grid's two orderings
  aggregated non-causally, then merged (mamba3_noncausal.py:181-222).

Tensors are float32 device tensors, laid out as for `mamba3_scan`.
"""

from typing import Optional

import torch

from . import _ffi
from .mamba3 import _check_shapes, _cos_sin
from .op import _CALLS, _c, _device_of, _ptr, _stream
from .ss2d import _MERGES, grid_to_views
from .ss2d_mamba3 import _check_grid, grid_to_views_time_major, views_to_grid_time_major


def _run_noncausal(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z):
    dev = _device_of(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z)
    b, length, groups, dqk = q.shape
    h, dv = v.shape[2], v.shape[3]
    dims = _ffi.ArmMamba3Dims(b, h, dv, dqk, length, 1, groups)
    out = torch.empty((b, length, h, dv), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _ffi.mamba3_noncausal_raw(
            dims,
            [q.data_ptr(), k.data_ptr(), v.data_ptr(), adt.data_ptr(), dt.data_ptr(),
             trap.data_ptr(), q_bias.data_ptr(), k_bias.data_ptr(), cos.data_ptr(),
             sin.data_ptr(), _ptr(d_skip), _ptr(z)],
            _ffi.BACKENDS["auto"], _ffi.THREADING["auto"], out.data_ptr(),
            stream=_stream(dev))
    _CALLS["n"] += 1
    return out


@torch.library.custom_op("arm_scan::mamba3_noncausal", mutates_args=())
def _mamba3_noncausal_op(
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
) -> torch.Tensor:
    return _run_noncausal(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z)


@_mamba3_noncausal_op.register_fake
def _(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2], v.shape[3]))


def noncausal_scan(q, k, v, adt, dt, trap, q_bias, k_bias, angles=None,
                   D=None, z=None, cos=None, sin=None):
    """Non-causal 1D aggregation in O(L): (b, l, h, dv)
    (python/arm_scan/mamba3_noncausal.py:89-98).

    q, k (b, l, g, dqk) or (b, l, dqk); the other arguments as for `mamba3_scan`.
    The angle pre-pass runs once and serves both traversals.
    """
    if q.dim() == 3:
        q = q.unsqueeze(2)
    if k.dim() == 3:
        k = k.unsqueeze(2)
    cos, sin = _cos_sin(angles, cos, sin, dt, q.shape[-1] // 2)
    _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D, z)
    return _mamba3_noncausal_op(
        _c(q), _c(k), _c(v), _c(adt), _c(dt), _c(trap), _c(q_bias), _c(k_bias), _c(cos),
        _c(sin), None if D is None else _c(D), None if z is None else _c(z))


def _rope_pairs(t, cos, sin):
    """Rotate interleaved pairs (2i, 2i+1) of t (b, l, h, dqk) by cos/sin (b, l, h, dqk/2)."""
    even, odd = t[..., 0::2], t[..., 1::2]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(-2)


def noncausal_scan_dense(q, k, v, adt, dt, trap, q_bias, k_bias, angles=None,
                         D=None, z=None, cos=None, sin=None, causal=False):
    """Non-causal 1D aggregation through the explicit (L, L) mask, O(L^2)
    (python/arm_scan/mamba3_noncausal.py:101-178): out = (M o Q K^T) V + D V, gated.

    M[t, s] is e^{c_t - c_s} scale_s for s < t (scale_s = gamma_s + dt_{s+1}
    (1 - sigmoid(trap_{s+1})), the forward trapezoid), gamma_t on the diagonal, and
    for s > t the backward traversal's weight e^{c'_s - c'_t} scale'_s with
    c' = c - adt (the sum of adt over t <= u < s) and scale'_s = gamma_s + dt_{s-1}
    (1 - sigmoid(trap_{s-1})). `causal=True` keeps the diagonal and below: the dual
    form of the causal scan.
    """
    if q.dim() == 3:
        q = q.unsqueeze(2)
    if k.dim() == 3:
        k = k.unsqueeze(2)
    dev = _device_of(q, k, v, adt, dt, trap, q_bias, k_bias, angles, cos, sin, D, z)
    b, length, g, dqk = q.shape
    h, dv = v.shape[2], v.shape[3]
    cos, sin = _cos_sin(angles, cos, sin, dt, dqk // 2)
    _check_shapes(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D, z)
    f32 = dict(dtype=torch.float32, device=dev)
    heads_of = torch.arange(h, device=dev) // (h // g)
    qh = _rope_pairs(q.to(**f32)[:, :, heads_of] + q_bias.to(**f32), cos.to(**f32),
                     sin.to(**f32))
    kh = _rope_pairs(k.to(**f32)[:, :, heads_of] + k_bias.to(**f32), cos.to(**f32),
                     sin.to(**f32))
    # (b, h, l, dqk) operands, the right one transposed and made contiguous
    qk = torch.matmul(qh.permute(0, 2, 1, 3).contiguous(),
                      kh.permute(0, 2, 3, 1).contiguous())  # (b, h, t, s)

    adt32, dt32 = adt.to(**f32), dt.to(**f32)
    lam = torch.sigmoid(trap.to(**f32))
    gamma = dt32 * lam
    carry = dt32 * (1.0 - lam)  # what step s hands its trapezoid neighbour
    scale_f = gamma.clone()
    scale_f[..., :-1] += carry[..., 1:]
    scale_b = gamma.clone()
    scale_b[..., 1:] += carry[..., :-1]
    c = torch.cumsum(adt32, dim=-1)
    ci, cj = c.unsqueeze(-1), c.unsqueeze(-2)  # [t, s]
    idx = torch.arange(length, device=dev)
    below = idx.view(-1, 1) > idx.view(1, -1)
    above = idx.view(-1, 1) < idx.view(1, -1)
    mask = torch.where(below, torch.exp(torch.where(below, ci - cj, 0.0)) *
                       scale_f.unsqueeze(-2), 0.0)
    if not causal:
        cp = c - adt32
        ei = torch.where(above, cp.unsqueeze(-2) - cp.unsqueeze(-1), 0.0)
        mask = mask + torch.where(above, torch.exp(ei) * scale_b.unsqueeze(-2), 0.0)
    mask = mask + torch.diag_embed(gamma)
    out = torch.matmul(mask * qk, v.to(**f32).permute(0, 2, 1, 3).contiguous())
    out = out.permute(0, 2, 1, 3)  # (b, l, h, dv)
    if D is not None:
        out = out + D.to(**f32).view(1, 1, h, 1) * v.to(**f32)
    if z is not None:
        z32 = z.to(**f32)
        out = out * (z32 * torch.sigmoid(z32))
    return out.contiguous()


def ss2d_noncausal_mamba3(q, k, v, adt, dt, trap, q_bias, k_bias, angles,
                          D=None, z=None, merge="sum"):
    """Non-causal 2D aggregation over a token grid
    (python/arm_scan/mamba3_noncausal.py:181-222): the row-major and column-major
    orderings, each aggregated non-causally (both stacked in one call of the
    non-causal kernel), then merged.

    Layouts as for `ss2d_scan_mamba3`: q, k (b, H, W, g, dqk); v, z (b, H, W, h, dv);
    adt, dt, trap (b, h, H, W); angles (b, H, W, h, r). merge "none" returns the two
    per-ordering planes (rows, cols), each (b, H, W, h, dv); "mean" halves the sum.
    """
    if merge not in _MERGES:
        raise ValueError(f"merge must be one of {_MERGES}, got {merge!r}")
    if q.dim() != 5:
        raise ValueError(f"q must be (b, H, W, groups, dqk), got {tuple(q.shape)}")
    b, hh, ww = q.shape[:3]
    for name, t in (("q", q), ("k", k), ("v", v), ("angles", angles)):
        _check_grid(name, t, b, hh, ww, 5)
    for name, t in (("adt", adt), ("dt", dt), ("trap", trap)):
        _check_grid(name, t, b, hh, ww, 4, head_major=True)
    if z is not None:
        _check_grid("z", z, b, hh, ww, 5)
    nc = noncausal_scan(
        grid_to_views_time_major(q), grid_to_views_time_major(k), grid_to_views_time_major(v),
        grid_to_views(adt), grid_to_views(dt), grid_to_views(trap), q_bias, k_bias,
        angles=grid_to_views_time_major(angles), D=D,
        z=None if z is None else grid_to_views_time_major(z))
    rows, cols = views_to_grid_time_major(nc[:b], nc[b:], hh, ww)
    if merge == "none":
        return rows, cols
    out = rows + cols
    return out if merge == "sum" else out * 0.5

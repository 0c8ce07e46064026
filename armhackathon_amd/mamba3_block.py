"""The Mamba-3 mixer on MI355X (apps/mamba3_lm/block.py:1-199): the block around the
scan, so that a Mamba-3 LM layer runs its whole mixer through this package.

The constructor arguments, parameter names and shapes are the reference's, which are
the published checkpoint's (block.py:24-44, 85-145): in_proj, out_proj, dt_bias, D,
B_bias, C_bias, B_norm.weight, C_norm.weight, and mimo_x / mimo_z / mimo_o for MIMO. A
state dict loads unchanged.

`Mamba3Mixer.forward` runs four launches where the reference runs about twenty torch
ops and four contiguous copies:

1. in_proj, a GEMM (torch.nn.functional.linear);
2. the front-end kernel (arm_scan_mamba3_block_frontend_f32). From the projection it
   writes dt, adt and trap head-major, q = C_norm(C) and k = B_norm(B). That covers
   the heavy-tail decay, the softplus, the A_floor clamp and the Q <- C / K <- B
   mapping (block.py:150-178);
3. the scan from raw angles (arm_scan_mamba3_scan_strided_f32). It reads x, z and the
   angles in place from the projection: the angles with head stride 0, as one set
   shared by every head (block.py:174). SISO fuses the angle pre-pass into the scan
   where the layout allows; otherwise the pre-pass kernels run first;
4. out_proj.

Computation is float32 on device tensors: the projection is taken in the input's
dtype and raised to float32 for the front-end, as the reference raises dd_A
(block.py:163-165).
"""

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _ffi
from .op import _CALLS, _device_of, _stream


def heavy_tail_activation(x: torch.Tensor) -> torch.Tensor:
    """f(x) = 1 + x for x >= 0, 1 / (1 - x) below (block.py:52-62), in torch ops. The
    mixer's forward evaluates it inside the front-end kernel."""
    return x.clamp_min(0) + torch.reciprocal(1 - x.clamp_max(0))


class RMSNorm(nn.Module):
    """RMSNorm over the last axis in float32 with eps inside the square root
    (block.py:65-82). It holds the `weight` the checkpoint names; the mixer applies the
    norm inside the front-end kernel and does not call this forward."""

    def __init__(self, hidden_size: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dtype = x.dtype
        x = x.float()
        rstd = torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + self.eps)
        return (x * rstd * self.weight.float()).to(dtype)


def _f32(t):
    # no detach: the op has no backward, so a graph that needs one fails loudly there
    return None if t is None else t.to(torch.float32).contiguous()


def _mixer_scan(proj, dt_bias, b_norm, c_norm, b_bias, c_bias, d_skip, psi, zeta, phi,
                heads, headdim, d_state, rank, groups, n_angles, a_floor, eps):
    dev = _device_of(proj, dt_bias, b_norm, c_norm, b_bias, c_bias, d_skip, psi, zeta, phi)
    b, length, row = proj.shape
    f32 = dict(dtype=torch.float32, device=dev)
    q = torch.empty((b, length, rank, groups, d_state), **f32)
    k = torch.empty_like(q)
    adt = torch.empty((b, heads, length), **f32)
    dt = torch.empty_like(adt)
    trap = torch.empty_like(adt)
    d_inner = heads * headdim
    col_ang = 2 * d_inner + 2 * rank * groups * d_state + 3 * heads
    out = torch.empty((b, length, heads, headdim), **f32)
    base, es = proj.data_ptr(), proj.element_size()
    with torch.cuda.device(dev):
        st = _stream(dev)
        _ffi.block_frontend_raw(
            base, b, length, row, heads, headdim, d_state, rank, groups, n_angles,
            dt_bias.data_ptr(), a_floor, b_norm.data_ptr(), c_norm.data_ptr(), eps,
            q.data_ptr(), k.data_ptr(), adt.data_ptr(), dt.data_ptr(), trap.data_ptr(),
            stream=st)
        dims = _ffi.ArmMamba3Dims(b, heads, headdim, d_state, length, rank, groups)
        mimo = psi is not None
        _ffi.mamba3_strided_raw(
            dims,
            [q.data_ptr(), k.data_ptr(), base + es * d_inner, adt.data_ptr(), dt.data_ptr(),
             trap.data_ptr(), c_bias.data_ptr(), b_bias.data_ptr(), base + es * col_ang,
             d_skip.data_ptr(), base, psi.data_ptr() if mimo else 0,
             zeta.data_ptr() if mimo else 0, phi.data_ptr() if mimo else 0],
            {"v": (length * row, row), "z": (length * row, row),
             "angles": (length * row, row, 0)},
            n_angles, _ffi.BACKENDS["auto"], _ffi.THREADING["auto"], out.data_ptr(),
            stream=st)
    _CALLS["n"] += 1
    return out


@torch.library.custom_op("arm_scan::mamba3_mixer_scan", mutates_args=())
def _mixer_scan_op(
    proj: torch.Tensor,
    dt_bias: torch.Tensor,
    b_norm: torch.Tensor,
    c_norm: torch.Tensor,
    b_bias: torch.Tensor,
    c_bias: torch.Tensor,
    d_skip: torch.Tensor,
    psi: Optional[torch.Tensor],
    zeta: Optional[torch.Tensor],
    phi: Optional[torch.Tensor],
    heads: int,
    headdim: int,
    d_state: int,
    rank: int,
    groups: int,
    n_angles: int,
    a_floor: float,
    eps: float,
) -> torch.Tensor:
    return _mixer_scan(proj, dt_bias, b_norm, c_norm, b_bias, c_bias, d_skip, psi, zeta, phi,
                       heads, headdim, d_state, rank, groups, n_angles, a_floor, eps)


@_mixer_scan_op.register_fake
def _(proj, dt_bias, b_norm, c_norm, b_bias, c_bias, d_skip, psi, zeta, phi, heads, headdim,
      d_state, rank, groups, n_angles, a_floor, eps):
    return proj.new_empty((proj.shape[0], proj.shape[1], heads, headdim),
                          dtype=torch.float32)


class Mamba3Mixer(nn.Module):
    """One Mamba-3 mixer (SISO, or rank-r MIMO with is_mimo), parameter names as the
    checkpoint's (block.py:85-145). forward: u (batch, seqlen, d_model) -> same shape."""

    def __init__(self, d_model=768, d_state=128, expand=2, headdim=64,
                 ngroups=1, rope_fraction=0.5, A_floor=1e-4, chunk_size=64,
                 layer_idx=None, is_mimo=False, mimo_rank=1):
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.headdim = headdim
        self.A_floor = A_floor
        self.chunk_size = chunk_size  # the reference's argument; the kernels pick their own
        self.layer_idx = layer_idx
        self.is_mimo = is_mimo
        self.d_inner = int(expand * d_model)
        if self.d_inner % headdim:
            raise ValueError(f"d_inner ({self.d_inner}) must be a multiple of headdim")
        self.nheads = self.d_inner // headdim
        self.num_bc_heads = ngroups
        if self.nheads % ngroups:
            raise ValueError(f"ngroups ({ngroups}) must divide the head count ({self.nheads})")
        self.mimo_rank = mimo_rank if is_mimo else 1
        if rope_fraction not in (0.5, 1.0):
            raise ValueError("rope_fraction must be 0.5 or 1.0")
        rotated = int(d_state * rope_fraction)
        rotated -= rotated % 2
        self.num_rope_angles = rotated // 2
        if self.num_rope_angles <= 0:
            raise ValueError("d_state leaves no rotary pairs")
        bc = d_state * self.num_bc_heads * self.mimo_rank
        self.split_sizes = [self.d_inner, self.d_inner, bc, bc, self.nheads, self.nheads,
                            self.nheads, self.num_rope_angles]
        self.in_proj = nn.Linear(d_model, sum(self.split_sizes), bias=False)
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False)
        self.dt_bias = nn.Parameter(torch.zeros(self.nheads))
        self.D = nn.Parameter(torch.ones(self.nheads))
        self.B_bias = nn.Parameter(torch.ones(self.nheads, self.mimo_rank, d_state))
        self.C_bias = nn.Parameter(torch.ones(self.nheads, self.mimo_rank, d_state))
        self.B_norm = RMSNorm(d_state, eps=1e-5)
        self.C_norm = RMSNorm(d_state, eps=1e-5)
        if is_mimo:
            shape = (self.nheads, self.mimo_rank, headdim)
            self.mimo_x = nn.Parameter(torch.ones(*shape) / self.mimo_rank)
            self.mimo_z = nn.Parameter(torch.ones(*shape))
            self.mimo_o = nn.Parameter(torch.ones(*shape) / self.mimo_rank)

    def forward(self, u: torch.Tensor) -> torch.Tensor:
        b, seqlen, _ = u.shape
        if self.B_norm.eps != self.C_norm.eps:
            raise ValueError("the front-end kernel takes one eps for B_norm and C_norm")
        proj = F.linear(u, self.in_proj.weight)
        proj = proj.to(torch.float32).contiguous()
        mimo = self.is_mimo
        y = _mixer_scan_op(
            proj, _f32(self.dt_bias), _f32(self.B_norm.weight), _f32(self.C_norm.weight),
            _f32(self.B_bias), _f32(self.C_bias), _f32(self.D),
            _f32(self.mimo_x) if mimo else None, _f32(self.mimo_z) if mimo else None,
            _f32(self.mimo_o) if mimo else None, self.nheads, self.headdim, self.d_state,
            self.mimo_rank, self.num_bc_heads, self.num_rope_angles, float(self.A_floor),
            float(self.B_norm.eps))
        y = y.reshape(b, seqlen, self.nheads * self.headdim)
        return self.out_proj(y.to(u.dtype))

"""Seeded synthetic inputs for the benchmark configurations of the scan path.

Each builder returns a dict of float32 numpy arrays in the layouts of the
C ABI (include/arm_scan_hip.h), drawn from numpy's PCG64 generator with a
fixed seed, so the same inputs can be handed to the HIP kernels and to the CPU
oracle. The distributions are the ones the configurations name:

  m1_op      Mamba-1 selective_scan: u ~ N(0,1); delta = softplus(0.5 N(0,1) - 4)
             (passed with delta_softplus off); A = -[1..N] per channel; B, C ~ N(0,1)
             shared by all channels (groups = 1); D ~ N(0,1); z ~ N(0,1).
  m1_layer   the bench step (one Mamba-130M prefill layer's scan): m1_op with a raw
             delta 0.5 N(0,1) - 4 and delta_bias ~ U(-0.5, 0.5), softplus in the scan.
  m3_siso    Mamba-3 SISO: dt = softplus(N(0,1) - 4); trap ~ N(0,1) (pre-sigmoid);
             A_h = -exp(N(0, 0.5)); adt = A_h dt; theta = cumsum_L(U(-pi, pi) dt) per
             rotation pair (float64), cos/sin float32; q, k ~ N(0,1)/sqrt(dqk) per head
             (groups = heads); v ~ N(0,1); zero q/k biases.
  m3_mimo    as m3_siso with rank-r q, k (b, l, r, heads, dqk), psi ~ N(0,1),
             zeta = 1, phi ~ N(0,1)/2.
  ss2d       four-direction 2D scan over an H x W grid: u, z ~ N(0,1); delta, A, D
             as m1_op; one B and one C per direction, (4, b, n, H, W).
"""

import numpy as np

F32 = np.float32


def _softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def m1_op(batch=1, dim=1536, length=2048, state=16, seed=0, z=True, D=True):
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((batch, dim, length), dtype=F32)
    delta = _softplus(rng.standard_normal((batch, dim, length), dtype=F32) * F32(0.5)
                      - F32(4.0)).astype(F32)
    A = np.broadcast_to(-np.arange(1, state + 1, dtype=F32), (dim, state)).copy()
    B = rng.standard_normal((batch, 1, state, length), dtype=F32)
    C = rng.standard_normal((batch, 1, state, length), dtype=F32)
    out = dict(u=u, delta=delta, A=A, B=B, C=C)
    out["D"] = rng.standard_normal(dim, dtype=F32) if D else None
    out["z"] = rng.standard_normal((batch, dim, length), dtype=F32) if z else None
    return out


def m1_layer(batch=8, dim=1536, length=2048, state=16, seed=0):
    """One Mamba-130M prefill layer's scan (config 2's scan shape, the bench step):
    m1_op's u, A, B, C, D, z, with delta the raw dt_proj output 0.5 N(0,1) - 4 and a
    delta_bias ~ U(-0.5, 0.5), to be scanned with delta_softplus on, as the Hugging
    Face mixer calls it (modeling_mamba.py: softplus inside the scan)."""
    x = m1_op(batch=batch, dim=dim, length=length, state=state, seed=seed)
    rng = np.random.default_rng(seed + 100)
    x["delta"] = (rng.standard_normal(x["u"].shape, dtype=F32) * F32(0.5) - F32(4.0))
    x["delta_bias"] = rng.uniform(-0.5, 0.5, dim).astype(F32)
    return x


def _m3_common(rng, batch, length, heads, dqk):
    dt = _softplus(rng.standard_normal((batch, heads, length)) - 4.0)
    trap = rng.standard_normal((batch, heads, length))
    A = -np.exp(rng.normal(0.0, 0.5, heads))
    adt = A[None, :, None] * dt
    dtheta = rng.uniform(-np.pi, np.pi, (batch, length, heads, dqk // 2)) \
        * dt.transpose(0, 2, 1)[..., None]
    theta = np.cumsum(dtheta, axis=1)
    return dict(adt=adt.astype(F32), dt=dt.astype(F32), trap=trap.astype(F32),
                cos=np.cos(theta).astype(F32), sin=np.sin(theta).astype(F32))


def m3_siso(batch=4, length=4096, heads=24, dv=64, dqk=128, seed=0):
    rng = np.random.default_rng(seed)
    x = _m3_common(rng, batch, length, heads, dqk)
    s = F32(1.0 / np.sqrt(dqk))
    x["q"] = rng.standard_normal((batch, length, heads, dqk), dtype=F32) * s
    x["k"] = rng.standard_normal((batch, length, heads, dqk), dtype=F32) * s
    x["v"] = rng.standard_normal((batch, length, heads, dv), dtype=F32)
    x["q_bias"] = np.zeros((heads, dqk), F32)
    x["k_bias"] = np.zeros((heads, dqk), F32)
    return x


def m3_mimo(batch=4, length=4096, heads=24, dv=64, dqk=128, rank=4, seed=0):
    rng = np.random.default_rng(seed)
    x = _m3_common(rng, batch, length, heads, dqk)
    s = F32(1.0 / np.sqrt(dqk))
    x["q"] = rng.standard_normal((batch, length, rank, heads, dqk), dtype=F32) * s
    x["k"] = rng.standard_normal((batch, length, rank, heads, dqk), dtype=F32) * s
    x["v"] = rng.standard_normal((batch, length, heads, dv), dtype=F32)
    x["q_bias"] = np.zeros((heads, rank, dqk), F32)
    x["k_bias"] = np.zeros((heads, rank, dqk), F32)
    x["psi"] = rng.standard_normal((heads, rank, dv), dtype=F32)
    x["zeta"] = np.ones((heads, rank, dv), F32)
    x["phi"] = rng.standard_normal((heads, rank, dv), dtype=F32) * F32(0.5)
    return x


def m3_with_angles(x, r=None, seed=0):
    """`x` (from m3_siso / m3_mimo) with raw rotary angles (b, l, h, r) in place of
    cos/sin, for the fused pre-pass: angle ~ N(0,1), so tanh(angle) * pi * dt is a
    spread of increments within (-pi, pi) * dt. r defaults to dqk/4, the published
    rotation fraction of 0.5 (python/arm_scan/mamba3.py:49-52)."""
    b, length, h = x["v"].shape[:3]
    r = x["q"].shape[-1] // 4 if r is None else r
    rng = np.random.default_rng(seed)
    y = {k: v for k, v in x.items() if k not in ("cos", "sin")}
    y["angles"] = rng.standard_normal((b, length, h, r), dtype=F32)
    return y


def ss2d(batch=16, dim=192, height=64, width=64, state=16, seed=0):
    rng = np.random.default_rng(seed)
    shape = (batch, dim, height, width)
    u = rng.standard_normal(shape, dtype=F32)
    delta = _softplus(rng.standard_normal(shape, dtype=F32) * F32(0.5) - F32(4.0)).astype(F32)
    A = np.broadcast_to(-np.arange(1, state + 1, dtype=F32), (dim, state)).copy()
    B4 = rng.standard_normal((4, batch, state, height, width), dtype=F32)
    C4 = rng.standard_normal((4, batch, state, height, width), dtype=F32)
    D = rng.standard_normal(dim, dtype=F32)
    z = rng.standard_normal(shape, dtype=F32)
    return dict(u=u, delta=delta, A=A, B4=B4, C4=C4, D=D, z=z)


def m1_bytes(batch, dim, length, state, groups=1, z=True, D=True, bias=False,
             last_state=True):
    """Algorithmic HBM bytes of one Mamba-1 scan: every input read once, every
    output written once, fp32."""
    row = batch * dim * length
    n = 4 * (row * (3 + (1 if z else 0))                      # u, delta, out (+ z)
             + 2 * batch * groups * state * length             # B, C
             + dim * state                                     # A
             + dim * ((1 if D else 0) + (1 if bias else 0))    # D, delta_bias
             + (batch * dim * state if last_state else 0))     # last_state
    return n


def m3_bytes(x, want_state=True):
    """Algorithmic HBM bytes of one Mamba-3 scan over the inputs `x` (SISO or
    MIMO, from m3_siso / m3_mimo): every input read once, the output (b, l, h, dv)
    and the final states written once, fp32."""
    b, length, h, dv = x["v"].shape
    dqk = x["q"].shape[-1]
    mimo = "psi" in x
    n = sum(v.nbytes for v in x.values())
    n += 4 * b * length * h * dv                       # out
    if want_state:
        n += 4 * b * h * dv * dqk                      # last_state
        if not mimo:
            n += 4 * b * h * dqk                       # last_bx
    return n


def ss2d_bytes(x, merge="sum", last_state=True):
    """Algorithmic HBM bytes of one four-direction SS2D scan over the inputs `x`
    (from ss2d): every input read once, the output and final states written once."""
    b, d, hh, ww = x["u"].shape
    n = sum(v.nbytes for v in x.values())
    n += 4 * b * d * hh * ww * (4 if merge == "none" else 1)
    if last_state:
        n += 4 * 4 * b * d * x["A"].shape[1]
    return n

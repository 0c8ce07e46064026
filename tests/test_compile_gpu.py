"""torch.compile composability of every arm_scan custom op, the check the reference
makes for its Mamba-3 op (tests/check_mamba3_op.py:76-95): the public call traced with
fullgraph=True (a graph break fails the test) through the ops' fake kernels and
bit-equal to eager. The backend is aot_eager: it traces through AOT autograd and
generates no code, so the only kernels that run are the ops' own HIP kernels. Plus
torch.library.opcheck's schema, fake-tensor and AOT-dispatch checks on each op."""

import pytest

from util import case

pytestmark = pytest.mark.gpu


def _rand(*shape, scale=1.0, seed=0):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed + sum(shape))
    return torch.randn(*shape, device="cuda", generator=g) * scale


def _cases():
    """(name, public call, the op it lowers to, that op's arguments)."""
    import torch
    import torch.nn.functional as F

    import armhackathon_amd as arm_scan
    from armhackathon_amd import mamba3, mamba3_noncausal, op  # noqa: F401 (registers ops)
    from armhackathon_amd.mamba3_block import Mamba3Mixer

    b, d, L, n = 2, 32, 96, 8
    u, dl, z = _rand(b, d, L), F.softplus(_rand(b, d, L, seed=1) - 3), _rand(b, d, L, seed=2)
    A = -torch.exp(_rand(d, n, scale=0.5, seed=3))
    B, C, D = _rand(b, n, L, seed=4), _rand(b, n, L, seed=5), _rand(d, seed=6)
    zt = _rand(b, L, 2 * d, seed=7)[..., d:].transpose(1, 2)  # a time-major view
    st = _rand(b, d, n, seed=8)
    x1, dt1, z1 = _rand(b, d, seed=9), _rand(b, d, seed=10), _rand(b, d, seed=11)
    B1, C1 = _rand(b, n, seed=12), _rand(b, n, seed=13)

    h, dv, dqk, Lm = 2, 16, 32, 40
    q, k = _rand(b, Lm, 1, dqk, scale=0.2, seed=14), _rand(b, Lm, 1, dqk, scale=0.2, seed=15)
    v, zz = _rand(b, Lm, h, dv, seed=16), _rand(b, Lm, h, dv, seed=17)
    dt = F.softplus(_rand(b, h, Lm, seed=18) - 3)
    adt, trap = -dt * 0.5, _rand(b, h, Lm, seed=19)
    qb, kb, Dm = _rand(h, dqk, scale=0.1, seed=20), _rand(h, dqk, scale=0.1, seed=21), _rand(h)
    ang = _rand(b, Lm, h, 8, seed=22)
    cos, sin = arm_scan.angles_to_cos_sin(ang, dt, dqk // 2)
    proj = _rand(b, Lm, 2 * h * dv + 8, seed=23)
    xv = proj[..., h * dv:2 * h * dv].view(b, Lm, h, dv)
    zv = proj[..., :h * dv].view(b, Lm, h, dv)
    angv = proj[..., -8:].unsqueeze(-2).expand(-1, -1, h, -1)

    xc = _rand(b, L, 2 * d, seed=25)[..., :d].transpose(1, 2)  # the mixer's conv input
    wc, bc = _rand(d, 4, seed=26), _rand(d, seed=27)
    cst = _rand(b, d, 4, seed=28)

    def conv_step():
        s = cst.clone()
        y = arm_scan.causal_conv1d_update(xc[..., 0], s, wc, bc, activation="silu")
        return y, s

    mixer = Mamba3Mixer(d_model=32, d_state=32, headdim=16).cuda()
    uin = _rand(b, Lm, 32, seed=24)

    ops = torch.ops.arm_scan
    m3 = (q, k, v, adt, dt, trap, qb, kb)
    return [
        ("selective_scan",
         lambda: arm_scan.selective_scan(u, dl, A, B, C, D=D, z=z),
         ops.selective_scan.default,
         (u, dl, A, B.unsqueeze(1), C.unsqueeze(1), D, z, None, None, False, False)),
        ("selective_scan_time_major",
         lambda: arm_scan.selective_scan_time_major(u, dl, A, B, C, D=D, z=zt),
         None, None),
        ("selective_scan_bidirectional",
         lambda: arm_scan.selective_scan_bidirectional(u, dl, A, B, C, D=D, z=z),
         None, None),
        ("selective_state_update",
         lambda: arm_scan.selective_state_update(st.clone(), x1, dt1, A, B1, C1, D=D, z=z1,
                                                 dt_softplus=True),
         None, None),
        ("mamba3_scan (cos/sin)",
         lambda: arm_scan.mamba3_scan(*m3, cos=cos, sin=sin, D=Dm, z=zz),
         ops.mamba3_scan.default, (*m3, cos, sin, Dm, zz, False)),
        ("mamba3_scan (fused angles)",
         lambda: arm_scan.mamba3_scan(*m3, angles=ang, D=Dm, z=zz),
         ops.mamba3_scan_angles.default, (*m3, ang, Dm, zz)),
        ("mamba3_scan (views)",
         lambda: arm_scan.mamba3_scan(q, k, xv, adt, dt, trap, qb, kb, angles=angv, D=Dm,
                                      z=zv),
         None, None),
        ("noncausal_scan",
         lambda: arm_scan.noncausal_scan(*m3, cos=cos, sin=sin, D=Dm, z=zz),
         ops.mamba3_noncausal.default, (*m3, cos, sin, Dm, zz)),
        ("Mamba3Mixer", lambda: mixer(uin), None, None),
        ("causal_conv1d",
         lambda: arm_scan.causal_conv1d(xc, wc, bc, activation="silu"),
         ops.causal_conv1d.default, (xc, wc, bc, True, True)),
        ("causal_conv1d_update", conv_step, None, None),
    ]


@pytest.mark.parametrize("idx", range(11))
def test_compile_fullgraph(idx):
    import torch

    name, fn, op, args = _cases()[idx]
    case(f"torch.compile fullgraph: {name}")
    torch._dynamo.reset()
    with torch.no_grad():
        eager = fn()
        compiled = torch.compile(fn, fullgraph=True, backend="aot_eager")()
    eager = eager if isinstance(eager, tuple) else (eager,)
    compiled = compiled if isinstance(compiled, tuple) else (compiled,)
    for e, c in zip(eager, compiled):
        assert e.shape == c.shape and torch.equal(e, c), name
    if op is not None:
        torch.library.opcheck(op, args, test_utils=("test_schema", "test_faketensor",
                                                    "test_aot_dispatch_dynamic"))

"""Write the Mamba-3 mixer fixtures (run once, in the build container only).

The reference's mixer, apps/mamba3_lm/block.py (`Mamba3Mixer.forward`,
:146-199), decides the projection's column split [z | x | B | C | dd_dt | dd_A |
trap | angles] (:113-118), the Q <- C / K <- B mapping and the casts around the
scan. Its own block-level captures (block_io_00/01 in its
tests/golden/mamba3/manifest.json) are not in its tree, and its model-level capture
needs the published checkpoint, so nothing else pins those choices.

This script imports that one file by path (never the reference's package, which
would pull in its loader) with its module-level `import arm_scan` bound to a stand-in
whose `mamba3_scan` / `mamba3_mimo_scan` are the oracle's float64 scans with the
float64 angle pre-pass (oracle.angles_to_cos_sin). It runs the reference's mixer in
float64 on seeded weights and inputs and writes the inputs, the weights and the
output as fixtures:

  mamba3_block/mixer_siso.npz   d_model 64, d_state 32, 8 heads of 16, B2 L48
  mamba3_block/mixer_mimo.npz   the same with MIMO rank 2, B1 L40

The reference never travels to the GPU box: the tests read these .npz files only.
`block.py` casts dd_A and the angles to float32 before use (:167, :175), so the
fixture carries that rounding (about 1e-7 relative).
"""

import importlib.util
import json
import sys
import types
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
BLOCK = Path("/root/reference/apps/mamba3_lm/block.py")

CASES = [
    ("mixer_siso", dict(d_model=64, d_state=32, headdim=16), 2, 48, 11),
    ("mixer_mimo", dict(d_model=64, d_state=32, headdim=16, is_mimo=True, mimo_rank=2), 1,
     40, 12),
]


def _stand_in():
    """An `arm_scan` module whose scans are the oracle's float64 ones."""
    import torch

    sys.path.insert(0, str(ROOT))
    import oracle

    def f64(t):
        return None if t is None else t.detach().cpu().double().numpy()

    def run(q, k, v, adt, dt, trap, q_bias, k_bias, angles, D, z, psi=None, zeta=None,
            phi=None):
        cos, sin = oracle.angles_to_cos_sin(f64(angles), f64(dt), q.shape[-1] // 2)
        out = oracle.mamba3_scan(f64(q), f64(k), f64(v), f64(adt), f64(dt), f64(trap),
                                 f64(q_bias), f64(k_bias), cos, sin, D=f64(D), z=f64(z),
                                 psi=f64(psi), zeta=f64(zeta), phi=f64(phi),
                                 dtype=np.float64)
        return torch.from_numpy(np.ascontiguousarray(out.transpose(0, 2, 1, 3)))

    def mamba3_scan(q, k, v, adt, dt, trap, q_bias, k_bias, angles=None, D=None, z=None,
                    reverse=False, cos=None, sin=None):
        assert angles is not None and not reverse and cos is None
        if q.dim() == 3:
            q, k = q.unsqueeze(2), k.unsqueeze(2)
        return run(q, k, v, adt, dt, trap, q_bias, k_bias, angles, D, z)

    def mamba3_mimo_scan(q, k, v, adt, dt, trap, q_bias, k_bias, psi, zeta, phi,
                         angles=None, D=None, z=None, reverse=False, cos=None, sin=None):
        assert angles is not None and not reverse and cos is None
        if q.dim() == 4:
            q, k = q.unsqueeze(3), k.unsqueeze(3)
        return run(q, k, v, adt, dt, trap, q_bias, k_bias, angles, D, z, psi, zeta, phi)

    mod = types.ModuleType("arm_scan")
    mod.mamba3_scan = mamba3_scan
    mod.mamba3_mimo_scan = mamba3_mimo_scan
    return mod


def _seeded(m, seed):
    """Weights away from their init values so every parameter matters."""
    import torch

    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, t in m.named_parameters():
            if name.endswith("proj.weight"):
                t.copy_(torch.randn(t.shape, generator=g, dtype=t.dtype) / t.shape[1] ** 0.5)
            elif name == "dt_bias":
                t.copy_(torch.rand(t.shape, generator=g, dtype=t.dtype) * 2.0 - 4.0)
            else:
                t.copy_(1.0 + 0.3 * torch.randn(t.shape, generator=g, dtype=t.dtype))


def main():
    import torch

    if not BLOCK.is_file():
        print(f"{BLOCK} not present; nothing to write")
        return 1
    sys.modules["arm_scan"] = _stand_in()
    spec = importlib.util.spec_from_file_location("ref_mamba3_block", BLOCK)
    block = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(block)
    out_dir = HERE / "mamba3_block"
    out_dir.mkdir(exist_ok=True)
    for name, kw, b, L, seed in CASES:
        m = block.Mamba3Mixer(**kw).double()
        _seeded(m, seed)
        u = np.random.default_rng(seed).standard_normal((b, L, kw["d_model"]))
        with torch.no_grad():
            y = m(torch.from_numpy(u)).numpy()
        params = {f"param:{k}": v.detach().numpy() for k, v in m.state_dict().items()}
        meta = dict(kwargs=kw, batch=b, len=L, seed=seed, nheads=m.nheads,
                    headdim=m.headdim, d_state=m.d_state, mimo_rank=m.mimo_rank,
                    ngroups=m.num_bc_heads, num_rope_angles=m.num_rope_angles,
                    A_floor=m.A_floor, eps=m.B_norm.eps,
                    source="apps/mamba3_lm/block.py Mamba3Mixer.forward, float64, "
                           "scans = oracle float64")
        np.savez_compressed(out_dir / f"{name}.npz", u=u, y=y,
                            meta_json=np.frombuffer(json.dumps(meta).encode(), np.uint8),
                            **params)
        print(f"{name}: u {u.shape} -> y {y.shape}, |y|max {np.abs(y).max():.3f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())

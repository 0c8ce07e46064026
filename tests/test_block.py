"""The Mamba-3 mixer's host side on the CPU: the checkpoint's parameter names and
shapes (apps/mamba3_lm/block.py:24-31 lists them for the published SISO model), and
the oracle's front-end pieces against closed forms."""

import numpy as np
import pytest

from oracle import naive


def test_mixer_parameters_match_the_checkpoint():
    torch = pytest.importorskip("torch")
    from armhackathon_amd.mamba3_block import Mamba3Mixer

    m = Mamba3Mixer()
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert shapes == {
        "in_proj.weight": (3432, 768), "out_proj.weight": (768, 1536), "dt_bias": (24,),
        "D": (24,), "B_bias": (24, 1, 128), "C_bias": (24, 1, 128),
        "B_norm.weight": (128,), "C_norm.weight": (128,)}
    assert m.split_sizes == [1536, 1536, 128, 128, 24, 24, 24, 32]
    mm = Mamba3Mixer(d_model=64, d_state=32, headdim=16, is_mimo=True, mimo_rank=4)
    s = {k: tuple(v.shape) for k, v in mm.state_dict().items()}
    assert s["mimo_x"] == s["mimo_z"] == s["mimo_o"] == (8, 4, 16)
    assert s["B_bias"] == (8, 4, 32) and mm.split_sizes[2] == 4 * 32
    assert Mamba3Mixer(d_state=128, rope_fraction=1.0).num_rope_angles == 64
    with pytest.raises(ValueError):
        Mamba3Mixer(rope_fraction=0.25)
    del torch


def test_heavy_tail_closed_forms():
    """f(x) = 1 + x (x >= 0), 1 / (1 - x) (x < 0): values, continuity and slope 1 at 0,
    positive everywhere (so -f is a decay)."""
    x = np.array([0.0, 2.0, -1.0, -3.0, 1e-9, -1e-9])
    np.testing.assert_allclose(naive.heavy_tail(x), [1.0, 3.0, 0.5, 0.25, 1.0, 1.0],
                               rtol=1e-12, atol=1e-8)
    h = 1e-6
    slope = (naive.heavy_tail(h) - naive.heavy_tail(-h)) / (2 * h)
    assert abs(slope - 1.0) < 1e-6
    grid = np.linspace(-50, 50, 1001)
    assert (naive.heavy_tail(grid) > 0).all()
    assert (np.diff(naive.heavy_tail(grid)) > 0).all()


def test_rms_norm_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 7, 32))
    y = naive.rms_norm(x, np.ones(32), 0.0)
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1.0, rtol=1e-12)
    np.testing.assert_allclose(naive.rms_norm(3.5 * x, np.ones(32), 0.0), y, rtol=1e-12)
    w = rng.standard_normal(32)
    np.testing.assert_allclose(naive.rms_norm(x, w, 0.0), y * w, rtol=1e-12)
    # eps inside the square root: a zero row stays finite (and zero)
    assert np.all(naive.rms_norm(np.zeros((1, 32)), w, 1e-5) == 0.0)


def test_frontend_rejects_short_rows():
    """The host check runs before any launch (fake, never dereferenced pointers)."""
    from armhackathon_amd import _ffi

    with pytest.raises(_ffi.ArmScanError) as e:
        _ffi.block_frontend_raw(16, 1, 4, 10, 2, 4, 4, 1, 1, 2, 16, 1e-4, 16, 16, 1e-5, 16, 16,
                                16, 16, 16)
    assert e.value.code == 2 and "row_stride" in str(e.value)


def test_grid_views_round_trip():
    """grid -> (row-major, column-major) views -> grid is exact, and the two orderings
    differ (a transpose that silently did nothing would pass the scan checks)."""
    torch = pytest.importorskip("torch")
    from armhackathon_amd.ss2d_mamba3 import grid_to_views_time_major, views_to_grid_time_major

    g = torch.arange(2 * 3 * 5 * 4, dtype=torch.float32).reshape(2, 3, 5, 4)
    views = grid_to_views_time_major(g)
    assert views.shape == (4, 15, 4)
    rows, cols = views_to_grid_time_major(views[:2], views[2:], 3, 5)
    assert torch.equal(rows, g) and torch.equal(cols, g)
    assert not torch.equal(views[:2], views[2:])


def test_use_arm_scan_swaps_and_restores():
    """use_arm_scan (python/arm_scan/ss2d.py:170-202): every block exposing scan_pair_fn
    or scan_fn gets this package's function, the count is returned, and enable=False
    puts the originals back."""
    torch = pytest.importorskip("torch")
    from armhackathon_amd import ss2d

    class Block(torch.nn.Module):
        def __init__(self, attr):
            super().__init__()
            setattr(self, attr, lambda *a, **k: "original")

    root = torch.nn.Sequential(Block("scan_pair_fn"), Block("scan_fn"), torch.nn.Linear(2, 2))
    assert ss2d.use_arm_scan(root) == 2
    assert root[0].scan_pair_fn is ss2d.scan_pair_arm and root[1].scan_fn is ss2d.scan_fn_arm
    assert ss2d.use_arm_scan(root) == 2  # idempotent: the originals stay remembered
    assert ss2d.use_arm_scan(root, enable=False) == 2
    assert root[0].scan_pair_fn() == "original" and root[1].scan_fn() == "original"
    assert not hasattr(root[0], "_arm_scan_saved_scan_pair_fn")


def test_causal_conv1d_oracle_closed_forms():
    """The oracle's causal convolution: an impulse at t returns the taps in order
    (w[d, K-1] at t, w[d, K-2] at t+1, ...), nothing before t (causality); width 1 is a
    per-channel scale; linear in x."""
    rng = np.random.default_rng(0)
    w = rng.standard_normal((3, 4))
    x = np.zeros((1, 3, 10))
    x[0, :, 5] = 1.0
    y = naive.causal_conv1d(x, w)
    assert np.all(y[0, :, :5] == 0.0)
    np.testing.assert_allclose(y[0, :, 5:9], w[:, ::-1], rtol=0, atol=0)
    x2 = rng.standard_normal((2, 3, 10))
    np.testing.assert_allclose(naive.causal_conv1d(x2, w[:, :1]), x2 * w[None, :, :1],
                               rtol=1e-15)
    x3 = rng.standard_normal((2, 3, 10))
    np.testing.assert_allclose(naive.causal_conv1d(2 * x2 - x3, w),
                               2 * naive.causal_conv1d(x2, w) - naive.causal_conv1d(x3, w),
                               rtol=1e-12, atol=1e-12)


def _mixer_fixture(golden_dir, name):
    import json

    z = np.load(golden_dir / "mamba3_block" / f"{name}.npz")
    meta = json.loads(bytes(z["meta_json"]).decode())
    params = {k[len("param:"):].replace(".weight", ""): z[k]
              for k in z.files if k.startswith("param:")}
    return z["u"], z["y"], params, meta


def _oracle_mixer(u, p, meta):
    return naive.m3_mixer(u, p, meta["nheads"], meta["headdim"], meta["d_state"],
                          meta["mimo_rank"], meta["ngroups"], meta["num_rope_angles"],
                          meta["A_floor"], meta["eps"])


def _swap_rows(w, a, b, n):
    """in_proj with its column blocks [a, a+n) and [b, b+n) exchanged."""
    w = w.copy()
    w[[*range(a, a + n), *range(b, b + n)]] = w[[*range(b, b + n), *range(a, a + n)]]
    return w


@pytest.mark.parametrize("name", ["mixer_siso", "mixer_mimo"])
def test_oracle_mixer_matches_reference_block(golden_dir, name):
    """naive.m3_mixer (the oracle's transcription of block.py:146-199) against the
    reference's own Mamba3Mixer.forward, captured with the oracle's float64 scans by
    tests/golden/gen_mixer_fixtures.py. That pins the column split and the
    Q <- C / K <- B mapping; planted mistakes in either must fail the same gate."""
    u, y, p, meta = _mixer_fixture(golden_dir, name)
    got = _oracle_mixer(u, p, meta)
    err = np.abs(got - y).max() / np.abs(y).max()
    assert err < 1e-6, err  # the reference casts dd_A and the angles to float32
    di = meta["nheads"] * meta["headdim"]
    bc = meta["d_state"] * meta["mimo_rank"] * meta["ngroups"]
    # Q <- B, K <- C instead: B and C column blocks (and their norms and biases) swapped
    q = dict(p, in_proj=_swap_rows(p["in_proj"], 2 * di, 2 * di + bc, bc),
             B_norm=p["C_norm"], C_norm=p["B_norm"], B_bias=p["C_bias"], C_bias=p["B_bias"])
    assert np.abs(_oracle_mixer(u, q, meta) - y).max() / np.abs(y).max() > 1e-2
    # x and z split the other way round
    q = dict(p, in_proj=_swap_rows(p["in_proj"], 0, di, di))
    assert np.abs(_oracle_mixer(u, q, meta) - y).max() / np.abs(y).max() > 1e-2

"""Shared helpers of the GPU parity tests."""

import numpy as np


def rel_err(got, ref):
    """Tensor-scale relative error max|got - ref| / max|ref|, the reference's
    own convention (golden.rs:103-110, check_mamba3_op.py:63-64)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def dev(x, device="cuda"):
    """numpy dict/array -> torch device tensors (None passes through)."""
    import torch

    if isinstance(x, dict):
        return {k: dev(v, device) for k, v in x.items()}
    if x is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def host(t):
    return t.detach().cpu().numpy()


def case(msg):
    """Print (and flush) which case a GPU step is on, so a failing run names it."""
    print(f"[case] {msg}", flush=True)
